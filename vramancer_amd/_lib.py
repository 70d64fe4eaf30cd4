"""ctypes binding of libvrm_paged.so (declared in include/vrm_paged.h).

The library is loaded once per process under a lock.  There is no fallback:
if the shared library is missing or a GPU is not present, the public
functions raise ``RuntimeError``.  Arguments are raw device pointers taken
from torch tensors, plus the HIP stream of ``torch.cuda.current_stream()``.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

from .build import LIB_PATH

VRM_ABI_VERSION = 2

VRM_KV_F32 = 0
VRM_KV_F16 = 1
VRM_KV_BF16 = 2
VRM_KV_I8 = 3
VRM_KV_FP8E4M3 = 4
VRM_KV_I8_INLINE = 5
VRM_KV_FP8E4M3_INLINE = 6

# size of the fixed split-K array of vrm_paged_decode_noalloc (VRM_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 64 << 20

VRM_SRC_F32 = 0
VRM_SRC_F16 = 1
VRM_SRC_BF16 = 2

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None

_p = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t
_ll = ctypes.c_longlong

# name -> (restype, argtypes); mirrors include/vrm_paged.h
SIGNATURES = {
    "vrm_abi_version": (_i, []),
    "vrm_last_error": (ctypes.c_char_p, []),
    "vrm_kv_slab_bytes": (_sz, [_i, _i, _i, _i]),
    "vrm_paged_decode_num_splits": (_i, [_i, _i, _i, _i, _i]),
    "vrm_paged_decode_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "vrm_paged_decode": (_i, [_p, _p, _p, _p, _p, _p, _p, _sz] + [_i] * 9 + [_f, _i, _p]),
    "vrm_paged_decode_noalloc": (_i, [_p, _p, _p, _p, _p, _p] + [_i] * 9 + [_f, _i, _p]),
    "vrm_paged_decode_balanced": (_i, [_p] * 7 + [_i] * 9 + [_f, _i, _p]),
    "vrm_paged_decode_balanced_loads": (_i, [_p] * 6 + [_i] * 9 + [_f, _i, _p]),
    "vrm_paged_decode_partitions": (_i, [_p, _p, _p, _p, _p, _p, _sz] + [_i] * 9 + [_f, _i, _p]),
    "vrm_paged_decode_merge": (_i, [_p, _p, _p, _sz] + [_i] * 6 + [_p]),
    "vrm_paged_decode_q4": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _sz] + [_i] * 9 + [_f, _p]),
    "vrm_kv_quant_append": (_i, [_p, _p, _i, _p, _p, _i, _p, _p, _i] + [_i] * 6 + [_p]),
    "vrm_kv_quant_pages": (_i, [_p, _p, _i, _p, _p, _i, _p, _p, _i] + [_i] * 6 + [_p]),
    "vrm_kv_dequant_pages": (_i, [_p, _p, _i, _p, _i, _p] + [_i] * 6 + [_p]),
    "vrm_turboquant_compress": (_i, [_p, _i, _i, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p]),
    "vrm_turboquant_decompress": (_i, [_p, _p, _i, _i, _i, _i, _i, _p, _p, _p, _i, _p]),
    "vrm_tq_slice_bytes": (_sz, [_i, _i, _i]),
    "vrm_tq_slice_bytes_ps": (_sz, [_i, _i, _i, _i]),
    "vrm_tq_quant_append": (_i, [_p, _p, _i, _p, _p, _i, _p] + [_i] * 8 + [_p, _p, _p, _p]),
    "vrm_tq_quant_pages": (_i, [_p, _p, _i, _p, _p, _i, _p] + [_i] * 8 + [_p, _p, _p, _p]),
    "vrm_tq_read_pages": (_i, [_p, _p, _i] + [_i] * 8 + [_p, _p, _p, _p, _p]),
    "vrm_paged_decode_tq": (_i, [_p, _p, _p, _p, _p, _p, _sz] + [_i] * 9 + [_f, _i, _i, _p, _p, _p, _p]),
    "vrm_tq_compress_pool": (_i, [_p, _i, _p, _p, _i, _p] + [_i] * 8 + [_p, _p, _p, _p]),
    "vrm_build_block_table": (_i, [_p, _i, _p, _p, _i, _i, _p, _p, _p]),
    "vrm_kv_write": (_i, [_p, _p, _i, _p, _p, _i, _p] + [_i] * 7 + [_p]),
    "vrm_turboquant_score_workspace_bytes": (_sz, [_i, _i, _i]),
    "vrm_turboquant_score": (_i, [_p, _i, _p, _p, _p, _p] + [_i] * 6 + [_p, _p, _p, _f, _p, _sz, _p, _p]),
    "vrm_topk_attend_workspace_bytes": (_sz, [_i, _i]),
    "vrm_topk_attend": (_i, [_p, _i, _i, _ll, _i, _p, _i, _ll, _p, _ll, _p, _sz, _p]),
    "vrm_paged_decode_lse": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _sz] + [_i] * 9 + [_f, _i, _p]),
    "vrm_paged_decode_tq_lse": (_i, [_p, _p, _p, _p, _p, _p, _p, _sz] + [_i] * 9 + [_f, _i, _i, _p, _p, _p, _i, _p]),
    "vrm_attn_combine": (_i, [_p, _p, _p, _p, _ll, _i, _p, _p, _p]),
    "vrm_pack_bits": (_i, [_p, _ll, _i, _i, _p, _p]),
    "vrm_unpack_bits": (_i, [_p, _ll, _i, _i, _p, _p]),
}


def library_path() -> str:
    return os.environ.get("VRM_LIB_PATH", LIB_PATH)


def load() -> ctypes.CDLL:
    """Loads and type-annotates the shared library (once); raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"libvrm_paged.so not found at {path}; build it with `python -m vramancer_amd.build`"
            )
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.vrm_abi_version()
        if ver != VRM_ABI_VERSION:
            raise RuntimeError(f"libvrm_paged.so ABI {ver} != expected {VRM_ABI_VERSION}")
        _lib = lib
        return lib


def available() -> bool:
    """True when the library loads and a GPU is visible to torch."""
    try:
        load()
    except (OSError, RuntimeError, AttributeError):
        return False
    import torch

    return torch.cuda.is_available()


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().vrm_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_of(t) -> int:
    """Raw handle of the current stream of t's device, the stream torch orders
    t's work on (torch's raw getter: the public Stream object costs about two
    microseconds per call)."""
    import torch

    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        return raw(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def require_cuda(*tensors) -> None:
    """The kernels run on the GPU only; CPU tensors are an error, not a fallback."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "vramancer_amd kernels run on the GPU; got a CPU tensor "
                f"(shape {tuple(t.shape)}, dtype {t.dtype})"
            )
    dev = None
    for t in tensors:
        if t is None:
            continue
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")


_KV_CODES: dict = {}


def kv_dtype_code(dtype) -> int:
    if not _KV_CODES:
        import torch

        _KV_CODES.update({
            torch.float32: VRM_KV_F32,
            torch.float16: VRM_KV_F16,
            torch.bfloat16: VRM_KV_BF16,
            torch.int8: VRM_KV_I8,
            torch.float8_e4m3fn: VRM_KV_FP8E4M3,
        })
    code = _KV_CODES.get(dtype)
    if code is None:
        raise RuntimeError(f"unsupported KV pool dtype {dtype}")
    return code


def src_dtype_code(dtype) -> int:
    import torch

    table = {torch.float32: VRM_SRC_F32, torch.float16: VRM_SRC_F16, torch.bfloat16: VRM_SRC_BF16}
    if dtype not in table:
        raise RuntimeError(f"unsupported K/V source dtype {dtype} (float32, float16, bfloat16)")
    return table[dtype]
