"""TurboQuant KV pages on MI355X: a paged pool of the reference's TurboQuant
codes, written by the GPU quantizer and attended in place by the paged decode.

The reference stores TurboQuant-compressed K/V as Python dicts per (page,
layer, slot) (``write_kv`` + ``flush_compression``, core/paged_attention.py:
568-675; ``compress_page_bulk``, :1420-1496) and attends them with
``compute_attention_turbo`` (:1259-1418), which gathers and decompresses on
the host side per call.  Here the same codes live in a device pool

    tq_pool[P, L, 2, KH, slice]   (uint8, slice = slice_bytes(bits) bytes)

one slice per (page, layer, K/V, kv-head) with the page's tokens: the
padded_dim - 1 angle bins, the fp16 radius and, for K, the QJL sign bits and
the fp16 residual norm.  The codes are those of ``KVCacheCompressor.compress``; the
decode computes compute_attention_turbo's attention (QJL-corrected scores on
the rotated query, dense decompressed values) with query head h reading
kv-head h // (H / KH), the mapping of the paged decode path.

Head_dim 33 .. 128 with the compressor's default QJL rows (padded_dim / 2:
32 at head_dim <= 64, 64 above), 2 to 4 bits per angle and pages of 16 tokens
use the tuned layouts and decode kernel; every other compressor setting
(head_dim 1 .. 256, 1 to 8 bits, QJL rows up to 256) and page size uses the
generic layout and kernels of the same library.
"""
from __future__ import annotations

import functools
import math
from typing import Any, Dict, Optional

from . import _lib
from .paged_attention_cuda import _check_lse, check_outputs, decode_workspace
from .turboquant_cuda import angle_lut

__all__ = [
    "slice_bytes",
    "allocate_pool",
    "quantize_append",
    "quantize_pages",
    "read_pages",
    "paged_attention_decode_turbo",
]

PAGE_SIZE = 16  # default tokens per page (the reference's)


@functools.lru_cache(maxsize=None)
def slice_bytes(bits_per_angle: int, head_dim: int = 128, qjl_dim: int = 64, page_size: int = PAGE_SIZE) -> int:
    """Bytes of one (page, layer, K/V, kv-head) slice for these settings."""
    n = _lib.load().vrm_tq_slice_bytes_ps(head_dim, bits_per_angle, qjl_dim, page_size)
    if n == 0:
        raise RuntimeError(f"TurboQuant pages take head_dim 1 .. 256, 1 .. 8 bits per angle, qjl_dim 1 .. 256 "
                           f"(got {head_dim}, {bits_per_angle}, {qjl_dim}, page {page_size})")
    return int(n)


def _check_compressor(compressor):
    if not (1 <= compressor.head_dim <= 256 and 1 <= compressor.bits_per_angle <= 8
            and 1 <= compressor.qjl_dim <= 256):
        raise RuntimeError("TurboQuant pages need a KVCacheCompressor with head_dim 1 .. 256, 1 .. 8 bits per "
                           f"angle and qjl_dim 1 .. 256 (got {compressor.head_dim}, {compressor.bits_per_angle}, "
                           f"{compressor.qjl_dim})")


def _slice(compressor, page_size: int) -> int:
    return slice_bytes(compressor.bits_per_angle, compressor.head_dim, compressor.qjl_dim, page_size)


def _buffers(compressor, device):
    """Float32 device copies of the compressor's Hadamard signs and JL matrix,
    and the angle table.  The copies are kept on the compressor per device and
    made again when either source tensor is replaced or changed in place, so a
    compressor that stays on the host costs one upload, not two per call."""
    import torch

    src_s, src_j = compressor._hadamard_signs, compressor.jl_matrix
    cache = compressor.__dict__.setdefault("_vrm_device_buffers", {})
    hit = cache.get(device)
    if (hit is None or hit[0] is not src_s or hit[1] is not src_j or hit[2] != (src_s._version, src_j._version)
            or hit[3] != compressor.bits_per_angle):
        dev = torch.device(device)
        follows_current = dev.type == "cuda" and dev.index is None  # not cached: the current device may change
        if follows_current:
            dev = torch.device("cuda", torch.cuda.current_device())
        signs = src_s.to(device=dev, dtype=torch.float32).contiguous()
        jl = src_j.to(device=dev, dtype=torch.float32).contiguous()
        hit = (src_s, src_j, (src_s._version, src_j._version), compressor.bits_per_angle,
               (signs, jl, angle_lut(compressor.bits_per_angle, dev)))
        if not follows_current:
            cache[device] = hit
    return hit[4]


def allocate_pool(num_pages: int, num_layers: int, num_kv_heads: int, compressor, device: Any = "cuda",
                  page_size: int = PAGE_SIZE):
    """Zero-initialised TurboQuant pool for ``compressor``'s settings."""
    import torch

    _check_compressor(compressor)
    return torch.zeros((num_pages, num_layers, 2, num_kv_heads, _slice(compressor, page_size)),
                       dtype=torch.uint8, device=device)


def _pool_dims(tq_pool, compressor, page_size):
    want = _slice(compressor, page_size)
    if tq_pool.dim() != 5 or tq_pool.shape[2] != 2 or tq_pool.shape[4] != want:
        raise RuntimeError(f"tq_pool must be [P, L, 2, KH, {want}] uint8 for page_size {page_size}")
    if not tq_pool.is_contiguous():
        raise RuntimeError("tq_pool must be contiguous (it is written in place)")
    P, L, _, KH, _ = tq_pool.shape
    return P, L, KH


def quantize_append(tq_pool, layer_idx: int, page_ids, slots, key, value, compressor,
                    page_size: int = PAGE_SIZE) -> None:
    """Compresses N new tokens ([N, KH, head_dim] K and V) into their (page,
    slot) of layer ``layer_idx`` (slots from append_token,
    core/paged_attention.py:431-459)."""
    import torch

    _check_compressor(compressor)
    _lib.require_cuda(tq_pool, page_ids, slots, key, value)
    P, L, KH = _pool_dims(tq_pool, compressor, page_size)
    D = compressor.head_dim
    if key.shape != value.shape or key.dim() != 3 or key.shape[1:] != (KH, D):
        raise RuntimeError(f"key/value must be [N, {KH}, {D}], got {tuple(key.shape)} / {tuple(value.shape)}")
    if key.dtype != value.dtype:
        raise RuntimeError("key and value must share a dtype")
    N = key.shape[0]
    page_ids = page_ids.to(torch.int32).contiguous()
    slots = slots.to(torch.int32).contiguous()
    if page_ids.shape != (N,) or slots.shape != (N,):
        raise RuntimeError("page_ids and slots must be [N]")
    key, value = key.contiguous(), value.contiguous()
    signs, jl, lut = _buffers(compressor, tq_pool.device)
    rc = _lib.load().vrm_tq_quant_append(
        _lib.ptr(key), _lib.ptr(value), _lib.src_dtype_code(key.dtype), _lib.ptr(page_ids), _lib.ptr(slots), N,
        _lib.ptr(tq_pool), KH, D, page_size, L, P, int(layer_idx), compressor.bits_per_angle, compressor.qjl_dim,
        _lib.ptr(signs), _lib.ptr(jl), _lib.ptr(lut), _lib.stream_of(tq_pool),
    )
    _lib.check(rc, "tq quantize_append")


def quantize_pages(tq_pool, layer_idx: int, page_ids, key_pages, value_pages, compressor,
                   n_valid: Optional[Any] = None, page_size: int = PAGE_SIZE) -> None:
    """Bulk write of whole pages ([NP, KH, page_size, head_dim] K and V); page
    n holds ``n_valid[n]`` tokens (default page_size), later slots get zero
    codes."""
    import torch

    _check_compressor(compressor)
    _lib.require_cuda(tq_pool, page_ids, key_pages, value_pages, n_valid)
    P, L, KH = _pool_dims(tq_pool, compressor, page_size)
    D = compressor.head_dim
    if key_pages.shape != value_pages.shape or key_pages.dim() != 4 or key_pages.shape[1:] != (KH, page_size, D):
        raise RuntimeError(f"key/value pages must be [NP, {KH}, {page_size}, {D}], got {tuple(key_pages.shape)}")
    if key_pages.dtype != value_pages.dtype:
        raise RuntimeError("key and value pages must share a dtype")
    NP = key_pages.shape[0]
    page_ids = page_ids.to(torch.int32).contiguous()
    if n_valid is None:
        n_valid = torch.full((NP,), page_size, dtype=torch.int32, device=tq_pool.device)
    n_valid = n_valid.to(torch.int32).contiguous()
    if page_ids.shape != (NP,) or n_valid.shape != (NP,):
        raise RuntimeError("page_ids and n_valid must be [NP]")
    key_pages, value_pages = key_pages.contiguous(), value_pages.contiguous()
    signs, jl, lut = _buffers(compressor, tq_pool.device)
    lib = _lib.load()
    step = max(1, (1 << 24) // (KH * page_size))  # rows of one launch stay well inside the grid limits
    for s in range(0, NP, step):
        e = min(NP, s + step)
        rc = lib.vrm_tq_quant_pages(
            _lib.ptr(key_pages[s:e]), _lib.ptr(value_pages[s:e]), _lib.src_dtype_code(key_pages.dtype),
            _lib.ptr(page_ids[s:e]), _lib.ptr(n_valid[s:e]), e - s, _lib.ptr(tq_pool), KH, D, page_size, L, P,
            int(layer_idx), compressor.bits_per_angle, compressor.qjl_dim, _lib.ptr(signs), _lib.ptr(jl),
            _lib.ptr(lut), _lib.stream_of(tq_pool),
        )
        _lib.check(rc, "tq quantize_pages")


def read_pages(tq_pool, layer_idx: int, page_ids, compressor, page_size: int = PAGE_SIZE) -> Dict[str, Any]:
    """Codes of the given pages in the reference's raw format, indexed
    [n, K/V, kv-head, token]: radius fp16, angles uint8 [.., padded_dim - 1]
    level-major, qjl_signs uint8 [.., qjl_dim], qjl_norms fp16 (zero for V)."""
    import torch

    _check_compressor(compressor)
    _lib.require_cuda(tq_pool, page_ids)
    P, L, KH = _pool_dims(tq_pool, compressor, page_size)
    page_ids = page_ids.to(torch.int32).contiguous()
    NP = page_ids.shape[0]
    dev = tq_pool.device
    shape = (NP, 2, KH, page_size)
    radius = torch.empty(shape, dtype=torch.float16, device=dev)
    angles = torch.empty(shape + (compressor._padded_dim - 1,), dtype=torch.uint8, device=dev)
    signs = torch.empty(shape + (compressor.qjl_dim,), dtype=torch.uint8, device=dev)
    norms = torch.empty(shape, dtype=torch.float16, device=dev)
    rc = _lib.load().vrm_tq_read_pages(
        _lib.ptr(tq_pool), _lib.ptr(page_ids), NP, KH, compressor.head_dim, page_size, L, P, int(layer_idx),
        compressor.bits_per_angle, compressor.qjl_dim, _lib.ptr(radius), _lib.ptr(angles), _lib.ptr(signs),
        _lib.ptr(norms), _lib.stream_of(tq_pool),
    )
    _lib.check(rc, "tq read_pages")
    return {"radius": radius, "angles": angles, "qjl_signs": signs, "qjl_norms": norms}


def paged_attention_decode_turbo(query, tq_pool, page_table, context_lens, layer_idx: int, compressor,
                                 scale: Optional[float] = None, out=None, workspace=None, lse=None,
                                 qjl: bool = True, page_size: int = PAGE_SIZE):
    """[B, H, head_dim] float32 attention over TurboQuant pages
    (compute_attention_turbo with dense values, core/paged_attention.py:
    1259-1418, for a batch).

    ``lse`` ([B, H] float32) receives ln sum_t exp(scale score_t); with
    ``qjl=False`` (only together with ``lse``) the scores are q . decompress(k)
    without the QJL correction, as the Hugging Face cache path attends."""
    import torch

    _check_compressor(compressor)
    _lib.require_cuda(query, tq_pool, page_table, context_lens)
    P, L, KH = _pool_dims(tq_pool, compressor, page_size)
    B, H, D = query.shape
    if D != compressor.head_dim:
        raise RuntimeError(f"query head_dim {D} does not match the compressor's {compressor.head_dim}")
    if H % KH:
        raise RuntimeError(f"num_heads {H} is not a multiple of num_kv_heads {KH}")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    query = query.float().contiguous()
    page_table = page_table.to(torch.int32).contiguous()
    context_lens = context_lens.to(torch.int32).contiguous()
    _lib.require_cuda(query, out, workspace, lse)
    check_outputs(query, out, workspace, page_table, context_lens)
    max_pp = page_table.shape[1]
    if out is None:
        out = torch.empty((B, H, D), dtype=torch.float32, device=query.device)
    if workspace is None:
        workspace = decode_workspace(B, H, KH, D, max_pp, query.device, page_size)
    signs, jl, lut = _buffers(compressor, query.device)
    lib = _lib.load()
    ws_bytes = workspace.numel() * workspace.element_size()
    qd = compressor.qjl_dim
    if lse is None:
        if not qjl:
            raise RuntimeError("qjl=False needs an lse output")
        rc = lib.vrm_paged_decode_tq(
            _lib.ptr(query), _lib.ptr(tq_pool), _lib.ptr(page_table), _lib.ptr(context_lens), _lib.ptr(out),
            _lib.ptr(workspace), ws_bytes, B, H, KH, D, page_size, L, P, max_pp, int(layer_idx), float(scale),
            compressor.bits_per_angle, qd, _lib.ptr(signs), _lib.ptr(jl), _lib.ptr(lut), _lib.stream_of(query),
        )
    else:
        _check_lse(lse, B, H, query.device)
        rc = lib.vrm_paged_decode_tq_lse(
            _lib.ptr(query), _lib.ptr(tq_pool), _lib.ptr(page_table), _lib.ptr(context_lens), _lib.ptr(out),
            _lib.ptr(lse), _lib.ptr(workspace), ws_bytes, B, H, KH, D, page_size, L, P, max_pp, int(layer_idx),
            float(scale), compressor.bits_per_angle, qd, _lib.ptr(signs), _lib.ptr(jl), _lib.ptr(lut),
            1 if qjl else 0, _lib.stream_of(query),
        )
    _lib.check(rc, "paged_attention_decode_turbo")
    return out
