"""TurboQuant codec on MI355X — drop-in for VRAMancer's ``core/turboquant_cuda.py``.

``CUDATurboQuantOps`` keeps the reference's static-method signatures
(core/turboquant_cuda.py:117-255) and result dictionaries (radius [N] fp16,
angles as a per-level list of uint8 views, qjl_signs [N, qjl_dim] uint8,
qjl_norms [N, 1] fp16), but computes them with the gfx950 kernels of
libvrm_paged.so.  The codes follow the reference's CPU path
(core/kv_quantizer.py:391-417), not its CUDA kernel: the residual is formed
from the fp32 radius, and ``attention_score_gpu`` uses the rotated query for
both the polar dot product and the QJL correction (the reference's CUDA
wrapper uses the unrotated query, core/turboquant_cuda.py:231-253).
"""
from __future__ import annotations

import math
import threading
from typing import Dict, Tuple

from . import _lib

__all__ = ["CUDATurboQuantOps", "has_cuda_turboquant", "angle_lut", "topk_attend"]

_lut_lock = threading.Lock()
_lut_cache: Dict[Tuple[int, str], "object"] = {}


def has_cuda_turboquant() -> bool:
    """True when the gfx950 library is loadable and a GPU is visible."""
    return _lib.available()


def bin_centres(bits_per_angle: int):
    """Dequantized angle of every bin, computed with the reference's float32
    expression ``lo + (idx.float() + 0.5) * (hi - lo) / n_bins``
    (core/kv_quantizer.py:289-295) for level 0 ([-pi, pi]) and levels >= 1
    ([0, pi/2])."""
    import torch

    n_bins = 1 << bits_per_angle
    idx = torch.arange(n_bins, dtype=torch.uint8)
    out = []
    for lo, hi in ((-math.pi, math.pi), (0.0, math.pi / 2)):
        out.append(lo + (idx.float() + 0.5) * (hi - lo) / n_bins)
    return out


def angle_lut(bits_per_angle: int, device) -> "object":
    """[2, 2, 2^bits] float32 table {level 0, levels >= 1} x {cos, sin} of the
    bin centres.

    The values are PyTorch's CPU cos/sin of the centres, which is what the
    reference's polar decode evaluates (core/kv_quantizer.py:301-302); those
    functions are not the C library's and have no device equivalent, so the
    table is built once on the host and cached per device.
    """
    import torch

    key = (bits_per_angle, str(device))
    with _lut_lock:
        lut = _lut_cache.get(key)
        if lut is None:
            rows = []
            for centres in bin_centres(bits_per_angle):
                rows.append(torch.stack([torch.cos(centres), torch.sin(centres)]))
            lut = torch.stack(rows).contiguous().to(device)
            _lut_cache[key] = lut
    return lut


def _split_levels(angles, padded_dim: int, n_levels: int):
    out = []
    offset = 0
    d = padded_dim
    for _ in range(n_levels):
        half = d // 2
        out.append(angles[:, offset:offset + half])
        offset += half
        d = half
    return out


def level_bins(levels, width: int):
    """The [N, width] uint8 bin array of a per-level list of [N, n_l] bins.

    When the list is the column views of one [N, width] array, as
    ``compress_gpu`` returns it, that array is used as is; any other list is
    concatenated into a new one.
    """
    import torch

    first = levels[0]
    N = first.shape[0] if first.dim() == 2 else -1
    if N > 0 and sum(t.shape[-1] for t in levels) == width:
        ptr = first.data_ptr()
        base = first.untyped_storage().data_ptr()
        for t in levels:
            if (t.dtype != torch.uint8 or t.dim() != 2 or t.shape[0] != N or t.stride() != (width, 1)
                    or t.device != first.device or t.untyped_storage().data_ptr() != base or t.data_ptr() != ptr):
                break
            ptr += t.shape[1]
        else:
            return torch.as_strided(first, (N, width), (width, 1))
    return torch.cat([a.to(torch.uint8) for a in levels], dim=-1).contiguous()


class CUDATurboQuantOps:
    """Fused gfx950 TurboQuant ops: one kernel launch per compress / decompress."""

    @staticmethod
    def compress_gpu(
        kv,              # [N, head_dim] or [..., head_dim]; float32 / float16 / bfloat16
        head_dim: int,
        padded_dim: int,
        n_levels: int,
        bits_per_angle: int,
        hadamard_signs,  # [padded_dim] +-1
        jl_matrix,       # [qjl_dim, padded_dim]
    ) -> dict:
        import torch

        _lib.require_cuda(kv)
        orig_shape = kv.shape
        flat = kv.reshape(-1, head_dim)
        if flat.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            flat = flat.float()
        flat = flat.contiguous()
        device = flat.device
        signs_f = hadamard_signs.to(device=device, dtype=torch.float32).contiguous()
        jl_f = jl_matrix.to(device=device, dtype=torch.float32).contiguous()
        qjl_dim = jl_f.shape[0]
        if signs_f.shape != (padded_dim,) or jl_f.shape != (qjl_dim, padded_dim):
            raise RuntimeError("hadamard_signs / jl_matrix shapes do not match padded_dim")
        N = flat.shape[0]
        radius = torch.empty(N, dtype=torch.float16, device=device)
        angles = torch.empty((N, padded_dim - 1), dtype=torch.uint8, device=device)
        qjl_signs = torch.empty((N, qjl_dim), dtype=torch.uint8, device=device)
        qjl_norms = torch.empty(N, dtype=torch.float16, device=device)
        lut = angle_lut(bits_per_angle, device)
        rc = _lib.load().vrm_turboquant_compress(
            _lib.ptr(flat), _lib.src_dtype_code(flat.dtype), N, head_dim, padded_dim, n_levels, bits_per_angle,
            qjl_dim, _lib.ptr(signs_f), _lib.ptr(jl_f), _lib.ptr(lut), _lib.ptr(radius), _lib.ptr(angles),
            _lib.ptr(qjl_signs), _lib.ptr(qjl_norms), _lib.stream_of(flat),
        )
        _lib.check(rc, "turboquant compress")
        return {
            "radius": radius,                          # [N] fp16
            "angles": _split_levels(angles, padded_dim, n_levels),
            "qjl_signs": qjl_signs,                    # [N, qjl_dim] uint8
            "qjl_norms": qjl_norms.unsqueeze(-1),      # [N, 1] fp16
            "shape": orig_shape,
        }

    @staticmethod
    def _decode(compressed: dict, head_dim: int, padded_dim: int, n_levels: int, bits_per_angle: int,
                hadamard_signs, rotated: bool):
        import torch

        radius = compressed["radius"].reshape(-1).to(torch.float16).contiguous()
        _lib.require_cuda(radius)
        device = radius.device
        angles = level_bins(compressed["angles"], padded_dim - 1)
        N = radius.shape[0]
        if angles.shape != (N, padded_dim - 1):
            raise RuntimeError(f"angles {tuple(angles.shape)} do not match padded_dim {padded_dim}")
        signs_f = hadamard_signs.to(device=device, dtype=torch.float32).contiguous()
        width = padded_dim if rotated else head_dim
        out = torch.empty((N, width), dtype=torch.float32, device=device)
        lut = angle_lut(bits_per_angle, device)
        rc = _lib.load().vrm_turboquant_decompress(
            _lib.ptr(radius), _lib.ptr(angles), N, head_dim, padded_dim, n_levels, bits_per_angle,
            _lib.ptr(signs_f), _lib.ptr(lut), _lib.ptr(out), 1 if rotated else 0, _lib.stream_of(radius),
        )
        _lib.check(rc, "turboquant decompress")
        return out

    @staticmethod
    def decompress_gpu(
        compressed: dict,
        head_dim: int,
        padded_dim: int,
        n_levels: int,
        bits_per_angle: int,
        hadamard_signs,
    ):
        out = CUDATurboQuantOps._decode(compressed, head_dim, padded_dim, n_levels, bits_per_angle,
                                        hadamard_signs, rotated=False)
        return out.reshape(compressed["shape"])

    @staticmethod
    def polar_keys_gpu(compressed: dict, head_dim: int, padded_dim: int, n_levels: int, bits_per_angle: int,
                       hadamard_signs):
        """Polar reconstruction in the rotated space, [N, padded_dim] float32."""
        return CUDATurboQuantOps._decode(compressed, head_dim, padded_dim, n_levels, bits_per_angle,
                                         hadamard_signs, rotated=True)

    @staticmethod
    def attention_score_gpu(
        q,
        compressed_k: dict,
        head_dim: int,
        padded_dim: int,
        n_levels: int,
        bits_per_angle: int,
        hadamard_signs,
        jl_matrix,
        qjl_dim: int,
        scale: float = 1.0,
    ):
        """[n_queries, N] scores = q_rot . k_polar + QJL correction
        (core/kv_quantizer.py:502-535), times ``scale``, in two kernels:
        query rotation and projection, then one wavefront per key."""
        import torch

        _lib.require_cuda(q)
        device = q.device
        flat_q = q.reshape(-1, head_dim).float().contiguous()
        radius = compressed_k["radius"].reshape(-1).to(torch.float16).contiguous()
        angles = level_bins(compressed_k["angles"], padded_dim - 1)
        qjl_signs = compressed_k["qjl_signs"].to(torch.uint8).contiguous()
        qjl_norms = compressed_k["qjl_norms"].reshape(-1).to(torch.float16).contiguous()
        _lib.require_cuda(flat_q, radius, angles, qjl_signs, qjl_norms)
        M, N = flat_q.shape[0], radius.shape[0]
        if angles.shape != (N, padded_dim - 1) or qjl_signs.shape != (N, qjl_dim) or qjl_norms.shape != (N,):
            raise RuntimeError("compressed key fields do not match padded_dim / qjl_dim")
        signs_f = hadamard_signs.to(device=device, dtype=torch.float32).contiguous()
        jl_f = jl_matrix.to(device=device, dtype=torch.float32).contiguous()
        lib = _lib.load()
        ws_bytes = lib.vrm_turboquant_score_workspace_bytes(M, padded_dim, qjl_dim)
        ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=device)
        scores = torch.empty((M, N), dtype=torch.float32, device=device)
        rc = lib.vrm_turboquant_score(
            _lib.ptr(flat_q), M, _lib.ptr(radius), _lib.ptr(angles), _lib.ptr(qjl_signs), _lib.ptr(qjl_norms), N,
            head_dim, padded_dim, n_levels, bits_per_angle, qjl_dim, _lib.ptr(signs_f), _lib.ptr(jl_f),
            _lib.ptr(angle_lut(bits_per_angle, device)), float(scale), _lib.ptr(ws), ws.numel() * 4,
            _lib.ptr(scores), _lib.stream_of(flat_q),
        )
        _lib.check(rc, "turboquant attention_score")
        return scores


def topk_attend(scores, k: int, values):
    """Renormalised top-k softmax attention: for each row of ``scores`` [M, N]
    the ``k`` largest scores are kept and ``out[m] = softmax(kept) @
    values[kept]`` ([M, D] float32, values [N, D]).  This is the value step of
    the reference's sparse V (core/kv_quantizer.py:537-562,
    core/paged_attention.py:1384-1400); ``k >= N`` is the dense softmax."""
    import torch

    _lib.require_cuda(scores, values)
    scores = scores.float().contiguous()
    values = values.float().contiguous()
    M, N = scores.shape
    if values.dim() != 2 or values.shape[0] != N:
        raise RuntimeError(f"values must be [{N}, D], got {tuple(values.shape)}")
    D = values.shape[1]
    k = max(1, min(int(k), N))
    out = torch.empty((M, D), dtype=torch.float32, device=scores.device)
    lib = _lib.load()
    ws_bytes = lib.vrm_topk_attend_workspace_bytes(M, k)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=scores.device)
    rc = lib.vrm_topk_attend(_lib.ptr(scores), M, N, N, k, _lib.ptr(values), D, D, _lib.ptr(out), D, _lib.ptr(ws),
                             ws.numel(), _lib.stream_of(scores))
    _lib.check(rc, "topk_attend")
    return out
