"""Restatement of the reference's TurboQuant CPU path (test oracle only).

Follows core/kv_quantizer.py op for op with PyTorch CPU tensors:
  bit packing           :46-105
  buffers               :217-236 (randint signs, then randn JL matrix)
  Hadamard / rotation   :240-258
  polar encode / bins   :262-309
  QJL                   :313-324
  pack / unpack dicts   :337-371
  compress              :391-417 (CPU branch: residual from the fp32 radius)
  decompress            :481-500
  attention_score       :502-535
  sparse_v_attend       :537-562
  bits_per_dim          :564-572
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F


@dataclass
class TQParams:
    head_dim: int
    bits_per_angle: int
    padded_dim: int
    n_levels: int
    qjl_dim: int
    signs: torch.Tensor      # [pd] float32 +-1
    jl_matrix: torch.Tensor  # [qjl, pd] float32


def make_params(head_dim: int, bits_per_angle: int = 3, qjl_dim: Optional[int] = None,
                seed: Optional[int] = None) -> TQParams:
    """Draws the buffers exactly as KVCacheCompressor.__init__; with ``seed``,
    ``torch.manual_seed(seed)`` is called first."""
    if seed is not None:
        torch.manual_seed(seed)
    pd = 1 << math.ceil(math.log2(max(head_dim, 2)))
    n_levels = int(math.log2(pd))
    qjl = qjl_dim or pd // 2
    signs = torch.randint(0, 2, (pd,)).float() * 2 - 1
    jl = torch.randn(qjl, pd) / math.sqrt(qjl)
    return TQParams(head_dim, bits_per_angle, pd, n_levels, qjl, signs, jl)


# -- bit packing --

def pack_bits(signs):
    *batch, M = signs.shape
    pad = (8 - M % 8) % 8
    if pad:
        signs = F.pad(signs, (0, pad))
    packed_M = signs.shape[-1] // 8
    signs = signs.reshape(*batch, packed_M, 8)
    weights = torch.tensor([128, 64, 32, 16, 8, 4, 2, 1], dtype=torch.uint8)
    return (signs * weights).sum(dim=-1).to(torch.uint8)


def unpack_bits(packed, M):
    *batch, packed_M = packed.shape
    bits = packed.unsqueeze(-1).expand(*batch, packed_M, 8)
    shifts = torch.tensor([7, 6, 5, 4, 3, 2, 1, 0], dtype=torch.uint8)
    return ((bits >> shifts) & 1).reshape(*batch, packed_M * 8)[..., :M]


def pack_angles(angles_list, bits_per_angle):
    if not angles_list:
        return torch.tensor([], dtype=torch.uint8)
    flat = torch.cat(angles_list, dim=-1)
    N = flat.shape[0]
    shifts = torch.arange(bits_per_angle - 1, -1, -1, dtype=torch.uint8)
    bits = ((flat.unsqueeze(-1) >> shifts) & 1).reshape(N, -1)
    return pack_bits(bits)


def unpack_angles(packed, N, level_dims, bits_per_angle):
    total_cols = sum(level_dims)
    bits = unpack_bits(packed, total_cols * bits_per_angle)
    shifts = torch.arange(bits_per_angle - 1, -1, -1, dtype=torch.uint8)
    flat = (bits.reshape(N, total_cols, bits_per_angle) * (1 << shifts)).sum(dim=-1).to(torch.uint8)
    out, offset = [], 0
    for d in level_dims:
        out.append(flat[:, offset:offset + d])
        offset += d
    return out


# -- rotation --

def hadamard(x):
    d = x.shape[-1]
    h = 1
    result = x.clone()
    while h < d:
        result = result.view(*result.shape[:-1], -1, 2, h)
        a = result[..., 0, :] + result[..., 1, :]
        b = result[..., 0, :] - result[..., 1, :]
        result = torch.stack([a, b], dim=-2).reshape(*x.shape[:-1], -1)
        h *= 2
    return result / math.sqrt(d)


def rotate(p: TQParams, x):
    return hadamard(x * p.signs)


def unrotate(p: TQParams, x):
    return hadamard(x) * p.signs


# -- polar --

def ieee_sqrt(t):
    """Correctly rounded float32 square root (float64 sqrt rounded once).

    PyTorch's CPU torch.sqrt goes through MKL's vector math library, which is
    not correctly rounded for about 0.6% of float32 inputs; passing this
    function as ``sqrt_fn`` evaluates the reference algorithm with IEEE sqrt."""
    return torch.sqrt(t.double()).float()


def polar_encode(p: TQParams, x, sqrt_fn=torch.sqrt):
    all_angles = []
    current = x
    for _ in range(p.n_levels):
        d_cur = current.shape[-1]
        pairs = current.view(*current.shape[:-1], d_cur // 2, 2)
        a, b = pairs[..., 0], pairs[..., 1]
        radii = sqrt_fn(a * a + b * b + 1e-12)
        angles = torch.atan2(b, a)
        all_angles.append(angles)
        current = radii
    return current, all_angles


def _bounds(level):
    return (-math.pi, math.pi) if level == 0 else (0.0, math.pi / 2)


def quantize_angle(p: TQParams, angle, level):
    n_bins = 1 << p.bits_per_angle
    lo, hi = _bounds(level)
    normalized = (angle - lo) / (hi - lo)
    return torch.clamp((normalized * n_bins).long(), 0, n_bins - 1).to(torch.uint8)


def dequantize_angle(p: TQParams, idx, level):
    n_bins = 1 << p.bits_per_angle
    lo, hi = _bounds(level)
    return lo + (idx.float() + 0.5) * (hi - lo) / n_bins


def polar_decode(p: TQParams, radius, q_angles):
    current = radius
    for level in range(p.n_levels - 1, -1, -1):
        angles = dequantize_angle(p, q_angles[level], level)
        a = current * torch.cos(angles)
        b = current * torch.sin(angles)
        current = torch.stack([a, b], dim=-1).reshape(*a.shape[:-1], angles.shape[-1] * 2)
    return current


# -- QJL --

def qjl_encode(p: TQParams, residual):
    projected = residual @ p.jl_matrix.t()
    signs = (projected > 0).to(torch.uint8)
    norms = torch.norm(residual, dim=-1, keepdim=True).half()
    return signs, norms, projected


def qjl_score_correction(p: TQParams, q, signs, norms):
    q_proj = q @ p.jl_matrix.t()
    raw = q_proj @ (signs.float() * 2 - 1).t()
    return raw * (math.sqrt(math.pi / 2) / p.qjl_dim) * norms.float().t()


# -- packed dicts --

def pack_compressed(p: TQParams, d):
    return {
        "radius": d["radius"],
        "angles_packed": pack_angles(d["angles"], p.bits_per_angle),
        "qjl_signs_packed": pack_bits(d["qjl_signs"]),
        "qjl_norms": d["qjl_norms"],
        "shape": d["shape"],
        "_N": d["qjl_signs"].shape[0],
        "_qjl_dim": d["qjl_signs"].shape[-1],
        "_level_dims": [a.shape[-1] for a in d["angles"]],
    }


def unpack_compressed(p: TQParams, d):
    if "angles" in d:
        return d
    return {
        "radius": d["radius"],
        "angles": unpack_angles(d["angles_packed"], d["_N"], d["_level_dims"], p.bits_per_angle),
        "qjl_signs": unpack_bits(d["qjl_signs_packed"], d["_qjl_dim"]),
        "qjl_norms": d["qjl_norms"],
        "shape": d["shape"],
    }


# -- public operations --

def angle_positions(p: TQParams, angles_list):
    """Unclamped, untruncated bin coordinates ((angle - lo) / (hi - lo)) * 2^bits
    of every level, for locating codes that sit on a bin edge."""
    n_bins = 1 << p.bits_per_angle
    out = []
    for level, a in enumerate(angles_list):
        lo, hi = _bounds(level)
        out.append((a - lo) / (hi - lo) * n_bins)
    return out


def compress(p: TQParams, kv, pack: bool = True, return_projection: bool = False, sqrt_fn=torch.sqrt):
    """core/kv_quantizer.py:391-417.  With return_projection, also returns the
    float32 QJL projections, the residual and the bin coordinates."""
    orig_shape = kv.shape
    flat = kv.reshape(-1, p.head_dim)
    if p.padded_dim > p.head_dim:
        flat = F.pad(flat, (0, p.padded_dim - p.head_dim))
    rotated = rotate(p, flat)
    radius, angles_list = polar_encode(p, rotated, sqrt_fn=sqrt_fn)
    q_angles = [quantize_angle(p, a, level) for level, a in enumerate(angles_list)]
    reconstructed = polar_decode(p, radius, q_angles)
    residual = rotated - reconstructed
    qjl_signs, qjl_norms, projected = qjl_encode(p, residual)
    raw = {
        "radius": radius.half(),
        "angles": q_angles,
        "qjl_signs": qjl_signs,
        "qjl_norms": qjl_norms,
        "shape": orig_shape,
    }
    out = pack_compressed(p, raw) if pack else raw
    if return_projection:
        return out, projected, residual, angle_positions(p, angles_list)
    return out


def decompress(p: TQParams, compressed):
    c = unpack_compressed(p, compressed)
    reconstructed = polar_decode(p, c["radius"].float(), c["angles"])
    unrotated = unrotate(p, reconstructed)
    if p.padded_dim > p.head_dim:
        unrotated = unrotated[..., :p.head_dim]
    return unrotated.reshape(c["shape"])


def attention_score(p: TQParams, q, compressed_k):
    c = unpack_compressed(p, compressed_k)
    flat_q = q.reshape(-1, p.head_dim)
    if p.padded_dim > p.head_dim:
        flat_q = F.pad(flat_q, (0, p.padded_dim - p.head_dim))
    q_rot = rotate(p, flat_q)
    k_polar = polar_decode(p, c["radius"].float(), c["angles"])
    return q_rot @ k_polar.t() + qjl_score_correction(p, q_rot, c["qjl_signs"], c["qjl_norms"])


def sparse_v_attend(p: TQParams, q, compressed_k, compressed_v_list, scale=None, sparse_v_ratio=0.1):
    if scale is None:
        scale = 1.0 / math.sqrt(p.head_dim)
    weights = torch.softmax(attention_score(p, q, compressed_k) * scale, dim=-1)
    seq_len = weights.shape[-1]
    k = max(1, int(math.ceil(sparse_v_ratio * seq_len)))
    if k >= seq_len:
        return weights @ torch.cat([decompress(p, cv) for cv in compressed_v_list], dim=0)
    topk_w, topk_idx = weights.topk(k, dim=-1)
    topk_w = topk_w / topk_w.sum(dim=-1, keepdim=True)
    v_mat = torch.cat([decompress(p, compressed_v_list[int(i)]) for i in topk_idx.squeeze(0)], dim=0)
    return topk_w @ v_mat


def bits_per_dim(p: TQParams):
    d = p.padded_dim
    return ((d - 1) * p.bits_per_angle + 16 + p.qjl_dim + 16) / p.head_dim
