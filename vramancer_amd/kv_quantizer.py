"""TurboQuant KV compressor (randomized Hadamard + PolarQuant + QJL) on
MI355X — drop-in for VRAMancer's ``core/kv_quantizer.py``.

``KVCacheCompressor`` keeps the reference's constructor, buffers and public
methods (core/kv_quantizer.py:207-576): the rotation signs and the JL matrix
are drawn from torch's global RNG in the same order (``randint`` then
``randn``), so a compressor built after ``torch.manual_seed(s)`` holds the
same buffers as the reference's.  Compression, decompression and the
rotated-space key reconstruction run in gfx950 kernels; the packed format
(MSB-first bit packing of angles and QJL signs, core/kv_quantizer.py:46-105)
is produced with tensor ops on the same device.

There is no CPU path: CPU tensors raise ``RuntimeError`` and ``force_cpu``
is rejected (the reference's CPU path is the oracle these kernels are tested
against, not a fallback).
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn

from . import _lib
from .turboquant_cuda import CUDATurboQuantOps, level_bins

__all__ = ["KVCacheCompressor", "TurboQuantCompressor"]


# Bit packing (MSB first): the byte layout of core/kv_quantizer.py:46-105.

def _pack_values(vals, bits: int):
    """[..., M] uint8 -> [..., ceil(M * bits / 8)] bytes: the low ``bits``
    bits of each value, most significant first, packed MSB-first
    (core/kv_quantizer.py:46-83), by the gfx950 pack kernel."""
    *batch, M = vals.shape
    flat = vals.reshape(-1, M).to(torch.uint8).contiguous()
    _lib.require_cuda(flat)
    nbytes = (M * bits + 7) // 8
    out = torch.empty((flat.shape[0], nbytes), dtype=torch.uint8, device=flat.device)
    rc = _lib.load().vrm_pack_bits(_lib.ptr(flat), flat.shape[0], M, bits, _lib.ptr(out), _lib.stream_of(flat))
    _lib.check(rc, "pack")
    return out.reshape(*batch, nbytes)


def _unpack_values(packed, M: int, bits: int):
    """Inverse of _pack_values: [..., nbytes] -> [..., M] uint8."""
    *batch, nbytes = packed.shape
    flat = packed.reshape(-1, nbytes).to(torch.uint8).contiguous()
    _lib.require_cuda(flat)
    if nbytes * 8 < M * bits:
        raise RuntimeError(f"{nbytes} bytes cannot hold {M} values of {bits} bits")
    out = torch.empty((flat.shape[0], M), dtype=torch.uint8, device=flat.device)
    rc = _lib.load().vrm_unpack_bits(_lib.ptr(flat), flat.shape[0], M, bits, _lib.ptr(out), _lib.stream_of(flat))
    _lib.check(rc, "unpack")
    return out.reshape(*batch, M)


def _pack_bits(signs):
    """[..., M] 0/1 uint8 -> [..., ceil(M/8)] bytes, first element in the MSB."""
    return _pack_values(signs, 1)


def _unpack_bits(packed, M):
    return _unpack_values(packed, M, 1)


def _pack_angles(angles_list, bits_per_angle):
    """Level-major concatenation of a row's angle bins, bits_per_angle bits each."""
    if not angles_list:
        return torch.tensor([], dtype=torch.uint8)
    return _pack_values(level_bins(angles_list, sum(a.shape[-1] for a in angles_list)), bits_per_angle)


def _unpack_angles(packed, N, level_dims, bits_per_angle):
    flat = _unpack_values(packed, sum(level_dims), bits_per_angle).reshape(N, -1)
    return list(torch.split(flat, list(level_dims), dim=-1))


def _split_rows(result: dict, rows: list, shapes: list) -> list:
    """Per-item dicts over the rows of one batched result, as device views.

    ``torch.split`` cuts every field in one call for all items, so the cost
    does not grow with the number of fields times items in Python; each item
    gets a plain dict of views (no copy) with its own input shape.  Works on
    raw results (radius / angles / qjl_signs / qjl_norms) and on packed ones
    (angles_packed / qjl_signs_packed), whose rows are packed independently.
    """
    columns = {}
    for key, val in result.items():
        if key == "shape" or key.startswith("_"):
            continue
        if isinstance(val, list):
            columns[key] = list(zip(*(torch.split(level, rows) for level in val)))
        else:
            columns[key] = torch.split(val, rows)
    items = []
    for i, (shape, n) in enumerate(zip(shapes, rows)):
        item = {key: (list(col[i]) if isinstance(result[key], list) else col[i]) for key, col in columns.items()}
        item["shape"] = shape
        for key in ("_qjl_dim", "_level_dims"):
            if key in result:
                item[key] = result[key]
        if "_N" in result:
            item["_N"] = n
        items.append(item)
    return items


class KVCacheCompressor(nn.Module):
    """TurboQuant KV compressor.

    Args:
        head_dim: attention head dimension (padded internally to a power of 2)
        bits_per_angle: bits per quantized polar angle (default 3)
        qjl_dim: JL projection rows (default padded_dim // 2)
        force_cpu: accepted for signature compatibility; must be False
    """

    def __init__(self, head_dim: int, bits_per_angle: int = 3, qjl_dim: Optional[int] = None,
                 force_cpu: bool = False):
        super().__init__()
        if force_cpu:
            raise ValueError("force_cpu=True is not supported: this codec runs on the GPU only")
        self.head_dim = head_dim
        self.bits_per_angle = bits_per_angle
        self._force_cpu = False
        self._padded_dim = 1 << math.ceil(math.log2(max(head_dim, 2)))
        self._n_levels = int(math.log2(self._padded_dim))
        self.qjl_dim = qjl_dim or self._padded_dim // 2
        # Same draws, in the same order, as core/kv_quantizer.py:231-236.
        signs = torch.randint(0, 2, (self._padded_dim,)).float() * 2 - 1
        self.register_buffer("_hadamard_signs", signs)
        P = torch.randn(self.qjl_dim, self._padded_dim) / math.sqrt(self.qjl_dim)
        self.register_buffer("jl_matrix", P)

    # -- helpers --

    def _ops_args(self):
        return self.head_dim, self._padded_dim, self._n_levels, self.bits_per_angle

    def _pack_compressed(self, d):
        N = d["qjl_signs"].shape[0]
        return {
            "radius": d["radius"],
            "angles_packed": _pack_angles(d["angles"], self.bits_per_angle),
            "qjl_signs_packed": _pack_bits(d["qjl_signs"]),
            "qjl_norms": d["qjl_norms"],
            "shape": d["shape"],
            "_N": N,
            "_qjl_dim": d["qjl_signs"].shape[-1],
            "_level_dims": [a.shape[-1] for a in d["angles"]],
        }

    def _unpack_compressed(self, d):
        if "angles" in d:
            return d
        N = d["_N"]
        return {
            "radius": d["radius"],
            "angles": _unpack_angles(d["angles_packed"], N, d["_level_dims"], self.bits_per_angle),
            "qjl_signs": _unpack_bits(d["qjl_signs_packed"], d["_qjl_dim"]),
            "qjl_norms": d["qjl_norms"],
            "shape": d["shape"],
        }

    # -- public API (core/kv_quantizer.py:375-572) --

    def compress(self, kv, pack: bool = True):
        """Compresses [..., head_dim] vectors; returns the packed dict by default."""
        result = CUDATurboQuantOps.compress_gpu(kv, *self._ops_args(), self._hadamard_signs, self.jl_matrix)
        return self._pack_compressed(result) if pack else result

    def compress_batch(self, kv_list: list, pack: bool = False) -> list:
        """Compresses several tensors with one kernel launch and returns one
        dict per tensor: raw codes (device views into the batch result), or,
        with ``pack=True``, packed dicts (the whole batch is packed by one
        launch per field, then split).  A one-element list returns
        ``[self.compress(kv)]`` (packed), as the reference does
        (core/kv_quantizer.py:443-444)."""
        if not kv_list:
            return []
        if len(kv_list) == 1:
            return [self.compress(kv_list[0])]
        shapes = [tuple(kv.shape) for kv in kv_list]
        flat = [kv.reshape(-1, self.head_dim) for kv in kv_list]
        rows = [f.shape[0] for f in flat]
        result = CUDATurboQuantOps.compress_gpu(torch.cat(flat, dim=0), *self._ops_args(), self._hadamard_signs,
                                                self.jl_matrix)
        if pack:
            result = self._pack_compressed(result)
        return _split_rows(result, rows, shapes)

    def decompress(self, compressed):
        """Approximate K/V from polar codes only (no QJL), shaped like the input."""
        compressed = self._unpack_compressed(compressed)
        return CUDATurboQuantOps.decompress_gpu(compressed, *self._ops_args(), self._hadamard_signs)

    def attention_score(self, q, compressed_k):
        """[n_queries, seq_len] scores from compressed keys plus the QJL correction."""
        compressed_k = self._unpack_compressed(compressed_k)
        return CUDATurboQuantOps.attention_score_gpu(
            q, compressed_k, *self._ops_args(), self._hadamard_signs, self.jl_matrix, self.qjl_dim)

    def sparse_v_attend(self, q, compressed_k, compressed_v_list, scale=None, sparse_v_ratio=0.1):
        """Scores from compressed keys, then the renormalised softmax over the
        top ceil(ratio * seq) scores applied to their values
        (core/kv_quantizer.py:537-562); every step runs in gfx950 kernels.
        The values are decompressed in one batch; rows of several queries are
        supported (the reference's sparse branch takes one)."""
        from .turboquant_cuda import topk_attend

        if scale is None:
            scale = 1.0 / math.sqrt(self.head_dim)
        compressed_k = self._unpack_compressed(compressed_k)
        scores = CUDATurboQuantOps.attention_score_gpu(
            q, compressed_k, *self._ops_args(), self._hadamard_signs, self.jl_matrix, self.qjl_dim, scale=scale)
        seq_len = scores.shape[-1]
        k = max(1, int(math.ceil(sparse_v_ratio * seq_len)))
        v_mat = self._decompress_list(compressed_v_list)
        if v_mat.shape[0] != seq_len:
            raise RuntimeError(f"{v_mat.shape[0]} value rows for {seq_len} keys")
        return topk_attend(scores, min(k, seq_len), v_mat)

    def _decompress_list(self, compressed_list):
        """Rows of every dict of the list, decompressed in one launch: [rows, head_dim]."""
        parts = [self._unpack_compressed(c) for c in compressed_list]
        if not parts:
            raise RuntimeError("empty value list")
        merged = {
            "radius": torch.cat([c["radius"].reshape(-1) for c in parts]),
            "angles": [torch.cat([c["angles"][l].reshape(-1, c["angles"][l].shape[-1]) for c in parts])
                       for l in range(len(parts[0]["angles"]))],
        }
        merged["shape"] = (merged["radius"].shape[0], self.head_dim)
        return CUDATurboQuantOps.decompress_gpu(merged, *self._ops_args(), self._hadamard_signs)

    def bits_per_dim(self):
        """((padded_dim - 1) * bits + 16 + qjl_dim + 16) / head_dim."""
        d = self._padded_dim
        total = (d - 1) * self.bits_per_angle + 16 + self.qjl_dim + 16
        return total / self.head_dim


TurboQuantCompressor = KVCacheCompressor
