"""Writes golden vectors of the reference's TurboQuant CPU codec.

Run from the repository root on a machine that holds the reference at
/root/reference (the tests only read the fixtures it writes):

    python tests/golden/make_golden.py

Imports ``core.kv_quantizer`` from the reference with VRM_MINIMAL_TEST=1 (no
JIT, stub package init) and records, for seeded inputs, the compressor
buffers, raw and packed codes, decompressed rows and attention scores.  Only
data is written (``turboquant_golden.npz``); the tests compare the oracle in
oracle/turboquant.py against it.
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "turboquant_golden.npz")

# (name, head_dim, bits, seed, rows, input kind)
CASES = [
    ("d128_b3_t", 128, 3, 1234, 160, "student_t_bf16"),
    ("d128_b4_t", 128, 4, 1234, 160, "student_t_bf16"),
    ("d128_b3_n", 128, 3, 7, 128, "normal_f32"),
    ("d96_b3_n", 96, 3, 42, 64, "normal_f32"),
    ("d64_b8_n", 64, 8, 42, 64, "normal_f32"),
    ("d64_b2_n", 64, 2, 5, 64, "normal_f32"),
    ("d128_b4_single", 128, 4, 99, 1, "normal_f32"),
    # head_dims below 33: padded to 32, 16, 8 and 2 (the smallest padded dim)
    ("d32_b3_n", 32, 3, 11, 96, "normal_f32"),
    ("d32_b4_t", 32, 4, 12, 96, "student_t_bf16"),
    ("d16_b3_n", 16, 3, 13, 96, "normal_f32"),
    ("d8_b3_n", 8, 3, 14, 96, "normal_f32"),
    ("d5_b4_n", 5, 4, 15, 96, "normal_f32"),
    ("d2_b3_n", 2, 3, 16, 96, "normal_f32"),
]


def make_input(kind: str, rows: int, head_dim: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed + 1)
    if kind == "student_t_bf16":
        # Student-t, df = 3, scaled to unit variance (variance of t_3 is 3)
        z = torch.randn(rows, head_dim, generator=g)
        chi2 = sum(torch.randn(rows, head_dim, generator=g) ** 2 for _ in range(3))
        t = z / torch.sqrt(chi2 / 3)
        return (t / math.sqrt(3.0)).to(torch.bfloat16)
    return torch.randn(rows, head_dim, generator=g)


def main() -> None:
    os.environ["VRM_MINIMAL_TEST"] = "1"
    sys.path.insert(0, REF)
    from core.kv_quantizer import KVCacheCompressor  # noqa: E402

    arrays = {}
    for name, head_dim, bits, seed, rows, kind in CASES:
        torch.manual_seed(seed)
        comp = KVCacheCompressor(head_dim=head_dim, bits_per_angle=bits)
        kv = make_input(kind, rows, head_dim, seed)
        raw = comp.compress(kv, pack=False)
        packed = comp.compress(kv, pack=True)
        dec = comp.decompress(raw)
        q = torch.randn(8, head_dim, generator=torch.Generator().manual_seed(seed + 2))
        score = comp.attention_score(q, raw)
        pre = name + "/"
        arrays[pre + "signs"] = comp._hadamard_signs.numpy()
        arrays[pre + "jl"] = comp.jl_matrix.numpy()
        arrays[pre + "kv"] = kv.float().numpy()
        arrays[pre + "kv_is_bf16"] = np.array(kv.dtype == torch.bfloat16)
        arrays[pre + "meta"] = np.array([head_dim, bits, seed, rows])
        arrays[pre + "radius"] = raw["radius"].view(torch.int16).numpy()
        arrays[pre + "angles"] = torch.cat(raw["angles"], dim=-1).numpy()
        arrays[pre + "qjl_signs"] = raw["qjl_signs"].numpy()
        arrays[pre + "qjl_norms"] = raw["qjl_norms"].view(torch.int16).numpy()
        arrays[pre + "angles_packed"] = packed["angles_packed"].numpy()
        arrays[pre + "qjl_signs_packed"] = packed["qjl_signs_packed"].numpy()
        arrays[pre + "decompress"] = dec.numpy()
        arrays[pre + "q"] = q.numpy()
        arrays[pre + "score"] = score.numpy()
        arrays[pre + "bits_per_dim"] = np.array(comp.bits_per_dim())
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
