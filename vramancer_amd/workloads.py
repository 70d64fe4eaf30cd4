"""Seeded synthetic decode workloads with the shapes of the benchmark
configurations (inputs only; no model weights are involved).

  fp32-plumbing  fp32 pool, B=4, H=KH=12, D=64, context 512, L=1
  7b-bf16        bf16 pool, B=32, H=28, KH=4, D=128, context ~ U[1024, 8192],
                 K/V ~ N(0, 0.5^2), pool with 10% spare pages, L=1
  14b-int8       int8 pool (per-token scale), B=64, H=40, KH=8, D=128,
                 context 4096, 16384 pages of the 48-layer page shape;
                 K/V ~ N(0, 1) in bf16 with 2 of 128 channels per head x20
  mixed-fp8      fp8-e4m3 pool (per-page scale), H=64, KH=8, D=128, 128
                 sequences with lognormal context (median 2048, sigma 1,
                 clipped to [16, 131072]) plus one of 131072, L=1
  14b-q4         the 14b-int8 shape and K/V over the reference's asymmetric
                 4-bit pool (nibble codes, per 32-dim group an fp16 scale and
                 zero point); the reference ships no Q4 writer, so the codes
                 come from a plain per-group min / max quantizer
  14b-turbo3/4   TurboQuant pages (3 / 4 bits per angle), B=16, context
                 32768, H=40, KH=8, D=128; K/V bf16 from a Student-t (df 3)
                 per channel scaled to unit variance; the compressor's
                 rotation comes from torch.manual_seed(seed) before it is built

Every page table is a seeded shuffle of the physical pages.  Tensors are
generated on ``device`` with a seeded generator; the page table, context
lengths and the pool contents are returned so a checker can copy them to the
host.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import torch

PAGE_SIZE = 16


@dataclass
class DecodeConfig:
    name: str
    batch: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    num_layers: int
    codec: str                       # "f32" | "f16" | "bf16" | "int8" | "fp8" | "q4" | "tq3" | "tq4"
    context: str                     # "fixed" | "uniform" | "lognormal"
    ctx_fixed: int = 0
    ctx_low: int = 0
    ctx_high: int = 0
    ctx_median: float = 0.0
    ctx_sigma: float = 0.0
    ctx_clip: Sequence[int] = (16, 131072)
    pinned_long: int = 0             # extra sequence of this length (0: none)
    kv_std: float = 1.0
    kv_dist: str = "normal"          # "normal" | "student_t3" (unit variance)
    outlier_channels: int = 0
    outlier_scale: float = 1.0
    spare_pages: float = 0.0
    page_size: int = PAGE_SIZE
    meta: Dict[str, str] = field(default_factory=dict)


CONFIGS: Dict[str, DecodeConfig] = {
    "fp32-plumbing": DecodeConfig("fp32-plumbing", 4, 12, 12, 64, 1, "f32", "fixed", ctx_fixed=512),
    "7b-bf16": DecodeConfig("7b-bf16", 32, 28, 4, 128, 1, "bf16", "uniform", ctx_low=1024, ctx_high=8192,
                            kv_std=0.5, spare_pages=0.10),
    "14b-int8": DecodeConfig("14b-int8", 64, 40, 8, 128, 48, "int8", "fixed", ctx_fixed=4096,
                             outlier_channels=2, outlier_scale=20.0),
    "14b-q4": DecodeConfig("14b-q4", 64, 40, 8, 128, 48, "q4", "fixed", ctx_fixed=4096,
                           outlier_channels=2, outlier_scale=20.0),
    "mixed-fp8": DecodeConfig("mixed-fp8", 128, 64, 8, 128, 1, "fp8", "lognormal", ctx_median=2048.0,
                              ctx_sigma=1.0, pinned_long=131072),
    "14b-turbo3": DecodeConfig("14b-turbo3", 16, 40, 8, 128, 1, "tq3", "fixed", ctx_fixed=32768,
                               kv_dist="student_t3"),
    "14b-turbo4": DecodeConfig("14b-turbo4", 16, 40, 8, 128, 1, "tq4", "fixed", ctx_fixed=32768,
                               kv_dist="student_t3"),
}


def scaled(cfg: DecodeConfig, batch: Optional[int] = None, ctx_div: int = 1, num_layers: Optional[int] = None,
           pinned_long: Optional[int] = None) -> DecodeConfig:
    """A smaller copy of a configuration with the same structure (for tests)."""
    c = DecodeConfig(**{k: getattr(cfg, k) for k in cfg.__dataclass_fields__})
    if batch is not None:
        c.batch = batch
    if num_layers is not None:
        c.num_layers = num_layers
    if ctx_div > 1:
        c.ctx_fixed = max(1, c.ctx_fixed // ctx_div)
        c.ctx_low = max(1, c.ctx_low // ctx_div)
        c.ctx_high = max(c.ctx_low, c.ctx_high // ctx_div)
        c.ctx_median = c.ctx_median / ctx_div
        c.ctx_clip = (max(1, c.ctx_clip[0] // ctx_div), max(1, c.ctx_clip[1] // ctx_div))
        c.pinned_long = c.pinned_long // ctx_div
    if pinned_long is not None:
        c.pinned_long = pinned_long
    return c


def context_lengths(cfg: DecodeConfig, seed: int) -> List[int]:
    g = torch.Generator().manual_seed(seed)
    if cfg.context == "fixed":
        lens = [cfg.ctx_fixed] * cfg.batch
    elif cfg.context == "uniform":
        lens = torch.randint(cfg.ctx_low, cfg.ctx_high + 1, (cfg.batch,), generator=g).tolist()
    else:
        z = torch.randn(cfg.batch, generator=g, dtype=torch.float64)
        vals = torch.exp(math.log(cfg.ctx_median) + cfg.ctx_sigma * z).round().long()
        lens = vals.clamp(cfg.ctx_clip[0], cfg.ctx_clip[1]).tolist()
    if cfg.pinned_long:
        lens = lens + [cfg.pinned_long]
    return [int(x) for x in lens]


def _pool_dtype(codec: str):
    return {
        "f32": torch.float32,
        "f16": torch.float16,
        "bf16": torch.bfloat16,
        "int8": torch.int8,
        "fp8": torch.float8_e4m3fn,
    }[codec]


def q4_quantize(x: torch.Tensor):
    """Codes of the reference's asymmetric 4-bit pool for float rows
    [..., D]: per 32-dim group scale = (max - min) / 15 and zero = -min / scale
    (float16), nibble = clamp(round(x / scale + zero), 0, 15), byte j holding
    dims 2j (low nibble) and 2j + 1 (high).  Returns (codes [..., D/2] uint8,
    scales [..., D/32] float16, zeros [..., D/32] float16)."""
    g = x.float().reshape(*x.shape[:-1], -1, 32)
    lo, hi = g.amin(-1), g.amax(-1)
    scale = ((hi - lo) / 15).clamp(min=1e-6).to(torch.float16)
    zero = (-lo / scale.float()).to(torch.float16)
    n = torch.clamp(torch.round(g / scale.float()[..., None] + zero.float()[..., None]), 0, 15).to(torch.uint8)
    n = n.reshape(x.shape)
    return n[..., 0::2] | (n[..., 1::2] << 4), scale, zero


def _kv_pages(cfg: DecodeConfig, n: int, gen: torch.Generator, device, outlier_idx) -> torch.Tensor:
    """[n, KH, PS, D] float32 K or V rows of the configured distribution."""
    shape = (n, cfg.num_kv_heads, cfg.page_size, cfg.head_dim)
    x = torch.randn(shape, generator=gen, device=device)
    if cfg.kv_dist == "student_t3":  # t(3) = z / sqrt(chi2_3 / 3), variance 3
        chi2 = sum(torch.randn(shape, generator=gen, device=device) ** 2 for _ in range(3))
        x = x / torch.sqrt(chi2 / 3) / math.sqrt(3.0)
    x = x * cfg.kv_std
    if cfg.outlier_channels:
        x[:, torch.arange(cfg.num_kv_heads, device=device)[:, None], :, outlier_idx] *= cfg.outlier_scale
    return x


def make_decode_inputs(cfg: DecodeConfig, device="cuda", seed: int = 0, layers: Sequence[int] = (0,),
                       chunk_pages: int = 2048, layout: Optional[str] = None) -> dict:
    """Builds (query, kv_pool, kv_scales, page_table, context_lens) on ``device``.

    Only the layers in ``layers`` are filled; the others stay zero (they are
    part of the page stride, not of the attended data).  Quantized pools are
    filled through the library's page quantizer from bf16 rows, in the given
    memory layout (``kv_quant.allocate_pool``: "inline", "plain", or None for
    the codec's default).
    """
    from . import kv_quant

    lens = context_lengths(cfg, seed)
    B = len(lens)
    PS = cfg.page_size
    pages_per_seq = [(n + PS - 1) // PS for n in lens]
    used = sum(pages_per_seq)
    P = max(1, int(math.ceil(used * (1.0 + cfg.spare_pages))))
    max_pp = max(1, max(pages_per_seq))
    g_cpu = torch.Generator().manual_seed(seed + 1)
    perm = torch.randperm(P, generator=g_cpu)
    table = torch.full((B, max_pp), -1, dtype=torch.int32)
    off = 0
    for b, npg in enumerate(pages_per_seq):
        table[b, :npg] = perm[off:off + npg].to(torch.int32)
        off += npg
    gen = torch.Generator(device=device).manual_seed(seed + 2)
    H, KH, D, L = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.num_layers
    query = torch.randn((B, H, D), generator=gen, device=device)
    outlier_idx = None
    if cfg.outlier_channels:
        outlier_idx = torch.stack([
            torch.randperm(D, generator=g_cpu)[:cfg.outlier_channels] for _ in range(KH)
        ]).to(device)
    kv_scales = None
    kv_zeros = None
    compressor = None
    if cfg.codec == "q4":
        kv_pool = torch.zeros((P, L, 2, KH, PS, D // 2), dtype=torch.uint8, device=device)
        kv_scales = torch.zeros((P, L, 2, KH, PS, D // 32), dtype=torch.float16, device=device)
        kv_zeros = torch.zeros_like(kv_scales)
    elif cfg.codec in ("tq3", "tq4"):
        from . import tq_pages
        from .kv_quantizer import KVCacheCompressor

        torch.manual_seed(seed)  # the rotation and JL matrix are fixed by the seed
        compressor = KVCacheCompressor(cfg.head_dim, int(cfg.codec[2]))
        kv_pool = tq_pages.allocate_pool(P, L, KH, compressor, device, PS)
        dtype = None
    elif cfg.codec in ("int8", "fp8"):
        dtype = _pool_dtype(cfg.codec)
        kv_pool, kv_scales = kv_quant.allocate_pool(P, L, KH, D, cfg.codec, PS, device, layout=layout)
    else:
        dtype = _pool_dtype(cfg.codec)
        kv_pool = torch.zeros((P, L, 2, KH, PS, D), dtype=dtype, device=device)
    page_ids_all = torch.arange(P, dtype=torch.int32, device=device)
    for layer in layers:
        for s in range(0, P, chunk_pages):
            e = min(P, s + chunk_pages)
            k = _kv_pages(cfg, e - s, gen, device, outlier_idx)
            v = _kv_pages(cfg, e - s, gen, device, outlier_idx)
            if cfg.codec == "q4":
                for kv, x in ((0, k), (1, v)):
                    codes, sc, zp = q4_quantize(x.to(torch.bfloat16))
                    kv_pool[s:e, layer, kv] = codes
                    kv_scales[s:e, layer, kv] = sc
                    kv_zeros[s:e, layer, kv] = zp
            elif compressor is not None:
                tq_pages.quantize_pages(kv_pool, layer, page_ids_all[s:e], k.to(torch.bfloat16),
                                        v.to(torch.bfloat16), compressor, page_size=PS)
            elif kv_scales is not None:
                # the quantized pools start from bf16 activations
                kv_quant.quantize_pages(kv_pool, kv_scales, layer, page_ids_all[s:e], k.to(torch.bfloat16),
                                        v.to(torch.bfloat16))
            else:
                kv_pool[s:e, layer, 0] = k.to(dtype)
                kv_pool[s:e, layer, 1] = v.to(dtype)
    return {
        "query": query,
        "kv_pool": kv_pool,
        "kv_scales": kv_scales,
        "kv_zeros": kv_zeros,
        "page_table": table.to(device),
        "context_lens": torch.tensor(lens, dtype=torch.int32, device=device),
        "layers": list(layers),
        "num_pages": P,
        "config": cfg,
        "compressor": compressor,
    }


def algorithmic_bytes(cfg: DecodeConfig, lens: Sequence[int]) -> Dict[str, float]:
    """Bytes one layer-step must move at minimum: valid-token K/V codes, their
    scales at their granularity, Q and O in float32, and the page-table
    entries read."""
    PS = cfg.page_size
    KH, D, H = cfg.num_kv_heads, cfg.head_dim, cfg.num_heads
    tokens = sum(lens)
    pages = sum((n + PS - 1) // PS for n in lens)
    if cfg.codec in ("tq3", "tq4"):
        # per token and kv-head: K angles + QJL sign bits + fp16 radius + fp16 norm, V angles + fp16
        # radius; padded_dim - 1 angles of `bits` bits, padded_dim / 2 QJL rows (the compressor's
        # defaults, core/kv_quantizer.py:225-229)
        bits = int(cfg.codec[2])
        pd = 2
        while pd < D:
            pd *= 2
        angles = ((pd - 1) * bits + 7) // 8
        signs = (pd // 2 + 7) // 8
        kv = tokens * KH * ((angles + signs + 2 + 2) + (angles + 2))
        scales = 0
        qo = 2 * len(lens) * H * D * 4
        table = pages * 4
        return {"kv": kv, "scales": scales, "qo": qo, "table": table, "total": kv + scales + qo + table,
                "tokens": tokens, "pages": pages}
    if cfg.codec == "q4":
        kv = tokens * KH * 2 * (D // 2)
        scales = tokens * KH * 2 * (D // 32) * 2 * 2  # float16 scale and zero per 32-dim group
        qo = 2 * len(lens) * H * D * 4
        table = pages * 4
        return {"kv": kv, "scales": scales, "qo": qo, "table": table, "total": kv + scales + qo + table,
                "tokens": tokens, "pages": pages}
    elem = {"f32": 4, "f16": 2, "bf16": 2, "int8": 1, "fp8": 1}[cfg.codec]
    kv = tokens * KH * 2 * D * elem
    if cfg.codec == "int8":
        scales = tokens * KH * 2 * 4
    elif cfg.codec == "fp8":
        scales = pages * KH * 2 * 4
    else:
        scales = 0
    qo = 2 * len(lens) * H * D * 4
    table = pages * 4
    return {"kv": kv, "scales": scales, "qo": qo, "table": table, "total": kv + scales + qo + table,
            "tokens": tokens, "pages": pages}
