"""int8 and fp8-e4m3 KV codecs as this build defines them (test oracle only).

The reference has no int8 or fp8 KV codec (core/kv_quantizer.py is
TurboQuant-only; fp8 exists only as vLLM's kv_cache_dtype,
benchmarks/_fp8_kv_worker.py:26-36), so these are the definitions the GPU
kernels must reproduce bit for bit, written with PyTorch CPU ops:

int8, per (token, kv-head) over head_dim:
    scale = amax(|x|) / 127                       (float32 division)
    code  = clamp(round_half_even(x / scale), -127, 127); scale == 0 -> codes 0
fp8-e4m3fn, per (page, layer, K/V, kv-head) over the page's valid tokens:
    scale = amax(|x|) / 448
    code  = (x / scale).to(float8_e4m3fn)         (round to nearest even)
pool layout: each (page, layer, K/V, kv-head) slice holds PS x D codes
    (PS a multiple of 4, D a multiple of 16); K is token-major like the reference's pool,
    V is tiled: the code of token t, dim d sits at byte
        ((t // 4 * 16 + d % 16) * (D // 16) + d // 16) * 4 + t % 4
    (four consecutive tokens of one dim share a dword; the 16 dims d % 16 of a
    token quad are D / 4 bytes apart).  ``v_token_major`` / ``v_pool_order``
    convert.
fp8 append of token x into slot s of a page with scale s_old (0 if s == 0):
    s_new = max(s_old, amax(|x|) / 448)
    if s_new > s_old: every code c in slots < s becomes e4m3((float(c) * s_old) / s_new)
    new row = e4m3(x / s_new)
"""
from __future__ import annotations

import torch


def quantize_int8(x):
    """x [..., D] -> (codes int8 [..., D], scale float32 [...])."""
    xf = x.float()
    amax = xf.abs().amax(dim=-1, keepdim=True)
    scale = amax / 127
    codes = torch.round(xf / scale).clamp(-127, 127)
    codes = torch.where(scale > 0, codes, torch.zeros_like(codes)).to(torch.int8)
    return codes, scale.squeeze(-1)


def dequantize_int8(codes, scale):
    return codes.float() * scale.unsqueeze(-1)


def e4m3(x):
    """float32 tensor -> e4m3fn codes as uint8 (torch's RNE cast)."""
    return x.float().to(torch.float8_e4m3fn).view(torch.uint8)


def e4m3_to_float(codes_u8):
    return codes_u8.view(torch.float8_e4m3fn).float()


def quantize_fp8_page(x_page, n_valid: int):
    """x_page [PS, D] -> (codes uint8 [PS, D], scale float32 0-dim)."""
    xf = x_page.float()
    codes = torch.zeros(xf.shape, dtype=torch.uint8)
    if n_valid <= 0:
        return codes, torch.tensor(0.0)
    amax = xf[:n_valid].abs().max()
    scale = amax / 448
    if scale > 0:
        codes[:n_valid] = e4m3(xf[:n_valid] / scale)
    return codes, scale


def fp8_append(page_codes, old_scale, slot: int, x):
    """Returns (new page codes uint8 [PS, D], new scale) after writing x [D] at slot."""
    codes = page_codes.clone()
    old = torch.tensor(0.0) if slot == 0 else old_scale.float().reshape(())
    want = x.float().abs().max() / 448
    new = torch.maximum(old, want)
    if slot > 0 and new > old:
        y = e4m3_to_float(codes[:slot]) * old
        codes[:slot] = e4m3(y / new)
    if new > 0:
        codes[slot] = e4m3(x.float() / new)
    else:
        codes[slot] = 0
    return codes, new


def dequantize_fp8(codes_u8, scale):
    return e4m3_to_float(codes_u8) * scale


def v_token_major(v_slices):
    """Physical V slices [..., PS, D] (tiled as the pool stores them) ->
    logical [..., PS, D] (token t, dim d at [t, d]); PS % 4 == 0, D % 16 == 0."""
    *lead, PS, D = v_slices.shape
    assert PS % 4 == 0 and D % 16 == 0, (PS, D)
    # physical axes (t // 4, d % 16, d // 16, t % 4) -> logical (t // 4, t % 4, d // 16, d % 16)
    tiles = v_slices.reshape(*lead, PS // 4, 16, D // 16, 4)
    return tiles.transpose(-1, -3).reshape(*lead, PS, D)


def v_pool_order(v_logical):
    """Logical V [..., PS, D] -> the pool's tiled physical [..., PS, D]."""
    *lead, PS, D = v_logical.shape
    assert PS % 4 == 0 and D % 16 == 0, (PS, D)
    tiles = v_logical.reshape(*lead, PS // 4, 4, D // 16, 16)
    return tiles.transpose(-1, -3).contiguous().reshape(*lead, PS, D)


def pool_to_logical(pool):
    """[P, L, 2, KH, PS, D] quantized pool -> same shape with V token-major."""
    out = pool.clone()
    out[:, :, 1] = v_token_major(pool[:, :, 1])
    return out


def pool_from_logical(pool_logical):
    out = pool_logical.clone()
    out[:, :, 1] = v_pool_order(pool_logical[:, :, 1])
    return out
