"""Restatement of the reference's PyTorch decode path (test oracle only).

``paged_attention_decode`` follows ``_pytorch_paged_attention_decode``
(core/paged_attention_cuda.py:187-231) op for op: per-sequence loop, page
gather -> [KH, ctx, D] float32, repeat_interleave for GQA (head h reads kv-head
h // (H / KH)), bmm -> softmax -> bmm.  Quantized pools are dequantized first
(int8: code * per-token scale; fp8: float(code) * per-page scale, with V
read in the tiled order those pools store it), as the reference's fused-dequant
contract implies.  ``paged_attention_decode_q4``
follows core/paged_attention_cuda.py:291-348.  ``dense_attention`` is an
independent fp64 closed form used to pin the restatement.
"""
from __future__ import annotations

import math
from typing import Optional

import torch


def _dequant_pages(kv_pool, kv_scales, page_ids, layer_idx, kv):
    pages = kv_pool[page_ids, layer_idx, kv]  # [n, KH, PS, D]
    if kv == 1 and kv_pool.dtype in (torch.int8, torch.float8_e4m3fn):
        # quantized pools keep V tiled inside each page-head slice
        from .kv_codecs import v_token_major
        pages = v_token_major(pages)
    if kv_pool.dtype == torch.int8:
        return pages.float() * kv_scales[page_ids, layer_idx, kv].unsqueeze(-1)
    if kv_pool.dtype == torch.float8_e4m3fn:
        return pages.float() * kv_scales[page_ids, layer_idx, kv][:, :, None, None]
    return pages.float()


def paged_attention_decode(query, kv_pool, page_table, context_lens, layer_idx, scale=None, kv_scales=None):
    """[B, H, D] float32 attention output; core/paged_attention_cuda.py:187-231."""
    batch_size, num_heads, head_dim = query.shape
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    query = query.float()
    num_kv_heads = kv_pool.shape[3]
    page_size = kv_pool.shape[4]
    kv_head_ratio = num_heads // num_kv_heads
    outputs = []
    for b in range(batch_size):
        ctx_len = int(context_lens[b].item())
        if ctx_len <= 0:
            outputs.append(torch.zeros(num_heads, head_dim))
            continue
        num_pages = (ctx_len + page_size - 1) // page_size
        page_ids = page_table[b, :num_pages].long()
        k_pages = _dequant_pages(kv_pool, kv_scales, page_ids, layer_idx, 0)
        v_pages = _dequant_pages(kv_pool, kv_scales, page_ids, layer_idx, 1)
        k_flat = k_pages.permute(1, 0, 2, 3).reshape(num_kv_heads, -1, head_dim)[:, :ctx_len, :]
        v_flat = v_pages.permute(1, 0, 2, 3).reshape(num_kv_heads, -1, head_dim)[:, :ctx_len, :]
        if kv_head_ratio > 1:
            k_flat = k_flat.repeat_interleave(kv_head_ratio, dim=0)
            v_flat = v_flat.repeat_interleave(kv_head_ratio, dim=0)
        q = query[b].unsqueeze(1)
        scores = torch.bmm(q, k_flat.transpose(1, 2)) * scale
        weights = torch.softmax(scores, dim=-1)
        outputs.append(torch.bmm(weights, v_flat).squeeze(1))
    return torch.stack(outputs)


def dequant_q4_page(packed, scales, zeros, group_size: int = 32):
    """[..., D/2] nibbles -> [..., D] float32; core/paged_attention_cuda.py:303-313."""
    lo = (packed & 0x0F).float()
    hi = ((packed >> 4) & 0x0F).float()
    vals = torch.stack([lo, hi], dim=-1).reshape(*packed.shape[:-1], -1)
    sc = scales.float().repeat_interleave(group_size, dim=-1)[..., :vals.shape[-1]]
    zp = zeros.float().repeat_interleave(group_size, dim=-1)[..., :vals.shape[-1]]
    return (vals - zp) * sc


def paged_attention_decode_q4(query, kv_pool_q4, kv_scales, kv_zeros, page_table, context_lens, layer_idx,
                              scale=None):
    """core/paged_attention_cuda.py:291-348."""
    batch_size, num_heads, head_dim = query.shape
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    query = query.float()
    num_kv_heads = kv_pool_q4.shape[3]
    page_size = kv_pool_q4.shape[4]
    ratio = num_heads // num_kv_heads
    outputs = []
    for b in range(batch_size):
        ctx_len = int(context_lens[b].item())
        if ctx_len <= 0:
            outputs.append(torch.zeros(num_heads, head_dim))
            continue
        num_pages = (ctx_len + page_size - 1) // page_size
        page_ids = page_table[b, :num_pages].long()
        k_pages = dequant_q4_page(kv_pool_q4[page_ids, layer_idx, 0], kv_scales[page_ids, layer_idx, 0],
                                  kv_zeros[page_ids, layer_idx, 0])
        v_pages = dequant_q4_page(kv_pool_q4[page_ids, layer_idx, 1], kv_scales[page_ids, layer_idx, 1],
                                  kv_zeros[page_ids, layer_idx, 1])
        k_flat = k_pages.permute(1, 0, 2, 3).reshape(num_kv_heads, -1, head_dim)[:, :ctx_len, :]
        v_flat = v_pages.permute(1, 0, 2, 3).reshape(num_kv_heads, -1, head_dim)[:, :ctx_len, :]
        if ratio > 1:
            k_flat = k_flat.repeat_interleave(ratio, dim=0)
            v_flat = v_flat.repeat_interleave(ratio, dim=0)
        q = query[b].unsqueeze(1)
        scores = torch.bmm(q, k_flat.transpose(1, 2)) * scale
        weights = torch.softmax(scores, dim=-1)
        outputs.append(torch.bmm(weights, v_flat).squeeze(1))
    return torch.stack(outputs)


def gather_sequence(pool_f32, page_table_row, ctx_len, layer_idx, skip_invalid: bool = False):
    """K, V of one sequence as [KH, n, D] float64 from a dequantized [P, L, 2,
    KH, PS, D] pool, token by token; with skip_invalid, tokens on pages whose
    id is < 0 or >= P are dropped."""
    P = pool_f32.shape[0]
    PS = pool_f32.shape[4]
    ks, vs = [], []
    for t in range(ctx_len):
        pid = int(page_table_row[t // PS])
        if not (0 <= pid < P):
            if skip_invalid:
                continue
            pid = pid % P
        ks.append(pool_f32[pid, layer_idx, 0, :, t % PS, :].double())
        vs.append(pool_f32[pid, layer_idx, 1, :, t % PS, :].double())
    if not ks:
        return None, None
    return torch.stack(ks, dim=1), torch.stack(vs, dim=1)


def dense_attention(q, K, V, scale):
    """fp64 softmax(scale q K^T) V for one sequence; q [H, D], K/V [KH, n, D];
    query head h uses kv-head h // (H / KH).  Independent of the restatement."""
    H, D = q.shape
    KH = K.shape[0]
    out = torch.zeros(H, D, dtype=torch.float64)
    for h in range(H):
        kh = h // (H // KH)
        s = (K[kh] @ q[h].double()) * scale
        s = s - s.max()
        w = torch.exp(s)
        out[h] = (w[:, None] * V[kh]).sum(0) / w.sum()
    return out


def paged_attention_decode_turbo(p, query, codes, page_table, context_lens, scale=None, head_map="div",
                                 sparse_v_ratio=1.0):
    """[B, H, D] float32 attention over TurboQuant pages, as
    PagedKVCacheManager.compute_attention_turbo (core/paged_attention.py:
    1259-1418) evaluates it with dense values (sparse_v_ratio 1.0): per kv-head,
    scores = attention_score(q_group, merged compressed keys) * scale (QJL-
    corrected, on the rotated query; core/kv_quantizer.py:502-535), softmax,
    then weights @ decompress(values) (core/kv_quantizer.py:481-500).  With
    head_map "div" query head h reads kv-head h // (H / KH), the paged
    decode's mapping; with "mod" it reads kv-head h % KH, the mapping of
    compute_attention_turbo itself (core/paged_attention.py:1374).  With
    sparse_v_ratio < 1 each head keeps its top ceil(ratio * seq) softmax
    weights, renormalised, over the values of those tokens (:1384-1400).

    ``p`` are the compressor's parameters (oracle.turboquant.make_params);
    ``codes`` holds one layer's raw codes indexed [page, K/V, kv-head, token]:
    radius fp16, angles uint8 [.., 127] level-major, qjl_signs uint8 [.., 64],
    qjl_norms fp16.  Pages whose id is < 0 or >= P are skipped.
    """
    from . import turboquant as TQ

    B, H, D = query.shape
    P, _, KH, PS = codes["radius"].shape
    ratio = H // KH
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    level_dims = [p.padded_dim >> (l + 1) for l in range(p.n_levels)]
    out = torch.zeros(B, H, D)
    for b in range(B):
        ctx = int(context_lens[b])
        if ctx <= 0:
            continue
        n = (ctx + PS - 1) // PS
        tokens = [(int(page_table[b, t // PS]), t % PS) for t in range(ctx)]
        tokens = [(pid, s) for pid, s in tokens if 0 <= pid < P]
        if not tokens:
            continue
        pids = torch.tensor([pid for pid, _ in tokens])
        slots = torch.tensor([s for _, s in tokens])

        def gather(kv, kvh):
            ang = codes["angles"][pids, kv, kvh, slots]
            return {
                "radius": codes["radius"][pids, kv, kvh, slots].reshape(-1, 1),
                "angles": list(torch.split(ang, level_dims, dim=-1)),
                "qjl_signs": codes["qjl_signs"][pids, kv, kvh, slots],
                "qjl_norms": codes["qjl_norms"][pids, kv, kvh, slots].reshape(-1, 1),
                "shape": (len(tokens), D),
            }

        for kvh in range(KH):
            ck, cv = gather(0, kvh), gather(1, kvh)
            if head_map == "div":
                group = list(range(kvh * ratio, (kvh + 1) * ratio))
            elif head_map == "mod":
                group = [h for h in range(H) if h % KH == kvh]
            else:
                raise ValueError(f"head_map {head_map!r}")
            q_group = query[b, group].float()
            scores = TQ.attention_score(p, q_group, ck) * scale
            weights = torch.softmax(scores, dim=-1)
            values = TQ.decompress(p, cv)
            seq = weights.shape[-1]
            k = max(1, int(math.ceil(sparse_v_ratio * seq)))
            if k < seq:
                for gi, h in enumerate(group):
                    top_w, top_i = weights[gi:gi + 1].topk(k, dim=-1)
                    top_w = top_w / top_w.sum(dim=-1, keepdim=True)
                    out[b, h] = (top_w @ values[top_i[0]])[0]
            else:
                out[b, group] = weights @ values
    return out
