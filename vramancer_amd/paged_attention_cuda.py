"""Paged-attention decode on MI355X — drop-in for VRAMancer's
``core/paged_attention_cuda.py``.

Same public names and arguments as the reference module
(``paged_attention_decode``, ``paged_attention_decode_q4``,
``has_cuda_paged_attention``; core/paged_attention_cuda.py:120-351), backed by
the gfx950 kernels of libvrm_paged.so instead of a JIT-compiled CUDA
extension.  Differences a caller can observe:

* bfloat16, int8 and float8_e4m3fn pools are supported; the quantized pools
  take their scales through the extra keyword ``kv_scales`` (int8: one
  float32 per (page, layer, K/V, kv-head, token); fp8: one per
  (page, layer, K/V, kv-head)), either as dense arrays or as the two views of
  one inline buffer that ``kv_quant.allocate_pool`` returns;
* there is no silent PyTorch fallback: CPU tensors or a missing library raise
  ``RuntimeError`` (the reference logs and falls back,
  core/paged_attention_cuda.py:178-183);
* page-table entries < 0 or >= num_pages mark absent pages whose tokens are
  skipped (the reference kernel stops at the first -1,
  csrc/paged_attention_kernel.cu:123; both agree when the table covers the
  context).
"""
from __future__ import annotations

import math
from typing import Any, Optional

from . import _lib

_VRM_ERR_UNSUPPORTED = -2

__all__ = [
    "paged_attention_decode",
    "prefer_balanced",
    "combine_attention",
    "paged_attention_decode_q4",
    "has_cuda_paged_attention",
    "decode_workspace",
]


def has_cuda_paged_attention() -> bool:
    """True when the gfx950 library is loadable and a GPU is visible."""
    return _lib.available()


def decode_workspace(batch: int, num_heads: int, num_kv_heads: int, head_dim: int, max_pages_per_seq: int,
                     device: Any, page_size: int = 16):
    """Allocates the split-K workspace a decode call of this shape needs.

    Callers that decode in a loop can allocate it once and pass it as
    ``workspace=`` to avoid a per-call allocation.
    """
    import torch

    lib = _lib.load()
    nsplit = lib.vrm_paged_decode_num_splits(batch, num_heads, num_kv_heads, max_pages_per_seq, page_size)
    nbytes = lib.vrm_paged_decode_workspace_bytes(batch, num_heads, head_dim, max(nsplit, 1))
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


# The balanced decode (one workgroup per sequence and kv-head, partitions
# merged in LDS; vrm_paged_decode_balanced) replaces the work-item decode when
# the caller knows the context lengths on the host and they are even: its time
# follows the longest sequence, the work-item decode's the mean.
BALANCED_MAX_SPREAD = 1.10   # longest context / mean context
BALANCED_MIN_PAIRS = 128     # sequences x kv-heads: enough workgroups to fill the GPU


def prefer_balanced(context_lens_host, num_kv_heads: int, kv_dtype) -> bool:
    """True when the balanced decode suits this batch: an int8 or fp8 pool, at
    least BALANCED_MIN_PAIRS (sequence, kv-head) pairs, and the longest context
    within BALANCED_MAX_SPREAD of the mean (host-side lengths, no device sync)."""
    import torch

    if kv_dtype not in (torch.int8, torch.float8_e4m3fn):
        return False
    # built-in reductions over a list of ints (this runs once per layer call,
    # so it avoids a per-element Python loop)
    lens = context_lens_host.tolist() if hasattr(context_lens_host, "tolist") else context_lens_host
    n = len(lens)
    if not n or n * num_kv_heads < BALANCED_MIN_PAIRS:
        return False
    total = sum(lens)
    if min(lens) < 0:
        total = sum(x for x in lens if x > 0)
    return total > 0 and max(lens) * n <= BALANCED_MAX_SPREAD * total


def check_outputs(query, out, workspace, page_table, context_lens) -> None:
    """Validates the caller-supplied tensors a decode writes or indexes through.

    ``out`` must be a contiguous float32 [B, H, D] tensor and ``workspace`` a
    contiguous tensor, both on the query's device: the kernels write through
    their raw pointers.  ``page_table`` must be [B, max_pages] and
    ``context_lens`` [B] (the kernels read B rows of max_pages entries)."""
    import torch

    B, H, D = query.shape
    if page_table.dim() != 2 or page_table.shape[0] != B or page_table.shape[1] < 1:
        raise RuntimeError(f"page_table must be [B={B}, max_pages >= 1], got {tuple(page_table.shape)}")
    if tuple(context_lens.shape) != (B,):
        raise RuntimeError(f"context_lens must be [B={B}], got {tuple(context_lens.shape)}")
    if out is not None:
        if (tuple(out.shape) != (B, H, D) or out.dtype != torch.float32 or not out.is_contiguous()
                or out.device != query.device):
            raise RuntimeError(f"out must be a contiguous float32 [{B}, {H}, {D}] tensor on {query.device}, got "
                               f"{out.dtype} {tuple(out.shape)} on {out.device}")
    if workspace is not None:
        if workspace.device != query.device or not workspace.is_contiguous():
            raise RuntimeError(f"workspace must be a contiguous tensor on {query.device}, got one on "
                               f"{workspace.device}")


def _prepare(query, page_table, context_lens, scale):
    import torch

    head_dim = query.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    if page_table.dtype != torch.int32:
        page_table = page_table.to(torch.int32)
    if context_lens.dtype != torch.int32:
        context_lens = context_lens.to(torch.int32)
    if query.dtype != torch.float32:
        query = query.float()
    return query.contiguous(), page_table.contiguous(), context_lens.contiguous(), float(scale)


def paged_attention_decode(
    query: Any,            # [B, H, D] (cast to float32)
    kv_pool: Any,          # [P, L, 2, KH, PS, D] float32/float16/bfloat16/int8/float8_e4m3fn
    page_table: Any,       # [B, max_pages_per_seq] (cast to int32)
    context_lens: Any,     # [B] (cast to int32)
    layer_idx: int,
    scale: Optional[float] = None,
    kv_scales: Any = None,  # int8: [P, L, 2, KH, PS] / fp8: [P, L, 2, KH] float32
    out: Any = None,
    workspace: Any = None,
    lse: Any = None,        # optional [B, H] float32 output: ln sum_t exp(scale q.k_t)
    context_lens_host: Any = None,  # optional host copy of context_lens (list / CPU tensor)
) -> Any:
    """Single-token attention straight from the paged KV pool.

    Mirrors core/paged_attention_cuda.py:129-184: ``scale`` defaults to
    1/sqrt(head_dim), query head h reads kv-head h // (H / KH), sequences with
    context length <= 0 produce zeros.  Returns [B, H, D] float32.

    ``context_lens_host``, when given, must equal ``context_lens``; it only
    selects the kernel (``prefer_balanced``): even batches over int8 / fp8
    pools take the balanced decode, which needs no workspace.
    """
    import torch

    query, page_table, context_lens, scale = _prepare(query, page_table, context_lens, scale)
    _lib.require_cuda(query, kv_pool, page_table, context_lens, kv_scales)
    if kv_pool.dim() != 6:
        raise RuntimeError(f"kv_pool must be [P, L, 2, KH, PS, D], got shape {tuple(kv_pool.shape)}")
    B, H, D = query.shape
    P, L, two, KH, PS, Dp = kv_pool.shape
    if two != 2 or Dp != D:
        raise RuntimeError(f"kv_pool shape {tuple(kv_pool.shape)} does not match query head_dim {D}")
    _lib.require_cuda(out, workspace)
    check_outputs(query, out, workspace, page_table, context_lens)
    code = _lib.kv_dtype_code(kv_pool.dtype)
    if code in (_lib.VRM_KV_I8, _lib.VRM_KV_FP8E4M3):
        from . import kv_quant

        want = (P, L, 2, KH, PS) if code == _lib.VRM_KV_I8 else (P, L, 2, KH)
        if kv_scales is None or tuple(kv_scales.shape) != want or kv_scales.dtype != torch.float32:
            raise RuntimeError(f"{kv_pool.dtype} pool needs float32 kv_scales of shape {want}")
        # plain (dense) or inline (the two views of kv_quant.allocate_pool) as
        # they are; any other strides are copied to the plain layout
        layout_code = kv_quant.pool_dtype_code(kv_pool, kv_scales)
        if layout_code is None:
            kv_pool, kv_scales = kv_pool.contiguous(), kv_scales.contiguous()
        else:
            code = layout_code
    elif kv_scales is not None:
        raise RuntimeError("kv_scales is only meaningful for int8 / float8_e4m3fn pools")
    else:
        kv_pool = kv_pool.contiguous()
    max_pp = page_table.shape[1]
    if out is None:
        out = torch.empty((B, H, D), dtype=torch.float32, device=query.device)
    lib = _lib.load()
    if context_lens_host is not None and prefer_balanced(context_lens_host, KH, kv_pool.dtype):
        if lse is not None:
            _check_lse(lse, B, H, query.device)
        rc = lib.vrm_paged_decode_balanced(
            _lib.ptr(query), _lib.ptr(kv_pool), _lib.ptr(kv_scales), _lib.ptr(page_table), _lib.ptr(context_lens),
            _lib.ptr(out), _lib.ptr(lse), B, H, KH, D, PS, L, P, max_pp, int(layer_idx), scale, code,
            _lib.stream_of(query),
        )
        if rc != _VRM_ERR_UNSUPPORTED:
            _lib.check(rc, "paged_attention_decode (balanced)")
            return out
    if workspace is None:
        workspace = decode_workspace(B, H, KH, D, max_pp, query.device, PS)
    ws_bytes = workspace.numel() * workspace.element_size()
    if lse is None:
        rc = lib.vrm_paged_decode(
            _lib.ptr(query), _lib.ptr(kv_pool), _lib.ptr(kv_scales), _lib.ptr(page_table), _lib.ptr(context_lens),
            _lib.ptr(out), _lib.ptr(workspace), ws_bytes, B, H, KH, D, PS, L, P, max_pp, int(layer_idx), scale, code,
            _lib.stream_of(query),
        )
    else:
        _check_lse(lse, B, H, query.device)
        rc = lib.vrm_paged_decode_lse(
            _lib.ptr(query), _lib.ptr(kv_pool), _lib.ptr(kv_scales), _lib.ptr(page_table), _lib.ptr(context_lens),
            _lib.ptr(out), _lib.ptr(lse), _lib.ptr(workspace), ws_bytes, B, H, KH, D, PS, L, P, max_pp,
            int(layer_idx), scale, code, _lib.stream_of(query),
        )
    _lib.check(rc, "paged_attention_decode")
    return out


def _check_lse(lse, B: int, H: int, device) -> None:
    import torch

    if tuple(lse.shape) != (B, H) or lse.dtype != torch.float32 or not lse.is_contiguous() or lse.device != device:
        raise RuntimeError(f"lse must be a contiguous float32 [{B}, {H}] tensor on {device}")


def combine_attention(out1: Any, lse1: Any, out2: Any, lse2: Any, lse_out: Any = None) -> Any:
    """Attention over the union of two disjoint token sets from the
    attentions over each ([..., D] float32 outputs with their [...] log-sum-exp
    of the scaled scores); rows where both sets are empty give zeros."""
    import torch

    _lib.require_cuda(out1, lse1, out2, lse2, lse_out)
    if out1.shape != out2.shape or lse1.shape != lse2.shape or tuple(out1.shape[:-1]) != tuple(lse1.shape):
        raise RuntimeError("combine_attention: mismatched shapes")
    o1, o2 = out1.float().contiguous(), out2.float().contiguous()
    l1, l2 = lse1.float().contiguous(), lse2.float().contiguous()
    D = o1.shape[-1]
    rows = o1.numel() // D
    out = torch.empty_like(o1)
    if lse_out is not None and (lse_out.shape != l1.shape or lse_out.dtype != torch.float32 or
                                not lse_out.is_contiguous()):
        raise RuntimeError("lse_out must be a contiguous float32 tensor shaped like lse1")
    rc = _lib.load().vrm_attn_combine(_lib.ptr(o1), _lib.ptr(l1), _lib.ptr(o2), _lib.ptr(l2), rows, D, _lib.ptr(out),
                                      _lib.ptr(lse_out), _lib.stream_of(o1))
    _lib.check(rc, "combine_attention")
    return out


def paged_attention_decode_q4(
    query: Any,            # [B, H, D]
    kv_pool_q4: Any,       # [P, L, 2, KH, PS, D/2] uint8 packed nibbles
    kv_scales: Any,        # [P, L, 2, KH, PS, D/32] float16
    kv_zeros: Any,         # [P, L, 2, KH, PS, D/32] float16
    page_table: Any,
    context_lens: Any,
    layer_idx: int,
    scale: Optional[float] = None,
    out: Any = None,
    workspace: Any = None,
) -> Any:
    """Paged decode over the reference's asymmetric 4-bit pool
    (core/paged_attention_cuda.py:238-288): value = (nibble - zero) * scale with
    groups of 32 along head_dim, low nibble = even index."""
    import torch

    query, page_table, context_lens, scale = _prepare(query, page_table, context_lens, scale)
    _lib.require_cuda(query, kv_pool_q4, kv_scales, kv_zeros, page_table, context_lens, out, workspace)
    check_outputs(query, out, workspace, page_table, context_lens)
    B, H, D = query.shape
    P, L, two, KH, PS, Dh = kv_pool_q4.shape
    if two != 2 or Dh * 2 != D or kv_pool_q4.dtype != torch.uint8:
        raise RuntimeError(f"kv_pool_q4 shape {tuple(kv_pool_q4.shape)} / dtype {kv_pool_q4.dtype} do not match D={D}")
    want = (P, L, 2, KH, PS, D // 32)
    for name, t in (("kv_scales", kv_scales), ("kv_zeros", kv_zeros)):
        if tuple(t.shape) != want or t.dtype != torch.float16:
            raise RuntimeError(f"{name} must be float16 of shape {want}")
    kv_pool_q4 = kv_pool_q4.contiguous()
    kv_scales = kv_scales.contiguous()
    kv_zeros = kv_zeros.contiguous()
    max_pp = page_table.shape[1]
    if out is None:
        out = torch.empty((B, H, D), dtype=torch.float32, device=query.device)
    lib = _lib.load()
    if workspace is None:
        workspace = decode_workspace(B, H, KH, D, max_pp, query.device, PS)
    rc = lib.vrm_paged_decode_q4(
        _lib.ptr(query), _lib.ptr(kv_pool_q4), _lib.ptr(kv_scales), _lib.ptr(kv_zeros), _lib.ptr(page_table),
        _lib.ptr(context_lens), _lib.ptr(out), _lib.ptr(workspace), workspace.numel() * workspace.element_size(),
        B, H, KH, D, PS, L, P, max_pp, int(layer_idx), scale, _lib.stream_of(query),
    )
    _lib.check(rc, "paged_attention_decode_q4")
    return out
