"""int8 / fp8-e4m3 paged KV pools: allocation, quantize-on-append, bulk page
writes and dequantization, all on the GPU.

VRAMancer has no int8 or fp8 KV codec (core/kv_quantizer.py is
TurboQuant-only and fp8 exists only as vLLM's kv_cache_dtype); this module
defines them in the style of the reference's pool API:

* the pool keeps the reference layout ``[P, L, 2, KH, PS, D]``
  (core/paged_attention.py:321-330) with int8 or float8_e4m3fn elements;
* int8 uses one float32 scale per (page, layer, K/V, kv-head, token):
  ``scale = amax / 127``, ``code = clamp(round_half_even(x / scale), -127, 127)``
  (amax == 0 gives scale 0 and codes 0);
* fp8 uses one float32 scale per (page, layer, K/V, kv-head):
  ``scale = amax / 448``, ``code = e4m3fn(x / scale)`` rounded to nearest even.
  On append the page scale only grows; when it grows, codes already in the
  page are re-encoded as ``e4m3fn(float(code) * old / new)``;
* each (page, layer, K/V, kv-head) slice holds PS x D codes; K is
  token-major as in the reference, V is tiled (token t, dim d at byte
  ``((t // 4 * 16 + d % 16) * (D // 16) + d // 16) * 4 + t % 4``) so that
  each lane of the decode kernel loads its matrix-core operand for one page
  as D / 4 consecutive bytes; ``logical_view`` returns the pool with V
  token-major for inspection;
* the write itself replaces the raw index-put of
  ``PagedKVCacheManager.write_kv`` (core/paged_attention.py:611-612).

Two memory layouts hold the same logical tensors:

* ``plain``: ``kv_pool`` a dense ``[P, L, 2, KH, PS, D]`` array and
  ``kv_scales`` a separate dense array;
* ``inline``: one byte buffer of ``P * L`` slabs, each holding per kv-head
  its K codes, V codes and K / V scales side by side (int8: ``PS * (2 D +
  8)`` bytes per kv-head; fp8: ``2 PS D + 128``), laid out layer by layer
  (slab ``l P + p`` holds page ``p`` of layer ``l``).  ``kv_pool`` and
  ``kv_scales`` are strided views of that buffer with the usual shapes, so
  indexing them reads the same values as in the plain layout.  A layer's page
  is one contiguous run per kv-head and a layer's pages one run: the balanced
  decodes read a sequence's pages in ascending page order, and workgroups
  streaming sequences of equal length then sweep that run together.

``allocate_pool`` makes int8 pools inline (the 14B decode over a 48-layer
pool: 98.0 -> 93.7 us per layer-step against the page-major order, and no
slower elsewhere measured) and fp8 pools
plain (the ragged work-item decode reads their one-float page scales faster
from the small separate array: 1-7 % in the measured shapes).
``pool_dtype_code`` tells the kernels which layout a pair of tensors has.
"""
from __future__ import annotations

from typing import Any, Optional, Tuple

from . import _lib

__all__ = [
    "logical_view",
    "allocate_pool",
    "default_layout",
    "abi_dtype_code",
    "pool_dtype_code",
    "pool_layout",
    "quantize_append",
    "quantize_pages",
    "dequantize_pages",
]

CODECS = ("int8", "fp8")


def _codec_dtype(codec: str):
    import torch

    if codec == "int8":
        return torch.int8
    if codec == "fp8":
        return torch.float8_e4m3fn
    raise ValueError(f"unknown codec {codec!r}; expected one of {CODECS}")


LAYOUTS = ("inline", "plain")


def _inline_geometry(num_pages: int, num_kv_heads: int, page_size: int, head_dim: int, fp8: bool):
    """(slab bytes, byte offset of the scales, code strides, scale strides) of
    the inline layout; strides in elements of the code / float32 views.  The
    slabs lie layer by layer: (page p, layer l) is slab l P + p."""
    P, KH, PS, D = num_pages, num_kv_heads, page_size, head_dim
    # per kv-head a record of K codes, V codes, K scales, V scales (fp8: one
    # scale each, the record padded to 128 bytes past the codes)
    head = 2 * PS * D + 128 if fp8 else PS * (2 * D + 8)
    slab = KH * head
    scale_off = 2 * PS * D
    if fp8:
        scales = (slab // 4, P * slab // 4, 1, head // 4)
    else:
        scales = (slab // 4, P * slab // 4, PS, head // 4, 1)
    codes = (slab, P * slab, PS * D, head, D, 1)
    return slab, scale_off, codes, scales


def default_layout(codec: str) -> str:
    """The memory layout ``allocate_pool`` picks for a codec."""
    _codec_dtype(codec)
    return "inline" if codec == "int8" else "plain"


def allocate_pool(num_pages: int, num_layers: int, num_kv_heads: int, head_dim: int, codec: str,
                  page_size: int = 16, device: Any = "cuda", layout: Optional[str] = None) -> Tuple[Any, Any]:
    """Zero-initialised (codes, scales) for a quantized pool, in the given
    layout ("inline" or "plain"; by default ``default_layout(codec)``)."""
    import torch

    dtype = _codec_dtype(codec)
    layout = layout or default_layout(codec)
    P, L, KH, PS, D = num_pages, num_layers, num_kv_heads, page_size, head_dim
    scale_shape = (P, L, 2, KH, PS) if codec == "int8" else (P, L, 2, KH)
    if layout == "plain":
        pool = torch.zeros((P, L, 2, KH, PS, D), dtype=torch.uint8, device=device).view(dtype)
        return pool, torch.zeros(scale_shape, dtype=torch.float32, device=device)
    if layout != "inline":
        raise ValueError(f"unknown layout {layout!r}; expected one of {LAYOUTS}")
    if D % 16 or PS % 4:
        raise ValueError(f"quantized pools need head_dim % 16 == 0 and page_size % 4 == 0 (got {D}, {PS})")
    slab, scale_off, code_strides, scale_strides = _inline_geometry(P, KH, PS, D, codec == "fp8")
    buf = torch.zeros(P * L * slab, dtype=torch.uint8, device=device)
    pool = buf.view(dtype).as_strided((P, L, 2, KH, PS, D), code_strides)
    scales = buf.view(torch.float32).as_strided(scale_shape, scale_strides, storage_offset=scale_off // 4)
    return pool, scales


def _same_strides(t, strides) -> bool:
    return all(n <= 1 or st == want for n, st, want in zip(t.shape, t.stride(), strides))


def pool_layout(kv_pool, kv_scales) -> Optional[str]:
    """``"plain"`` when both tensors are dense, ``"inline"`` when they are the
    two views of one inline buffer, ``None`` otherwise."""
    if kv_pool.is_contiguous() and kv_scales.is_contiguous():
        return "plain"
    if kv_pool.dim() != 6:
        return None
    P, L, two, KH, PS, D = kv_pool.shape
    fp8 = _lib.kv_dtype_code(kv_pool.dtype) == _lib.VRM_KV_FP8E4M3
    _, scale_off, code_strides, scale_strides = _inline_geometry(P, KH, PS, D, fp8)
    if (_same_strides(kv_pool, code_strides) and _same_strides(kv_scales, scale_strides)
            and kv_scales.data_ptr() == kv_pool.data_ptr() + scale_off):
        return "inline"
    return None


def abi_dtype_code(kv_pool, kv_scales=None) -> int:
    """kv_dtype code of the C ABI for any pool: the float pools by element
    type, the quantized ones by element type and layout (``RuntimeError`` for
    a quantized pair in neither layout)."""
    if kv_scales is None:
        return _lib.kv_dtype_code(kv_pool.dtype)
    code = pool_dtype_code(kv_pool, kv_scales)
    if code is None:
        raise RuntimeError("kv_pool / kv_scales are neither dense arrays nor the views allocate_pool returns")
    return code


def pool_dtype_code(kv_pool, kv_scales) -> Optional[int]:
    """The kv_dtype code of the C ABI for a quantized pool and its scales
    (VRM_KV_I8 / VRM_KV_FP8E4M3 plain, VRM_KV_*_INLINE inline), ``None``
    when they are in neither layout."""
    code = _lib.kv_dtype_code(kv_pool.dtype)
    layout = pool_layout(kv_pool, kv_scales)
    if layout is None or code not in (_lib.VRM_KV_I8, _lib.VRM_KV_FP8E4M3):
        return None
    if layout == "plain":
        return code
    return _lib.VRM_KV_I8_INLINE if code == _lib.VRM_KV_I8 else _lib.VRM_KV_FP8E4M3_INLINE


def logical_view(kv_pool):
    """Copy of a quantized pool with V token-major ([.., PS, D] as indexed)."""
    P, L, two, KH, PS, D = kv_pool.shape
    raw = kv_pool.view(torch_uint8())
    out = raw.clone()
    # physical axes (t // 4, d % 16, d // 16, t % 4) -> (t // 4, t % 4, d // 16, d % 16)
    tiles = raw[:, :, 1].reshape(P, L, KH, PS // 4, 16, D // 16, 4)
    out[:, :, 1] = tiles.transpose(-1, -3).reshape(P, L, KH, PS, D)
    return out.view(kv_pool.dtype)


def torch_uint8():
    import torch

    return torch.uint8


def _check_pool(kv_pool, kv_scales):
    import torch

    code = _lib.kv_dtype_code(kv_pool.dtype)
    if code not in (_lib.VRM_KV_I8, _lib.VRM_KV_FP8E4M3):
        raise RuntimeError(f"kv_pool dtype {kv_pool.dtype} is not a quantized pool (int8, float8_e4m3fn)")
    P, L, two, KH, PS, D = kv_pool.shape
    want = (P, L, 2, KH, PS) if code == _lib.VRM_KV_I8 else (P, L, 2, KH)
    if tuple(kv_scales.shape) != want or kv_scales.dtype != torch.float32:
        raise RuntimeError(f"kv_scales must be float32 of shape {want}")
    layout_code = pool_dtype_code(kv_pool, kv_scales)
    if layout_code is None:
        raise RuntimeError("kv_pool and kv_scales must be dense arrays or the two views allocate_pool returns "
                           "(they are written in place)")
    return layout_code, P, L, KH, PS, D


def quantize_append(kv_pool: Any, kv_scales: Any, layer_idx: int, page_ids: Any, slots: Any,
                    key: Any, value: Any) -> None:
    """Quantizes N new tokens into their (page, slot) of layer ``layer_idx``.

    ``key``/``value`` are [N, KH, D] float32/float16/bfloat16 on the pool's
    device; ``page_ids``/``slots`` are [N] integer tensors (as returned by the
    reference's ``append_token``, core/paged_attention.py:431-459).  For fp8
    pools, tokens of one call must go to distinct pages.
    """
    import torch

    _lib.require_cuda(kv_pool, kv_scales, page_ids, slots, key, value)
    code, P, L, KH, PS, D = _check_pool(kv_pool, kv_scales)
    if key.shape != value.shape or key.dim() != 3 or key.shape[1:] != (KH, D):
        raise RuntimeError(f"key/value must be [N, {KH}, {D}], got {tuple(key.shape)} / {tuple(value.shape)}")
    if key.dtype != value.dtype:
        raise RuntimeError("key and value must share a dtype")
    N = key.shape[0]
    page_ids = page_ids.to(torch.int32).contiguous()
    slots = slots.to(torch.int32).contiguous()
    if page_ids.shape != (N,) or slots.shape != (N,):
        raise RuntimeError("page_ids and slots must be [N]")
    key = key.contiguous()
    value = value.contiguous()
    rc = _lib.load().vrm_kv_quant_append(
        _lib.ptr(key), _lib.ptr(value), _lib.src_dtype_code(key.dtype), _lib.ptr(page_ids), _lib.ptr(slots), N,
        _lib.ptr(kv_pool), _lib.ptr(kv_scales), code, KH, D, PS, L, P, int(layer_idx), _lib.stream_of(kv_pool),
    )
    _lib.check(rc, "quantize_append")


def quantize_pages(kv_pool: Any, kv_scales: Any, layer_idx: int, page_ids: Any, key_pages: Any, value_pages: Any,
                   n_valid: Optional[Any] = None) -> None:
    """Bulk (prefill) write of whole pages.

    ``key_pages``/``value_pages`` are [NP, KH, PS, D]; page n is written to
    physical page ``page_ids[n]`` and holds ``n_valid[n]`` tokens (default: a
    full page).  Slots past ``n_valid`` get code 0; the fp8 page scale is taken
    over the valid tokens only.
    """
    import torch

    _lib.require_cuda(kv_pool, kv_scales, page_ids, key_pages, value_pages, n_valid)
    code, P, L, KH, PS, D = _check_pool(kv_pool, kv_scales)
    if key_pages.shape != value_pages.shape or key_pages.dim() != 4 or key_pages.shape[1:] != (KH, PS, D):
        raise RuntimeError(f"key/value pages must be [NP, {KH}, {PS}, {D}], got {tuple(key_pages.shape)}")
    if key_pages.dtype != value_pages.dtype:
        raise RuntimeError("key and value pages must share a dtype")
    NP = key_pages.shape[0]
    page_ids = page_ids.to(torch.int32).contiguous()
    if n_valid is None:
        n_valid = torch.full((NP,), PS, dtype=torch.int32, device=kv_pool.device)
    n_valid = n_valid.to(torch.int32).contiguous()
    if page_ids.shape != (NP,) or n_valid.shape != (NP,):
        raise RuntimeError("page_ids and n_valid must be [NP]")
    key_pages = key_pages.contiguous()
    value_pages = value_pages.contiguous()
    lib = _lib.load()
    # The kernels index rows with a 16-bit grid dimension; split large writes.
    step = 65535
    for s in range(0, NP, step):
        e = min(NP, s + step)
        rc = lib.vrm_kv_quant_pages(
            _lib.ptr(key_pages[s:e]), _lib.ptr(value_pages[s:e]), _lib.src_dtype_code(key_pages.dtype),
            _lib.ptr(page_ids[s:e]), _lib.ptr(n_valid[s:e]), e - s, _lib.ptr(kv_pool), _lib.ptr(kv_scales), code,
            KH, D, PS, L, P, int(layer_idx), _lib.stream_of(kv_pool),
        )
        _lib.check(rc, "quantize_pages")


def dequantize_pages(kv_pool: Any, kv_scales: Any, layer_idx: int, page_ids: Any) -> Any:
    """Returns float32 [NP, 2, KH, PS, D] = codes * scale of the given pages."""
    import torch

    _lib.require_cuda(kv_pool, kv_scales, page_ids)
    code, P, L, KH, PS, D = _check_pool(kv_pool, kv_scales)
    page_ids = page_ids.to(torch.int32).contiguous()
    NP = page_ids.shape[0]
    out = torch.empty((NP, 2, KH, PS, D), dtype=torch.float32, device=kv_pool.device)
    lib = _lib.load()
    step = 65535
    for s in range(0, NP, step):
        e = min(NP, s + step)
        rc = lib.vrm_kv_dequant_pages(
            _lib.ptr(kv_pool), _lib.ptr(kv_scales), code, _lib.ptr(page_ids[s:e]), e - s, _lib.ptr(out[s:e]),
            KH, D, PS, L, P, int(layer_idx), _lib.stream_of(kv_pool),
        )
        _lib.check(rc, "dequantize_pages")
    return out
