"""Host tests of the quantized pools' two memory layouts (no GPU): the inline
layout's views put every code and scale at the byte the C ABI documents
(include/vrm_paged.h: per (page, layer) slab, the slabs layer by layer, per
kv-head a record of K codes, V codes, K scales, V scales), the sizes agree with the library's
vrm_kv_slab_bytes, and the layout detection tells inline, plain and other
strides apart."""
import pytest
import torch

from vramancer_amd import _lib, kv_quant


def _buffer(t):
    """The whole byte buffer under a view."""
    return torch.empty(0, dtype=torch.uint8).set_(t.untyped_storage())


@pytest.mark.parametrize("codec", ["int8", "fp8"])
@pytest.mark.parametrize("P,L,KH,PS,D", [(3, 2, 2, 8, 32), (2, 3, 3, 4, 48), (2, 1, 8, 16, 128)])
def test_inline_views_hit_the_documented_bytes(codec, P, L, KH, PS, D):
    pool, sc = kv_quant.allocate_pool(P, L, KH, D, codec, PS, device="cpu", layout="inline")
    fp8 = codec == "fp8"
    head = 2 * PS * D + 128 if fp8 else PS * (2 * D + 8)
    slab = KH * head
    buf = _buffer(pool)
    assert buf.numel() == P * L * slab
    g = torch.Generator().manual_seed(P * 100 + D)
    raw = pool.view(torch.uint8)
    for _ in range(200):
        p, l, kv, h = (int(torch.randint(n, (1,), generator=g)) for n in (P, L, 2, KH))
        t, d = int(torch.randint(PS, (1,), generator=g)), int(torch.randint(D, (1,), generator=g))
        val = int(torch.randint(1, 255, (1,), generator=g))
        raw[p, l, kv, h, t, d] = val
        off = (l * P + p) * slab + h * head + kv * PS * D + t * D + d
        assert int(buf[off]) == val
        raw[p, l, kv, h, t, d] = 0
        s = (torch.rand(1, generator=g) + 0.5).item()  # a float32 value
        idx = (p, l, kv, h) if fp8 else (p, l, kv, h, t)
        sc[idx] = s
        soff = (l * P + p) * slab + h * head + 2 * PS * D + (kv * 4 if fp8 else kv * PS * 4 + t * 4)
        assert buf[soff:soff + 4].view(torch.float32).item() == s
        sc[idx] = 0
    assert int(buf.count_nonzero()) == 0  # nothing else was touched
    assert kv_quant.pool_layout(pool, sc) == "inline"
    want = _lib.VRM_KV_FP8E4M3_INLINE if fp8 else _lib.VRM_KV_I8_INLINE
    assert kv_quant.pool_dtype_code(pool, sc) == want == kv_quant.abi_dtype_code(pool, sc)


def test_inline_slab_matches_the_library():
    lib = _lib.load()
    for codec, code in (("int8", _lib.VRM_KV_I8_INLINE), ("fp8", _lib.VRM_KV_FP8E4M3_INLINE)):
        for KH, PS, D in ((8, 16, 128), (3, 4, 48), (1, 32, 256)):
            pool, _ = kv_quant.allocate_pool(2, 3, KH, D, codec, PS, device="cpu", layout="inline")
            assert _buffer(pool).numel() == 2 * 3 * lib.vrm_kv_slab_bytes(code, KH, PS, D)


def test_default_layouts():
    """int8 pools are inline by default, fp8 pools plain."""
    assert kv_quant.default_layout("int8") == "inline" and kv_quant.default_layout("fp8") == "plain"
    p8, s8 = kv_quant.allocate_pool(2, 2, 2, 32, "int8", 8, device="cpu")
    pf, sf = kv_quant.allocate_pool(2, 2, 2, 32, "fp8", 8, device="cpu")
    assert kv_quant.pool_layout(p8, s8) == "inline" and kv_quant.pool_layout(pf, sf) == "plain"


def test_layout_detection():
    pool, sc = kv_quant.allocate_pool(4, 3, 2, 32, "int8", 8, device="cpu", layout="plain")
    assert pool.is_contiguous() and sc.is_contiguous()
    assert kv_quant.pool_layout(pool, sc) == "plain"
    assert kv_quant.pool_dtype_code(pool, sc) == _lib.VRM_KV_I8
    ipool, isc = kv_quant.allocate_pool(4, 3, 2, 32, "int8", 8, device="cpu")
    assert not ipool.is_contiguous()
    # one layer's slabs are a run of their own: a layer slice is a one-layer inline pool
    assert kv_quant.pool_layout(ipool[:, 1:2], isc[:, 1:2]) == "inline"
    # a page slice keeps the layer stride of all 4 pages, which 2 pages do not have
    assert kv_quant.pool_layout(ipool[:2], isc[:2]) is None
    # views of two different buffers, or mixed layouts
    other, osc = kv_quant.allocate_pool(4, 3, 2, 32, "int8", 8, device="cpu")
    assert kv_quant.pool_layout(ipool, osc) is None
    assert kv_quant.pool_layout(ipool, sc) is None
    with pytest.raises(RuntimeError):
        kv_quant.abi_dtype_code(ipool, osc)
    # copies of inline views are plain arrays with the same values
    ipool.view(torch.uint8)[1, 2, 1, 0, 3, 5] = 7
    isc[1, 2, 1, 0, 3] = 2.5
    cp, csc = ipool.contiguous(), isc.contiguous()
    assert kv_quant.pool_layout(cp, csc) == "plain"
    assert int(cp.view(torch.uint8)[1, 2, 1, 0, 3, 5]) == 7 and csc[1, 2, 1, 0, 3].item() == 2.5
    # float pools take their dtype code
    assert kv_quant.abi_dtype_code(torch.zeros(2, 1, 2, 1, 4, 8, dtype=torch.bfloat16)) == _lib.VRM_KV_BF16
    with pytest.raises(ValueError):
        kv_quant.allocate_pool(2, 1, 1, 40, "int8", 8, device="cpu")  # head_dim not a multiple of 16
    with pytest.raises(ValueError):
        kv_quant.allocate_pool(2, 1, 1, 32, "int8", 8, device="cpu", layout="strided")


def test_logical_view_of_an_inline_pool():
    """logical_view undoes the V tiling the same way for both layouts."""
    P, L, KH, PS, D = 2, 2, 2, 8, 32
    ip, isc = kv_quant.allocate_pool(P, L, KH, D, "int8", PS, device="cpu")
    pp, psc = kv_quant.allocate_pool(P, L, KH, D, "int8", PS, device="cpu", layout="plain")
    vals = torch.randint(-127, 128, (P, L, 2, KH, PS, D), generator=torch.Generator().manual_seed(1),
                         dtype=torch.int8)
    ip.copy_(vals)
    pp.copy_(vals)
    assert torch.equal(kv_quant.logical_view(ip), kv_quant.logical_view(pp))
