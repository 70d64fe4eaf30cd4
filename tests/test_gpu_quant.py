"""GPU quantize-on-append / page writes / dequantization: codes and scales
bit-identical to the codec definitions in oracle/kv_codecs.py."""
import pytest
import torch

from oracle import kv_codecs as KC
from vramancer_amd import kv_quant

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _src(shape, dtype, seed, outliers=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if outliers:
        x[..., 3] *= 20
        x[..., 77 % shape[-1]] *= 20
    x.view(-1, shape[-1])[0] = 0  # an all-zero row
    return x.to(dtype)


# the two memory layouts of the quantized pools (kv_quant.allocate_pool)
LAYOUTS = ["inline", "plain"]


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float16, torch.float32],
                         ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_int8_append_bit_exact(src_dtype, D, layout):
    _say(f"int8 append {src_dtype} D{D} {layout}")
    P, L, KH, PS, N = 12, 3, 4, 16, 9
    pool, scales = kv_quant.allocate_pool(P, L, KH, D, "int8", device=DEV, layout=layout)
    k = _src((N, KH, D), src_dtype, 1)
    v = _src((N, KH, D), src_dtype, 2)
    page_ids = torch.tensor([3, 3, 7, 0, 11, 5, 5, 9, 1], dtype=torch.int32)
    slots = torch.tensor([0, 15, 4, 2, 9, 1, 3, 0, 8], dtype=torch.int32)
    kv_quant.quantize_append(pool, scales, 2, page_ids.to(DEV), slots.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    pool_c, sc_c = kv_quant.logical_view(pool).cpu(), scales.cpu()
    for n in range(N):
        for kv, src in ((0, k), (1, v)):
            codes, s = KC.quantize_int8(src[n])
            assert torch.equal(pool_c[page_ids[n], 2, kv, :, slots[n]], codes), (n, kv)
            assert torch.equal(sc_c[page_ids[n], 2, kv, :, slots[n]], s), (n, kv)
    # nothing else was written
    mask = torch.zeros(P, L, 2, KH, PS, dtype=torch.bool)
    mask[page_ids.long(), 2, :, :, slots.long()] = True
    assert (sc_c[~mask] == 0).all()
    assert (pool_c.view(torch.uint8)[~mask] == 0).all()


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("codec", ["int8", "fp8"])
def test_quantize_pages_bit_exact(codec, layout):
    _say(f"pages {codec} {layout}")
    P, L, KH, PS, D, NP = 20, 2, 8, 16, 128, 7
    pool, scales = kv_quant.allocate_pool(P, L, KH, D, codec, device=DEV, layout=layout)
    kp = _src((NP, KH, PS, D), torch.bfloat16, 3)
    vp = _src((NP, KH, PS, D), torch.bfloat16, 4)
    page_ids = torch.tensor([19, 0, 4, 8, 15, 2, 11], dtype=torch.int32)
    n_valid = torch.tensor([16, 16, 1, 9, 16, 0, 15], dtype=torch.int32)
    kv_quant.quantize_pages(pool, scales, 1, page_ids.to(DEV), kp.to(DEV), vp.to(DEV), n_valid.to(DEV))
    torch.cuda.synchronize()
    pool_c = kv_quant.logical_view(pool).cpu().view(torch.uint8)
    sc_c = scales.cpu()
    for n in range(NP):
        pid, nv = int(page_ids[n]), int(n_valid[n])
        for kv, src in ((0, kp), (1, vp)):
            for h in range(KH):
                if codec == "int8":
                    codes, s = KC.quantize_int8(src[n, h])
                    codes = codes.view(torch.uint8).clone()
                    s = s.clone()
                    codes[nv:] = 0
                    s[nv:] = 0
                    assert torch.equal(pool_c[pid, 1, kv, h], codes), (n, kv, h)
                    assert torch.equal(sc_c[pid, 1, kv, h], s), (n, kv, h)
                else:
                    codes, s = KC.quantize_fp8_page(src[n, h], nv)
                    assert torch.equal(pool_c[pid, 1, kv, h], codes), (n, kv, h)
                    assert sc_c[pid, 1, kv, h].item() == s.item(), (n, kv, h)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_fp8_append_sequence_bit_exact(layout):
    """Token-by-token appends into fp8 pages, with the scale growing on some
    appends, match the oracle's append policy code for code."""
    _say(f"fp8 append sequence {layout}")
    P, L, KH, PS, D = 4, 1, 2, 16, 128
    pool, scales = kv_quant.allocate_pool(P, L, KH, D, "fp8", device=DEV, layout=layout)
    g = torch.Generator().manual_seed(5)
    ref_codes = torch.zeros(P, 2, KH, PS, D, dtype=torch.uint8)
    ref_scale = torch.zeros(P, 2, KH)
    pages = [2, 0]
    for t in range(PS + 5):
        # growing magnitudes on some steps force re-encoding of earlier codes
        mag = 1.0 + (t % 4 == 3) * t * 0.7
        k = (torch.randn(len(pages), KH, D, generator=g) * mag).to(torch.bfloat16)
        v = (torch.randn(len(pages), KH, D, generator=g) * mag).to(torch.bfloat16)
        slot = t % PS
        page_ids = torch.tensor(pages, dtype=torch.int32) if t < PS else torch.tensor([1, 3], dtype=torch.int32)
        kv_quant.quantize_append(pool, scales, 0, page_ids.to(DEV), torch.full((2,), slot, dtype=torch.int32).to(DEV),
                                 k.to(DEV), v.to(DEV))
        for i, pid in enumerate(page_ids.tolist()):
            for kv, src in ((0, k), (1, v)):
                for h in range(KH):
                    c, s = KC.fp8_append(ref_codes[pid, kv, h], ref_scale[pid, kv, h], slot, src[i, h])
                    ref_codes[pid, kv, h] = c
                    ref_scale[pid, kv, h] = s
    torch.cuda.synchronize()
    assert torch.equal(kv_quant.logical_view(pool).cpu().view(torch.uint8)[:, 0], ref_codes)
    assert torch.equal(scales.cpu()[:, 0], ref_scale)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("codec", ["int8", "fp8"])
def test_dequantize_pages_exact(codec, layout):
    _say(f"dequant {codec} {layout}")
    P, L, KH, PS, D = 6, 2, 4, 16, 64
    pool, scales = kv_quant.allocate_pool(P, L, KH, D, codec, device=DEV, layout=layout)
    kp = _src((P, KH, PS, D), torch.float32, 6)
    vp = _src((P, KH, PS, D), torch.float32, 7)
    ids = torch.arange(P, dtype=torch.int32, device=DEV)
    kv_quant.quantize_pages(pool, scales, 1, ids, kp.to(DEV), vp.to(DEV))
    out = kv_quant.dequantize_pages(pool, scales, 1, torch.tensor([5, 0, 3], dtype=torch.int32, device=DEV)).cpu()
    pc, sc = kv_quant.logical_view(pool).cpu(), scales.cpu()
    for i, pid in enumerate([5, 0, 3]):
        if codec == "int8":
            ref = KC.dequantize_int8(pc[pid, 1], sc[pid, 1])
        else:
            ref = KC.dequantize_fp8(pc[pid, 1].view(torch.uint8), sc[pid, 1][..., None, None])
        assert torch.equal(out[i], ref)


@pytest.mark.parametrize("codec", ["int8", "fp8"])
@pytest.mark.parametrize("D,PS", [(80, 16), (96, 8), (112, 32), (48, 4), (128, 32)])
def test_quant_other_head_dims_and_page_sizes(codec, D, PS):
    """Whole-page writes, appends and dequantization at head_dims and page
    sizes beside 64 / 128 / 256 and 16 (any multiple of 16, and of 4): codes
    and scales bit-identical to the codec definitions."""
    _say(f"quant {codec} D{D} PS{PS}")
    P, L, KH, NP = 9, 2, 3, 4
    pool, scales = kv_quant.allocate_pool(P, L, KH, D, codec, PS, device=DEV)
    kp = _src((NP, KH, PS, D), torch.bfloat16, D + PS)
    vp = _src((NP, KH, PS, D), torch.bfloat16, D + PS + 1)
    page_ids = torch.tensor([8, 0, 5, 2], dtype=torch.int32)
    n_valid = torch.tensor([PS, 1, PS - 1, PS // 2], dtype=torch.int32)
    kv_quant.quantize_pages(pool, scales, 1, page_ids.to(DEV), kp.to(DEV), vp.to(DEV), n_valid.to(DEV))
    # one appended token into the half-full page (int8: slot PS // 2 of page 2)
    kn = _src((1, KH, D), torch.float16, 3 * D)
    vn = _src((1, KH, D), torch.float16, 3 * D + 1)
    if codec == "int8":
        kv_quant.quantize_append(pool, scales, 1, torch.tensor([2], dtype=torch.int32, device=DEV),
                                 torch.tensor([PS // 2], dtype=torch.int32, device=DEV), kn.to(DEV), vn.to(DEV))
    torch.cuda.synchronize()
    pool_c = kv_quant.logical_view(pool).cpu().view(torch.uint8)
    sc_c = scales.cpu()
    for n in range(NP):
        pid, nv = int(page_ids[n]), int(n_valid[n])
        for kv, src in ((0, kp), (1, vp)):
            for h in range(KH):
                if codec == "int8":
                    codes, s = KC.quantize_int8(src[n, h])
                    codes = codes.view(torch.uint8).clone()
                    s = s.clone()
                    codes[nv:] = 0
                    s[nv:] = 0
                    if pid == 2:
                        c1, s1 = KC.quantize_int8((kn if kv == 0 else vn)[0, h])
                        codes[PS // 2] = c1.view(torch.uint8)
                        s[PS // 2] = s1
                    assert torch.equal(pool_c[pid, 1, kv, h], codes), (n, kv, h)
                    assert torch.equal(sc_c[pid, 1, kv, h], s), (n, kv, h)
                else:
                    codes, s = KC.quantize_fp8_page(src[n, h], nv)
                    assert torch.equal(pool_c[pid, 1, kv, h], codes), (n, kv, h)
                    assert sc_c[pid, 1, kv, h].item() == s.item(), (n, kv, h)
    out = kv_quant.dequantize_pages(pool, scales, 1, page_ids.to(DEV)).cpu()
    pc = kv_quant.logical_view(pool).cpu()
    for i, pid in enumerate(page_ids.tolist()):
        if codec == "int8":
            ref = KC.dequantize_int8(pc[pid, 1], sc_c[pid, 1])
        else:
            ref = KC.dequantize_fp8(pc[pid, 1].view(torch.uint8), sc_c[pid, 1][..., None, None])
        assert torch.equal(out[i], ref)
