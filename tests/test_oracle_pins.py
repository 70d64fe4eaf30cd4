"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Each oracle function is checked against something it does not restate: the
reference's own outputs (tests/golden/turboquant_golden.npz, written by
tests/golden/make_golden.py from core/kv_quantizer.py), an fp64 closed-form
attention, textbook objects (the Sylvester Hadamard matrix), hand-derived
tiny cases, torch's float8_e4m3fn cast, and invariants chosen so that a
dropped term, a wrong index or a swapped operand fails.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import kv_codecs as KC
from oracle import paged_decode as PD
from oracle import turboquant as TQ

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "turboquant_golden.npz")


# ---------------------------------------------------------------------------
# paged decode restatement vs fp64 closed form
# ---------------------------------------------------------------------------

def _random_paged(B, H, KH, D, ctxs, L=2, layer=1, dtype=torch.float32, seed=0, spare=3):
    g = torch.Generator().manual_seed(seed)
    PS = 16
    npages = [(c + PS - 1) // PS for c in ctxs]
    P = sum(npages) + spare
    pool = torch.randn(P, L, 2, KH, PS, D, generator=g).to(dtype)
    perm = torch.randperm(P, generator=g)
    table = torch.full((B, max(max(npages), 1) + 1), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(npages):
        table[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = torch.randn(B, H, D, generator=g)
    return q, pool, table, torch.tensor(ctxs, dtype=torch.int32)


@pytest.mark.parametrize("B,H,KH,D,ctxs", [
    (2, 12, 12, 64, [48, 37]),
    (3, 32, 8, 128, [64, 1, 17]),
    (2, 40, 8, 128, [100, 256]),
    (1, 28, 4, 128, [33]),
])
def test_decode_restatement_matches_fp64_closed_form(B, H, KH, D, ctxs):
    q, pool, table, lens = _random_paged(B, H, KH, D, ctxs)
    scale = 1.0 / math.sqrt(D)
    out = PD.paged_attention_decode(q, pool, table, lens, 1, scale)
    for b in range(B):
        K, V = PD.gather_sequence(pool, table[b], int(lens[b]), 1)
        ref = PD.dense_attention(q[b], K, V, scale)
        torch.testing.assert_close(out[b].double(), ref, atol=2e-5, rtol=1e-5)


def test_decode_gqa_mapping_is_integer_division():
    # A mapping of h % KH would differ from h // (H / KH) on this case.
    q, pool, table, lens = _random_paged(1, 8, 2, 64, [40])
    scale = 0.125
    out = PD.paged_attention_decode(q, pool, table, lens, 1, scale)
    K, V = PD.gather_sequence(pool, table[0], 40, 1)
    wrong = torch.zeros(8, 64, dtype=torch.float64)
    for h in range(8):
        s = (K[h % 2] @ q[0, h].double()) * scale
        w = torch.softmax(s, 0)
        wrong[h] = w @ V[h % 2]
    assert (out[0].double() - wrong).abs().max() > 1e-2


def test_decode_zero_context_gives_zeros():
    # tests/test_cuda_tp.py:102-115 of the reference
    q, pool, table, _ = _random_paged(2, 4, 4, 64, [16, 16])
    out = PD.paged_attention_decode(q, pool, table, torch.tensor([0, 0], dtype=torch.int32), 1, 0.125)
    assert out.shape == (2, 4, 64) and (out == 0).all()


def test_decode_single_token_returns_its_value():
    # one token: softmax weight 1, output = V of that token for every head of its group
    q, pool, table, lens = _random_paged(1, 4, 2, 64, [1])
    out = PD.paged_attention_decode(q, pool, table, lens, 1, 0.125)
    pid = int(table[0, 0])
    for h in range(4):
        torch.testing.assert_close(out[0, h], pool[pid, 1, 1, h // 2, 0].float())


def test_decode_quantized_pools_dequantize_first():
    g = torch.Generator().manual_seed(3)
    P, L, KH, PS, D = 6, 1, 2, 16, 64
    x = torch.randn(P, L, 2, KH, PS, D, generator=g)
    codes, scales = KC.quantize_int8(x)
    q = torch.randn(1, 4, D, generator=g)
    table = torch.tensor([[4, 1, 3]], dtype=torch.int32)
    lens = torch.tensor([40], dtype=torch.int32)
    # the pool stores V tiled; the closed form reads the logical codes
    out = PD.paged_attention_decode(q, KC.pool_from_logical(codes), table, lens, 0, 0.125, kv_scales=scales)
    deq = KC.dequantize_int8(codes, scales)
    K, V = PD.gather_sequence(deq, table[0], 40, 0)
    torch.testing.assert_close(out[0].double(), PD.dense_attention(q[0], K, V, 0.125), atol=2e-5, rtol=1e-5)


def test_quantized_pool_v_layout_by_hand():
    # V of a page-head slice is tiled: token t, dim d at
    # ((t // 4 * 16 + d % 16) * (D // 16) + d // 16) * 4 + t % 4
    D = 32
    logical = torch.arange(2 * 16 * D, dtype=torch.int32).reshape(1, 1, 2, 1, 16, D)
    phys = KC.pool_from_logical(logical)
    assert torch.equal(phys[0, 0, 0], logical[0, 0, 0])          # K untouched
    flat = phys[0, 0, 1, 0].reshape(-1)
    seen = set()
    for t in range(16):
        for d in range(D):
            off = ((t // 4 * 16 + d % 16) * (D // 16) + d // 16) * 4 + t % 4
            assert flat[off] == logical[0, 0, 1, 0, t, d]
            seen.add(off)
    assert len(seen) == 16 * D
    # lane (col, grp) of the decode reads tokens 4 grp .. 4 grp + 3 of dims
    # col, col + 16, ... as D / 4 consecutive bytes
    col, grp = 5, 2
    run = flat[(grp * 16 + col) * (D // 4):(grp * 16 + col + 1) * (D // 4)].reshape(D // 16, 4)
    for blk in range(D // 16):
        assert torch.equal(run[blk], logical[0, 0, 1, 0, 4 * grp:4 * grp + 4, 16 * blk + col])
    assert torch.equal(KC.pool_to_logical(phys), logical)


def test_q4_dequant_by_hand():
    # byte 0x4B: low nibble 0xB = 11 is d=0, high nibble 4 is d=1
    packed = torch.full((1, 16), 0x4B, dtype=torch.uint8)
    scales = torch.tensor([[0.5]], dtype=torch.float16)
    zeros = torch.tensor([[3.0]], dtype=torch.float16)
    vals = PD.dequant_q4_page(packed, scales, zeros)
    assert vals.shape == (1, 32)
    assert vals[0, 0].item() == (11 - 3) * 0.5 and vals[0, 1].item() == (4 - 3) * 0.5


def test_q4_restatement_matches_closed_form():
    g = torch.Generator().manual_seed(9)
    P, L, KH, PS, D = 5, 1, 2, 16, 64
    packed = torch.randint(0, 256, (P, L, 2, KH, PS, D // 2), generator=g, dtype=torch.uint8)
    sc = (torch.rand(P, L, 2, KH, PS, D // 32, generator=g) * 0.2 + 0.01).half()
    zp = (torch.rand(P, L, 2, KH, PS, D // 32, generator=g) * 15).half()
    q = torch.randn(1, 4, D, generator=g)
    table = torch.tensor([[2, 0, 4]], dtype=torch.int32)
    lens = torch.tensor([35], dtype=torch.int32)
    out = PD.paged_attention_decode_q4(q, packed, sc, zp, table, lens, 0, 0.125)
    # explicit nibble loop
    pool = torch.zeros(P, L, 2, KH, PS, D)
    for d in range(D):
        nib = (packed[..., d // 2] >> (4 * (d % 2))) & 0xF
        pool[..., d] = (nib.float() - zp[..., d // 32].float()) * sc[..., d // 32].float()
    K, V = PD.gather_sequence(pool, table[0], 35, 0)
    torch.testing.assert_close(out[0].double(), PD.dense_attention(q[0], K, V, 0.125), atol=2e-5, rtol=1e-5)


# ---------------------------------------------------------------------------
# int8 / fp8 codecs
# ---------------------------------------------------------------------------

def test_int8_codec_identities():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 128, generator=g).to(torch.bfloat16)
    codes, scale = KC.quantize_int8(x)
    xf = x.float()
    amax = xf.abs().amax(-1)
    assert torch.equal(scale, amax / 127)
    # the element of largest magnitude maps to +-127 exactly
    idx = xf.abs().argmax(-1)
    assert torch.equal(codes.gather(1, idx[:, None]).abs().squeeze(1).to(torch.int32),
                       torch.full((64,), 127, dtype=torch.int32))
    err = (KC.dequantize_int8(codes, scale) - xf).abs()
    # half a quantization step, plus the rounding of code * scale in float32
    assert (err <= scale[:, None] * 0.5 + xf.abs() * 2.0 ** -23).all()


def test_int8_codec_by_hand():
    x = torch.tensor([[1.0, -2.0, 0.0, 0.5, 2.54]])
    codes, scale = KC.quantize_int8(x)
    s = np.float32(2.54) / np.float32(127)
    assert scale.item() == pytest.approx(float(s), rel=0, abs=0)
    expect = [round(v / float(s)) for v in (1.0, -2.0, 0.0, 0.5)] + [127]
    assert codes[0].tolist() == expect
    # round half to even: 2.5 -> 2, 3.5 -> 4
    y = torch.tensor([[127.0, 2.5, 3.5, -2.5]])
    c, s = KC.quantize_int8(y)
    assert s.item() == 1.0 and c[0].tolist() == [127, 2, 4, -2]


def test_int8_zero_row():
    codes, scale = KC.quantize_int8(torch.zeros(2, 64))
    assert (codes == 0).all() and (scale == 0).all()


def test_fp8_codec_pinned_by_torch_cast():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(16, 128, generator=g) * 3
    codes, scale = KC.quantize_fp8_page(x, 16)
    assert scale.item() == (x.abs().max() / 448).item()
    ref = (x / scale).to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(codes, ref)
    # the largest element encodes to +-448 (0x7e / 0xfe)
    i = x.abs().argmax()
    assert int(codes.flatten()[i]) & 0x7F == 0x7E
    # partial page: tail slots are code 0, scale over the valid rows only
    c2, s2 = KC.quantize_fp8_page(x, 5)
    assert s2.item() == (x[:5].abs().max() / 448).item() and (c2[5:] == 0).all()


def test_fp8_append_growth_by_hand():
    page = torch.zeros(16, 4, dtype=torch.uint8)
    c, s = KC.fp8_append(page, torch.tensor(0.0), 0, torch.tensor([448.0, 1.0, -2.0, 0.0]))
    assert s.item() == 1.0 and c[0].tolist() == [0x7E, 0x38, 0xC0, 0x00]
    # smaller token: scale unchanged, existing codes untouched
    c2, s2 = KC.fp8_append(c, s, 1, torch.tensor([224.0, 0.0, 0.0, 0.0]))
    assert s2.item() == 1.0 and torch.equal(c2[0], c[0]) and c2[1, 0].item() == 0x76  # 224
    # larger token doubles the scale: old 448 -> 224, 1 -> 0.5, -2 -> -1
    c3, s3 = KC.fp8_append(c2, s2, 2, torch.tensor([896.0, 0.0, 0.0, 0.0]))
    assert s3.item() == 2.0
    assert c3[0].tolist() == [0x76, 0x30, 0xB8, 0x00] and c3[2, 0].item() == 0x7E


# ---------------------------------------------------------------------------
# TurboQuant restatement
# ---------------------------------------------------------------------------

def _golden():
    return np.load(GOLDEN, allow_pickle=False)


def _golden_cases():
    g = _golden()
    return sorted({k.split("/")[0] for k in g.files})


@pytest.mark.parametrize("case", _golden_cases())
def test_turboquant_restatement_matches_reference_goldens(case):
    g = _golden()
    hd, bits, seed, rows = (int(v) for v in g[case + "/meta"])
    p = TQ.make_params(hd, bits, seed=seed)
    assert np.array_equal(p.signs.numpy(), g[case + "/signs"])
    assert np.array_equal(p.jl_matrix.numpy(), g[case + "/jl"])
    kv = torch.from_numpy(g[case + "/kv"])
    if bool(g[case + "/kv_is_bf16"]):
        kv = kv.to(torch.bfloat16)
    raw = TQ.compress(p, kv, pack=False)
    packed = TQ.compress(p, kv, pack=True)
    assert np.array_equal(raw["radius"].view(torch.int16).numpy(), g[case + "/radius"])
    assert np.array_equal(torch.cat(raw["angles"], -1).numpy(), g[case + "/angles"])
    assert np.array_equal(raw["qjl_signs"].numpy(), g[case + "/qjl_signs"])
    assert np.array_equal(raw["qjl_norms"].view(torch.int16).numpy(), g[case + "/qjl_norms"])
    assert np.array_equal(packed["angles_packed"].numpy(), g[case + "/angles_packed"])
    assert np.array_equal(packed["qjl_signs_packed"].numpy(), g[case + "/qjl_signs_packed"])
    assert np.array_equal(TQ.decompress(p, raw).numpy(), g[case + "/decompress"])
    # scores are sums of float32 products whose order the host's BLAS picks
    # (it differs between CPU models), so they are pinned to float32 rounding
    score = TQ.attention_score(p, torch.from_numpy(g[case + "/q"]), raw)
    np.testing.assert_allclose(score.numpy(), g[case + "/score"], rtol=1e-5, atol=1e-5)
    assert TQ.bits_per_dim(p) == float(g[case + "/bits_per_dim"])


def _sylvester(d):
    H = torch.ones(1, 1, dtype=torch.float64)
    while H.shape[0] < d:
        H = torch.cat([torch.cat([H, H], 1), torch.cat([H, -H], 1)], 0)
    return H


@pytest.mark.parametrize("d", [2, 4, 8, 16, 64])
def test_hadamard_is_normalised_sylvester(d):
    out = TQ.hadamard(torch.eye(d, dtype=torch.float64))
    torch.testing.assert_close(out, _sylvester(d) / math.sqrt(d))


def test_rotation_orthogonal_and_inverse():
    p = TQ.make_params(64, 3, seed=42)
    x = torch.randn(50, 64)
    r = TQ.rotate(p, x)
    torch.testing.assert_close(r.norm(dim=-1), x.norm(dim=-1), atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(TQ.unrotate(p, r), x, atol=1e-5, rtol=1e-5)


def test_polar_roundtrip_high_bits_and_shapes():
    p = TQ.make_params(128, 8, seed=42)
    x = TQ.rotate(p, torch.randn(16, 128))
    radius, angles = TQ.polar_encode(p, x)
    assert radius.shape == (16, 1) and (radius >= 0).all()
    assert [a.shape[-1] for a in angles] == [64, 32, 16, 8, 4, 2, 1]
    q = [TQ.quantize_angle(p, a, lvl) for lvl, a in enumerate(angles)]
    rec = TQ.polar_decode(p, radius, q)
    assert ((x - rec).norm() / x.norm()) < 0.05
    # the radius is the row norm (up to the 1e-12 per level)
    torch.testing.assert_close(radius.squeeze(1), x.norm(dim=-1), atol=1e-4, rtol=1e-5)


def test_polar_bins_tiny_by_hand():
    p = TQ.TQParams(2, 3, 2, 1, 1, torch.ones(2), torch.ones(1, 2))
    cases = {(1.0, 0.0): 4, (0.0, 1.0): 6, (-1.0, 0.0): 7, (0.0, -1.0): 2, (1.0, -1e-6): 3}
    for (a, b), want in cases.items():
        radius, angles = TQ.polar_encode(p, torch.tensor([[a, b]]))
        assert int(TQ.quantize_angle(p, angles[0], 0)) == want, (a, b)
    # level >= 1 bins span [0, pi/2]: angle pi/4 is the middle (bin 4 of 8); pi/2 clamps to 7
    assert int(TQ.quantize_angle(p, torch.tensor([math.pi / 4]), 1)) == 4
    assert int(TQ.quantize_angle(p, torch.tensor([math.pi / 2]), 1)) == 7
    # centres
    c = TQ.dequantize_angle(p, torch.tensor([0, 7], dtype=torch.uint8), 0)
    torch.testing.assert_close(c, torch.tensor([-math.pi + math.pi / 8, math.pi - math.pi / 8]))


def test_bit_packing_msb_first():
    assert TQ.pack_bits(torch.tensor([[1, 0, 0, 0, 0, 0, 0, 1]], dtype=torch.uint8)).tolist() == [[0x81]]
    assert TQ.pack_bits(torch.tensor([[1, 1, 0]], dtype=torch.uint8)).tolist() == [[0xC0]]
    assert TQ.pack_angles([torch.tensor([[5]], dtype=torch.uint8)], 3).tolist() == [[0xA0]]
    a = [torch.randint(0, 8, (3, n), dtype=torch.uint8) for n in (4, 2, 1)]
    packed = TQ.pack_angles(a, 3)
    back = TQ.unpack_angles(packed, 3, [4, 2, 1], 3)
    assert all(torch.equal(x, y) for x, y in zip(a, back))


def test_bits_per_dim_closed_form():
    assert TQ.bits_per_dim(TQ.make_params(128, 3, seed=0)) == (127 * 3 + 16 + 64 + 16) / 128
    assert TQ.bits_per_dim(TQ.make_params(128, 4, seed=0)) == (127 * 4 + 16 + 64 + 16) / 128


def test_qjl_estimator_correlates():
    # tests/test_turboquant.py:111-138 of the reference
    p = TQ.make_params(64, 3, qjl_dim=256, seed=7)
    keys, queries = torch.randn(500, 64), torch.randn(50, 64)
    signs, norms, _ = TQ.qjl_encode(p, keys)
    est = TQ.qjl_score_correction(p, queries, signs, norms)
    corr = torch.corrcoef(torch.stack([(queries @ keys.t()).flatten(), est.flatten()]))[0, 1]
    assert corr > 0.3


def _turbo_codes(p, P, KH, seed):
    """Raw codes of random K/V pages, indexed [page, K/V, kv-head, token]."""
    g = torch.Generator().manual_seed(seed)
    codes = {}
    parts = []
    for kv in range(2):
        x = torch.randn(P * KH * 16, 128, generator=g)
        parts.append(TQ.compress(p, x, pack=False))
    codes["radius"] = torch.stack([c["radius"].reshape(P, KH, 16) for c in parts], 1)
    codes["angles"] = torch.stack([torch.cat(c["angles"], -1).reshape(P, KH, 16, 127) for c in parts], 1)
    codes["qjl_signs"] = torch.stack([c["qjl_signs"].reshape(P, KH, 16, 64) for c in parts], 1)
    codes["qjl_norms"] = torch.stack([c["qjl_norms"].reshape(P, KH, 16) for c in parts], 1)
    return codes


def test_turbo_paged_oracle_without_qjl_is_dense_attention_over_decompressed_kv():
    # with zero residual norms the score is q_rot . k_polar = q . decompress(k)
    # (the rotation is orthonormal), so the paged turbo attention reduces to
    # the fp64 closed form over the decompressed keys and values
    p = TQ.make_params(128, 3, seed=5)
    P, KH, H = 6, 2, 6
    codes = _turbo_codes(p, P, KH, 1)
    codes["qjl_norms"].zero_()
    g = torch.Generator().manual_seed(2)
    q = torch.randn(2, H, 128, generator=g)
    table = torch.tensor([[4, 1, 3], [0, 5, -1]], dtype=torch.int32)
    lens = torch.tensor([40, 20], dtype=torch.int32)
    out = PD.paged_attention_decode_turbo(p, q, codes, table, lens, scale=0.09)
    out_mod = PD.paged_attention_decode_turbo(p, q, codes, table, lens, scale=0.09, head_map="mod")
    for b in range(2):
        ks, vs = [], []
        for t in range(int(lens[b])):
            pid, s = int(table[b, t // 16]), t % 16
            rows = []
            for kv in range(2):
                c = {"radius": codes["radius"][pid, kv, :, s].reshape(-1, 1),
                     "angles": list(torch.split(codes["angles"][pid, kv, :, s], [64, 32, 16, 8, 4, 2, 1], -1)),
                     "shape": (KH, 128)}
                rows.append(TQ.decompress(p, c))
            ks.append(rows[0])
            vs.append(rows[1])
        K = torch.stack(ks, 1).double()
        V = torch.stack(vs, 1).double()
        ref = PD.dense_attention(q[b], K, V, 0.09)
        torch.testing.assert_close(out[b].double(), ref, atol=2e-5, rtol=1e-5)
        # compute_attention_turbo's own mapping: head h reads kv-head h % KH
        for h in range(H):
            w = torch.softmax(0.09 * (K[h % KH] @ q[b, h].double()), 0)
            torch.testing.assert_close(out_mod[b, h].double(), w @ V[h % KH], atol=2e-5, rtol=1e-5)


def test_turbo_paged_oracle_relabel_invariance():
    p = TQ.make_params(128, 4, seed=6)
    P, KH, H = 5, 1, 3
    codes = _turbo_codes(p, P, KH, 3)
    q = torch.randn(1, H, 128, generator=torch.Generator().manual_seed(4))
    table = torch.tensor([[2, 0, 4]], dtype=torch.int32)
    lens = torch.tensor([45], dtype=torch.int32)
    out = PD.paged_attention_decode_turbo(p, q, codes, table, lens)
    perm = torch.tensor([3, 4, 0, 1, 2])  # new page i holds old page perm[i]
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(P)
    codes2 = {k: v[perm] for k, v in codes.items()}
    out2 = PD.paged_attention_decode_turbo(p, q, codes2, inv[table.long()].to(torch.int32), lens)
    assert torch.equal(out, out2)


def test_turbo_paged_oracle_sparse_v_closed_forms():
    # sparse V keeps the top-k softmax weights of each head and renormalises
    # them: with zero residual norms this is the fp64 softmax over the k
    # largest scores of the decompressed keys; k = 1 returns the value row of
    # the best-scoring token; a ratio reaching every token is the dense path
    p = TQ.make_params(128, 3, seed=9)
    P, KH, H = 5, 2, 4
    codes = _turbo_codes(p, P, KH, 12)
    codes["qjl_norms"].zero_()
    q = torch.randn(1, H, 128, generator=torch.Generator().manual_seed(13))
    table = torch.tensor([[3, 0, 4, 1]], dtype=torch.int32)
    lens = torch.tensor([57], dtype=torch.int32)
    dense = PD.paged_attention_decode_turbo(p, q, codes, table, lens, scale=0.1, head_map="mod")
    full = PD.paged_attention_decode_turbo(p, q, codes, table, lens, scale=0.1, head_map="mod", sparse_v_ratio=0.999)
    assert torch.equal(dense, full)  # ceil(0.999 * 57) = 57 keeps every token
    ks, vs = [], []
    for t in range(57):
        pid, s = int(table[0, t // 16]), t % 16
        rows = []
        for kv in range(2):
            c = {"radius": codes["radius"][pid, kv, :, s].reshape(-1, 1),
                 "angles": list(torch.split(codes["angles"][pid, kv, :, s], [64, 32, 16, 8, 4, 2, 1], -1)),
                 "shape": (KH, 128)}
            rows.append(TQ.decompress(p, c).double())
        ks.append(rows[0])
        vs.append(rows[1])
    K, V = torch.stack(ks, 1), torch.stack(vs, 1)
    for ratio, k in ((0.3, 18), (0.01, 1)):
        out = PD.paged_attention_decode_turbo(p, q, codes, table, lens, scale=0.1, head_map="mod",
                                              sparse_v_ratio=ratio)
        for h in range(H):
            s = 0.1 * (K[h % KH] @ q[0, h].double())
            top = torch.argsort(s, descending=True)[:k]
            w = torch.softmax(s[top], 0)
            torch.testing.assert_close(out[0, h].double(), w @ V[h % KH][top], atol=2e-5, rtol=1e-5)
            if k == 1:
                torch.testing.assert_close(out[0, h].double(), V[h % KH][int(s.argmax())], atol=1e-6, rtol=1e-6)
