"""Native TurboQuant scores and top-k (sparse V) attention on the GPU.

* vrm_turboquant_score against the oracle's attention_score
  (core/kv_quantizer.py:502-535 restated in oracle/turboquant.py) on the same
  codes: float32 tolerance, |gpu - oracle| <= 1e-4 (1 + |oracle|), since the
  dot products are summed in another order than the oracle's BLAS.
* vrm_topk_attend against an independent float64 evaluation on the CPU: the
  kept set is exactly the k largest scores (lowest indices first among equal
  scores), and the output matches softmax-over-kept @ values within 1e-5.
* The manager's sparse V over TurboQuant pages against the oracle's
  compute_attention_turbo restatement with sparse_v_ratio, within
  |gpu - oracle| <= 2e-3 + 1e-2 |oracle|.
"""
import math

import pytest
import torch

from oracle import paged_decode as PD
from oracle import turboquant as TQ
from vramancer_amd import tq_pages
from vramancer_amd.paged_attention import PagedKVCacheManager, PagedKVConfig
from vramancer_amd.turboquant_cuda import CUDATurboQuantOps, topk_attend

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("head_dim,bits,qjl,M,N", [(128, 3, None, 5, 700), (64, 4, 96, 70, 129), (96, 2, None, 1, 33),
                                                    (256, 4, None, 3, 300), (128, 4, None, 40, 4101),
                                                    (128, 2, None, 17, 33), (128, 3, None, 1, 1), (128, 8, None, 3, 50),
                                                    (32, 3, None, 5, 70), (16, 4, 24, 3, 33), (8, 3, None, 2, 17),
                                                    (2, 3, None, 3, 9)])
def test_native_score_matches_oracle(head_dim, bits, qjl, M, N):
    _say(f"score d{head_dim} b{bits} qjl {qjl} M{M} N{N}")
    p = TQ.make_params(head_dim, bits, qjl_dim=qjl, seed=head_dim + bits)
    g = torch.Generator().manual_seed(3)
    keys = torch.randn(N, head_dim, generator=g)
    q = torch.randn(M, head_dim, generator=g)
    ck = TQ.compress(p, keys, pack=False)
    want = TQ.attention_score(p, q, ck)
    gk = {"radius": ck["radius"].to(DEV), "angles": [a.to(DEV) for a in ck["angles"]],
          "qjl_signs": ck["qjl_signs"].to(DEV), "qjl_norms": ck["qjl_norms"].to(DEV)}
    got = CUDATurboQuantOps.attention_score_gpu(q.to(DEV), gk, head_dim, p.padded_dim, p.n_levels, bits,
                                                p.signs.to(DEV), p.jl_matrix.to(DEV), p.qjl_dim, scale=0.5).cpu()
    assert got.shape == (M, N)
    err = (got - 0.5 * want).abs()
    assert (err <= 1e-4 * (1 + (0.5 * want).abs())).all(), f"max err {err.max():.3e}"


def test_native_score_unaligned_codes_take_the_serial_kernel():
    """Angle bytes and sign bytes that start off their 4- / 16-byte alignment
    (views into a larger buffer) are scored by the serial-order kernels, to
    the same bar."""
    _say("score unaligned codes")
    p = TQ.make_params(128, 3, seed=5)
    g = torch.Generator().manual_seed(6)
    keys = torch.randn(300, 128, generator=g)
    q = torch.randn(7, 128, generator=g)
    ck = TQ.compress(p, keys, pack=False)
    want = TQ.attention_score(p, q, ck)
    ang = torch.cat(ck["angles"], -1)
    buf = torch.zeros(ang.numel() + 1, dtype=torch.uint8, device=DEV)
    buf[1:] = ang.reshape(-1).to(DEV)
    ang_off = buf[1:].view(300, 127)  # one byte past an aligned start
    sbuf = torch.zeros(ck["qjl_signs"].numel() + 4, dtype=torch.uint8, device=DEV)
    sbuf[4:] = ck["qjl_signs"].reshape(-1).to(DEV)
    gk = {"radius": ck["radius"].to(DEV), "angles": [ang_off], "qjl_signs": sbuf[4:].view(300, 64),
          "qjl_norms": ck["qjl_norms"].to(DEV)}
    got = CUDATurboQuantOps.attention_score_gpu(q.to(DEV), gk, 128, 128, 7, 3, p.signs.to(DEV), p.jl_matrix.to(DEV),
                                                64).cpu()
    err = (got - want).abs()
    assert (err <= 1e-4 * (1 + want.abs())).all(), f"max err {err.max():.3e}"


def _topk_reference(s, k, v):
    """float64: the k largest of each row (lowest index first among ties)."""
    out = torch.zeros(s.shape[0], v.shape[1], dtype=torch.float64)
    for m in range(s.shape[0]):
        order = sorted(range(s.shape[1]), key=lambda n: (-float(s[m, n]), n))[:k]
        idx = torch.tensor(order)
        w = torch.softmax(s[m, idx].double(), 0)
        out[m] = w @ v[idx].double()
    return out


@pytest.mark.parametrize("M,N,D,k", [(3, 1000, 128, 100), (2, 77, 7, 1), (4, 300, 256, 300), (1, 5000, 64, 4999),
                                     (70, 40, 128, 13), (2, 600, 300, 57), (40, 32768, 128, 3277)])
def test_topk_attend_matches_float64(M, N, D, k):
    _say(f"topk M{M} N{N} D{D} k{k}")
    g = torch.Generator().manual_seed(N + k)
    s = torch.randn(M, N, generator=g) * 3
    v = torch.randn(N, D, generator=g)
    got = topk_attend(s.to(DEV), k, v.to(DEV)).cpu()
    torch.testing.assert_close(got.double(), _topk_reference(s, k, v), atol=1e-5, rtol=1e-5)


def test_topk_attend_ties_and_negative_zero():
    _say("topk ties")
    s = torch.tensor([[1.0, 3.0, 2.0, 3.0, 3.0, -0.5, 3.0, 0.0],
                      [-1.0, -1.0, -1.0, -1.0, -2.0, -3.0, -1.0, -1.0]])
    v = torch.eye(8)
    for k in (1, 2, 3, 4, 5, 8):
        got = topk_attend(s.to(DEV), k, v.to(DEV)).cpu()
        torch.testing.assert_close(got.double(), _topk_reference(s, k, v), atol=1e-6, rtol=1e-6)
        kept = got > 0
        assert int(kept[0].sum()) == k and int(kept[1].sum()) == k


def _codes(m, layer):
    P = m.config.max_pages
    c = tq_pages.read_pages(m._tq_pool, layer, torch.arange(P, dtype=torch.int32, device=DEV), m._kv_compressor)
    return {k: t.cpu() for k, t in c.items()}


@pytest.mark.parametrize("ratio", [0.3, 0.05, 0.999])
def test_manager_sparse_v_matches_oracle(ratio):
    _say(f"manager sparse V ratio {ratio}")
    torch.manual_seed(21)
    cfg = PagedKVConfig(page_size=16, num_layers=2, num_kv_heads=2, head_dim=128, max_pages=32, device=DEV,
                        dtype="bfloat16", kv_compression="turboquant", compression_bits=3, sparse_v_ratio=ratio)
    m = PagedKVCacheManager(cfg)
    g = torch.Generator().manual_seed(5)
    for rid, n in (("a", 70), ("b", 3)):
        m.allocate(rid)
        for _ in range(n):
            page, slot = m.append_token(rid)
            for layer in range(2):
                m.write_kv(rid, layer, page, slot, torch.randn(2, 128, generator=g).to(DEV),
                           torch.randn(2, 128, generator=g).to(DEV))
        m.flush_compression()
    comp = m._kv_compressor
    p = TQ.TQParams(128, 3, 128, 7, 64, comp._hadamard_signs.cpu(), comp.jl_matrix.cpu())
    q = torch.randn(3, 6, 128, generator=g)
    for i, rid in enumerate(("a", "b")):
        out = m.compute_attention_turbo(q[i].to(DEV), rid, 1)
        e = m._page_tables[rid]
        table = torch.tensor([e.pages], dtype=torch.int32)
        ref = PD.paged_attention_decode_turbo(p, q[i:i + 1], _codes(m, 1), table,
                                              torch.tensor([e.num_tokens], dtype=torch.int32), head_map="mod",
                                              sparse_v_ratio=ratio)[0]
        err = (out.cpu() - ref).abs()
        assert (err <= 2e-3 + 1e-2 * ref.abs()).all(), f"{rid}: max err {err.max():.3e}"
    batch = m.compute_attention_turbo_batch(q[:2].to(DEV), ["a", "b"], 1)
    for i, rid in enumerate(("a", "b")):
        single = m.compute_attention_turbo(q[i].to(DEV), rid, 1)
        assert torch.allclose(batch[i], single, atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("bits,M", [(1, 64), (1, 13), (3, 127), (4, 127), (2, 5), (8, 9), (5, 31)])
def test_pack_kernels_match_numpy_packbits(bits, M):
    """The packed format against numpy's packbits (big bit order), a library
    routine: each value's low `bits` bits, MSB first, then bytes MSB-first."""
    import numpy as np

    from vramancer_amd.kv_quantizer import _pack_values, _unpack_values

    _say(f"pack bits {bits} M {M}")
    g = np.random.default_rng(bits * 100 + M)
    vals = g.integers(0, 256, size=(37, M), dtype=np.uint8)
    stream = np.unpackbits(vals[..., None], axis=-1)[..., 8 - bits:].reshape(37, M * bits)
    want = np.packbits(stream, axis=-1, bitorder="big")
    got = _pack_values(torch.from_numpy(vals).to(DEV), bits).cpu().numpy()
    assert np.array_equal(got, want)
    back = _unpack_values(torch.from_numpy(want).to(DEV), M, bits).cpu().numpy()
    assert np.array_equal(back, vals & ((1 << bits) - 1))
