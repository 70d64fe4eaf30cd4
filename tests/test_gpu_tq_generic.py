"""TurboQuant pages of every compressor setting: head_dim 33 .. 256
(padded_dim 64 / 128 / 256), 1 .. 8 bits per angle, qjl_dim 1 .. 256, any
page size.  head_dim 33 .. 64 with 32 QJL rows and 65 .. 128 with 64 (the
compressor's default qjl_dim), 2 .. 4 bits and 16-token pages use the tuned
slices and kernel; everything else the generic layout.

* Codes written into pages equal, bit for bit, the standalone GPU
  compressor's codes (CUDATurboQuantOps.compress_gpu, itself checked against
  the reference's CPU path in test_gpu_turboquant.py) for the same rows;
  unwritten slots and the QJL fields of value rows read as zero.
* The paged decode matches the oracle's restatement of compute_attention_turbo
  (oracle/paged_decode.py) on the codes read back from the pool, within
  |gpu - oracle| <= 2e-3 + 1e-2 |oracle| elementwise, at D in {64, 96, 256}
  and other settings, with the log-sum-exp output and without the QJL term
  (the Hugging Face cache's scores) checked the same way.
* The cache manager replays the reference's head_dim 96 / 4-token page
  scenario (tests/test_turboquant_integration.py:232-252) and its head_dim 64,
  four-layer one (:254-273), then attends the codes it wrote.
"""
import math

import pytest
import torch

from oracle import paged_decode as PD
from oracle import turboquant as TQ
from vramancer_amd import tq_pages
from vramancer_amd.kv_quantizer import KVCacheCompressor
from vramancer_amd.paged_attention import PagedKVCacheManager, PagedKVConfig
from vramancer_amd.turboquant_cuda import CUDATurboQuantOps

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ATOL, RTOL = 2e-3, 1e-2

# head_dim, bits per angle, qjl_dim (None: the compressor's padded_dim / 2), page size
SETTINGS = [
    (64, 3, None, 16), (96, 3, None, 4), (256, 4, None, 16), (128, 1, None, 16), (128, 3, 32, 16),
    (128, 3, 64, 8), (80, 8, 100, 5), (200, 5, 256, 3), (33, 2, 7, 1), (128, 6, None, 32),
    # head_dim 65 .. 128 at 64 QJL rows, 2-4 bits and 16-token pages share the tuned slice of head_dim 128,
    # head_dim 33 .. 64 at 32 QJL rows that of head_dim 64
    (96, 3, None, 16), (80, 4, None, 16), (65, 2, None, 16), (64, 2, None, 16), (48, 4, None, 16),
    (33, 3, None, 16),
    # head_dim 1 .. 32: padded dims 2 .. 32, generic slices
    (32, 3, None, 16), (32, 4, 40, 5), (17, 2, None, 16), (16, 3, None, 8), (8, 4, None, 16), (5, 3, 3, 4),
    (2, 3, None, 16), (1, 8, None, 3),
]


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _student_t(shape, seed):
    """bf16 rows, Student-t (df 3) per channel scaled to unit variance."""
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(*shape, generator=g)
    chi2 = sum(torch.randn(*shape, generator=g) ** 2 for _ in range(3))
    return (z / torch.sqrt(chi2 / 3) / math.sqrt(3.0)).to(torch.bfloat16)


def _compressor(head_dim, bits, qjl=None, seed=1234):
    torch.manual_seed(seed)
    return KVCacheCompressor(head_dim, bits, qjl)


def _params(comp):
    return TQ.TQParams(comp.head_dim, comp.bits_per_angle, comp._padded_dim, comp._n_levels, comp.qjl_dim,
                       comp._hadamard_signs.cpu(), comp.jl_matrix.cpu())


def _assert_close(got, want, what):
    got, want = got.float().cpu(), want.float().cpu()
    err = (got - want).abs()
    bad = err > ATOL + RTOL * want.abs()
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.numel()} outside tolerance, max abs err {err.max():.3e}"


def _ref_codes(comp, x):
    """Standalone GPU compressor codes of rows x [N, head_dim] (host)."""
    r = CUDATurboQuantOps.compress_gpu(x.to(DEV), comp.head_dim, comp._padded_dim, comp._n_levels,
                                       comp.bits_per_angle, comp._hadamard_signs, comp.jl_matrix)
    return {"radius": r["radius"].cpu().reshape(-1), "angles": torch.cat([a.cpu() for a in r["angles"]], -1),
            "qjl_signs": r["qjl_signs"].cpu(), "qjl_norms": r["qjl_norms"].cpu().reshape(-1)}


def _read(pool, comp, layer, ids, ps):
    c = tq_pages.read_pages(pool, layer, ids.to(torch.int32).to(DEV), comp, ps)
    return {k: t.cpu() for k, t in c.items()}


def _sid(s):
    return f"d{s[0]}-b{s[1]}-q{s[2]}-ps{s[3]}"


@pytest.mark.parametrize("setting", SETTINGS, ids=_sid)
def test_generic_page_codes_equal_compressor_codes(setting):
    hd, bits, qjl, ps = setting
    _say(f"generic page codes {_sid(setting)}")
    comp = _compressor(hd, bits, qjl)
    P, L, KH, NP = 9, 2, 3, 5
    pool = tq_pages.allocate_pool(P, L, KH, comp, DEV, ps)
    assert pool.shape == (P, L, 2, KH, tq_pages.slice_bytes(bits, hd, comp.qjl_dim, ps))
    k = _student_t((NP, KH, ps, hd), 1)
    v = _student_t((NP, KH, ps, hd), 2)
    ids = torch.tensor([7, 0, 4, 8, 2], dtype=torch.int32)
    n_valid = torch.tensor([ps, ps, max(ps // 3, 1), 1, ps], dtype=torch.int32)
    tq_pages.quantize_pages(pool, 1, ids.to(DEV), k.to(DEV), v.to(DEV), comp, n_valid.to(DEV), page_size=ps)
    got = _read(pool, comp, 1, ids, ps)
    pd, qd = comp._padded_dim, comp.qjl_dim
    assert got["angles"].shape == (NP, 2, KH, ps, pd - 1) and got["qjl_signs"].shape == (NP, 2, KH, ps, qd)
    for kv, src in ((0, k), (1, v)):
        ref = _ref_codes(comp, src.reshape(-1, hd))
        r_rad = ref["radius"].reshape(NP, KH, ps)
        r_ang = ref["angles"].reshape(NP, KH, ps, pd - 1)
        r_sgn = ref["qjl_signs"].reshape(NP, KH, ps, qd)
        r_nrm = ref["qjl_norms"].reshape(NP, KH, ps)
        for n in range(NP):
            nv = int(n_valid[n])
            assert torch.equal(got["radius"][n, kv, :, :nv].view(torch.int16), r_rad[n, :, :nv].view(torch.int16))
            assert torch.equal(got["angles"][n, kv, :, :nv], r_ang[n, :, :nv]), (kv, n)
            assert (got["radius"][n, kv, :, nv:] == 0).all() and (got["angles"][n, kv, :, nv:] == 0).all()
            if kv == 0:
                assert torch.equal(got["qjl_signs"][n, 0, :, :nv], r_sgn[n, :, :nv]), n
                assert torch.equal(got["qjl_norms"][n, 0, :, :nv].view(torch.int16),
                                   r_nrm[n, :, :nv].view(torch.int16)), n
    assert (got["qjl_signs"][:, 1] == 0).all() and (got["qjl_norms"][:, 1] == 0).all()
    # layer 0 and the pages never written stay zero
    assert (pool[:, 0] == 0).all() and (pool[[1, 3, 5, 6], 1] == 0).all()


@pytest.mark.parametrize("setting", [(96, 3, None, 4), (256, 5, None, 8), (64, 1, 17, 16)], ids=_sid)
def test_generic_append_equals_page_write(setting):
    hd, bits, qjl, ps = setting
    _say(f"generic append vs pages {_sid(setting)}")
    comp = _compressor(hd, bits, qjl)
    KH = 2
    k = _student_t((1, KH, ps, hd), 3)
    v = _student_t((1, KH, ps, hd), 4)
    a = tq_pages.allocate_pool(4, 1, KH, comp, DEV, ps)
    b = tq_pages.allocate_pool(4, 1, KH, comp, DEV, ps)
    pid = torch.tensor([2], dtype=torch.int32, device=DEV)
    tq_pages.quantize_pages(a, 0, pid, k.to(DEV), v.to(DEV), comp, page_size=ps)
    for t in range(ps):  # token by token, as a decode loop appends
        tq_pages.quantize_append(b, 0, pid, torch.tensor([t], dtype=torch.int32, device=DEV),
                                 k[:, :, t].to(DEV).contiguous(), v[:, :, t].to(DEV).contiguous(), comp,
                                 page_size=ps)
    # slots outside [0, ps) and pages outside [0, P) are dropped
    tq_pages.quantize_append(b, 0, torch.tensor([2, 9, -1], dtype=torch.int32, device=DEV),
                             torch.tensor([ps, 0, 0], dtype=torch.int32, device=DEV),
                             k[0, :, :3].transpose(0, 1).to(DEV).contiguous(),
                             v[0, :, :3].transpose(0, 1).to(DEV).contiguous(), comp, page_size=ps)
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), b.cpu())


@pytest.mark.parametrize("setting", [(96, 3, None, 4), (256, 4, None, 16), (64, 7, None, 32)], ids=_sid)
def test_generic_bulk_page_write_equals_small_writes(setting):
    """40 pages of 8 kv-heads written at once equal the same pages written 5
    at a time."""
    hd, bits, qjl, ps = setting
    _say(f"generic bulk write {_sid(setting)}")
    comp = _compressor(hd, bits, qjl)
    P, L, KH, NP = 48, 2, 8, 40
    k = _student_t((NP, KH, ps, hd), 11).to(DEV)
    v = _student_t((NP, KH, ps, hd), 12).to(DEV)
    ids = torch.randperm(P, generator=torch.Generator().manual_seed(3))[:NP].to(torch.int32).to(DEV)
    n_valid = torch.randint(1, ps + 1, (NP,), generator=torch.Generator().manual_seed(4)).to(torch.int32).to(DEV)
    a = tq_pages.allocate_pool(P, L, KH, comp, DEV, ps)
    b = tq_pages.allocate_pool(P, L, KH, comp, DEV, ps)
    tq_pages.quantize_pages(a, 1, ids, k, v, comp, n_valid, page_size=ps)
    for s in range(0, NP, 5):
        tq_pages.quantize_pages(b, 1, ids[s:s + 5], k[s:s + 5], v[s:s + 5], comp, n_valid[s:s + 5], page_size=ps)
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), b.cpu())


def _turbo_case(comp, B, H, KH, ctxs, seed, ps, L=1, layer=0, spare=2):
    g = torch.Generator().manual_seed(seed)
    hd = comp.head_dim
    npages = [(c + ps - 1) // ps for c in ctxs]
    P = sum(npages) + spare
    pool = tq_pages.allocate_pool(P, L, KH, comp, DEV, ps)
    k = _student_t((P, KH, ps, hd), seed + 1)
    v = _student_t((P, KH, ps, hd), seed + 2)
    tq_pages.quantize_pages(pool, layer, torch.arange(P, dtype=torch.int32, device=DEV), k.to(DEV), v.to(DEV), comp,
                            page_size=ps)
    perm = torch.randperm(P, generator=g)
    table = torch.full((B, max(max(npages), 1)), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(npages):
        table[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = torch.randn(B, H, hd, generator=g)
    lens = torch.tensor(ctxs, dtype=torch.int32)
    return pool, q, table, lens


def _codes(pool, comp, layer, ps):
    return _read(pool, comp, layer, torch.arange(pool.shape[0]), ps)


DECODE = [  # head_dim, bits, qjl_dim, page size, H, KH
    (64, 3, None, 16, 8, 2), (96, 3, None, 4, 12, 4), (256, 4, None, 16, 16, 2), (96, 2, None, 16, 40, 8),
    (64, 1, None, 8, 8, 8), (256, 8, 100, 5, 4, 1), (128, 3, 64, 32, 40, 8), (80, 5, 33, 3, 6, 3),
    (128, 3, 32, 16, 8, 2), (96, 3, None, 16, 40, 8), (80, 4, None, 16, 12, 4), (65, 2, None, 16, 8, 1),
    (64, 2, None, 16, 32, 4), (64, 4, None, 16, 16, 2), (48, 3, None, 16, 12, 3), (33, 4, None, 16, 8, 1),
    (64, 3, None, 16, 40, 8), (64, 3, 16, 16, 28, 4),
    (32, 3, None, 16, 8, 2), (32, 4, None, 16, 40, 8), (24, 2, 20, 5, 6, 3), (16, 4, None, 16, 12, 4),
    (8, 3, None, 8, 8, 2), (3, 5, None, 16, 4, 4), (2, 3, None, 16, 4, 1),
]


@pytest.mark.parametrize("case", DECODE, ids=lambda c: _sid(c[:4]) + f"-h{c[4]}-kh{c[5]}")
def test_generic_decode_turbo_matches_oracle(case):
    hd, bits, qjl, ps, H, KH = case
    _say(f"generic turbo decode {case}")
    comp = _compressor(hd, bits, qjl, seed=bits + hd)
    pool, q, table, lens = _turbo_case(comp, 3, H, KH, [37, 300, 1], seed=H + bits, ps=ps)
    out = tq_pages.paged_attention_decode_turbo(q.to(DEV), pool, table.to(DEV), lens.to(DEV), 0, comp, page_size=ps)
    torch.cuda.synchronize()
    ref = PD.paged_attention_decode_turbo(_params(comp), q, _codes(pool, comp, 0, ps), table, lens)
    _assert_close(out, ref, f"decode {case}")


@pytest.mark.parametrize("setting", [(96, 3, None, 4), (64, 2, None, 16), (256, 4, None, 8), (64, 4, None, 16),
                                     (56, 3, None, 16), (32, 3, None, 16), (8, 4, None, 4)], ids=_sid)
def test_generic_decode_turbo_lse_and_no_qjl(setting):
    """The log-sum-exp output, with and without the QJL term: lse equals
    ln sum_t exp(scale score_t) of the oracle's scores, and without the QJL
    term the output equals softmax attention over the decompressed keys."""
    hd, bits, qjl, ps = setting
    _say(f"generic turbo lse {_sid(setting)}")
    comp = _compressor(hd, bits, qjl, seed=5)
    B, H, KH = 3, 8, 2
    pool, q, table, lens = _turbo_case(comp, B, H, KH, [50, 129, 7], seed=31, ps=ps)
    codes = _codes(pool, comp, 0, ps)
    p = _params(comp)
    scale = 0.11
    for qjl_on in (True, False):
        lse = torch.empty(B, H, device=DEV)
        out = tq_pages.paged_attention_decode_turbo(q.to(DEV), pool, table.to(DEV), lens.to(DEV), 0, comp,
                                                    scale=scale, lse=lse, qjl=qjl_on, page_size=ps)
        torch.cuda.synchronize()
        want_out = torch.zeros(B, H, hd)
        want_lse = torch.zeros(B, H)
        for b in range(B):
            n = int(lens[b])
            pids = torch.tensor([int(table[b, t // ps]) for t in range(n)])
            slots = torch.arange(n) % ps
            for kvh in range(KH):
                group = list(range(kvh * (H // KH), (kvh + 1) * (H // KH)))

                def gather(kv):
                    ang = codes["angles"][pids, kv, kvh, slots]
                    return {"radius": codes["radius"][pids, kv, kvh, slots].reshape(-1, 1),
                            "angles": list(torch.split(ang, [p.padded_dim >> (l + 1) for l in range(p.n_levels)],
                                                       dim=-1)),
                            "qjl_signs": codes["qjl_signs"][pids, kv, kvh, slots],
                            "qjl_norms": codes["qjl_norms"][pids, kv, kvh, slots].reshape(-1, 1),
                            "shape": (n, hd)}

                ck, cv = gather(0), gather(1)
                qg = q[b, group].float()
                if qjl_on:
                    s = TQ.attention_score(p, qg, ck) * scale
                else:
                    s = (qg @ TQ.decompress(p, ck).float().T) * scale
                want_lse[b, group] = torch.logsumexp(s.double(), -1).float()
                want_out[b, group] = torch.softmax(s, -1) @ TQ.decompress(p, cv).float()
        _assert_close(out, want_out, f"out qjl={qjl_on}")
        assert (lse.cpu() - want_lse).abs().max() <= 2e-3 + 1e-3 * want_lse.abs().max(), f"lse qjl={qjl_on}"


def test_generic_decode_turbo_edge_cases_and_long_contexts():
    """Zero context, an absent page (-1), a layer other than 0, and long
    contexts split over many partitions, at head_dim 96 with 4-token pages."""
    _say("generic turbo edges / long")
    comp = _compressor(96, 3, seed=9)
    pool, q, table, lens = _turbo_case(comp, 4, 8, 2, [0, 64, 17, 3000], seed=9, ps=4, L=3, layer=2)
    table[1, 1] = -1  # an absent page: its tokens are skipped
    out = tq_pages.paged_attention_decode_turbo(q.to(DEV), pool, table.to(DEV), lens.to(DEV), 2, comp, scale=0.3,
                                                page_size=4)
    torch.cuda.synchronize()
    assert (out[0] == 0).all()
    ref = PD.paged_attention_decode_turbo(_params(comp), q, _codes(pool, comp, 2, 4), table, lens, scale=0.3)
    _assert_close(out, ref, "edge cases")
    comp = _compressor(256, 2, seed=3)
    pool, q, table, lens = _turbo_case(comp, 2, 16, 4, [5000, 900], seed=13, ps=16)
    out = tq_pages.paged_attention_decode_turbo(q.to(DEV), pool, table.to(DEV), lens.to(DEV), 0, comp)
    torch.cuda.synchronize()
    ref = PD.paged_attention_decode_turbo(_params(comp), q, _codes(pool, comp, 0, 16), table, lens)
    _assert_close(out, ref, "long contexts d256")


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_tuned_d64_decode_edge_cases_and_long_contexts(bits):
    """The tuned head_dim-64 slice: zero context, an absent page (-1), a
    layer other than 0, a partial last page and contexts split over many
    partitions, with 5 query heads per kv-head."""
    _say(f"tuned d64 edges / long b{bits}")
    comp = _compressor(64, bits, seed=21 + bits)
    pool, q, table, lens = _turbo_case(comp, 5, 20, 4, [0, 64, 17, 4100, 1601], seed=9 + bits, ps=16, L=3, layer=1)
    table[1, 2] = -1  # absent pages: their tokens are skipped
    table[3, 5] = -1
    out = tq_pages.paged_attention_decode_turbo(q.to(DEV), pool, table.to(DEV), lens.to(DEV), 1, comp, scale=0.2)
    torch.cuda.synchronize()
    assert (out[0] == 0).all()
    ref = PD.paged_attention_decode_turbo(_params(comp), q, _codes(pool, comp, 1, 16), table, lens, scale=0.2)
    _assert_close(out, ref, f"tuned d64 b{bits}")


def _mgr_codes_match(m, rows, layer):
    """Codes of rows {(page, slot): (k [KH, D], v [KH, D])} in the manager's
    pool equal the standalone compressor's."""
    comp, cfg = m._kv_compressor, m.config
    got = _read(m._tq_pool, comp, layer, torch.arange(cfg.max_pages), cfg.page_size)
    items = list(rows.items())
    KH = cfg.num_kv_heads
    for kv in (0, 1):
        ref = _ref_codes(comp, torch.cat([it[1][kv].reshape(KH, -1) for it in items]))
        for i, ((p, s), _) in enumerate(items):
            sl = slice(i * KH, (i + 1) * KH)
            assert torch.equal(got["radius"][p, kv, :, s].view(torch.int16), ref["radius"][sl].view(torch.int16))
            assert torch.equal(got["angles"][p, kv, :, s], ref["angles"][sl]), (layer, p, s, kv)
            if kv == 0:
                assert torch.equal(got["qjl_signs"][p, 0, :, s], ref["qjl_signs"][sl])
    return got


@pytest.mark.parametrize("head_dim", [96, 16])
def test_manager_head_dim_96_page_4(head_dim):
    """The reference's tests/test_turboquant_integration.py:232-252: a
    manager with head_dim 96, 4-token pages, one layer and one kv-head takes
    a token through write_kv and flush_compression, and the slot then holds
    codes; here the codes are also checked against the compressor's and the
    request (grown to 11 tokens, three pages) is attended.  The same scenario
    at head_dim 16 (padded dim 16, 8 QJL rows)."""
    _say(f"manager d{head_dim} ps4")
    torch.manual_seed(21)
    m = PagedKVCacheManager(PagedKVConfig(page_size=4, num_layers=1, num_kv_heads=1, head_dim=head_dim, max_pages=8,
                                          device=DEV, kv_compression="turboquant"))
    assert m.kv_compression_active is True
    m.allocate("edge1")
    page_id, slot = m.append_token("edge1")
    g = torch.Generator().manual_seed(1)
    key, value = torch.randn(1, head_dim, generator=g), torch.randn(1, head_dim, generator=g)
    m.write_kv("edge1", 0, page_id, slot, key.to(DEV), value.to(DEV))
    m.flush_compression()
    torch.cuda.synchronize()
    assert m._tq_slots[page_id, 0] & (1 << slot)
    rows = {(page_id, slot): (key, value)}
    for _ in range(10):
        page_id, slot = m.append_token("edge1")
        key, value = torch.randn(1, head_dim, generator=g), torch.randn(1, head_dim, generator=g)
        m.write_kv("edge1", 0, page_id, slot, key.to(DEV), value.to(DEV))
        rows[(page_id, slot)] = (key, value)
    m.flush_compression()
    torch.cuda.synchronize()
    pages = m._page_tables["edge1"].pages
    assert len(pages) == 3 and m.stats()["compressed_pages"] == 3
    codes = _mgr_codes_match(m, rows, 0)
    q = torch.randn(2, head_dim, generator=g)
    out = m.compute_attention_turbo(q.to(DEV), "edge1", 0)
    torch.cuda.synchronize()
    table = torch.tensor([pages], dtype=torch.int32)
    ref = PD.paged_attention_decode_turbo(_params(m._kv_compressor), q[None], codes, table,
                                          torch.tensor([11], dtype=torch.int32), head_map="mod")
    assert out.shape == (2, head_dim)
    _assert_close(out, ref[0], f"manager d{head_dim} ps4")


def test_manager_head_dim_64_four_layers():
    """The reference's tests/test_turboquant_integration.py:254-273: head_dim
    64, 4-token pages, four layers of two kv-heads; one token written to
    every layer is compressed in every layer."""
    _say("manager d64 ps4 four layers")
    torch.manual_seed(22)
    m = PagedKVCacheManager(PagedKVConfig(page_size=4, num_layers=4, num_kv_heads=2, head_dim=64, max_pages=8,
                                          device=DEV, kv_compression="turboquant"))
    m.allocate("multi")
    page_id, slot = m.append_token("multi")
    g = torch.Generator().manual_seed(2)
    written = {}
    for layer in range(4):
        key, value = torch.randn(2, 64, generator=g), torch.randn(2, 64, generator=g)
        m.write_kv("multi", layer, page_id, slot, key.to(DEV), value.to(DEV))
        written[layer] = (key, value)
    m.flush_compression()
    torch.cuda.synchronize()
    for layer in range(4):
        assert m._tq_slots[page_id, layer] != 0
        _mgr_codes_match(m, {(page_id, slot): written[layer]}, layer)


def test_manager_generic_lazy_bulk_compression():
    """Pages filled without a flush are compressed from the raw pool on the
    first turbo attention (compress_page_bulk at head_dim 96, 8-token pages)."""
    _say("manager generic lazy bulk")
    torch.manual_seed(23)
    m = PagedKVCacheManager(PagedKVConfig(page_size=8, num_layers=2, num_kv_heads=2, head_dim=96, max_pages=16,
                                          device=DEV, dtype="float16", kv_compression="turboquant",
                                          compression_bits=4))
    m.allocate("a")
    g = torch.Generator().manual_seed(5)
    for _ in range(29):
        pid, slot = m.append_token("a")
        for layer in range(2):
            m.write_kv("a", layer, pid, slot, torch.randn(2, 96, generator=g).to(DEV),
                       torch.randn(2, 96, generator=g).to(DEV))
    m._pending_compress.clear()  # never flushed: attention compresses the raw pages on demand
    q = torch.randn(4, 96, generator=g)
    out = m.compute_attention_turbo(q.to(DEV), "a", 1)
    torch.cuda.synchronize()
    pages = m._page_tables["a"].pages
    assert all(m._tq_slots[p, l] == 0xFF for p in pages for l in range(2))
    raw = m._gpu_pool.cpu()
    codes = _mgr_codes_match(m, {(p, s): (raw[p, 1, 0, :, s], raw[p, 1, 1, :, s]) for p in pages for s in range(8)},
                             1)
    table = torch.tensor([pages], dtype=torch.int32)
    ref = PD.paged_attention_decode_turbo(_params(m._kv_compressor), q[None], codes, table,
                                          torch.tensor([29], dtype=torch.int32), head_map="mod")
    _assert_close(out, ref[0], "lazy bulk d96")


@pytest.mark.parametrize("head_dim,bits", [(64, 3), (96, 2), (256, 5), (32, 3), (16, 4), (8, 2)])
def test_hf_cache_generic_decode_attention_matches_materialised(head_dim, bits):
    """The Hugging Face TurboQuant cache at other head dims: the paged decode
    step (TurboQuant pages + residual merged by log-sum-exp) against
    attention over the same cache's materialised keys/values."""
    from vramancer_amd.turboquant_cache import TurboQuantCache

    _say(f"hf cache d{head_dim} b{bits}")
    torch.manual_seed(11)
    cache = TurboQuantCache(2, head_dim, bits_per_angle=bits, residual_length=32, device=DEV, paged_attention=True)
    layer = cache.layers[0]
    g = torch.Generator().manual_seed(4)
    for s in (40, 1, 30, 1, 60, 1):
        k = torch.randn(2, 2, s, head_dim, generator=g).to(DEV)
        layer.update(k, torch.randn(2, 2, s, head_dim, generator=g).to(DEV))
        q = torch.randn(2, 4, 1, head_dim, generator=g).to(DEV)
        got = layer.attend_decode(q, 0.08)[:, 0].float().cpu()
        K, V = layer.materialize()
        Kr = K.float().cpu().repeat_interleave(2, dim=1)
        Vr = V.float().cpu().repeat_interleave(2, dim=1)
        w = torch.softmax(0.08 * (Kr @ q.float().cpu()[:, :, 0, :, None])[..., 0], -1)
        want = (w[..., None] * Vr).sum(2)
        err = (got - want).abs()
        assert (err <= 2e-3 + 1e-2 * want.abs()).all(), f"step {s}: max err {err.max():.3e} view {layer._view}"
