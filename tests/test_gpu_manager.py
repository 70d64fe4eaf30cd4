"""The paged cache manager on the GPU: device block table, slot writes,
TurboQuant flush / bulk compression and the decode entry points.

* Block tables and raw float writes are bit-exact against the host build and
  torch's dtype conversion.
* Decode outputs match the oracle (oracle/paged_decode.py) on the pool the
  manager filled, within |gpu - oracle| <= 2e-3 + 1e-2 |oracle|.
* TurboQuant codes written by flush_compression / compress_page_bulk equal,
  bit for bit, the standalone GPU compressor's codes of the same rows.
"""
import math

import numpy as np
import pytest
import torch

from oracle import paged_decode as PD
from oracle import turboquant as TQ
from vramancer_amd import _lib, tq_pages
from vramancer_amd.paged_attention import PagedKVCacheManager, PagedKVConfig
from vramancer_amd.turboquant_cuda import CUDATurboQuantOps

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ATOL, RTOL = 2e-3, 1e-2


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _assert_close(got, want, what):
    got, want = got.float().cpu(), want.float().cpu()
    err = (got - want).abs()
    bad = err > ATOL + RTOL * want.abs()
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.numel()} outside tolerance, max abs err {err.max():.3e}"


def _mgr(**kw):
    cfg = dict(page_size=16, num_layers=2, num_kv_heads=2, head_dim=128, max_pages=64, device=DEV)
    cfg.update(kw)
    return PagedKVCacheManager(PagedKVConfig(**cfg))


def _host_table(m, rids):
    lists = [m._page_tables[r].pages if r in m._page_tables else [] for r in rids]
    ntok = [m._page_tables[r].num_tokens if r in m._page_tables else 0 for r in rids]
    table = torch.full((len(rids), max(len(p) for p in lists)), -1, dtype=torch.int32)
    for b, p in enumerate(lists):
        table[b, :len(p)] = torch.tensor(p, dtype=torch.int32)
    return table, torch.tensor(ntok, dtype=torch.int32)


def _fill(m, rids, lens, src_dtype, seed, layers=None):
    """Appends lens[i] tokens to rids[i], one decode step at a time (batched
    append + one batched write per layer); returns the rows written as
    {(layer, page, slot): (k [KH, D], v [KH, D])} on the host."""
    g = torch.Generator().manual_seed(seed)
    cfg = m.config
    layers = range(cfg.num_layers) if layers is None else layers
    for r in rids:
        m.allocate(r)
    rows = {}
    for t in range(max(lens)):
        active = [r for r, n in zip(rids, lens) if t < n]
        pids, slots = m.append_tokens(active)
        hp, hs = pids.tolist(), slots.tolist()
        for l in layers:
            k = torch.randn(len(active), cfg.num_kv_heads, cfg.head_dim, generator=g).to(src_dtype)
            v = torch.randn(len(active), cfg.num_kv_heads, cfg.head_dim, generator=g).to(src_dtype)
            m.write_kv_batch(l, pids, slots, k.to(DEV), v.to(DEV), host_slots=list(zip(hp, hs)))
            for i in range(len(active)):
                rows[(l, hp[i], hs[i])] = (k[i], v[i])
    return rows


def test_build_block_table_entry_point():
    _say("vrm_build_block_table")
    g = np.random.default_rng(3)
    lists = [list(g.integers(0, 1000, n)) for n in (0, 5, 1, 300, 0, 17)]
    ntok = [0, 70, 3, 4790, 9, 260]
    B, max_pp = len(lists), 301
    flat = torch.tensor([p for l in lists for p in l], dtype=torch.int32, device=DEV)
    offs = torch.tensor(np.concatenate([[0], np.cumsum([len(l) for l in lists])]), dtype=torch.int32, device=DEV)
    nt = torch.tensor(ntok, dtype=torch.int32, device=DEV)
    table = torch.full((B, max_pp), 7, dtype=torch.int32, device=DEV)
    ctx = torch.full((B,), 7, dtype=torch.int32, device=DEV)
    s = torch.cuda.current_stream().cuda_stream
    lib = _lib.load()
    _lib.check(lib.vrm_build_block_table(flat.data_ptr(), flat.numel(), offs.data_ptr(), nt.data_ptr(), B, max_pp,
                                         table.data_ptr(), ctx.data_ptr(), s), "build")
    torch.cuda.synchronize()
    want = torch.full((B, max_pp), -1, dtype=torch.int32)
    for b, l in enumerate(lists):
        want[b, :len(l)] = torch.tensor(l, dtype=torch.int32)
    assert torch.equal(table.cpu(), want) and ctx.cpu().tolist() == ntok
    # a list running past the flat array gives an absent row instead of a read past it
    bad = torch.tensor([0, 5, 10**6], dtype=torch.int32, device=DEV)
    _lib.check(lib.vrm_build_block_table(flat.data_ptr(), flat.numel(), bad.data_ptr(), nt.data_ptr(), 2, max_pp,
                                         table.data_ptr(), ctx.data_ptr(), s), "build")
    torch.cuda.synchronize()
    assert (table[1].cpu() == -1).all()
    assert torch.equal(table[0, :5].cpu(), flat[:5].cpu()) and (table[0, 5:].cpu() == -1).all()


@pytest.mark.parametrize("pool_dtype", ["float16", "bfloat16", "float32"])
@pytest.mark.parametrize("src", [torch.float32, torch.bfloat16, torch.float16], ids=lambda d: str(d).split(".")[-1])
def test_write_kv_float_pools_bit_exact(pool_dtype, src):
    _say(f"write_kv {pool_dtype} <- {src}")
    m = _mgr(dtype=pool_dtype, num_kv_heads=3, head_dim=64)
    m.allocate("a")
    g = torch.Generator().manual_seed(1)
    special = torch.tensor([0.0, -0.0, 1e-30, -5e-8, 65504.0, 65520.0, 7e4, float("inf"), float("nan"),
                            1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 3.4e38])
    for layer in (1, 0):
        page, slot = m.append_token("a")
        k = torch.randn(3, 64, generator=g) * 100
        k.view(-1)[:special.numel()] = special
        k = k.to(src)
        v = torch.randn(3, 64, generator=g).to(src)
        m.write_kv("a", layer, page, slot, k.to(DEV), v.to(DEV))
        torch.cuda.synchronize()
        pool = m._gpu_pool.cpu()
        dt = getattr(torch, pool_dtype)
        want_k, want_v = k.to(dt), v.to(dt)
        got_k, got_v = pool[page, layer, 0, :, slot], pool[page, layer, 1, :, slot]
        assert torch.equal(got_k.view(torch.uint8), want_k.contiguous().view(torch.uint8)) or \
            (torch.equal(torch.isnan(got_k), torch.isnan(want_k)) and
             torch.equal(got_k[~torch.isnan(got_k)], want_k[~torch.isnan(want_k)]))
        assert torch.equal(got_v, want_v)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32", "int8", "fp8"])
def test_compute_attention_decode_matches_oracle(dtype):
    _say(f"compute_attention_decode {dtype}")
    m = _mgr(dtype=dtype, num_kv_heads=4, max_pages=96, num_layers=2)
    rids = ["r0", "r1", "r2", "r3"]
    _fill(m, rids, [37, 200, 1, 64], torch.bfloat16, seed=4)
    m.free("r3")  # its pages go back to the free list; the request decodes as empty
    H = 12
    q = torch.randn(4, H, 128, generator=torch.Generator().manual_seed(5))
    order = ["r1", "missing", "r0", "r2"]
    out = m.compute_attention_decode(q.to(DEV), order, 1)
    table, ctx = m._block_table(order, torch.device(DEV))
    want_t, want_c = _host_table(m, order)
    w = want_t.shape[1]
    assert table.shape[1] >= w and (table[:, w:] == -1).all()
    assert torch.equal(table[:, :w].cpu(), want_t) and torch.equal(ctx.cpu(), want_c)
    # unchanged page lists: the device table is reused, not rebuilt
    assert m._block_table(order, torch.device(DEV))[0] is table
    torch.cuda.synchronize()
    sc = None if m._kv_scales is None else m._kv_scales.cpu()
    ref = PD.paged_attention_decode(q, m._gpu_pool.cpu(), want_t, want_c, 1, kv_scales=sc)
    assert (out[1] == 0).all()
    _assert_close(out, ref, dtype)
    # one more token changes the table
    m.append_token("r2")
    assert m._block_table(order, torch.device(DEV))[1].cpu().tolist() == [200, 0, 37, 2]


def test_block_table_patched_on_growth():
    """Decode-style growth (token counts + 1, a page appended now and then)
    patches the kept device table in place; a shrink, a freed request or a
    list past the width rebuilds it.  Every state is compared with the table
    built on the host from the page lists."""
    _say("block table growth patches")
    m = _mgr(num_kv_heads=2, max_pages=400, num_layers=1)
    rids = ["a", "b", "c"]
    for rid, n in zip(rids, [15, 16, 40]):
        m.allocate(rid, num_tokens=n)
    dev = torch.device(DEV)

    def check(order):
        table, ctx = m._block_table(order, dev)
        want_t, want_c = _host_table(m, order)
        w = want_t.shape[1]
        assert (table[:, w:] == -1).all()
        assert torch.equal(table[:, :w].cpu(), want_t) and torch.equal(ctx.cpu(), want_c)
        return table

    first = check(rids)
    width = first.shape[1]
    for step in range(40):  # pages appended by a, b and c at different steps
        for rid in rids:
            m.append_token(rid)
        assert check(rids) is first
    m.allocate("d", num_tokens=3)
    assert check(rids + ["d"]) is not first  # another batch: rebuilt
    assert check(rids) is not first
    again = check(rids)
    m.free("b")
    m.allocate("b", num_tokens=5)  # a new entry under the same id
    assert check(rids) is not again
    grown = check(rids)
    while len(m._page_tables["c"].pages) <= grown.shape[1]:  # past the width
        m.append_token("c")
    assert check(rids) is not grown
    assert width >= 16


def test_compute_attention_decode_without_pages_is_none():
    m = _mgr()
    m.allocate("a")
    assert m.compute_attention_decode(torch.zeros(1, 2, 128, device=DEV), ["a", "b"], 0) is None


def _params(comp):
    return TQ.TQParams(128, comp.bits_per_angle, 128, 7, 64, comp._hadamard_signs.cpu(), comp.jl_matrix.cpu())


def _codes(m, layer):
    P = m.config.max_pages
    c = tq_pages.read_pages(m._tq_pool, layer, torch.arange(P, dtype=torch.int32, device=DEV), m._kv_compressor)
    return {k: t.cpu() for k, t in c.items()}


def _ref_codes(comp, x):
    """Standalone GPU compressor codes of rows x [N, 128]."""
    r = CUDATurboQuantOps.compress_gpu(x.to(DEV), 128, 128, 7, comp.bits_per_angle, comp._hadamard_signs,
                                       comp.jl_matrix)
    return {"radius": r["radius"].cpu().reshape(-1), "angles": torch.cat([a.cpu() for a in r["angles"]], -1),
            "qjl_signs": r["qjl_signs"].cpu(), "qjl_norms": r["qjl_norms"].cpu().reshape(-1)}


def _check_codes(m, rows):
    comp = m._kv_compressor
    by_layer = {}
    for (l, p, s), kv in rows.items():
        by_layer.setdefault(l, []).append((p, s, kv))
    for l, items in by_layer.items():
        got = _codes(m, l)
        for kv in (0, 1):
            ref = _ref_codes(comp, torch.cat([it[2][kv] for it in items]))
            KH = m.config.num_kv_heads
            for i, (p, s, _) in enumerate(items):
                sl = slice(i * KH, (i + 1) * KH)
                assert torch.equal(got["radius"][p, kv, :, s].view(torch.int16), ref["radius"][sl].view(torch.int16))
                assert torch.equal(got["angles"][p, kv, :, s], ref["angles"][sl]), (l, p, s, kv)
                if kv == 0:
                    assert torch.equal(got["qjl_signs"][p, 0, :, s], ref["qjl_signs"][sl])
                    assert torch.equal(got["qjl_norms"][p, 0, :, s].view(torch.int16),
                                       ref["qjl_norms"][sl].view(torch.int16))


@pytest.mark.parametrize("bits", [3, 4])
def test_turbo_flush_codes_and_attention(bits):
    _say(f"turbo flush bits {bits}")
    torch.manual_seed(100 + bits)
    m = _mgr(dtype="bfloat16", kv_compression="turboquant", compression_bits=bits, num_kv_heads=2, num_layers=3)
    rows = _fill(m, ["a", "b"], [40, 7], torch.bfloat16, seed=bits, layers=[0, 2])
    # one more token through the single-token write of the reference's API
    page, slot = m.append_token("b")
    g = torch.Generator().manual_seed(9)
    for l in (0, 2):
        k = torch.randn(2, 128, generator=g).to(torch.bfloat16)
        v = torch.randn(2, 128, generator=g).to(torch.bfloat16)
        m.write_kv("b", l, page, slot, k.to(DEV), v.to(DEV))
        rows[(l, page, slot)] = (k, v)
    m.flush_compression()
    torch.cuda.synchronize()
    assert not m._pending_compress
    _check_codes(m, rows)
    assert m.stats()["compressed_pages"] == len(m._page_tables["a"].pages) + len(m._page_tables["b"].pages)
    comp = m._kv_compressor
    H = 6
    q = torch.randn(H, 128, generator=g)
    for rid in ("a", "b"):
        out = m.compute_attention_turbo(q.to(DEV), rid, 2)
        torch.cuda.synchronize()
        table, ctx = _host_table(m, [rid])
        ref = PD.paged_attention_decode_turbo(_params(comp), q[None], _codes(m, 2), table, ctx, head_map="mod")
        assert out.shape == (H, 128)
        _assert_close(out, ref[0], f"turbo {rid}")


def test_turbo_lazy_bulk_compression_from_raw_pool():
    _say("turbo lazy compress_page_bulk")
    torch.manual_seed(7)
    m = _mgr(dtype="float16", kv_compression="turboquant", compression_bits=3, num_kv_heads=2, num_layers=2)
    _fill(m, ["a"], [45], torch.float32, seed=2)
    m._pending_compress.clear()  # never flushed: attention compresses the raw pages on demand
    q = torch.randn(4, 128, generator=torch.Generator().manual_seed(3))
    out = m.compute_attention_turbo(q.to(DEV), "a", 1)
    torch.cuda.synchronize()
    pages = m._page_tables["a"].pages
    assert all(m._tq_slots[p, l] == 0xFFFF for p in pages for l in range(2))
    raw = m._gpu_pool.cpu()
    rows = {(l, p, s): (raw[p, l, 0, :, s], raw[p, l, 1, :, s]) for p in pages for l in range(2) for s in range(16)}
    _check_codes(m, rows)
    table, ctx = _host_table(m, ["a"])
    ref = PD.paged_attention_decode_turbo(_params(m._kv_compressor), q[None], _codes(m, 1), table, ctx,
                                          head_map="mod")
    _assert_close(out, ref[0], "lazy bulk")
    # a page already compressed for a layer is left alone; free pages are refused
    assert m.compress_page_bulk(pages[0]) is True
    assert m.compress_page_bulk(0) is False


def test_turbo_reused_pages_are_compressed_afresh():
    """A freed page goes back with its compression state cleared: when
    from_hf_cache fills it for a new request (compression deferred), the turbo
    decode compresses the new contents instead of reading the old codes."""
    _say("turbo page reuse after free")
    torch.manual_seed(9)
    m = _mgr(dtype="float16", kv_compression="turboquant", compression_bits=3, num_kv_heads=2, num_layers=2)
    _fill(m, ["a"], [40], torch.float32, seed=6)
    m.flush_compression()
    old_pages = list(m._page_tables["a"].pages)
    assert all(m._tq_slots[p, 0] != 0 for p in old_pages)
    m.free("a")
    assert all(m._tq_slots[p].sum() == 0 for p in old_pages)
    g = torch.Generator().manual_seed(10)
    past = tuple((torch.randn(1, 2, 40, 128, generator=g).to(DEV), torch.randn(1, 2, 40, 128, generator=g).to(DEV))
                 for _ in range(2))
    m.from_hf_cache("b", past)
    assert set(m._page_tables["b"].pages) == set(old_pages)
    q = torch.randn(4, 128, generator=torch.Generator().manual_seed(11))
    out = m.compute_attention_turbo(q.to(DEV), "b", 1)
    torch.cuda.synchronize()
    raw = m._gpu_pool.cpu()
    pages = m._page_tables["b"].pages
    _check_codes(m, {(l, p, s): (raw[p, l, 0, :, s], raw[p, l, 1, :, s]) for p in pages[:2] for l in range(2)
                     for s in range(16)})
    table, ctx = _host_table(m, ["b"])
    ref = PD.paged_attention_decode_turbo(_params(m._kv_compressor), q[None], _codes(m, 1), table, ctx,
                                          head_map="mod")
    _assert_close(out, ref[0], "reused pages")


def test_compress_page_bulk_valid_slots():
    _say("compress_page_bulk num_valid_slots")
    torch.manual_seed(8)
    m = _mgr(dtype="bfloat16", kv_compression="turboquant", compression_bits=4, num_kv_heads=2, num_layers=2)
    _fill(m, ["a"], [16], torch.bfloat16, seed=5)
    page = m._page_tables["a"].pages[0]
    assert m.compress_page_bulk(page, num_valid_slots=5)
    torch.cuda.synchronize()
    raw = m._gpu_pool.cpu()
    _check_codes(m, {(l, page, s): (raw[page, l, 0, :, s], raw[page, l, 1, :, s]) for l in range(2) for s in range(5)})
    got = _codes(m, 1)
    assert (got["radius"][page, :, :, 5:] == 0).all() and (got["angles"][page, :, :, 5:] == 0).all()
    assert m._tq_slots[page, 0] == 0x1F


def test_turbo_batch_matches_single_requests():
    _say("turbo batch")
    torch.manual_seed(11)
    m = _mgr(dtype="bfloat16", kv_compression="turboquant", compression_bits=3, num_kv_heads=4, num_layers=1,
             max_pages=128)
    _fill(m, ["a", "b", "c"], [300, 17, 129], torch.bfloat16, seed=6)
    m.flush_compression()
    q = torch.randn(3, 8, 128, generator=torch.Generator().manual_seed(2))
    rids = ["a", "none", "b", "c"]
    qb = torch.cat([q[:1], torch.zeros(1, 8, 128), q[1:]])
    out = m.compute_attention_turbo_batch(qb.to(DEV), rids, 0)
    torch.cuda.synchronize()
    assert (out[1] == 0).all()
    for i, rid in enumerate(rids):
        if rid == "none":
            continue
        single = m.compute_attention_turbo(qb[i].to(DEV), rid, 0)
        _assert_close(out[i], single, rid)
    table, ctx = _host_table(m, rids)
    ref = PD.paged_attention_decode_turbo(_params(m._kv_compressor), qb, _codes(m, 0), table, ctx, head_map="mod")
    _assert_close(out, ref, "batch vs oracle")


@pytest.mark.parametrize("dtype", ["bfloat16", "float32", "int8", "fp8"])
@pytest.mark.parametrize("D,PS", [(96, 8), (80, 32)])
def test_manager_decode_other_head_dims_and_page_sizes(dtype, D, PS):
    """The manager's pool, writes, block table and decode at head_dim 96 with
    pages of 8 tokens and head_dim 80 with pages of 32 (the reference's
    PagedKVConfig takes any page_size and head_dim)."""
    _say(f"manager {dtype} D{D} PS{PS}")
    m = _mgr(dtype=dtype, num_kv_heads=4, max_pages=128, num_layers=2, head_dim=D, page_size=PS)
    rids = ["a", "b", "c"]
    _fill(m, rids, [3 * PS + 5, 1, 90], torch.bfloat16, seed=D + PS)
    q = torch.randn(3, 8, D, generator=torch.Generator().manual_seed(9))
    out = m.compute_attention_decode(q.to(DEV), rids, 1)
    torch.cuda.synchronize()
    table, ctx = _host_table(m, rids)
    sc = None if m._kv_scales is None else m._kv_scales.cpu()
    _assert_close(out, PD.paged_attention_decode(q, m._gpu_pool.cpu(), table, ctx, 1, kv_scales=sc),
                  f"{dtype} D{D} PS{PS}")


@pytest.mark.parametrize("dtype", ["int8", "fp8"])
def test_manager_even_batch_takes_the_balanced_decode(dtype):
    """32 requests of equal length over 4 kv-heads (128 pairs): the manager
    hands its token counts to the decode, which takes the balanced kernel;
    the output matches the oracle."""
    from vramancer_amd.paged_attention_cuda import prefer_balanced

    _say(f"manager balanced {dtype}")
    m = _mgr(dtype=dtype, num_kv_heads=4, max_pages=160, num_layers=2, head_dim=128)
    rids = [f"r{i}" for i in range(32)]
    _fill(m, rids, [40] * 32, torch.bfloat16, seed=21, layers=[1])
    q = torch.randn(32, 12, 128, generator=torch.Generator().manual_seed(2))
    out = m.compute_attention_decode(q.to(DEV), rids, 1)
    torch.cuda.synchronize()
    assert prefer_balanced(m._table_cache["ntok"], 4, m._gpu_pool.dtype)
    table, ctx = _host_table(m, rids)
    _assert_close(out, PD.paged_attention_decode(q, m._gpu_pool.cpu(), table, ctx, 1, kv_scales=m._kv_scales.cpu()),
                  f"balanced {dtype}")
