"""TurboQuant pages on the GPU.

* Codes written into pages equal, bit for bit, the codes of the standalone
  GPU compressor (CUDATurboQuantOps.compress_gpu, itself checked against the
  reference's CPU path in test_gpu_turboquant.py) for the same rows; value rows
  carry no QJL fields.
* The paged decode matches the oracle's restatement of compute_attention_turbo
  (oracle/paged_decode.py), evaluated on the codes read back from the pool,
  within |gpu - oracle| <= 2e-3 + 1e-2 |oracle| elementwise.
"""
import math

import pytest
import torch

from oracle import paged_decode as PD
from oracle import turboquant as TQ
from vramancer_amd import tq_pages
from vramancer_amd.kv_quantizer import KVCacheCompressor
from vramancer_amd.turboquant_cuda import CUDATurboQuantOps

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ATOL, RTOL = 2e-3, 1e-2


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _student_t(shape, seed):
    """bf16 rows, Student-t (df 3) per channel scaled to unit variance."""
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(*shape, generator=g)
    chi2 = sum(torch.randn(*shape, generator=g) ** 2 for _ in range(3))
    return (z / torch.sqrt(chi2 / 3) / math.sqrt(3.0)).to(torch.bfloat16)


def _compressor(bits, seed=1234):
    torch.manual_seed(seed)
    return KVCacheCompressor(128, bits)


def _params(comp):
    return TQ.TQParams(128, comp.bits_per_angle, 128, 7, 64, comp._hadamard_signs.cpu(), comp.jl_matrix.cpu())


def _assert_close(got, want, what):
    got, want = got.float().cpu(), want.float().cpu()
    err = (got - want).abs()
    bad = err > ATOL + RTOL * want.abs()
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.numel()} outside tolerance, max abs err {err.max():.3e}"


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_page_codes_equal_compressor_codes(bits):
    _say(f"page codes bits {bits}")
    comp = _compressor(bits)
    P, L, KH, NP = 9, 2, 3, 5
    pool = tq_pages.allocate_pool(P, L, KH, comp, DEV)
    k = _student_t((NP, KH, 16, 128), 1)
    v = _student_t((NP, KH, 16, 128), 2)
    ids = torch.tensor([7, 0, 4, 8, 2], dtype=torch.int32)
    n_valid = torch.tensor([16, 16, 5, 1, 16], dtype=torch.int32)
    tq_pages.quantize_pages(pool, 1, ids.to(DEV), k.to(DEV), v.to(DEV), comp, n_valid.to(DEV))
    got = {key: t.cpu() for key, t in tq_pages.read_pages(pool, 1, ids.to(DEV), comp).items()}
    for kv, src in ((0, k), (1, v)):
        ref = CUDATurboQuantOps.compress_gpu(src.to(DEV).reshape(-1, 128), 128, 128, 7, bits, comp._hadamard_signs,
                                             comp.jl_matrix)
        r_rad = ref["radius"].cpu().reshape(NP, KH, 16)
        r_ang = torch.cat([a.cpu() for a in ref["angles"]], -1).reshape(NP, KH, 16, 127)
        r_sgn = ref["qjl_signs"].cpu().reshape(NP, KH, 16, 64)
        r_nrm = ref["qjl_norms"].cpu().reshape(NP, KH, 16)
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


def test_append_equals_page_write():
    _say("append vs pages")
    comp = _compressor(3)
    P, L, KH = 4, 1, 2
    k = _student_t((1, KH, 16, 128), 3)
    v = _student_t((1, KH, 16, 128), 4)
    a = tq_pages.allocate_pool(P, L, KH, comp, DEV)
    b = tq_pages.allocate_pool(P, L, KH, comp, DEV)
    tq_pages.quantize_pages(a, 0, torch.tensor([2], dtype=torch.int32, device=DEV), k.to(DEV), v.to(DEV), comp)
    for t in range(16):  # token by token, as a decode loop appends
        tq_pages.quantize_append(b, 0, torch.tensor([2], dtype=torch.int32, device=DEV),
                                 torch.tensor([t], dtype=torch.int32, device=DEV),
                                 k[:, :, t].to(DEV).contiguous(), v[:, :, t].to(DEV).contiguous(), comp)
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), b.cpu())


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_bulk_page_write_equals_small_writes(bits):
    """40 pages of 8 kv-heads (5,120 rows per side, several rows per
    workgroup) written at once equal the same pages written 5 at a time."""
    _say(f"bulk page write bits {bits}")
    comp = _compressor(bits)
    P, L, KH, NP = 48, 2, 8, 40
    k = _student_t((NP, KH, 16, 128), 11).to(DEV)
    v = _student_t((NP, KH, 16, 128), 12).to(DEV)
    ids = torch.randperm(P, generator=torch.Generator().manual_seed(3))[:NP].to(torch.int32).to(DEV)
    n_valid = torch.randint(1, 17, (NP,), generator=torch.Generator().manual_seed(4)).to(torch.int32).to(DEV)
    a = tq_pages.allocate_pool(P, L, KH, comp, DEV)
    b = tq_pages.allocate_pool(P, L, KH, comp, DEV)
    tq_pages.quantize_pages(a, 1, ids, k, v, comp, n_valid)
    for s in range(0, NP, 5):
        tq_pages.quantize_pages(b, 1, ids[s:s + 5], k[s:s + 5], v[s:s + 5], comp, n_valid[s:s + 5])
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), b.cpu())


def test_device_buffers_cached_and_refreshed():
    """The compressor's signs and JL matrix are uploaded once per device and
    uploaded again after an in-place change or a replacement; pages written
    after the change carry codes of the changed matrix."""
    _say("device buffer cache")
    comp = _compressor(3)
    s1, j1, _ = tq_pages._buffers(comp, DEV)
    s2, j2, _ = tq_pages._buffers(comp, DEV)
    assert s1 is s2 and j1 is j2
    comp.jl_matrix.neg_()
    _, j3, _ = tq_pages._buffers(comp, DEV)
    assert j3 is not j1 and torch.equal(j3.cpu(), comp.jl_matrix)
    comp.jl_matrix = torch.flip(comp.jl_matrix, [0]).contiguous()
    _, j4, _ = tq_pages._buffers(comp, DEV)
    assert torch.equal(j4.cpu(), comp.jl_matrix)
    k = _student_t((1, 2, 16, 128), 5)
    pool = tq_pages.allocate_pool(1, 1, 2, comp, DEV)
    tq_pages.quantize_pages(pool, 0, torch.zeros(1, dtype=torch.int32, device=DEV), k.to(DEV), k.to(DEV), comp)
    got = tq_pages.read_pages(pool, 0, torch.zeros(1, dtype=torch.int32, device=DEV), comp)["qjl_signs"][0, 0].cpu()
    ref = CUDATurboQuantOps.compress_gpu(k.to(DEV).reshape(-1, 128), 128, 128, 7, 3, comp._hadamard_signs,
                                         comp.jl_matrix)["qjl_signs"].cpu().reshape(2, 16, 64)
    assert torch.equal(got, ref)


def _turbo_case(comp, B, H, KH, ctxs, seed, L=1, layer=0, spare=2):
    g = torch.Generator().manual_seed(seed)
    npages = [(c + 15) // 16 for c in ctxs]
    P = sum(npages) + spare
    pool = tq_pages.allocate_pool(P, L, KH, comp, DEV)
    k = _student_t((P, KH, 16, 128), seed + 1)
    v = _student_t((P, KH, 16, 128), seed + 2)
    tq_pages.quantize_pages(pool, layer, torch.arange(P, dtype=torch.int32, device=DEV), k.to(DEV), v.to(DEV), comp)
    perm = torch.randperm(P, generator=g)
    table = torch.full((B, max(max(npages), 1)), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(npages):
        table[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = torch.randn(B, H, 128, generator=g)
    lens = torch.tensor(ctxs, dtype=torch.int32)
    return pool, q, table, lens


def _codes(pool, comp, layer):
    P = pool.shape[0]
    c = tq_pages.read_pages(pool, layer, torch.arange(P, dtype=torch.int32, device=DEV), comp)
    return {k: t.cpu() for k, t in c.items()}


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("H,KH", [(40, 8), (16, 2), (8, 8)])
def test_decode_turbo_matches_oracle(bits, H, KH):
    _say(f"turbo decode bits {bits} H {H} KH {KH}")
    comp = _compressor(bits, seed=bits)
    pool, q, table, lens = _turbo_case(comp, 3, H, KH, [37, 300, 1], seed=H + bits)
    out = tq_pages.paged_attention_decode_turbo(q.to(DEV), pool, table.to(DEV), lens.to(DEV), 0, comp)
    torch.cuda.synchronize()
    ref = PD.paged_attention_decode_turbo(_params(comp), q, _codes(pool, comp, 0), table, lens)
    _assert_close(out, ref, f"bits {bits} H {H} KH {KH}")


def test_decode_turbo_zero_context_absent_page_and_layer():
    _say("turbo edge cases")
    comp = _compressor(3)
    pool, q, table, lens = _turbo_case(comp, 4, 8, 2, [0, 64, 17, 5], seed=9, L=3, layer=2)
    table[1, 1] = -1  # an absent page: its tokens are skipped
    out = tq_pages.paged_attention_decode_turbo(q.to(DEV), pool, table.to(DEV), lens.to(DEV), 2, comp, scale=0.3)
    torch.cuda.synchronize()
    assert (out[0] == 0).all()
    ref = PD.paged_attention_decode_turbo(_params(comp), q, _codes(pool, comp, 2), table, lens, scale=0.3)
    _assert_close(out, ref, "edge cases")


def test_decode_turbo_long_contexts_many_partitions():
    """14B TurboQuant shape (40/8 heads) at a reduced batch and context: many
    work items per sequence, merged by the partition merge."""
    _say("turbo long contexts")
    comp = _compressor(3)
    pool, q, table, lens = _turbo_case(comp, 2, 40, 8, [8192, 2900], seed=21)
    out = tq_pages.paged_attention_decode_turbo(q.to(DEV), pool, table.to(DEV), lens.to(DEV), 0, comp)
    torch.cuda.synchronize()
    ref = PD.paged_attention_decode_turbo(_params(comp), q, _codes(pool, comp, 0), table, lens)
    _assert_close(out, ref, "long contexts")


@pytest.mark.parametrize("name", ["14b-turbo3", "14b-turbo4"])
def test_decode_turbo_full_size_sampled_parity(name):
    """The TurboQuant benchmark at its full size (B=16 x 32768 tokens, 40/8
    heads): two sequences match the oracle on the codes read back from their
    own pages."""
    from vramancer_amd import workloads

    cfg = workloads.CONFIGS[name]
    _say(f"{name} full size")
    inp = workloads.make_decode_inputs(cfg, DEV, seed=4, layers=(0,))
    q, pool, table, lens, comp = (inp["query"], inp["kv_pool"], inp["page_table"], inp["context_lens"],
                                  inp["compressor"])
    out = tq_pages.paged_attention_decode_turbo(q, pool, table, lens, 0, comp)
    torch.cuda.synchronize()
    for b in (0, 11):
        n = (int(lens[b]) + 15) // 16
        codes = {k: t.cpu() for k, t in tq_pages.read_pages(pool, 0, table[b, :n].contiguous(), comp).items()}
        ref = PD.paged_attention_decode_turbo(_params(comp), q[b:b + 1].cpu(), codes,
                                              torch.arange(n, dtype=torch.int32)[None], lens[b:b + 1].cpu())
        _assert_close(out[b:b + 1], ref, f"{name} seq {b}")
