"""GPU parity of the split-K paged decode against the CPU oracle.

Tolerance (attention outputs): |gpu - oracle| <= 2e-3 + 1e-2 * |oracle|
elementwise (max-abs 2e-3 / rel 1e-2), the oracle being the reference's
PyTorch decode path restated in oracle/paged_decode.py, evaluated on the very
same pool contents (for quantized pools, on the same codes and scales).
"""
import math

import pytest
import torch

from oracle import paged_decode as PD
from vramancer_amd import _lib, kv_quant, workloads
from vramancer_amd.paged_attention_cuda import paged_attention_decode, paged_attention_decode_q4

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-3, 1e-2
DEV = "cuda:0"


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _assert_close(got, want, what):
    got = got.float().cpu()
    want = want.float().cpu()
    err = (got - want).abs()
    bound = ATOL + RTOL * want.abs()
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.numel()} outside tolerance, "
                          f"max abs err {err.max().item():.3e}")


def _shared_pages(dtype, D, PS):
    """True where the int8 / fp8 decode runs on workgroups whose wavefronts
    take page pairs as they free up (page 16, head_dim 64 .. 128): which
    wavefront sums which pages varies from run to run, so two runs agree to
    rounding, not bit for bit.  Every other path is deterministic."""
    return dtype in (torch.int8, torch.float8_e4m3fn) and PS == 16 and 64 <= D <= 128


def _assert_rerun(a, b, shared, what):
    """Two decodes of the same logical inputs: bit-identical on the
    deterministic paths; on the shared-page ones within rounding of the
    output's scale, |a - b| <= 1e-5 max|b| + 1e-6.  (The decode's error
    against the oracle is about 5e-5 wherever the x20 outlier channels make
    outputs reach 40-50, whatever the row; two runs differ by as much.)"""
    if shared:
        a, b = a.float(), b.float()
        fin = torch.isfinite(b)
        bar = 1e-5 * b[fin].abs().max() + 1e-6 if fin.any() else 0.0
        ok = (a == b) | (fin & ((a - b).abs() <= bar))  # equal (infinities included) or close
        err = torch.where(fin, (a - b).abs(), torch.zeros_like(b))
        assert ok.all(), f"{what}: {int((~ok).sum())} outside, max abs diff {err.max().item():.3e}"
    else:
        assert torch.equal(a, b), what


def _oracle(inp, layer):
    pool = inp["kv_pool"].cpu()
    sc = inp["kv_scales"].cpu() if inp["kv_scales"] is not None else None
    return PD.paged_attention_decode(inp["query"].cpu(), pool, inp["page_table"].cpu(),
                                     inp["context_lens"].cpu(), layer, kv_scales=sc)


CASES = [
    ("fp32-plumbing", dict()),
    ("7b-bf16", dict(batch=4, ctx_div=4)),
    ("14b-int8", dict(batch=4, ctx_div=8, num_layers=3)),
    ("mixed-fp8", dict(batch=6, ctx_div=32)),
]


@pytest.mark.parametrize("name,kw", CASES, ids=[c[0] for c in CASES])
def test_decode_matches_oracle_on_benchmark_shapes(name, kw):
    cfg = workloads.scaled(workloads.CONFIGS[name], **kw)
    layer = cfg.num_layers - 1
    _say(f"{name} scaled {kw} layer {layer}")
    inp = workloads.make_decode_inputs(cfg, DEV, seed=11, layers=(layer,))
    out = paged_attention_decode(inp["query"], inp["kv_pool"], inp["page_table"], inp["context_lens"], layer,
                                 kv_scales=inp["kv_scales"])
    torch.cuda.synchronize()
    _assert_close(out, _oracle(inp, layer), name)


def _pool_case(dtype, B, H, KH, D, ctxs, L=2, layer=1, seed=0, spare=3, table_pad=1, v_mag=None, PS=16):
    g = torch.Generator().manual_seed(seed)
    npages = [(max(c, 0) + PS - 1) // PS for c in ctxs]
    P = sum(npages) + spare
    base = torch.randn(P, L, 2, KH, PS, D, generator=g)
    if v_mag is not None:  # V magnitude: a number, or one factor per page [P]
        base[:, :, 1] *= torch.as_tensor(v_mag, dtype=torch.float32).reshape(-1, 1, 1, 1, 1)
    scales = None
    if dtype == torch.int8:
        from oracle.kv_codecs import pool_from_logical, quantize_int8
        pool, scales = quantize_int8(base)
        pool = pool_from_logical(pool)  # quantized pools keep V tiled
    elif dtype == torch.float8_e4m3fn:
        from oracle.kv_codecs import pool_from_logical
        amax = base.abs().amax(dim=(-2, -1))
        scales = amax / 448
        pool = (base / scales[..., None, None]).to(torch.float8_e4m3fn)
        pool = pool_from_logical(pool.view(torch.uint8)).view(torch.float8_e4m3fn)
    else:
        pool = base.to(dtype)
    perm = torch.randperm(P, generator=g)
    table = torch.full((B, max(max(npages), 1) + table_pad), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(npages):
        table[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = torch.randn(B, H, D, generator=g)
    return q, pool, scales, table, torch.tensor(ctxs, dtype=torch.int32)


def _run_both(q, pool, scales, table, lens, layer, scale=None):
    out = paged_attention_decode(q.to(DEV), pool.to(DEV), table.to(DEV), lens.to(DEV), layer, scale=scale,
                                 kv_scales=None if scales is None else scales.to(DEV))
    torch.cuda.synchronize()
    ref = PD.paged_attention_decode(q, pool, table, lens, layer, scale=scale, kv_scales=scales)
    return out.cpu(), ref


DTYPES = [torch.float32, torch.float16, torch.bfloat16, torch.int8, torch.float8_e4m3fn]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("H,KH,D", [(12, 12, 64), (32, 8, 128), (40, 8, 128), (28, 4, 128), (64, 8, 128),
                                    (16, 1, 128), (8, 2, 256), (6, 3, 64)])
def test_decode_dtypes_gqa_and_head_dims(dtype, H, KH, D):
    _say(f"dtype {dtype} H {H} KH {KH} D {D}")
    q, pool, sc, table, lens = _pool_case(dtype, 3, H, KH, D, [37, 160, 1], seed=H + D)
    out, ref = _run_both(q, pool, sc, table, lens, 1)
    _assert_close(out, ref, f"{dtype} H{H} KH{KH} D{D}")


def test_decode_zero_and_single_token_contexts():
    _say("ctx 0 and 1")
    q, pool, sc, table, lens = _pool_case(torch.bfloat16, 4, 8, 2, 128, [0, 1, 16, 0], seed=3)
    out, ref = _run_both(q, pool, sc, table, lens, 1)
    assert (out[0] == 0).all() and (out[3] == 0).all()
    _assert_close(out, ref, "ctx 0/1")
    # a single token returns its V row for every head of the group
    pid = int(table[1, 0])
    for h in range(8):
        torch.testing.assert_close(out[1, h], pool[pid, 1, 1, h // 4, 0].float(), atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn], ids=lambda d: str(d).split(".")[-1])
def test_decode_merge_starts_the_longest_sequence_first(dtype):
    """The merge runs the sequence with the most partials in its first
    workgroup row (swapped with sequence 0): the longest sequence in the
    middle of the batch, a tie for the longest, sequence 0 empty and a
    one-token one, all against the oracle."""
    _say(f"merge order {dtype}")
    for ctxs in ([0, 300, 12000, 40, 1, 12000, 900], [5000, 17, 0, 4999, 64]):
        q, pool, sc, table, lens = _pool_case(dtype, len(ctxs), 16, 4, 128, ctxs, L=1, layer=0, seed=len(ctxs))
        out, ref = _run_both(q, pool, sc, table, lens, 0)
        _assert_close(out, ref, f"{dtype} {ctxs}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.int8, torch.float8_e4m3fn],
                         ids=lambda d: str(d).split(".")[-1])
def test_decode_long_context_many_partitions(dtype):
    _say(f"long context {dtype}")
    q, pool, sc, table, lens = _pool_case(dtype, 2, 16, 2, 128, [20011, 3000], L=1, layer=0, seed=5)
    out, ref = _run_both(q, pool, sc, table, lens, 0)
    _assert_close(out, ref, "long context")


def test_decode_custom_scale_and_layer():
    _say("custom scale")
    q, pool, sc, table, lens = _pool_case(torch.float32, 2, 8, 8, 64, [100, 33], L=3, layer=2, seed=8)
    out, ref = _run_both(q, pool, sc, table, lens, 2, scale=0.37)
    _assert_close(out, ref, "scale 0.37")


def test_decode_absent_pages_are_skipped():
    _say("absent pages")
    q, pool, sc, table, lens = _pool_case(torch.float32, 2, 4, 2, 64, [64, 48], L=1, layer=0, seed=9)
    P = pool.shape[0]
    table[0, 1] = -1       # negative id
    table[1, 2] = P + 5    # out of range id
    out = paged_attention_decode(q.to(DEV), pool.to(DEV), table.to(DEV), lens.to(DEV), 0)
    torch.cuda.synchronize()
    for b in range(2):
        K, V = PD.gather_sequence(pool, table[b], int(lens[b]), 0, skip_invalid=True)
        ref = PD.dense_attention(q[b], K, V, 1 / 8)
        _assert_close(out[b].cpu(), ref, f"absent pages b{b}")


def test_partitions_then_merge_equals_fused_call():
    _say("partitions + merge")
    q, pool, sc, table, lens = _pool_case(torch.int8, 3, 40, 8, 128, [300, 2000, 17], L=1, layer=0, seed=4)
    q, pool, sc, table, lens = (t.to(DEV) for t in (q, pool, sc, table, lens))
    out = paged_attention_decode(q, pool, table, lens, 0, kv_scales=sc)
    lib = _lib.load()
    B, H, D = q.shape
    P, L, _, KH, PS, _ = pool.shape
    from vramancer_amd.paged_attention_cuda import decode_workspace
    ws = decode_workspace(B, H, KH, D, table.shape[1], q.device)
    out2 = torch.empty_like(out)
    s = _lib.stream_of(q)
    rc = lib.vrm_paged_decode_partitions(q.data_ptr(), pool.data_ptr(), sc.data_ptr(), table.data_ptr(),
                                         lens.data_ptr(), ws.data_ptr(), ws.numel(), B, H, KH, D, PS, L, P,
                                         table.shape[1], 0, 1 / math.sqrt(D), _lib.VRM_KV_I8, s)
    _lib.check(rc, "partitions")
    rc = lib.vrm_paged_decode_merge(lens.data_ptr(), out2.data_ptr(), ws.data_ptr(), ws.numel(), B, H, KH, D, PS,
                                    table.shape[1], s)
    _lib.check(rc, "merge")
    torch.cuda.synchronize()
    _assert_rerun(out, out2, _shared_pages(torch.int8, D, PS), "partitions + merge")


@pytest.mark.parametrize("dtype", [torch.int8, torch.float8_e4m3fn], ids=["int8", "fp8"])
@pytest.mark.parametrize("H,KH,D", [(16, 8, 128), (32, 4, 128), (24, 8, 96), (16, 4, 64)])
def test_shared_items_many_sequences(dtype, H, KH, D):
    """More sequences than a resident round has rows of two-unit workgroups:
    the shared-items pass runs four kv-head units per workgroup over rows of
    equal page runs (ragged lengths, empty sequences, one long sequence over
    many rows); the fused call, and partitions + merge, match the oracle."""
    _say(f"shared items, many sequences {dtype} H{H} KH{KH} D{D}")
    g = torch.Generator().manual_seed(H * 7 + D)
    ctxs = [int(x) for x in torch.randint(1, 400, (150,), generator=g)]
    for i in (3, 40, 77):
        ctxs[i] = 0
    ctxs[100] = 6000
    q, pool, sc, table, lens = _pool_case(dtype, len(ctxs), H, KH, D, ctxs, L=1, layer=0, seed=H + D)
    d = [t.to(DEV) for t in (q, pool, sc, table, lens)]
    out = paged_attention_decode(d[0], d[1], d[3], d[4], 0, kv_scales=d[2])
    lib = _lib.load()
    B = len(ctxs)
    P, L, _, _, PS, _ = pool.shape
    from vramancer_amd.paged_attention_cuda import decode_workspace
    ws = decode_workspace(B, H, KH, D, table.shape[1], DEV)
    out2 = torch.full_like(out, float("nan"))
    s = _lib.stream_of(d[0])
    code = kv_quant.abi_dtype_code(d[1], d[2])
    rc = lib.vrm_paged_decode_partitions(d[0].data_ptr(), d[1].data_ptr(), d[2].data_ptr(), d[3].data_ptr(),
                                         d[4].data_ptr(), ws.data_ptr(), ws.numel(), B, H, KH, D, PS, L, P,
                                         table.shape[1], 0, 1 / math.sqrt(D), code, s)
    _lib.check(rc, "partitions")
    rc = lib.vrm_paged_decode_merge(d[4].data_ptr(), out2.data_ptr(), ws.data_ptr(), ws.numel(), B, H, KH, D, PS,
                                    table.shape[1], s)
    _lib.check(rc, "merge")
    torch.cuda.synchronize()
    ref = PD.paged_attention_decode(q, pool, table, lens, 0, kv_scales=sc)
    _assert_close(out.cpu(), ref, "fused call")
    _assert_close(out2.cpu(), ref, "partitions + merge")
    assert not out[torch.tensor(ctxs) == 0].any(), "empty sequences give zero rows"


@pytest.mark.parametrize("H,KH,D", [(16, 4, 128), (40, 8, 128), (12, 2, 128), (14, 2, 128), (10, 2, 64),
                                    (12, 2, 256)])
def test_decode_q4_matches_oracle(H, KH, D):
    """Head groups per wave: 4, 5, 6, 1 (7 heads per kv-head), 5 and 6 at the
    other head dims."""
    _say(f"q4 H={H} KH={KH} D={D}")
    g = torch.Generator().manual_seed(12)
    B, PS, L = 3, 16, 2
    ctxs = [70, 1, 400]
    npages = [(c + PS - 1) // PS for c in ctxs]
    P = sum(npages) + 2
    packed = torch.randint(0, 256, (P, L, 2, KH, PS, D // 2), generator=g, dtype=torch.uint8)
    sc = (torch.rand(P, L, 2, KH, PS, D // 32, generator=g) * 0.1 + 0.01).half()
    zp = (torch.rand(P, L, 2, KH, PS, D // 32, generator=g) * 15).half()
    perm = torch.randperm(P, generator=g)
    table = torch.full((B, max(npages)), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(npages):
        table[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = torch.randn(B, H, D, generator=g)
    lens = torch.tensor(ctxs, dtype=torch.int32)
    out = paged_attention_decode_q4(q.to(DEV), packed.to(DEV), sc.to(DEV), zp.to(DEV), table.to(DEV), lens.to(DEV), 1)
    torch.cuda.synchronize()
    ref = PD.paged_attention_decode_q4(q, packed, sc, zp, table, lens, 1)
    _assert_close(out.cpu(), ref, "q4")


@pytest.mark.parametrize("v_mag", [1e-4, 1e5, "per-page"])
def test_decode_q4_v_scale_independence(v_mag):
    """Q4 V scales (fp16) at magnitudes from about 1e-6 to 1e4, and, "per-page",
    with each page's V scales multiplied by its own 10^u, u ~ U[-4, 4]: the
    output keeps the relative precision of V's codes, and scales above the
    fp16 range of a plain weight (p * s up to 8 * 65504) do not overflow.
    Bar: |gpu - oracle| <= 1e-3 * max|oracle| per sequence."""
    _say(f"q4 V magnitude {v_mag}")
    g = torch.Generator().manual_seed(31)
    B, H, KH, D, PS, L = 3, 40, 8, 128, 16, 2
    ctxs = [37, 1600, 333]
    npages = [(c + PS - 1) // PS for c in ctxs]
    P = sum(npages) + 2
    packed = torch.randint(0, 256, (P, L, 2, KH, PS, D // 2), generator=g, dtype=torch.uint8)
    sc = torch.rand(P, L, 2, KH, PS, D // 32, generator=g) * 0.1 + 0.01
    zp = (torch.rand(P, L, 2, KH, PS, D // 32, generator=g) * 15).half()
    if v_mag == "per-page":
        mag = torch.pow(10.0, torch.rand(P, generator=g) * 8 - 4).reshape(P, 1, 1, 1, 1)
    else:
        mag = torch.tensor(float(v_mag))
    sc[:, :, 1] = sc[:, :, 1] * mag
    sc = sc.half()
    assert torch.isfinite(sc).all()
    perm = torch.randperm(P, generator=g)
    table = torch.full((B, max(npages)), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(npages):
        table[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = torch.randn(B, H, D, generator=g)
    lens = torch.tensor(ctxs, dtype=torch.int32)
    out = paged_attention_decode_q4(q.to(DEV), packed.to(DEV), sc.to(DEV), zp.to(DEV), table.to(DEV), lens.to(DEV), 1)
    torch.cuda.synchronize()
    ref = PD.paged_attention_decode_q4(q, packed, sc, zp, table, lens, 1)
    out = out.cpu()
    assert torch.isfinite(out).all()
    for b in range(B):
        err = (out[b] - ref[b]).abs().max().item()
        bar = 1e-3 * ref[b].abs().max().item()
        assert err <= bar, f"seq {b}: max abs err {err:.3e} > {bar:.3e}"


def test_decode_full_size_int8_sampled_parity_and_relabel_invariance():
    """14B int8 at its full size (B=64, context 4096, 16384 pages): the output of
    a sample of sequences matches the oracle, and relabelling the physical pages
    (pool rows permuted, table remapped) leaves the output bit-identical."""
    cfg = workloads.scaled(workloads.CONFIGS["14b-int8"], num_layers=2)
    _say("14b-int8 full size, L=2")
    inp = workloads.make_decode_inputs(cfg, DEV, seed=21, layers=(1,))
    q, pool, sc, table, lens = inp["query"], inp["kv_pool"], inp["kv_scales"], inp["page_table"], inp["context_lens"]
    out = paged_attention_decode(q, pool, table, lens, 1, kv_scales=sc)
    torch.cuda.synchronize()
    for b in (0, 37, 63):
        pages = table[b].long()
        sub_pool = pool[pages].cpu()
        sub_sc = sc[pages].cpu()
        sub_table = torch.arange(pages.numel(), dtype=torch.int32)[None]
        ref = PD.paged_attention_decode(q[b:b + 1].cpu(), sub_pool, sub_table, lens[b:b + 1].cpu(), 1,
                                        kv_scales=sub_sc)
        _assert_close(out[b:b + 1], ref, f"full-size seq {b}")
    P = pool.shape[0]
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(3)).to(DEV)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(P, device=DEV)
    pool2 = pool[perm]       # new page i holds old page perm[i]
    sc2 = sc[perm]
    table2 = inv[table.long()].to(torch.int32)
    out2 = paged_attention_decode(q, pool2, table2, lens, 1, kv_scales=sc2)
    torch.cuda.synchronize()
    _assert_rerun(out, out2, _shared_pages(torch.int8, 128, 16), "relabelled pool")


def test_decode_full_size_q4_sampled_parity_and_relabel_invariance():
    """The 14B shape over the 4-bit pool at full size (B=64, context 4096,
    16384 pages): sampled sequences match the oracle, and relabelling the
    physical pages leaves the output bit-identical."""
    cfg = workloads.scaled(workloads.CONFIGS["14b-q4"], num_layers=2)
    _say("14b-q4 full size, L=2")
    inp = workloads.make_decode_inputs(cfg, DEV, seed=23, layers=(1,))
    q, pool, sc, zp = inp["query"], inp["kv_pool"], inp["kv_scales"], inp["kv_zeros"]
    table, lens = inp["page_table"], inp["context_lens"]
    out = paged_attention_decode_q4(q, pool, sc, zp, table, lens, 1)
    torch.cuda.synchronize()
    for b in (0, 29, 63):
        pages = table[b].long()
        sub_table = torch.arange(pages.numel(), dtype=torch.int32)[None]
        ref = PD.paged_attention_decode_q4(q[b:b + 1].cpu(), pool[pages].cpu(), sc[pages].cpu(), zp[pages].cpu(),
                                           sub_table, lens[b:b + 1].cpu(), 1)
        _assert_close(out[b:b + 1], ref, f"q4 full-size seq {b}")
    P = pool.shape[0]
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(4)).to(DEV)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(P, device=DEV)
    out2 = paged_attention_decode_q4(q, pool[perm], sc[perm], zp[perm], inv[table.long()].to(torch.int32), lens, 1)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


def test_decode_q4_ignores_garbage_past_context():
    """Scales and zeros of slots past the context, and of a page the table
    marks absent, may hold anything (here NaN and inf); the output must equal
    the oracle's, which never reads them."""
    _say("q4 garbage past context")
    g = torch.Generator().manual_seed(41)
    B, H, KH, D, PS, L = 3, 40, 8, 128, 16, 1
    ctxs = [37, 160, 5]
    npages = [(c + PS - 1) // PS for c in ctxs]
    P = sum(npages) + 1
    packed = torch.randint(0, 256, (P, L, 2, KH, PS, D // 2), generator=g, dtype=torch.uint8)
    sc = (torch.rand(P, L, 2, KH, PS, D // 32, generator=g) * 0.1 + 0.01).half()
    zp = (torch.rand(P, L, 2, KH, PS, D // 32, generator=g) * 15).half()
    table = torch.full((B, max(npages)), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(npages):
        table[b, :n] = torch.arange(off, off + n, dtype=torch.int32)
        off += n
    for b, c in enumerate(ctxs):
        last = int(table[b, (c - 1) // PS])
        sc[last, 0, :, :, c % PS or PS:] = float("nan")
        zp[last, 0, :, :, c % PS or PS:] = float("inf")
    sc[P - 1] = float("nan")  # a page the table never references
    table[1, 3] = -1  # an absent page in the middle of sequence 1
    q = torch.randn(B, H, D, generator=g)
    lens = torch.tensor(ctxs, dtype=torch.int32)
    out = paged_attention_decode_q4(q.to(DEV), packed.to(DEV), sc.to(DEV), zp.to(DEV), table.to(DEV), lens.to(DEV), 0)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    ref = PD.paged_attention_decode_q4(q, packed, sc, zp, table, lens, 0)
    _assert_close(out.cpu(), ref, "q4 garbage")


def test_decode_q4_unaligned_scales_take_the_valu_kernel():
    """Scales and zeros that start 2 bytes off an 8-byte boundary (views into
    larger buffers) are decoded by the VALU kernel, to the same bar."""
    _say("q4 unaligned scales")
    g = torch.Generator().manual_seed(43)
    B, H, KH, D, PS, L = 2, 40, 8, 128, 16, 1
    ctxs = [70, 300]
    npages = [(c + PS - 1) // PS for c in ctxs]
    P = sum(npages)
    packed = torch.randint(0, 256, (P, L, 2, KH, PS, D // 2), generator=g, dtype=torch.uint8)
    sc = (torch.rand(P, L, 2, KH, PS, D // 32, generator=g) * 0.1 + 0.01).half()
    zp = (torch.rand(P, L, 2, KH, PS, D // 32, generator=g) * 15).half()
    table = torch.full((B, max(npages)), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(npages):
        table[b, :n] = torch.arange(off, off + n, dtype=torch.int32)
        off += n
    q = torch.randn(B, H, D, generator=g)
    lens = torch.tensor(ctxs, dtype=torch.int32)

    def shifted(t):  # the same values, one float16 past an aligned start
        buf = torch.zeros(t.numel() + 1, dtype=t.dtype, device=DEV)
        buf[1:] = t.reshape(-1).to(DEV)
        return buf[1:].view(t.shape)

    out = paged_attention_decode_q4(q.to(DEV), packed.to(DEV), shifted(sc), shifted(zp), table.to(DEV),
                                    lens.to(DEV), 0)
    torch.cuda.synchronize()
    _assert_close(out.cpu(), PD.paged_attention_decode_q4(q, packed, sc, zp, table, lens, 0), "q4 unaligned")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("D", [128, 80])
def test_decode_float_pool_ignores_garbage_past_context(dtype, D):
    """Slots past the context in the last page, and pages the table marks
    absent, may hold anything (here NaN and inf); the output must equal the
    oracle's, which never reads them."""
    _say(f"garbage past context {dtype} D {D}")
    q, pool, sc, table, lens = _pool_case(dtype, 3, 16, 2, D, [37, 160, 5], seed=31)
    for b, c in enumerate(lens.tolist()):
        last = int(table[b, (c - 1) // 16])
        pool[last, 1, :, :, c % 16 or 16:, :] = float("nan")
    spare = sorted(set(range(pool.shape[0])) - set(table[table >= 0].tolist()))[0]
    pool[spare, 1] = float("inf")  # a page the table never references
    table[1, 3] = -1  # an absent page in the middle of sequence 1
    out = paged_attention_decode(q.to(DEV), pool.to(DEV), table.to(DEV), lens.to(DEV), 1)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    for b in range(3):
        K, V = PD.gather_sequence(pool, table[b], int(lens[b]), 1, skip_invalid=True)
        ref = PD.dense_attention(q[b], K, V, 1 / math.sqrt(D))
        _assert_close(out[b].cpu(), ref, f"seq {b}")


def test_decode_full_size_bf16_sampled_parity():
    """7B bf16 at its full size (B=32, 28/4 heads, context ~U[1024, 8192]):
    a sample of sequences matches the oracle."""
    cfg = workloads.CONFIGS["7b-bf16"]
    _say("7b-bf16 full size")
    inp = workloads.make_decode_inputs(cfg, DEV, seed=5, layers=(0,))
    q, pool, table, lens = inp["query"], inp["kv_pool"], inp["page_table"], inp["context_lens"]
    out = paged_attention_decode(q, pool, table, lens, 0)
    torch.cuda.synchronize()
    for b in (0, 13, 31):
        n = (int(lens[b]) + 15) // 16
        pages = table[b, :n].long()
        sub_pool = pool[pages].cpu()
        sub_table = torch.arange(n, dtype=torch.int32)[None]
        ref = PD.paged_attention_decode(q[b:b + 1].cpu(), sub_pool, sub_table, lens[b:b + 1].cpu(), 0)
        _assert_close(out[b:b + 1], ref, f"7b seq {b} ctx {int(lens[b])}")


def test_decode_full_size_fp8_sampled_parity():
    """Mixed-length fp8 at its full size (128 lognormal contexts plus one of
    131072 tokens, 64/8 heads): the longest, the shortest and a median
    sequence match the oracle on their own pages."""
    cfg = workloads.CONFIGS["mixed-fp8"]
    _say("mixed-fp8 full size")
    inp = workloads.make_decode_inputs(cfg, DEV, seed=9, layers=(0,))
    q, pool, sc, table, lens = inp["query"], inp["kv_pool"], inp["kv_scales"], inp["page_table"], inp["context_lens"]
    out = paged_attention_decode(q, pool, table, lens, 0, kv_scales=sc)
    torch.cuda.synchronize()
    order = torch.argsort(lens.cpu())
    picks = [int(order[-1]), int(order[0]), int(order[len(order) // 2])]
    assert int(lens[picks[0]]) == 131072
    for b in picks:
        n = (int(lens[b]) + 15) // 16
        pages = table[b, :n].long()
        ref = PD.paged_attention_decode(q[b:b + 1].cpu(), pool[pages].cpu(), torch.arange(n, dtype=torch.int32)[None],
                                        lens[b:b + 1].cpu(), 0, kv_scales=sc[pages].cpu())
        _assert_close(out[b:b + 1], ref, f"fp8 seq {b} ctx {int(lens[b])}")


def _dequant_pool(pool, sc, layer):
    """Float32 copy of one layer of a quantized pool (V token-major), garbage included."""
    f = torch.zeros(pool.shape, dtype=torch.float32)
    ids = torch.arange(pool.shape[0])
    for kv in (0, 1):
        f[:, layer, kv] = PD._dequant_pages(pool, sc, ids, layer, kv)
    return f


@pytest.mark.parametrize("dtype", [torch.int8, torch.float8_e4m3fn], ids=["int8", "fp8"])
@pytest.mark.parametrize("D", [128, 96, 112])
def test_decode_quantized_pool_ignores_garbage_past_context(dtype, D):
    """Codes and scales of slots past the context, of a page the table marks
    absent and of a page it never references may hold anything: NaN and inf
    scales, and for fp8 the NaN code 0x7f (0x7f is int8's largest code).  The
    output must equal the oracle's, which never reads them."""
    from oracle.kv_codecs import pool_from_logical, pool_to_logical

    _say(f"garbage past context {dtype} D {D}")
    q, pool, sc, table, lens = _pool_case(dtype, 3, 16, 2, D, [37, 160, 5], seed=31)
    raw = pool_to_logical(pool.view(torch.uint8))
    for b, c in enumerate(lens.tolist()):
        last = int(table[b, (c - 1) // 16])
        raw[last, 1, :, :, c % 16 or 16:, :] = 0x7F
        if dtype == torch.int8:
            sc[last, 1, 0, :, c % 16 or 16:] = float("inf")
            sc[last, 1, 1, :, c % 16 or 16:] = float("nan")
    spare = sorted(set(range(pool.shape[0])) - set(table[table >= 0].tolist()))[0]
    raw[spare, 1] = 0x7F
    sc[spare, 1] = float("nan")
    table[1, 3] = -1  # an absent page in the middle of sequence 1
    pool = pool_from_logical(raw).view(dtype)
    out = paged_attention_decode(q.to(DEV), pool.to(DEV), table.to(DEV), lens.to(DEV), 1, kv_scales=sc.to(DEV))
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    f = _dequant_pool(pool, sc, 1)
    for b in range(3):
        K, V = PD.gather_sequence(f, table[b], int(lens[b]), 1, skip_invalid=True)
        ref = PD.dense_attention(q[b], K, V, 1 / math.sqrt(D))
        _assert_close(out[b].cpu(), ref, f"{dtype} seq {b}")


@pytest.mark.parametrize("dtype", [torch.int8, torch.float8_e4m3fn], ids=["int8", "fp8"])
@pytest.mark.parametrize("v_mag", [1e-4, 1e5, 1e7, "per-page"])
def test_decode_quantized_v_scale_independence(dtype, v_mag):
    """V drawn at magnitudes from 1e-4 to 1e7 (and, "per-page", with each page
    scaled by its own factor 10^u, u ~ U[-4, 4], so the V scales of one
    partition span eight decades): the output keeps the relative precision
    of V's codes.  Bar: |gpu - oracle| <= 1e-3 * max|oracle| over each
    sequence's outputs, the oracle evaluated on the same codes and scales."""
    ctxs = [37, 1600, 333]
    if v_mag == "per-page":
        g = torch.Generator().manual_seed(77)
        n = sum((c + 15) // 16 for c in ctxs) + 3
        v_mag = torch.pow(10.0, torch.rand(n, generator=g) * 8 - 4)
    _say(f"V magnitude {dtype} {v_mag if not torch.is_tensor(v_mag) else 'per-page'}")
    q, pool, sc, table, lens = _pool_case(dtype, 3, 40, 8, 128, ctxs, seed=52, v_mag=v_mag)
    out, ref = _run_both(q, pool, sc, table, lens, 1)
    assert torch.isfinite(out).all()
    for b in range(3):
        err = (out[b] - ref[b]).abs().max().item()
        bar = 1e-3 * ref[b].abs().max().item()
        assert err <= bar, f"seq {b}: max abs err {err:.3e} > {bar:.3e}"


def test_decode_full_size_int8_48_layer_bench_pool():
    """The 14B int8 pool exactly as the benchmark times it: 48 layers of
    16384 pages (29 GB of codes and scales, page stride 1.5 MB, offsets far
    past 4 GiB), layers 0 / 12 / 24 / 36 filled.  Three sequences of each
    filled layer match the oracle on their own pages, and relabelling the
    physical pages of the whole pool leaves layer 36's output bit-identical."""
    cfg = workloads.CONFIGS["14b-int8"]
    layers = (0, 12, 24, 36)
    _say("14b-int8 full 48-layer pool")
    inp = workloads.make_decode_inputs(cfg, DEV, seed=0, layers=layers)
    q, pool, sc, table, lens = inp["query"], inp["kv_pool"], inp["kv_scales"], inp["page_table"], inp["context_lens"]
    assert pool.shape[:2] == (16384, 48)
    for layer in layers:
        out = paged_attention_decode(q, pool, table, lens, layer, kv_scales=sc)
        torch.cuda.synchronize()
        for b in (1, 30, 62):
            pages = table[b].long()
            sub_pool = pool[pages, layer:layer + 1].cpu()
            sub_sc = sc[pages, layer:layer + 1].cpu()
            sub_table = torch.arange(pages.numel(), dtype=torch.int32)[None]
            ref = PD.paged_attention_decode(q[b:b + 1].cpu(), sub_pool, sub_table, lens[b:b + 1].cpu(), 0,
                                            kv_scales=sub_sc)
            _assert_close(out[b:b + 1], ref, f"48-layer pool, layer {layer}, seq {b}")
    # the balanced decode (what the manager picks for this even batch), layer 36
    out_bal = paged_attention_decode(q, pool, table, lens, 36, kv_scales=sc, context_lens_host=lens.tolist())
    torch.cuda.synchronize()
    for b in (1, 30, 62):
        pages = table[b].long()
        ref = PD.paged_attention_decode(q[b:b + 1].cpu(), pool[pages, 36:37].cpu(),
                                        torch.arange(pages.numel(), dtype=torch.int32)[None], lens[b:b + 1].cpu(), 0,
                                        kv_scales=sc[pages, 36:37].cpu())
        _assert_close(out_bal[b:b + 1], ref, f"48-layer pool, balanced, seq {b}")
    P = pool.shape[0]
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(5)).to(DEV)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(P, device=DEV)
    table2 = inv[table.long()].to(torch.int32)
    pool2 = pool[perm]
    sc2 = sc[perm]
    del inp
    out2 = paged_attention_decode(q, pool2, table2, lens, 36, kv_scales=sc2)
    torch.cuda.synchronize()
    _assert_rerun(out, out2, _shared_pages(torch.int8, 128, 16), "relabelled 48-layer pool")


def test_wrappers_reject_bad_out_workspace_and_tables():
    """A wrong out (dtype, shape, device), a host workspace, or a page table /
    context-length array of the wrong batch is refused before any launch."""
    _say("wrapper argument checks")
    q, pool, sc, table, lens = (t.to(DEV) for t in _pool_case(torch.int8, 2, 8, 2, 128, [40, 20], seed=1))
    run = lambda **kw: paged_attention_decode(q, pool, kw.get("table", table), kw.get("lens", lens), 1,  # noqa: E731
                                              kv_scales=sc, out=kw.get("out"), workspace=kw.get("ws"))
    ref = run()
    for kw in (dict(out=torch.empty(2, 8, 128, dtype=torch.float16, device=DEV)),
               dict(out=torch.empty(2, 8, 64, device=DEV)),
               dict(out=torch.empty(2, 8, 128)),
               dict(ws=torch.empty(1 << 24, dtype=torch.uint8)),
               dict(table=table[:1]),
               dict(lens=lens[:1])):
        with pytest.raises(RuntimeError):
            run(**kw)
    _assert_rerun(run(out=torch.empty(2, 8, 128, device=DEV)), ref, _shared_pages(torch.int8, 128, 16),
                  "caller-supplied out")
    packed = torch.zeros(pool.shape[:-1] + (64,), dtype=torch.uint8, device=DEV)
    s4 = torch.ones(pool.shape[:-1] + (4,), dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError):
        paged_attention_decode_q4(q, packed, s4, s4, table[:1], lens, 1)
    with pytest.raises(RuntimeError):
        paged_attention_decode_q4(q, packed, s4, s4, table, lens, 1, out=torch.empty(2, 8, 128, device=DEV)[:, :4])


def _balanced(q, pool, sc, table, lens, layer, lse=None, scale=None):
    """vrm_paged_decode_balanced through the C ABI (device tensors)."""
    lib = _lib.load()
    B, H, D = q.shape
    P, L, _, KH, PS, _ = pool.shape
    out = torch.full((B, H, D), float("nan"), device=DEV)
    scale = 1 / math.sqrt(D) if scale is None else scale
    rc = lib.vrm_paged_decode_balanced(q.data_ptr(), pool.data_ptr(), sc.data_ptr(), table.data_ptr(),
                                       lens.data_ptr(), out.data_ptr(), _lib.ptr(lse), B, H, KH, D, PS, L, P,
                                       table.shape[1], layer, scale, kv_quant.abi_dtype_code(pool, sc),
                                       _lib.stream_of(q))
    _lib.check(rc, "vrm_paged_decode_balanced")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dtype", [torch.int8, torch.float8_e4m3fn], ids=["int8", "fp8"])
@pytest.mark.parametrize("H,KH,D,ctxs", [
    (40, 8, 128, [37, 1600, 333, 0, 1, 4096]),   # ragged: correct for any lengths
    (64, 8, 128, [512] * 20),                    # even
    (16, 1, 128, [3000, 2999, 17]),              # one kv-head, 16 heads per wave: 4-wave workgroups fit the LDS
    (8, 2, 64, [100, 260]),
    (12, 12, 64, [64, 65, 700]),
    (28, 4, 128, [8192, 8000, 1]),               # 512 pages in LDS
    (40, 8, 96, [700, 333, 5]),                  # head_dims between 64 and 128
    (16, 2, 80, [260, 17]),
    (24, 4, 112, [1000, 999]),
    # 12-wavefront workgroups of 768 threads sort a sequence's whole pages
    # when there are 4 .. 768 of them: 1000 pages (read in table order), 768
    # whole pages and a partial one, exactly 768, and 3 pages
    (16, 2, 128, [16000, 12289, 12288, 48]),
])
def test_balanced_decode_matches_oracle(dtype, H, KH, D, ctxs):
    """The balanced decode (one workgroup per sequence and kv-head, partitions
    merged in LDS, pages read in page order) against the oracle, at the
    decode bar."""
    _say(f"balanced {dtype} H {H} KH {KH} D {D} B {len(ctxs)}")
    q, pool, sc, table, lens = _pool_case(dtype, len(ctxs), H, KH, D, ctxs, seed=H + D + len(ctxs))
    out = _balanced(*(t.to(DEV) for t in (q, pool, sc, table, lens)), 1)
    ref = PD.paged_attention_decode(q, pool, table, lens, 1, kv_scales=sc)
    assert torch.isfinite(out).all()
    _assert_close(out, ref, f"balanced {dtype}")


@pytest.mark.parametrize("dtype", [torch.int8, torch.float8_e4m3fn], ids=["int8", "fp8"])
def test_balanced_decode_garbage_absent_pages_and_lse(dtype):
    """NaN / inf scales and 0x7f codes past the context, an absent page and an
    unreferenced page are ignored; the lse output equals the work-item
    decode's."""
    from oracle.kv_codecs import pool_from_logical, pool_to_logical

    _say(f"balanced garbage + lse {dtype}")
    q, pool, sc, table, lens = _pool_case(dtype, 3, 16, 2, 128, [37, 160, 5], seed=31)
    raw = pool_to_logical(pool.view(torch.uint8))
    for b, c in enumerate(lens.tolist()):
        last = int(table[b, (c - 1) // 16])
        raw[last, 1, :, :, c % 16 or 16:, :] = 0x7F
        if dtype == torch.int8:
            sc[last, 1, :, :, c % 16 or 16:] = float("nan")
    table[1, 3] = -1
    pool = pool_from_logical(raw).view(dtype)
    d = [t.to(DEV) for t in (q, pool, sc, table, lens)]
    lse = torch.empty(3, 16, device=DEV)
    out = _balanced(*d, 1, lse=lse)
    lse_ref = torch.empty(3, 16, device=DEV)
    ref_items = paged_attention_decode(d[0], d[1], d[3], d[4], 1, kv_scales=d[2], lse=lse_ref)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    f = _dequant_pool(pool, sc, 1)
    for b in range(3):
        K, V = PD.gather_sequence(f, table[b], int(lens[b]), 1, skip_invalid=True)
        _assert_close(out[b].cpu(), PD.dense_attention(q[b], K, V, 1 / math.sqrt(128)), f"seq {b}")
    torch.testing.assert_close(lse, lse_ref, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(out, ref_items, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.int8, torch.float8_e4m3fn], ids=["int8", "fp8"])
@pytest.mark.parametrize("D,PS", [(128, 16), (64, 16), (96, 16), (128, 32), (256, 16), (48, 8), (80, 4)])
def test_inline_layout_decodes_like_the_plain_layout(dtype, D, PS):
    """The same codes and scales copied into the inline layout give the same
    outputs and lse through every decode path that reads the pool: the
    work-item kernels (pages of 16 and 32 tokens), the generic kernel (other
    head_dims and pages), the no-allocation entry and the balanced decode
    (bit-identical where the path is deterministic, within 1e-5 where pages
    are handed out as wavefronts free up); and they match the oracle."""
    _say(f"inline vs plain {dtype} D{D} PS{PS}")
    codec = "int8" if dtype == torch.int8 else "fp8"
    ctxs = [300, 17, 1000, 0, 129, 64]
    B, H, KH = len(ctxs), 16, 2
    q, pool, sc, table, lens = _pool_case(dtype, B, H, KH, D, ctxs, seed=D + PS, PS=PS)
    P, L = pool.shape[:2]
    ip, isc = kv_quant.allocate_pool(P, L, KH, D, codec, PS, DEV, layout="inline")
    ip.copy_(pool.to(DEV))
    isc.copy_(sc.to(DEV))
    assert kv_quant.pool_layout(ip, isc) == "inline"
    d = [t.to(DEV) for t in (q, pool, sc, table, lens)]
    lib = _lib.load()
    scale = 1 / math.sqrt(D)
    outs = {}
    for name, (pp, ss) in (("plain", (d[1], d[2])), ("inline", (ip, isc))):
        lse = torch.empty(B, H, device=DEV)
        got = [paged_attention_decode(d[0], pp, d[3], d[4], 1, kv_scales=ss, lse=lse), lse]
        na = torch.full((B, H, D), float("nan"), device=DEV)
        ns = lib.vrm_paged_decode_num_splits(B, H, KH, d[3].shape[1], PS)
        if lib.vrm_paged_decode_workspace_bytes(B, H, D, ns) <= _lib.NOALLOC_SCRATCH_BYTES:
            rc = lib.vrm_paged_decode_noalloc(d[0].data_ptr(), pp.data_ptr(), ss.data_ptr(), d[3].data_ptr(),
                                              d[4].data_ptr(), na.data_ptr(), B, H, KH, D, PS, L, P, d[3].shape[1],
                                              1, scale, kv_quant.abi_dtype_code(pp, ss), _lib.stream_of(d[0]))
            _lib.check(rc, "vrm_paged_decode_noalloc")
        else:  # the fixed scratch array is too small for this shape
            na.zero_()
        got.append(na)
        if PS == 16 and D <= 128:
            lse_b = torch.empty(B, H, device=DEV)
            got += [_balanced(d[0], pp, ss, d[3], d[4], 1, lse=lse_b), lse_b]
        outs[name] = got
    torch.cuda.synchronize()
    # the balanced decode (outputs 3, 4) and the work items at page 16 and
    # head_dim 64 .. 128 hand page pairs out as their wavefronts free up, so
    # their summation order (and last bits) vary from run to run whatever the
    # layout; the other paths are bit-identical
    for i, (a, b) in enumerate(zip(outs["plain"], outs["inline"])):
        _assert_rerun(a, b, i >= 3 or _shared_pages(dtype, D, PS), f"output {i} of the two layouts")
    _assert_close(outs["inline"][0], PD.paged_attention_decode(q, pool, table, lens, 1, kv_scales=sc), "oracle")


def test_balanced_decode_refuses_d256_and_the_api_falls_back():
    """D = 256 is outside the balanced decode (VRM_ERR_UNSUPPORTED); the
    Python API then runs the work-item decode for the same even batch."""
    _say("balanced D=256 fallback")
    q, pool, sc, table, lens = _pool_case(torch.int8, 64, 4, 2, 256, [80] * 64, seed=7)
    d = [t.to(DEV) for t in (q, pool, sc, table, lens)]
    with pytest.raises(RuntimeError, match="status -2"):
        _balanced(*d, 1)
    out = paged_attention_decode(d[0], d[1], d[3], d[4], 1, kv_scales=d[2], context_lens_host=[80] * 64)
    torch.cuda.synchronize()
    _assert_close(out, PD.paged_attention_decode(q, pool, table, lens, 1, kv_scales=sc), "D=256 fallback")


def test_api_takes_the_balanced_decode_for_even_batches():
    """paged_attention_decode with host lengths picks the balanced decode for an
    even int8 batch (no workspace is allocated) and the work-item decode for a
    ragged one; both match the oracle."""
    from vramancer_amd import paged_attention_cuda as PAC

    for ctxs, want in (([300] * 32, True), ([30, 3000] * 16, False)):
        _say(f"api balanced choice {want}")
        q, pool, sc, table, lens = _pool_case(torch.int8, len(ctxs), 40, 8, 128, ctxs, seed=len(set(ctxs)))
        assert PAC.prefer_balanced(ctxs, 8, torch.int8) is want
        out = paged_attention_decode(q.to(DEV), pool.to(DEV), table.to(DEV), lens.to(DEV), 1, kv_scales=sc.to(DEV),
                                     context_lens_host=ctxs)
        torch.cuda.synchronize()
        _assert_close(out, PD.paged_attention_decode(q, pool, table, lens, 1, kv_scales=sc), f"api {want}")


# Head dims and page sizes outside the tuned kernels' (page 16, head_dim 64 /
# 128 / 256): the reference kernel takes any head_dim <= 256 and the pool's
# page size (csrc/paged_attention_kernel.cu:102-111, 460-466).  int8 / fp8
# pools need D % 16 == 0 and PS % 4 == 0 (their tiled V).
SHAPES_ALL = [(80, 16), (96, 16), (112, 16), (96, 8), (128, 8), (128, 32), (64, 32), (48, 4), (96, 64), (112, 128)]
SHAPES_FLOAT = [(100, 16), (72, 7), (256, 5), (30, 32), (1, 16)]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("D,PS", SHAPES_ALL, ids=[f"D{d}-PS{p}" for d, p in SHAPES_ALL])
def test_decode_other_head_dims_and_page_sizes(dtype, D, PS):
    _say(f"shape {dtype} D {D} PS {PS}")
    ctxs = [5 * PS + 3, 1, 700, 0]
    q, pool, sc, table, lens = _pool_case(dtype, 4, 12, 4, D, ctxs, seed=D * 7 + PS, PS=PS)
    out, ref = _run_both(q, pool, sc, table, lens, 1)
    _assert_close(out, ref, f"{dtype} D{D} PS{PS}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("D,PS", SHAPES_FLOAT, ids=[f"D{d}-PS{p}" for d, p in SHAPES_FLOAT])
def test_decode_float_pools_any_head_dim_and_page_size(dtype, D, PS):
    """Float pools at head_dims that are not multiples of 4 or 16 and odd
    page sizes, including the reference's maximum head_dim 256 at page 5."""
    _say(f"float shape {dtype} D {D} PS {PS}")
    ctxs = [3 * PS + 1, 260, 17]
    q, pool, sc, table, lens = _pool_case(dtype, 3, 8, 2, D, ctxs, seed=D + PS, PS=PS)
    out, ref = _run_both(q, pool, sc, table, lens, 1)
    _assert_close(out, ref, f"{dtype} D{D} PS{PS}")


@pytest.mark.parametrize("D,PS", [(96, 16), (64, 8), (128, 32), (160, 4)])
def test_decode_q4_other_head_dims_and_page_sizes(D, PS):
    _say(f"q4 D={D} PS={PS}")
    g = torch.Generator().manual_seed(D + PS)
    B, H, KH, L = 3, 8, 2, 2
    ctxs = [70, 1, 400]
    npages = [(c + PS - 1) // PS for c in ctxs]
    P = sum(npages) + 2
    packed = torch.randint(0, 256, (P, L, 2, KH, PS, D // 2), generator=g, dtype=torch.uint8)
    sc = (torch.rand(P, L, 2, KH, PS, D // 32, generator=g) * 0.1 + 0.01).half()
    zp = (torch.rand(P, L, 2, KH, PS, D // 32, generator=g) * 15).half()
    perm = torch.randperm(P, generator=g)
    table = torch.full((B, max(npages)), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(npages):
        table[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = torch.randn(B, H, D, generator=g)
    lens = torch.tensor(ctxs, dtype=torch.int32)
    out = paged_attention_decode_q4(q.to(DEV), packed.to(DEV), sc.to(DEV), zp.to(DEV), table.to(DEV), lens.to(DEV), 1)
    torch.cuda.synchronize()
    _assert_close(out.cpu(), PD.paged_attention_decode_q4(q, packed, sc, zp, table, lens, 1), f"q4 D{D} PS{PS}")


def test_decode_other_shapes_absent_pages_and_many_partitions():
    """D = 96, page 8: a long context split over many work items, an absent
    page, and the int8 pool written through the quantizer."""
    _say("D96 PS8 long + absent")
    q, pool, sc, table, lens = _pool_case(torch.int8, 2, 16, 2, 96, [9001, 2000], L=1, layer=0, seed=13, PS=8)
    table[0, 7] = -1
    out = paged_attention_decode(q.to(DEV), pool.to(DEV), table.to(DEV), lens.to(DEV), 0, kv_scales=sc.to(DEV))
    torch.cuda.synchronize()
    f = _dequant_pool(pool, sc, 0)
    for b in range(2):
        K, V = PD.gather_sequence(f, table[b], int(lens[b]), 0, skip_invalid=True)
        _assert_close(out[b].cpu(), PD.dense_attention(q[b], K, V, 1 / math.sqrt(96)), f"seq {b}")
