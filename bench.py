"""Benchmark: paged-attention decode over an int8 KV cache, 14B shape, one MI355X.

Workload (the configuration the headline metric is quoted on): Qwen2.5-14B-
shaped decode attention, 64 sequences x 4096 tokens of context, 40 query heads
over 8 KV heads, head_dim 128, page 16, in a 48-layer pool of 16384 pages
(25.8 GB of int8 codes + per-token fp32 scales, kept side by side per kv-head
in 33 KB (page, layer) slabs: the library's inline layout).  K/V are bf16 N(0, 1) with 2
of 128 channels per head scaled by 20, quantized to int8 with one scale per
(token, head).  One step = one layer-step: every sequence attends once for one
new query token over one layer.  Steps rotate over 4 filled layers so that the
working set (4 x 556 MB) does not fit the 256 MB Infinity Cache.  After the
warm-up the decode keeps running untimed for --settle seconds, so that the
timed region starts on quiet HBM (see settle()).

Prints one JSON line.  value = microseconds per layer-step (lower is better);
the line also carries the achieved HBM bandwidth on algorithmic bytes, the
tokens/s this implies for a 48-layer model, the roofline of the dominant
kernel (the split-K partition pass, timed alone with events on its stream)
and the reference's CPU path (the oracle restatement) timed on a sample.

``--workload`` measures one of the other decode shapes the same way (7b-bf16:
B=32, 28/4 heads, bf16 pool, context ~U[1024, 8192]; mixed-fp8: 129
sequences, 64/8 heads, fp8 pool, lognormal contexts plus one of 131072;
fp32-plumbing); the default line is 14b-int8.  ``--batcher`` times one layer
of a batched decode step of the 7b-bf16 batch through the pages against the
reference batcher's pad-and-concat step, on the same GPU.  ``--codecs`` times
the codec kernels beside the decode (fp8 append, TurboQuant compress, pack,
decompress, scores, sparse V) with the oracle's CPU time on a sample.
``--hf-cache`` times one layer of a decode step through the Hugging Face
TurboQuant cache at the 14b-turbo3 shape, paged attention against the
materialised keys/values + SDPA the reference's cache hands a model.
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from vramancer_amd import _lib, kv_quant, tq_pages, workloads  # noqa: E402
from vramancer_amd.paged_attention_cuda import decode_workspace, prefer_balanced  # noqa: E402

METRIC = "paged-attn decode µs/layer-step + HBM GB/s (% of peak), 14B-shape quantized KV"
PEAK_HBM_GBPS = 8000.0
LAYERS_FILLED = (0, 12, 24, 36)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_14b_int8.json")
# wave64 VALU instructions per launch of the VALU-bound kernels (rocprofv3 SQ counters)
VALU_FILE = os.path.join(ROOT, "profiles", "valu_counts.json")
# one wave64 VALU instruction per SIMD per 4 cycles: 256 CUs x 4 SIMDs at 2.4 GHz (the flat
# rate; a workload whose entry carries issue_ns_per_inst, the measured issue cost of each
# instruction kind weighted by the kernel loop's own mix, is priced at that instead)
N_SIMDS = 256 * 4
PEAK_VALU_GINST = N_SIMDS * 2.4 / 4
KV_CODE = {"f32": _lib.VRM_KV_F32, "f16": _lib.VRM_KV_F16, "bf16": _lib.VRM_KV_BF16, "int8": _lib.VRM_KV_I8,
           "fp8": _lib.VRM_KV_FP8E4M3}
KV_NAME = {"f32": "K_F32", "f16": "K_F16", "bf16": "K_BF16", "int8": "K_I8", "fp8": "K_FP8", "q4": "K_Q4"}
KERNEL = {"int8": "decode_stream_kernel<K_I8,{D}>", "fp8": "decode_stream_kernel<K_FP8,{D}>",
          "tq3": "decode_tq_kernel<3,{PD}> + merge", "tq4": "decode_tq_kernel<4,{PD}> + merge",
          "bf16": "decode_stream_float_kernel<K_BF16,{D}>", "f16": "decode_stream_float_kernel<K_F16,{D}>",
          "f32": "decode_split_kernel<K_F32,{D},G>", "q4": "decode_stream_q4_kernel + merge"}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_events(fn, steps):
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(steps):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / steps  # microseconds per call


def settle(fn, seconds):
    """Runs fn untimed for about `seconds` (synchronising every 50 calls) and
    returns (calls, elapsed seconds).  The timed region starts once the HBM is
    quiet: the kernel driver clears the memory an earlier process freed in the
    background, which on MI355X slows this decode's reads by about 4 % for
    about a second after a 30 GB pool is freed (the driver's round runs the
    GPU tests, each with such pools, just before the benchmark)."""
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(50):
            fn(n)
            n += 1
        torch.cuda.synchronize()
    return n, time.perf_counter() - t0


def host_us(fn, n):
    """Host microseconds per call to enqueue fn n times (no synchronisation
    inside the loop), the Python and ctypes cost a decode loop pays per layer."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(n):
        fn(i)
    t1 = time.perf_counter()
    torch.cuda.synchronize()
    return (t1 - t0) * 1e6 / n


def cpu_baseline(inp, layer, n_seq, reps, page_size=16):
    """The reference's PyTorch decode path (restated in oracle/) on the host
    cores, over the first n_seq sequences of the same workload.  Returns
    microseconds per context token and the thread count."""
    from oracle import paged_decode as PD

    torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
    threads = torch.get_num_threads()
    table = inp["page_table"][:n_seq]
    pages = torch.unique(table[table >= 0]).long()
    # copy only the pages the sample reads, relabelled 0..n-1
    remap = torch.full((inp["num_pages"],), -1, dtype=torch.long, device=pages.device)
    remap[pages] = torch.arange(pages.numel(), device=pages.device)
    tbl = remap[table.long()].to(torch.int32).cpu()
    q = inp["query"][:n_seq].cpu()
    lens = inp["context_lens"][:n_seq].cpu()
    comp = inp.get("compressor")
    if comp is not None:  # TurboQuant pages: the vectorised decompress + dense attention of the oracle
        from oracle import turboquant as TQ

        codes = {k: v.cpu() for k, v in tq_pages.read_pages(inp["kv_pool"], layer, pages.to(torch.int32),
                                                               comp, page_size).items()}
        p = TQ.TQParams(comp.head_dim, comp.bits_per_angle, comp._padded_dim, comp._n_levels, comp.qjl_dim,
                        comp._hadamard_signs.cpu(), comp.jl_matrix.cpu())
        PD.paged_attention_decode_turbo(p, q, codes, tbl, lens)  # warm-up
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            PD.paged_attention_decode_turbo(p, q, codes, tbl, lens)
            times.append(time.perf_counter() - t0)
        times.sort()
        return times[len(times) // 2] / max(1, int(lens.sum())) * 1e6, threads
    pool = inp["kv_pool"][pages][:, layer:layer + 1].cpu()
    if inp.get("kv_zeros") is not None:  # Q4: the oracle's dequantize-then-attend path
        sc = inp["kv_scales"][pages][:, layer:layer + 1].cpu()
        zp = inp["kv_zeros"][pages][:, layer:layer + 1].cpu()
        PD.paged_attention_decode_q4(q, pool, sc, zp, tbl, lens, 0)  # warm-up
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            PD.paged_attention_decode_q4(q, pool, sc, zp, tbl, lens, 0)
            times.append(time.perf_counter() - t0)
        times.sort()
        return times[len(times) // 2] / max(1, int(lens.sum())) * 1e6, threads
    scales = None
    if inp["kv_scales"] is not None:
        scales = inp["kv_scales"][pages][:, layer:layer + 1].cpu()
    PD.paged_attention_decode(q, pool, tbl, lens, 0, kv_scales=scales)  # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        PD.paged_attention_decode(q, pool, tbl, lens, 0, kv_scales=scales)
        times.append(time.perf_counter() - t0)
    times.sort()
    per_token_us = times[len(times) // 2] / max(1, int(lens.sum())) * 1e6
    return per_token_us, threads


def batcher_step(args):
    """``--batcher``: one layer of a continuous-batching decode step over the
    7b-bf16 batch (B=32, H=28, KH=4, D=128, context ~U[1024, 8192]), two ways
    on the GPU, with the same K/V:

    * paged: the new token's K/V rows written into the pages
      (``vrm_kv_write``), then the paged decode (``vrm_paged_decode``), bf16;
    * pad-and-concat, the reference batcher's step
      (core/continuous_batcher.py:711-756, 828-867): each request's cache
      [1, KH, len, D] left-padded with zeros to the longest and concatenated
      into the batch, the new token appended (``DynamicCache.update``'s
      ``torch.cat``), then transformers' SDPA attention with the padding mask,
      which repeats K/V to H heads.  Run in float16, the same bytes per
      element as bfloat16.

    The manager's bookkeeping, once per step for all layers, is timed on its
    own: the slot mapping of one new token per request (``append_tokens``)
    and the device block table, patched with the new token counts and pages
    (``manager_step_us``); a full rebuild of the table from every page list
    (``vrm_build_block_table``) for comparison."""
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    lib = _lib.load()
    dev = torch.device("cuda:0")
    cfg = workloads.CONFIGS["7b-bf16"]
    inp = workloads.make_decode_inputs(cfg, dev, seed=0)
    q, pool, table, lens = inp["query"], inp["kv_pool"], inp["page_table"], inp["context_lens"]
    B, H, D = q.shape
    P, L, _, KH, PS, _ = pool.shape
    max_pp = table.shape[1]
    scale = 1.0 / math.sqrt(D)
    lens_list = lens.tolist()
    stream = _lib.stream_of(q)
    out = torch.empty((B, H, D), dtype=torch.float32, device=dev)
    ws = decode_workspace(B, H, KH, D, max_pp, dev, PS)
    gen = torch.Generator(device=dev).manual_seed(7)
    knew = torch.randn((B, KH, D), generator=gen, device=dev).to(torch.bfloat16)
    vnew = torch.randn((B, KH, D), generator=gen, device=dev).to(torch.bfloat16)
    last = (lens - 1).clamp(min=0)
    pid = table.gather(1, (last // PS).long()[:, None]).squeeze(1).contiguous()
    slot = (last % PS).to(torch.int32).contiguous()

    def paged(i):
        rc = lib.vrm_kv_write(knew.data_ptr(), vnew.data_ptr(), _lib.VRM_SRC_BF16, pid.data_ptr(), slot.data_ptr(),
                              B, pool.data_ptr(), _lib.VRM_KV_BF16, KH, D, PS, L, P, 0, stream)
        rc = rc or lib.vrm_paged_decode(q.data_ptr(), pool.data_ptr(), None, table.data_ptr(), lens.data_ptr(),
                                        out.data_ptr(), ws.data_ptr(), ws.numel(), B, H, KH, D, PS, L, P, max_pp, 0,
                                        scale, _lib.VRM_KV_BF16, stream)
        if rc:
            _lib.check(rc, "paged step")

    # the manager's per-step bookkeeping for the same batch: slot mapping of
    # one new token per request, then the device block table (patched)
    from vramancer_amd.paged_attention import PagedKVCacheManager, PagedKVConfig

    mgr = PagedKVCacheManager(PagedKVConfig(page_size=PS, num_layers=1, num_kv_heads=KH, head_dim=D,
                                            max_pages=P + B * 8, device="cuda:0", dtype="bfloat16"))
    rids = [f"r{b}" for b in range(B)]
    for rid, n in zip(rids, lens_list):
        mgr.allocate(rid, num_tokens=n)

    def bookkeeping(i):
        mgr.append_tokens(rids)
        mgr._block_table(rids, dev)

    def rebuild(i):
        mgr._table_cache = None
        mgr._block_table(rids, dev)

    # per-request caches of layer 0, [1, KH, len, D] float16
    caches = []
    for b, n in enumerate(lens_list):
        pages = pool[table[b, :(n + PS - 1) // PS].long(), 0]  # [np, 2, KH, PS, D]
        kv = pages.permute(1, 2, 0, 3, 4).reshape(2, KH, -1, D)[:, :, :n].to(torch.float16)
        caches.append((kv[0].unsqueeze(0).contiguous(), kv[1].unsqueeze(0).contiguous()))
    maxlen = max(lens_list)
    keep = torch.zeros((B, maxlen + 1), dtype=torch.bool, device=dev)
    for b, n in enumerate(lens_list):
        keep[b, maxlen - n:] = True
    mask = keep[:, None, None, :]  # [B, 1, 1, maxlen + 1], True = attend
    q16 = q.to(torch.float16).unsqueeze(2)  # [B, H, 1, D]
    k16, v16 = knew.to(torch.float16).unsqueeze(2), vnew.to(torch.float16).unsqueeze(2)

    class _Attn:  # what sdpa_attention_forward reads from the attention module
        num_key_value_groups = H // KH
        is_causal = True

    def pad_concat(i):
        ks, vs = [], []
        for (k, v), n in zip(caches, lens_list):
            if n < maxlen:
                z = torch.zeros((1, KH, maxlen - n, D), dtype=k.dtype, device=dev)
                k, v = torch.cat([z, k], dim=2), torch.cat([z, v], dim=2)
            ks.append(k)
            vs.append(v)
        K = torch.cat([torch.cat(ks, dim=0), k16], dim=2)
        V = torch.cat([torch.cat(vs, dim=0), v16], dim=2)
        sdpa_attention_forward(_Attn, q16, K, V, mask, scaling=scale)

    for fn in (paged, rebuild, bookkeeping, pad_concat):
        for i in range(3):
            fn(i)
    torch.cuda.synchronize()
    log("timing the batcher step")
    us_paged = time_events(paged, args.steps)
    us_rebuild = time_events(rebuild, 20)
    us_book = time_events(bookkeeping, 100)  # 100 steps: every request opens 6 or 7 pages
    us_pad = time_events(pad_concat, 10)
    result = {
        "metric": "batched decode step, attention of one layer: paged vs pad-and-concat",
        "value": round(us_paged, 3),
        "unit": "us/layer-step",
        "higher_is_better": False,
        "pad_concat_us": round(us_pad, 1),
        "speedup": round(us_pad / us_paged, 1),
        "manager_step_us": round(us_book, 2),
        "block_table_rebuild_us": round(us_rebuild, 2),
        "dtype": "bf16 (pad-and-concat: f16)",
        "data": "synthetic",
        "config": {"workload": "7b-bf16 batch: B=32, H=28, KH=4, D=128, context ~U[1024, 8192], page 16",
                   "context_tokens": int(sum(lens_list)), "max_context": maxlen},
    }
    print(json.dumps(result), flush=True)


def codec_bench(args):
    """``--codecs``: the codec kernels beside the decode, each timed with HIP
    events on its stream at a size taken from the decode workloads, with its
    algorithmic bytes (inputs read + outputs written) and the oracle's CPU
    time on a bounded sample scaled to the same size:

    * fp8 append: one bf16 token per sequence and kv-head into the last page
      of each of the 129 mixed-fp8 sequences (8 kv-heads, D=128);
    * TurboQuant (3 bits, D=128) over 65,536 bf16 rows (16 sequences x 512
      tokens x 8 kv-heads): compress to the raw codes; pack angles and QJL
      signs; decompress;
    * attention_score: 40 query heads against 32,768 compressed keys;
    * sparse V: the same scores, softmax over the top 10 %, decompressed
      values.
    """
    from oracle import kv_codecs as KC
    from oracle import turboquant as TQ
    from vramancer_amd.kv_quantizer import KVCacheCompressor, _pack_angles, _pack_bits
    from vramancer_amd.turboquant_cuda import CUDATurboQuantOps

    dev = torch.device("cuda:0")
    torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
    threads = torch.get_num_threads()
    g = torch.Generator(device=dev).manual_seed(3)
    rows = []

    def gpu_us(fn, reps=20):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        return time_events(lambda i: fn(), reps)

    def cpu_us(fn, reps=3):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        ts.sort()
        return ts[len(ts) // 2] * 1e6

    def add(name, us, nbytes, cpu, scale_cpu, sample):
        rows.append({"name": name, "us": round(us, 2), "bytes": int(nbytes),
                     "gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "frac_of_8TBs": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4),
                     "cpu_us": round(cpu * scale_cpu, 1), "cpu_sample": sample})
        log(f"{name}: {us:.2f} us, cpu {cpu * scale_cpu:.0f} us")

    # fp8 append, mixed-fp8 shape
    Bq, KH, D, PS = 129, 8, 128, 16
    pool, scales = kv_quant.allocate_pool(Bq, 1, KH, D, "fp8", PS, dev)
    kn = torch.randn((Bq, KH, D), generator=g, device=dev).to(torch.bfloat16)
    vn = torch.randn((Bq, KH, D), generator=g, device=dev).to(torch.bfloat16)
    pid = torch.arange(Bq, dtype=torch.int32, device=dev)
    slot = torch.full((Bq,), 7, dtype=torch.int32, device=dev)
    us = gpu_us(lambda: kv_quant.quantize_append(pool, scales, 0, pid, slot, kn, vn))
    page0 = torch.zeros((PS, D), dtype=torch.uint8)
    kc = kn.cpu()

    def cpu_fp8():
        for b in range(16):
            for h in range(KH):
                KC.fp8_append(page0, torch.tensor(0.1), 7, kc[b, h])

    add("fp8_append", us, 2 * Bq * KH * D * (2 + 1) + 2 * Bq * KH * 4, cpu_us(cpu_fp8), 2 * Bq / 16,
        "oracle fp8_append of 16 of the 129 K rows (all 8 heads), scaled to K and V of 129")

    # TurboQuant over 65,536 rows
    torch.manual_seed(0)
    comp = KVCacheCompressor(128, 3).to(dev)
    p = TQ.TQParams(128, 3, 128, 7, 64, comp._hadamard_signs.cpu(), comp.jl_matrix.cpu())
    N = 65536
    x = torch.randn((N, 128), generator=g, device=dev).to(torch.bfloat16)
    args_ = (128, 128, 7, 3, comp._hadamard_signs, comp.jl_matrix)
    raw = CUDATurboQuantOps.compress_gpu(x, *args_)
    S = 2048
    xs = x[:S].float().cpu()
    add("tq_compress", gpu_us(lambda: CUDATurboQuantOps.compress_gpu(x, *args_)), N * (256 + 195),
        cpu_us(lambda: TQ.compress(p, xs, pack=False)), N / S, f"oracle compress of {S} rows, scaled")
    raw_s = TQ.compress(p, xs, pack=False)
    add("tq_pack", gpu_us(lambda: (_pack_angles(raw["angles"], 3), _pack_bits(raw["qjl_signs"]))),
        N * (127 + 64 + 48 + 8),
        cpu_us(lambda: (TQ.pack_angles(raw_s["angles"], 3), TQ.pack_bits(raw_s["qjl_signs"]))), N / S,
        f"oracle pack_angles + pack_bits of {S} rows, scaled")
    add("tq_decompress", gpu_us(lambda: CUDATurboQuantOps.decompress_gpu(raw, 128, 128, 7, 3, comp._hadamard_signs)),
        N * (2 + 127 + 512), cpu_us(lambda: TQ.decompress(p, raw_s)), N / S,
        f"oracle decompress of {S} rows, scaled")

    # scores and sparse V: 40 heads against 32,768 keys
    Nk, M = 32768, 40
    ck = {k: (v[:Nk] if torch.is_tensor(v) else [a[:Nk] for a in v] if isinstance(v, list) else v)
          for k, v in raw.items()}
    ck["shape"] = (Nk, 128)
    cv = {k: (v[Nk:2 * Nk] if torch.is_tensor(v) else [a[Nk:2 * Nk] for a in v] if isinstance(v, list) else v)
          for k, v in raw.items()}
    cv["shape"] = (Nk, 128)
    q = torch.randn((M, 128), generator=g, device=dev)
    ks = TQ.compress(p, x[:4096].float().cpu(), pack=False)
    qc = q.cpu()
    add("tq_attention_score",
        gpu_us(lambda: CUDATurboQuantOps.attention_score_gpu(q, ck, *args_, 64)),
        Nk * 195 + M * Nk * 4 + M * 128 * 4, cpu_us(lambda: TQ.attention_score(p, qc, ks)), Nk / 4096,
        "oracle attention_score of the 40 heads against 4096 keys, scaled")
    vs = [TQ.compress(p, r[None], pack=False) for r in x[4096:4096 + 4096].float().cpu()]
    add("tq_sparse_v_attend",
        gpu_us(lambda: comp.sparse_v_attend(q, ck, [cv], sparse_v_ratio=0.1)),
        Nk * (195 + 129) + M * Nk * 4 + M * 128 * 4,
        cpu_us(lambda: TQ.sparse_v_attend(p, qc[:1], ks, vs, sparse_v_ratio=0.1), reps=1), M * Nk / 4096,
        "oracle sparse_v_attend of 1 head over 4096 keys (per-token value dicts), scaled to 40 x 32768")
    print(json.dumps({"metric": "codec kernels: us, algorithmic GB/s, and the oracle on the CPU",
                      "n_gpus": 1, "data": "synthetic", "cpu_threads": threads, "rows": rows}), flush=True)


def hf_cache_step(args):
    """``--hf-cache``: one layer of a decode step through the Hugging Face
    TurboQuant cache (``TurboQuantLayer``, core/turboquant_cache.py:78-299) at
    the 14b-turbo3 shape: B=16, H=40, KH=8, D=128, 3 bits per angle, 32,768
    compressed tokens per sequence, a residual of 256, float16 activations.
    Two layers are filled with the same tokens and stepped two ways:

    * paged: ``update`` writes the new token into the residual pages, then
      ``turbo_paged_attention`` (the function ``enable_paged_attention``
      registers) runs the TurboQuant decode over the compressed pages and the
      float decode over the residual, merged by log-sum-exp;
    * materialised, what the reference's cache hands the model
      (core/turboquant_cache.py:176-230): ``update`` returns the full keys and
      values with the compressed part decompressed, and transformers' SDPA
      attends over them (K/V repeated to H heads, all-true padding mask).

    Steps are timed between spills; the spill (256 residual tokens of every
    sequence compressed into pages, once per 256 steps) is timed on its own."""
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    from vramancer_amd.kv_quantizer import KVCacheCompressor
    from vramancer_amd.turboquant_cache import TurboQuantLayer, turbo_paged_attention

    dev = torch.device("cuda:0")
    B, H, KH, D, ctx, bits, R = 16, 40, 8, 128, 32768, 3, 256
    dt = torch.float16
    scale = 1.0 / math.sqrt(D)
    torch.manual_seed(0)
    comp = KVCacheCompressor(D, bits).to(dev)
    gen = torch.Generator(device=dev).manual_seed(3)
    paged_layer = TurboQuantLayer(comp, R, paged_attention=True)
    mat_layer = TurboQuantLayer(comp, R, paged_attention=False)
    log(f"filling two cache layers with {ctx} tokens of {B} sequences")
    chunk = 4096
    for s in range(0, ctx, chunk):
        k = torch.randn((B, KH, chunk, D), generator=gen, device=dev).to(dt)
        v = torch.randn((B, KH, chunk, D), generator=gen, device=dev).to(dt)
        paged_layer.update(k, v)
        mat_layer.update(k, v)
        del k, v
    q = torch.randn((B, H, 1, D), generator=gen, device=dev).to(dt)
    kn = torch.randn((B, KH, 1, D), generator=gen, device=dev).to(dt)
    vn = torch.randn((B, KH, 1, D), generator=gen, device=dev).to(dt)

    class _Attn:  # what the attention functions read from the attention module
        num_key_value_groups = H // KH
        is_causal = True

    def paged(i):
        k, v = paged_layer.update(kn, vn)
        turbo_paged_attention(_Attn, q, k, v, None, scaling=scale)

    def materialised(i):
        k, v = mat_layer.update(kn, vn)
        mask = torch.ones((B, 1, 1, k.shape[2]), dtype=torch.bool, device=dev)
        sdpa_attention_forward(_Attn, q, k, v, mask, scaling=scale)

    # the first step of each spills the last prefill chunk; the residual then
    # holds 1 token and grows by one per step
    warm_p, warm_m = 4, 3
    for i in range(warm_p):
        paged(i)
    for i in range(warm_m):
        materialised(i)
    torch.cuda.synchronize()
    n_paged = min(args.steps, R - warm_p - 1)
    log(f"timing {n_paged} paged steps and 5 materialised steps")
    us_paged = time_events(paged, n_paged)
    us_mat = time_events(materialised, 5)
    for i in range(R - warm_p - n_paged):  # up to a full residual: the next update spills
        paged(i)
    us_spill = time_events(lambda i: paged_layer.update(kn, vn), 1)
    result = {
        "metric": "HF TurboQuant cache decode step, one layer: paged attention vs materialised K/V + SDPA",
        "value": round(us_paged, 3),
        "unit": "us/layer-step",
        "higher_is_better": False,
        "materialised_us": round(us_mat, 1),
        "speedup": round(us_mat / us_paged, 1),
        "spill_us": round(us_spill, 1),
        "spill_per_step_us": round(us_spill / R, 2),
        "dtype": "tq3-polar codes, f16 activations",
        "data": "synthetic",
        "config": {"workload": "14b-turbo3 shape through the HF cache: B=16, H=40, KH=8, D=128, 32,768 "
                               "compressed tokens per sequence, residual 256, 3 bits per angle",
                   "compressed_tokens": ctx, "residual_length": R},
    }
    print(json.dumps(result), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--pool-layout", default=None, choices=("inline", "plain"),
                    help="memory layout of the int8 / fp8 pools (default: kv_quant.default_layout of the codec)")
    ap.add_argument("--settle", type=float, default=2.0,
                    help="seconds of further untimed decode steps after the warm-up, so that the timed region "
                         "starts on quiet HBM (0: none)")
    ap.add_argument("--cpu-seqs", type=int, default=32, help="sequences in the CPU-baseline sample")
    ap.add_argument("--cpu-reps", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--workload", default="14b-int8", choices=sorted(workloads.CONFIGS),
                    help="decode shape to measure (the headline line is 14b-int8)")
    ap.add_argument("--codecs", action="store_true",
                    help="time the codec kernels (fp8 append, TurboQuant compress / pack / decompress / scores / "
                         "sparse V) beside the oracle on the CPU")
    ap.add_argument("--batcher", action="store_true",
                    help="time one layer of a batched decode step, paged vs the reference's pad-and-concat")
    ap.add_argument("--hf-cache", action="store_true",
                    help="time one layer of a decode step through the HF TurboQuant cache, paged attention vs "
                         "materialised K/V + SDPA")
    ap.add_argument("--head-dim", type=int, default=None,
                    help="override the workload's head_dim (any value <= 256; int8 / fp8 need a multiple of 16, "
                         "4-bit a multiple of 32, TurboQuant 33..256)")
    ap.add_argument("--page-size", type=int, default=None,
                    help="override the workload's page size (int8 / fp8 need a multiple of 4)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 10 plain 1 GiB device-to-device copies (known HBM traffic) for counter scaling")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the decode here has no multi-GPU path "
              "(it would shard by sequence or by kv-head, with no exchange); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    if args.batcher:
        batcher_step(args)
        return
    if args.codecs:
        codec_bench(args)
        return
    if args.hf_cache:
        hf_cache_step(args)
        return
    lib = _lib.load()
    dev = torch.device("cuda:0")
    cfg = workloads.CONFIGS[args.workload]
    shape_override = args.head_dim is not None or args.page_size is not None
    if shape_override:
        cfg = dataclasses.replace(cfg, head_dim=args.head_dim or cfg.head_dim,
                                  page_size=args.page_size or cfg.page_size)
    if cfg.num_layers < 4:
        # steps rotate over 4 layers so that consecutive steps never hit in the Infinity Cache
        cfg = workloads.scaled(cfg, num_layers=4)
    layers = LAYERS_FILLED if cfg.num_layers > max(LAYERS_FILLED) else tuple(range(4))
    turbo = cfg.codec in ("tq3", "tq4")
    q4 = cfg.codec == "q4"
    # TurboQuant pages are filled on one layer (compression is the slow part of
    # the set-up); the zero codes of the other layers cost the decode the same.
    fill = (layers[0],) if turbo else layers
    log(f"building {cfg.name} pool ({cfg.num_layers} layers, filling {fill}, rotating {layers})")
    inp = workloads.make_decode_inputs(cfg, dev, seed=0, layers=fill, layout=args.pool_layout)
    torch.cuda.synchronize()
    q, pool, sc, table, lens = inp["query"], inp["kv_pool"], inp["kv_scales"], inp["page_table"], inp["context_lens"]
    zp = inp["kv_zeros"]
    B, H, D = q.shape
    if turbo:
        P, L, _, KH, _ = pool.shape
        PS = cfg.page_size
        comp = inp["compressor"]
        tq_signs, tq_jl, tq_lut = tq_pages._buffers(comp, dev)
    else:
        P, L, _, KH, PS, _ = pool.shape
    max_pp = table.shape[1]
    scale = 1.0 / math.sqrt(D)
    out = torch.empty((B, H, D), dtype=torch.float32, device=dev)
    ws = decode_workspace(B, H, KH, D, max_pp, dev, PS)
    nsplit = lib.vrm_paged_decode_num_splits(B, H, KH, max_pp, PS)
    stream = _lib.stream_of(q)
    code = KV_CODE.get(cfg.codec)
    if cfg.codec in ("int8", "fp8"):
        code = kv_quant.abi_dtype_code(pool, sc)  # the pool's layout (inline, as allocate_pool makes it)
    sc_ptr = sc.data_ptr() if sc is not None else None
    lens_list = lens.tolist()
    ab = workloads.algorithmic_bytes(cfg, lens_list)
    log(f"pool {P} pages, {nsplit} partitions/sequence, algorithmic bytes/layer-step {ab['total'] / 1e6:.2f} MB")

    # even batches over int8 / fp8 pools take the balanced decode (one
    # workgroup per sequence and kv-head, no merge pass), as the manager does
    balanced = (not turbo and not q4 and D in (64, 80, 96, 112, 128) and PS == 16 and
                prefer_balanced(lens_list, KH, pool.dtype))
    log(f"decode mode: {'balanced' if balanced else 'work items + merge'}")

    def full(i):
        layer = layers[i % len(layers)]
        if balanced:
            rc = lib.vrm_paged_decode_balanced(q.data_ptr(), pool.data_ptr(), sc_ptr, table.data_ptr(),
                                               lens.data_ptr(), out.data_ptr(), None, B, H, KH, D, PS, L, P, max_pp,
                                               layer, scale, code, stream)
            if rc:
                _lib.check(rc, "balanced decode")
            return
        if turbo:
            rc = lib.vrm_paged_decode_tq(q.data_ptr(), pool.data_ptr(), table.data_ptr(), lens.data_ptr(),
                                         out.data_ptr(), ws.data_ptr(), ws.numel(), B, H, KH, D, PS, L, P, max_pp,
                                         layer, scale, comp.bits_per_angle, comp.qjl_dim, tq_signs.data_ptr(),
                                         tq_jl.data_ptr(), tq_lut.data_ptr(), stream)
            if rc:
                _lib.check(rc, "turbo decode")
            return
        if q4:
            rc = lib.vrm_paged_decode_q4(q.data_ptr(), pool.data_ptr(), sc.data_ptr(), zp.data_ptr(), table.data_ptr(),
                                         lens.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), B, H, KH, D, PS,
                                         L, P, max_pp, layer, scale, stream)
            if rc:
                _lib.check(rc, "q4 decode")
            return
        rc = lib.vrm_paged_decode(q.data_ptr(), pool.data_ptr(), sc_ptr, table.data_ptr(), lens.data_ptr(),
                                  out.data_ptr(), ws.data_ptr(), ws.numel(), B, H, KH, D, PS, L, P, max_pp, layer,
                                  scale, code, stream)
        if rc:
            _lib.check(rc, "decode")

    def partitions(i):
        layer = layers[i % len(layers)]
        rc = lib.vrm_paged_decode_partitions(q.data_ptr(), pool.data_ptr(), sc_ptr, table.data_ptr(),
                                             lens.data_ptr(), ws.data_ptr(), ws.numel(), B, H, KH, D, PS, L, P,
                                             max_pp, layer, scale, code, stream)
        if rc:
            _lib.check(rc, "partitions")

    for i in range(args.warmup):
        full(i)
    torch.cuda.synchronize()
    settled = settle(full, args.settle)
    log(f"settle: {settled[0]} more untimed layer-steps over {settled[1]:.2f} s")
    # int8 / fp8 at page 16 and head_dim 64 .. 128 without host lengths: the
    # shared-items pass (rows of equal page runs, cut into pieces per sequence)
    shared = not balanced and cfg.codec in ("int8", "fp8") and PS == 16 and D in (64, 80, 96, 112, 128)
    if balanced:
        pps, n_items = None, None
    else:
        # partition geometry the kernel chose (header): pages per partition and
        # work items, or for the shared-items pass pages per row and pieces
        pps, n_items = ws[:8].view(torch.int32).tolist()
    log(f"timing {args.steps} layer-steps")
    us_step = time_events(full, args.steps)
    # TurboQuant, Q4 and the balanced decode: one kernel, whose time is the whole decode
    us_part = us_step if (turbo or q4 or balanced) else time_events(partitions, args.steps)
    # The balanced decode's loads alone (same grid, addresses, order and ring,
    # no computation): what its access pattern costs on this GPU.
    us_loads = None
    if balanced:
        def loads(i):
            rc = lib.vrm_paged_decode_balanced_loads(q.data_ptr(), pool.data_ptr(), sc_ptr, table.data_ptr(),
                                                     lens.data_ptr(), out.data_ptr(), B, H, KH, D, PS, L, P, max_pp,
                                                     layers[i % len(layers)], scale, code, stream)
            if rc:
                _lib.check(rc, "load-only pass")

        for i in range(10):
            loads(i)
        us_loads = time_events(loads, args.steps)
        log(f"load-only pass of the same pattern {us_loads:.2f} us")
    log(f"decode {us_step:.2f} us/layer-step, partition kernel {us_part:.2f} us")

    # The drop-in Python call: the same decode through the module API, with the
    # wrapper allocating out + workspace per call, and with both preallocated.
    from vramancer_amd.paged_attention_cuda import paged_attention_decode, paged_attention_decode_q4

    def api(i, prealloc, host_lens=True):
        layer = layers[i % len(layers)]
        kw = dict(out=out, workspace=ws) if prealloc else {}
        if turbo:
            tq_pages.paged_attention_decode_turbo(q, pool, table, lens, layer, comp, page_size=PS, **kw)
        elif q4:
            paged_attention_decode_q4(q, pool, sc, zp, table, lens, layer, **kw)
        elif host_lens:
            paged_attention_decode(q, pool, table, lens, layer, kv_scales=sc, context_lens_host=lens_list, **kw)
        else:
            # the reference's own call: device lengths only, out and workspace made by the wrapper
            paged_attention_decode(q, pool, table, lens, layer, kv_scales=sc, **kw)

    for i in range(5):  # also loads the kernels each variant launches first
        api(i, False)
        api(i, True)
        api(i, False, False)
    n_host = 50
    n_api = max(args.steps, 200)
    python_api = {
        "host_us_per_call": {
            "c_abi": round(host_us(full, n_host), 2),
            "python": round(host_us(lambda i: api(i, False), n_host), 2),
            "python_preallocated": round(host_us(lambda i: api(i, True), n_host), 2),
        },
        # over at least 200 calls whatever --steps says: a short window would carry the cost of
        # filling the launch queue from Python (13 us of host time per call) into the average
        "us_per_layer_step_python_preallocated": round(time_events(lambda i: api(i, True), n_api), 3),
        # paged_attention_decode(query, kv_pool, page_table, context_lens, layer_idx, kv_scales=...) as the
        # reference's callers write it: no host copy of the lengths, no preallocated buffers
        "us_per_layer_step_reference_signature": round(time_events(lambda i: api(i, False, False), n_api), 3),
        "calls_timed": n_api,
    }
    log(f"python API: {python_api}")

    us_append = None
    if turbo:
        kn = torch.randn((B, KH, D), device=dev).to(torch.bfloat16)
        vn = torch.randn((B, KH, D), device=dev).to(torch.bfloat16)
        last = (lens - 1).clamp(min=0)
        pid = table.gather(1, (last // PS).long()[:, None]).squeeze(1).contiguous()
        slot = (last % PS).to(torch.int32).contiguous()

        def append(i):
            tq_pages.quantize_append(pool, layers[0], pid, slot, kn, vn, comp, page_size=PS)

        for i in range(5):
            append(i)
        us_append = time_events(append, 50)
    elif sc is not None and not q4:  # the reference has no Q4 writer
        # append one token per sequence (quantize-on-append), timed separately
        kn = torch.randn((B, KH, D), device=dev).to(torch.bfloat16)
        vn = torch.randn((B, KH, D), device=dev).to(torch.bfloat16)
        last = (lens - 1).clamp(min=0)
        pid = table.gather(1, (last // PS).long()[:, None]).squeeze(1).contiguous()
        slot = (last % PS).to(torch.int32).contiguous()

        def append(i):
            rc = lib.vrm_kv_quant_append(kn.data_ptr(), vn.data_ptr(), _lib.VRM_SRC_BF16, pid.data_ptr(),
                                         slot.data_ptr(), B, pool.data_ptr(), sc.data_ptr(), code, KH, D, PS, L, P,
                                         layers[0], stream)
            if rc:
                _lib.check(rc, "append")

        for i in range(5):
            append(i)
        us_append = time_events(append, 50)

    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        log("copy calibration: 10 x 1 GiB device copies done")

    achieved = ab["total"] / (us_part * 1e-6) / 1e9
    overall = ab["total"] / (us_step * 1e-6) / 1e9
    traffic = None
    if cfg.name == "14b-int8" and not shape_override and os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    cpu = None
    if not args.no_cpu:
        log(f"CPU baseline on {args.cpu_seqs} sequences")
        per_token_us, threads = cpu_baseline(inp, layers[0], min(args.cpu_seqs, B), args.cpu_reps, PS)
        cpu = {
            "value": round(per_token_us * sum(lens_list), 1),
            "unit": "us/layer-step",
            "cores": threads,
            "kind": "port",
            "sample": ((f"oracle restatement of compute_attention_turbo (per kv-head: QJL-corrected scores "
                        f"of the rotated query, softmax, decompressed values; fp32) over the first "
                        if cfg.codec.startswith("tq") else
                        f"oracle restatement of the reference's PyTorch decode ({cfg.codec} dequant + gather + "
                        f"repeat_interleave + bmm/softmax/bmm, fp32) over the first ")
                       + f"{min(args.cpu_seqs, B)} of the {B} sequences, median of {args.cpu_reps}, scaled by the "
                         "batch's total context"),
        }
    elem = {"f32": "f32", "f16": "f16", "bf16": "bf16", "int8": "int8", "fp8": "fp8e4m3", "tq3": "tq3-polar",
            "tq4": "tq4-polar", "q4": "u4-asym"}[cfg.codec]
    desc = {
        "14b-int8": ("14b-int8 paged decode: B=64, H=40, KH=8, D=128, context 4096, page 16, "
                     "48-layer pool of 16384 pages, int8 codes + per-token fp32 scales in the inline slab layout"),
        "14b-q4": ("14b-q4 paged decode: B=64, H=40, KH=8, D=128, context 4096, page 16, 48-layer pool of "
                   "16384 pages, 4-bit asymmetric codes + per-32-dim-group fp16 scale and zero"),
        "7b-bf16": "7b-bf16 paged decode: B=32, H=28, KH=4, D=128, context ~U[1024, 8192], page 16, bf16 pool",
        "mixed-fp8": ("mixed-fp8 paged decode: 128 sequences lognormal(median 2048, sigma 1) + one of 131072, "
                      "H=64, KH=8, D=128, page 16, fp8 e4m3fn codes + per-page fp32 scales"),
        "fp32-plumbing": "fp32-plumbing paged decode: B=4, H=KH=12, D=64, context 512, page 16, fp32 pool",
        "14b-turbo3": ("14b-turbo3 paged decode over TurboQuant pages: B=16, H=40, KH=8, D=128, context 32768, "
                       "page 16, 3 bits per angle, Student-t(3) K/V"),
        "14b-turbo4": ("14b-turbo4 paged decode over TurboQuant pages: B=16, H=40, KH=8, D=128, context 32768, "
                       "page 16, 4 bits per angle, Student-t(3) K/V"),
    }[cfg.name]
    if shape_override:
        desc += f" (head_dim set to {D}, page size to {PS})"
    if cfg.codec in ("int8", "fp8") and (args.pool_layout or kv_quant.default_layout(cfg.codec)) != "inline":
        desc = desc.replace("in the inline slab layout", "in the plain layout (separate scale array)")
    elif cfg.codec in ("int8", "fp8") and "inline" not in desc:
        desc += " in the inline slab layout"
    if turbo:
        pd = 1 << max(6, (D - 1).bit_length())
        tuned = pd in (64, 128) and comp.qjl_dim == pd // 2 and comp.bits_per_angle in (2, 3, 4) and PS == 16
        kname = KERNEL[cfg.codec].format(PD=pd) if tuned else f"decode_tq_gen_kernel<{pd}> + merge"
    elif (PS == 16 and D in (64, 128, 256)) or (
            PS in (16, 32, 64, 128, 256, 512, 1024) and D in (64, 80, 96, 112, 128, 256)
            and (cfg.codec in ("int8", "fp8") or (cfg.codec in ("bf16", "f16") and D <= 128))):
        kname = KERNEL[cfg.codec].format(D=D)
        if balanced:
            kname = kname.replace(">", ",balanced>")
        elif shared:
            kname = kname.replace(">", ",shared items>")
    else:
        kname = f"decode_generic_kernel<{KV_NAME[cfg.codec]}>" + (" + merge" if q4 else "")
    G = next(g for g in range(16, 0, -1) if (H // KH) % g == 0)
    roofline = {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": PEAK_HBM_GBPS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBPS, 4),
        "traffic": traffic,
        "kernel": kname + (f" (G={G}, whole decode)" if (turbo or q4 or balanced) else f" (G={G}, partition pass)"),
        "kernel_us": round(us_part, 3),
    }
    if us_loads is not None:
        # the access pattern's own time and the kernel's speed as a fraction of it
        roofline["pattern_loads_us"] = round(us_loads, 3)
        roofline["frac_of_pattern"] = round(us_loads / us_part, 4)
    valu = None
    if (turbo or q4) and os.path.exists(VALU_FILE):
        # counts per workload at its own shape ("<workload>") or another ("<workload>@d<D>-ps<PS>")
        key = cfg.name if not shape_override else f"{cfg.name}@d{D}-ps{PS}"
        with open(VALU_FILE) as f:
            valu = json.load(f)["workloads"].get(key)
    if valu is not None:
        # These kernels rebuild or unpack every code on the vector ALU: the
        # binding roofline is VALU issue, the HBM figures stay as context.
        ginst = valu["valu_insts_per_launch"] / (us_part * 1e-6) / 1e9
        ns_inst = valu.get("issue_ns_per_inst")
        peak = N_SIMDS / ns_inst if ns_inst else PEAK_VALU_GINST
        roofline.update({
            "bound": "valu",
            "achieved": round(ginst, 1),
            "peak": round(peak, 1),
            "unit": "Ginst/s",
            "frac": round(ginst / peak, 4),
            "valu_insts_per_launch": valu["valu_insts_per_launch"],
            "issue_ns_per_inst": ns_inst,
            "floor_us": round(valu["valu_insts_per_launch"] / peak / 1e3, 2),
            "frac_flat_4_cycles": round(ginst / PEAK_VALU_GINST, 4),
            "hbm_achieved_gbps": round(achieved, 1),
            "hbm_frac": round(achieved / PEAK_HBM_GBPS, 4),
        })
    result = {
        "metric": METRIC,
        "value": round(us_step, 3),
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"steps": settled[0], "seconds": round(settled[1], 2)},
        "ms_per_step": round(us_step / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": elem,
        "data": "synthetic",
        "config": {
            "workload": desc,
            "batch": B, "num_heads": H, "num_kv_heads": KH, "head_dim": D, "context_tokens": int(sum(lens_list)),
            "page_size": PS, "num_layers": L, "num_pages": P, "pages_per_partition": pps, "work_items": n_items,
            "decode_mode": "balanced" if balanced else "shared-items" if shared else "work-items",
            "layers_rotated": list(layers),
        },
        "hbm_gbps": round(overall, 1),
        "pct_of_peak": round(100 * overall / PEAK_HBM_GBPS, 2),
        "tokens_per_s": round(B / (us_step * 1e-6 * L), 1) if L > 1 else None,
        "append_us": round(us_append, 2) if us_append is not None else None,
        "algorithmic_bytes": int(ab["total"]),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "python_api": python_api,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
