"""vrm_paged_decode_noalloc: the decode entry point that takes no workspace
(its split-K partials live in a fixed array inside the library).

Parity bar: its output equals vrm_paged_decode's with a caller workspace
(same kernels, same work split) bit for bit on the deterministic bf16 path,
and within rounding (1e-5 of the output's largest magnitude) on the int8 /
fp8 path, whose workgroups hand page pairs to wavefronts as they free up; on
consecutive calls whose
second input is smaller than the first, so stale partials of the first call
cannot leak into the second (a leak would be far outside either bar).
Shapes whose partials exceed the array are rejected on the host.
"""
import math

import pytest
import torch

from vramancer_amd import _lib, kv_quant, workloads
from vramancer_amd.paged_attention_cuda import decode_workspace

DEV = "cuda:0"


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _inputs(name, seed, **kw):
    cfg = workloads.scaled(workloads.CONFIGS[name], **kw)
    inp = workloads.make_decode_inputs(cfg, DEV, seed=seed, layers=(cfg.num_layers - 1,))
    return cfg.num_layers - 1, inp


def _both(layer, inp):
    lib = _lib.load()
    q, pool, sc = inp["query"], inp["kv_pool"], inp["kv_scales"]
    table, lens = inp["page_table"], inp["context_lens"]
    B, H, D = q.shape
    P, L, _, KH, PS, _ = pool.shape
    max_pp = table.shape[1]
    code = kv_quant.abi_dtype_code(pool, sc)
    scale = 1.0 / math.sqrt(D)
    s = _lib.stream_of(q)
    ws = decode_workspace(B, H, KH, D, max_pp, q.device, PS)
    ref = torch.empty((B, H, D), dtype=torch.float32, device=DEV)
    rc = lib.vrm_paged_decode(q.data_ptr(), pool.data_ptr(), _lib.ptr(sc), table.data_ptr(), lens.data_ptr(),
                              ref.data_ptr(), ws.data_ptr(), ws.numel(), B, H, KH, D, PS, L, P, max_pp, layer, scale,
                              code, s)
    _lib.check(rc, "vrm_paged_decode")
    got = torch.full((B, H, D), float("nan"), dtype=torch.float32, device=DEV)
    rc = lib.vrm_paged_decode_noalloc(q.data_ptr(), pool.data_ptr(), _lib.ptr(sc), table.data_ptr(),
                                      lens.data_ptr(), got.data_ptr(), B, H, KH, D, PS, L, P, max_pp, layer, scale,
                                      code, s)
    _lib.check(rc, "vrm_paged_decode_noalloc")
    torch.cuda.synchronize()
    return got, ref


@pytest.mark.gpu
@pytest.mark.parametrize("name,big,small", [
    ("14b-int8", dict(batch=16, ctx_div=2, num_layers=2), dict(batch=3, ctx_div=16, num_layers=2)),
    ("mixed-fp8", dict(batch=24, ctx_div=8), dict(batch=2, ctx_div=64)),
    ("7b-bf16", dict(batch=8, ctx_div=2), dict(batch=1, ctx_div=32)),
], ids=["int8", "fp8", "bf16"])
def test_noalloc_equals_workspace_decode_on_consecutive_calls(name, big, small):
    for tag, kw, seed in (("larger", big, 5), ("smaller", small, 6)):
        layer, inp = _inputs(name, seed, **kw)
        _say(f"noalloc {name} {tag} B={inp['query'].shape[0]}")
        got, ref = _both(layer, inp)
        if name == "7b-bf16":  # deterministic path: bit-identical
            assert torch.equal(got, ref), f"{name} {tag}: max abs diff {(got - ref).abs().max().item():.3e}"
        else:  # int8 / fp8 at page 16: page pairs go to wavefronts as they free up, so the last bits vary
            err = (got - ref).abs()
            assert (err <= 1e-5 * ref.abs().max() + 1e-6).all(), f"{name} {tag}: max abs diff {err.max().item():.3e}"


def test_noalloc_rejects_shapes_beyond_its_array_on_the_host():
    """Checked before any HIP call, so this runs without a GPU."""
    lib = _lib.load()
    limit = (64 << 20)
    B, H, KH, D = 512, 64, 1, 256
    need = lib.vrm_paged_decode_workspace_bytes(B, H, D, lib.vrm_paged_decode_num_splits(B, H, KH, 64, 16))
    assert need > limit
    rc = lib.vrm_paged_decode_noalloc(1, 1, None, 1, 1, 1, B, H, KH, D, 16, 1, 8, 64, 0, 0.1, _lib.VRM_KV_BF16,
                                      None)
    assert rc == -3 and b"scratch" in lib.vrm_last_error()
    rc = lib.vrm_paged_decode_noalloc(None, 1, None, 1, 1, 1, 2, 8, 2, 128, 16, 1, 8, 4, 0, 0.1, _lib.VRM_KV_BF16,
                                      None)
    assert rc == -1 and b"null" in lib.vrm_last_error()
