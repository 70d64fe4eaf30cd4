"""The Hugging Face TurboQuant cache on the GPU, end to end on a tiny random
Llama (head_dim 128, GQA 2:1, two layers), teacher-forced: prompt, then one
token per step.

The oracle is the reference's cache restated on the CPU
(oracle/turboquant_cache.py) driving the same model on the CPU with eager
attention.  The scenario spills exactly once (prompt of 40 tokens, residual
of 64, 30 decode steps), so the reference's re-quantisation of older tokens
at later spills does not arise and both caches hold the same codes.

Logits of every step agree within |gpu - oracle| <= 2e-2 + 2e-2 |oracle|:
the attention outputs themselves meet 2e-3 + 1e-2 |ref| (the paged decode
bar), propagated through two layers and the output projection.
"""
import copy

import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM

from oracle import turboquant as TQ
from oracle.turboquant_cache import OracleTurboQuantCache
from vramancer_amd.turboquant_cache import TurboQuantCache, enable_paged_attention

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _model():
    cfg = LlamaConfig(vocab_size=256, hidden_size=512, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=128, max_position_embeddings=512)
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).eval()


@torch.no_grad()
def _run(model, cache, ids, steps):
    out = [model(ids[:, :-steps], past_key_values=cache, use_cache=True).logits[:, -1].float().cpu()]
    for i in range(steps, 0, -1):
        pos = ids.shape[1] - i
        out.append(model(ids[:, pos:pos + 1], past_key_values=cache, use_cache=True).logits[:, -1].float().cpu())
    return torch.stack(out, 1)


def _close(got, want, what):
    err = (got - want).abs()
    bad = err > 2e-2 + 2e-2 * want.abs()
    assert not bad.any(), f"{what}: {int(bad.sum())} logits off, max err {err.max():.3e}"


@pytest.fixture(scope="module")
def setting():
    model = _model()
    ids = torch.randint(0, 256, (2, 70), generator=torch.Generator().manual_seed(3))
    oracle = OracleTurboQuantCache(2, TQ.make_params(128, 3, seed=11), residual_length=64)
    ref = _run(model, oracle, ids, 30)
    assert oracle.layers[0].spills == 1
    return model, ids, ref


@pytest.mark.parametrize("paged", [True, False], ids=["paged-decode", "materialised"])
def test_turboquant_cache_matches_reference_cache(setting, paged):
    model, ids, ref = setting
    _say(f"hf cache paged={paged}")
    gpu_model = copy.deepcopy(model).to(DEV)
    if paged:
        enable_paged_attention(gpu_model)
    else:
        gpu_model.set_attn_implementation("sdpa")
    torch.manual_seed(11)  # the compressor draws its rotation as the reference's does
    cache = TurboQuantCache(2, 128, bits_per_angle=3, residual_length=64, device=DEV, paged_attention=paged)
    got = _run(gpu_model, cache, ids.to(DEV), 30)
    assert cache.get_seq_length() == 70
    layer = cache.layers[1]
    assert (layer._n_comp, layer._res_len) == (64, 6)
    _close(got, ref, f"paged={paged}")


def test_turboquant_cache_decode_attention_matches_materialised(setting):
    """The paged decode step (TurboQuant pages + residual merged by
    log-sum-exp) against SDPA over the same cache's materialised keys/values."""
    model, ids, _ = setting
    _say("paged step vs materialised")
    torch.manual_seed(11)
    cache = TurboQuantCache(2, 128, bits_per_angle=3, residual_length=32, device=DEV, paged_attention=True)
    layer = cache.layers[0]
    g = torch.Generator().manual_seed(4)
    # prompt, then steps that spill and refill the residual; the 60-token update grows the
    # residual pool while it holds a token (copy, new page / slot table), the next one spills it
    for s in (40, 1, 1, 30, 1, 60, 1):
        k = torch.randn(2, 2, s, 128, generator=g).to(DEV)
        layer.update(k, torch.randn(2, 2, s, 128, generator=g).to(DEV))
        q = torch.randn(2, 4, 1, 128, generator=g).to(DEV)
        got = layer.attend_decode(q, 0.08)[:, 0].float().cpu()
        K, V = layer.materialize()
        Kr = K.float().cpu().repeat_interleave(2, dim=1)
        Vr = V.float().cpu().repeat_interleave(2, dim=1)
        w = torch.softmax(0.08 * (Kr @ q.float().cpu()[:, :, 0, :, None])[..., 0], -1)
        want = (w[..., None] * Vr).sum(2)
        err = (got - want).abs()
        assert (err <= 2e-3 + 1e-2 * want.abs()).all(), f"step {s}: max err {err.max():.3e} view {layer._view}"
