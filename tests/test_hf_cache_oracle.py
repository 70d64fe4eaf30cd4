"""Pins of the restated Hugging Face TurboQuant cache (oracle/turboquant_cache.py)
on a tiny random Llama, on the CPU.

* Without a spill the cache holds every token uncompressed, so the logits
  equal, bit for bit, those of transformers' own DynamicCache.
* With 8 bits per angle the codec is close to lossless; after a spill the
  logits stay within 2e-2 of DynamicCache's, which a token/head mix-up in the
  compress/decompress reshapes would break by orders of magnitude.
"""
import pytest
import torch
from transformers import DynamicCache, LlamaConfig, LlamaForCausalLM

from oracle import turboquant as TQ
from oracle.turboquant_cache import OracleTurboQuantCache


def _model():
    cfg = LlamaConfig(vocab_size=128, hidden_size=256, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=2, num_key_value_heads=1, head_dim=128, max_position_embeddings=256)
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).eval()


def _run(model, cache, ids, steps):
    out = [model(ids[:, :-steps], past_key_values=cache, use_cache=True).logits[:, -1]]
    for i in range(steps, 0, -1):
        pos = ids.shape[1] - i
        out.append(model(ids[:, pos:pos + 1], past_key_values=cache, use_cache=True).logits[:, -1])
    return torch.stack(out, 1)


@torch.no_grad()
def test_oracle_cache_without_spill_is_dynamic_cache():
    model = _model()
    ids = torch.randint(0, 128, (2, 30), generator=torch.Generator().manual_seed(1))
    ref = _run(model, DynamicCache(), ids, 10)
    cache = OracleTurboQuantCache(2, TQ.make_params(128, 3, seed=5), residual_length=1000)
    got = _run(model, cache, ids, 10)
    assert torch.equal(got, ref)
    assert cache.layers[0].spills == 0 and cache.get_seq_length() == 30


@torch.no_grad()
def test_oracle_cache_spill_is_near_lossless_at_8_bits():
    model = _model()
    ids = torch.randint(0, 128, (1, 40), generator=torch.Generator().manual_seed(2))
    ref = _run(model, DynamicCache(), ids, 20)
    cache = OracleTurboQuantCache(2, TQ.make_params(128, 8, seed=6), residual_length=24)
    got = _run(model, cache, ids, 20)
    assert cache.layers[0].spills == 1
    assert (got - ref).abs().max() < 2e-2
    assert not torch.equal(got, ref)
