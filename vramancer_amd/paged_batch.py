"""Batched decode of Hugging Face models over the paged KV cache: the decode
step of VRAMancer's continuous batcher (core/continuous_batcher.py:693-816)
with the paged kernel in place of pad-and-concat.

The reference coalesces the decode requests into one forward by
concatenating their per-request Hugging Face caches, padding the shorter ones
to the longest with zeros (left padding) and masking the padding (:711-756,
:818-891), so every step copies every request's whole cache; the model then
places every request's new token at the padded length.  Here the requests' K/V stay
in the pages of a ``PagedKVCacheManager``, and ``PagedBatchCache`` is the
Hugging Face ``Cache`` of an ordered batch of request ids:

* the update of layer 0 starts a step: the manager appends one token to every
  request (``append_tokens``: a page id and slot each, a page allocated where
  the last one is full);
* each layer's update writes its new K/V rows into those slots with one
  ``vrm_kv_write`` launch (``write_kv_batch``) and tags the key it returns
  with the batch and the layer;
* the attention function registered as ``"vramancer_paged"``
  (``enable_paged_attention``) sees the tag and runs the paged decode of that
  layer over the batch's block table, which the manager builds on the device
  once per step.  Each request attends exactly its own tokens: no padding, no
  mask, no copy of the cache.

``decode_step`` runs one step of a batch, each request at its own position
(its token count, as a request decoded alone by ``_forward_single`` is), and
returns the last-position logits; ``prefill`` runs a
request's prompt through the model with an ordinary cache and stores the
result in its pages (``from_hf_cache``), as the reference batcher does after
its prefill (:594-597).

Only decode steps (one new token per request) go through the pages; a
multi-token update of a ``PagedBatchCache`` raises.  Calls of the attention
function on any other cache attend with PyTorch's SDPA, causal and unmasked
(prefill one request at a time, as the reference does).
"""
from __future__ import annotations

import math
from typing import Any, Optional, Sequence, Tuple

import numpy as np
import torch
from transformers.cache_utils import Cache, CacheLayerMixin

from .paged_attention import PagedKVCacheManager

__all__ = ["PagedBatchCache", "PagedBatchLayer", "decode_step", "prefill", "paged_attention_forward",
           "enable_paged_attention", "ATTENTION_NAME"]

ATTENTION_NAME = "vramancer_paged"


class PagedBatchLayer(CacheLayerMixin):
    """One layer of a ``PagedBatchCache``: writes the step's K/V rows into
    the manager's pages and returns the new states, tagged."""

    is_sliding = False

    def __init__(self, cache: "PagedBatchCache", layer_idx: int):
        super().__init__()
        self.cache = cache
        self.layer_idx = layer_idx

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        self.dtype, self.device = key_states.dtype, key_states.device
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs
               ) -> Tuple[torch.Tensor, torch.Tensor]:
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        B, _, q, _ = key_states.shape
        if q != 1:
            raise RuntimeError(f"PagedBatchCache takes decode steps of one token per request (got {q}); "
                               "prefill with an ordinary cache and PagedKVCacheManager.from_hf_cache")
        if B != len(self.cache.request_ids):
            raise RuntimeError(f"batch of {B} rows for {len(self.cache.request_ids)} request ids")
        if self.layer_idx == 0:
            self.cache._begin_step()
        page_ids, slots = self.cache._step_slots()
        self.cache.manager.write_kv_batch(self.layer_idx, page_ids, slots, key_states[:, :, 0],
                                          value_states[:, :, 0])
        key_states._vrm_paged_batch = (self.cache, self.layer_idx)
        return key_states, value_states

    def get_seq_length(self) -> int:
        return self.cache.get_seq_length()

    def get_max_length(self) -> int:
        return -1

    def get_max_cache_shape(self) -> int:
        return -1

    def get_mask_sizes(self, query_length) -> Tuple[int, int]:
        q = query_length if isinstance(query_length, int) else query_length.shape[0]
        return self.get_seq_length() + q, 0


class PagedBatchCache(Cache):
    """Hugging Face cache of a batch of requests held by a
    ``PagedKVCacheManager``; batch row i is ``request_ids[i]``.  The cache
    keeps no tensors of its own and can be kept across steps while the batch
    stays the same."""

    def __init__(self, manager: PagedKVCacheManager, request_ids: Sequence[str]):
        if manager.gpu_pool is None:
            raise RuntimeError("PagedBatchCache needs a manager with a GPU pool")
        known = manager.request_ids()
        missing = [rid for rid in request_ids if rid not in known]
        if missing:
            raise KeyError(f"unknown request ids {missing}")
        self.manager = manager
        self.request_ids = list(request_ids)
        self._slots: Optional[Tuple[torch.Tensor, torch.Tensor]] = None
        super().__init__(layers=[PagedBatchLayer(self, i) for i in range(manager.config.num_layers)])

    def token_counts(self) -> np.ndarray:
        """Each request's token count (the position of its next token)."""
        return self.manager.token_counts(self.request_ids)

    def _begin_step(self) -> None:
        self._slots = self.manager.append_tokens(self.request_ids, strict=True)

    def _step_slots(self) -> Tuple[torch.Tensor, torch.Tensor]:
        if self._slots is None:
            raise RuntimeError("a decode step starts with the update of layer 0")
        return self._slots

    def get_seq_length(self, layer_idx: int = 0) -> int:
        counts = self.token_counts()
        return int(counts.max()) if counts.size else 0

    def get_max_cache_shape(self, layer_idx: int = 0) -> int:
        return -1

    def attend(self, query: torch.Tensor, layer_idx: int, scale: float) -> torch.Tensor:
        """Paged decode of one layer: query [B, H, 1, D] -> [B, 1, H, D] in
        the query's dtype, the layout attention functions return."""
        out = self.manager.compute_attention_decode(query[:, :, 0].contiguous(), self.request_ids, layer_idx, scale)
        if out is None:
            raise RuntimeError("paged decode over a batch with no pages")
        return out.to(query.dtype).unsqueeze(1)


def paged_attention_forward(module, query, key, value, attention_mask, dropout: float = 0.0,
                            scaling: Optional[float] = None, **kwargs):
    """Attention function for ``attn_implementation="vramancer_paged"``.

    Keys returned by a ``PagedBatchCache`` are attended by the paged decode
    over the batch's pages; any other call attends with SDPA."""
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    tag = getattr(key, "_vrm_paged_batch", None)
    if scaling is None:
        scaling = 1.0 / math.sqrt(query.shape[-1])
    if tag is None:
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                      **kwargs)
    if dropout or kwargs.get("softcap") is not None or kwargs.get("sliding_window") is not None:
        raise NotImplementedError("paged decode supports neither dropout, softcap nor sliding windows")
    cache, layer_idx = tag
    return cache.attend(query, layer_idx, float(scaling)), None


def enable_paged_attention(model) -> None:
    """Registers ``paged_attention_forward`` and selects it for ``model``."""
    from transformers import AttentionInterface

    AttentionInterface.register(ATTENTION_NAME, paged_attention_forward)
    model.set_attn_implementation(ATTENTION_NAME)


def decode_step(model, manager: PagedKVCacheManager, request_ids: Sequence[str], input_ids: torch.Tensor,
                cache: Optional[PagedBatchCache] = None) -> torch.Tensor:
    """One batched decode step (core/continuous_batcher.py:693-770): token
    ``input_ids[i]`` of request ``request_ids[i]`` at position = that
    request's token count; one forward over the batch.  Returns the logits
    [B, vocab].  The model must use ``enable_paged_attention``; pass the
    ``cache`` of the previous step to reuse it."""
    if cache is None or cache.request_ids != list(request_ids):
        cache = PagedBatchCache(manager, request_ids)
    ids = input_ids.reshape(len(request_ids), 1)
    pos = torch.from_numpy(cache.token_counts()).to(ids.device).reshape(-1, 1)
    out = model(ids, position_ids=pos, past_key_values=cache, use_cache=True)
    logits = out.logits if hasattr(out, "logits") else out[0]
    return logits[:, -1]


def prefill(model, manager: PagedKVCacheManager, request_id: str, input_ids: torch.Tensor) -> torch.Tensor:
    """Runs a request's prompt [1, S] through the model with an ordinary
    cache and stores its K/V in the request's pages (``from_hf_cache``).
    Returns the last-position logits [1, vocab]."""
    out = model(input_ids.reshape(1, -1), use_cache=True)
    manager.from_hf_cache(request_id, out.past_key_values)
    return out.logits[:, -1]
