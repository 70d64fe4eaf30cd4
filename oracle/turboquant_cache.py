"""Restatement of the reference's Hugging Face TurboQuant cache (test oracle only).

``OracleTurboQuantLayer`` follows ``TurboQuantLayer`` of
core/turboquant_cache.py:78-299 on the local path (no offloader) step for
step, with the CPU codec of oracle/turboquant.py:

* update (:142-174): append the new states to the residual;
* _update_local (:176-196): keys_out = decompress(compressed) ++ residual
  (or the residual alone); when the residual holds residual_length tokens or
  more, compressed = compress(keys_out) (every token, the older ones
  re-quantised from their decompressed values) and the residual is emptied;
  keys_out is returned;
* _compress_tensor / _decompress_tensor (:120-138): rows of
  [B, H, S, D].float() compressed unpacked; decompressed rows reshaped and
  cast back to the states' dtype.

Only tests import this module.
"""
from __future__ import annotations

from typing import Any, Optional, Tuple

import torch
from transformers.cache_utils import Cache, CacheLayerMixin

from . import turboquant as TQ


class OracleTurboQuantLayer(CacheLayerMixin):
    is_sliding = False

    def __init__(self, params: TQ.TQParams, residual_length: int = 128):
        super().__init__()
        self.p = params
        self.residual_length = residual_length
        self.cumulative_length = 0
        self.compressed_keys: Optional[Tuple[dict, int, torch.dtype]] = None
        self.compressed_values: Optional[Tuple[dict, int, torch.dtype]] = None
        self.spills = 0

    def lazy_initialization(self, key_states, value_states) -> None:
        self.dtype, self.device = key_states.dtype, key_states.device
        self.keys = torch.tensor([], dtype=self.dtype, device=self.device)
        self.values = torch.tensor([], dtype=self.dtype, device=self.device)
        self.is_initialized = True

    def _compress(self, t):
        B, H, S, D = t.shape
        return TQ.compress(self.p, t.reshape(-1, D).float(), pack=False), S, t.dtype

    def _decompress(self, c, B, H):
        data, S, dtype = c
        return TQ.decompress(self.p, data).reshape(B, H, S, -1).to(dtype)

    def update(self, key_states, value_states, *args, **kwargs):
        self.cumulative_length += key_states.shape[-2]
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        B, H = key_states.shape[0], key_states.shape[1]
        if self.keys.numel() == 0:
            self.keys, self.values = key_states, value_states
        else:
            self.keys = torch.cat([self.keys, key_states], dim=-2)
            self.values = torch.cat([self.values, value_states], dim=-2)
        if self.compressed_keys is not None:
            keys_out = torch.cat([self._decompress(self.compressed_keys, B, H), self.keys], dim=-2)
            values_out = torch.cat([self._decompress(self.compressed_values, B, H), self.values], dim=-2)
        else:
            keys_out, values_out = self.keys, self.values
        if self.keys.shape[-2] >= self.residual_length:
            self.compressed_keys = self._compress(keys_out)
            self.compressed_values = self._compress(values_out)
            self.keys = torch.tensor([], dtype=self.dtype, device=self.device)
            self.values = torch.tensor([], dtype=self.dtype, device=self.device)
            self.spills += 1
        return keys_out, values_out

    def get_seq_length(self) -> int:
        return self.cumulative_length

    def get_max_length(self) -> int:
        return -1

    def get_mask_sizes(self, cache_position) -> Tuple[int, int]:
        q = cache_position if isinstance(cache_position, int) else cache_position.shape[0]
        return self.get_seq_length() + q, 0


class OracleTurboQuantCache(Cache):
    """TurboQuantCache restated (core/turboquant_cache.py:306-423), one
    compressor for every layer."""

    def __init__(self, num_layers: int, params: TQ.TQParams, residual_length: int = 128):
        super().__init__(layers=[OracleTurboQuantLayer(params, residual_length) for _ in range(num_layers)])

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.layers[layer_idx].get_seq_length() if layer_idx < len(self.layers) else 0
