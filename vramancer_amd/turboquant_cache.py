"""TurboQuant KV cache for Hugging Face models on MI355X: drop-in for
VRAMancer's ``core/turboquant_cache.py`` (``TurboQuantLayer``,
``TurboQuantCache``, ``from_model_config``).

As in the reference, each layer keeps the most recent tokens uncompressed in a
residual buffer and, once the buffer reaches ``residual_length`` tokens, moves
every buffered token into TurboQuant codes (core/turboquant_cache.py:
176-196).  Here both stores are paged device pools of this library:

* the residual is a paged float pool of the model's dtype (16-token pages,
  written by ``vrm_kv_write``);
* compressed tokens are TurboQuant pages (``tq_pages`` layout, written by
  ``vrm_tq_quant_append``); page j of sequence b is pool page j * B + b.

Attention of a decode step sees what the reference's ``update`` returns: the
compressed tokens so far plus the residual including the new token; a spill
triggered by this step takes effect at the next update, so this step still
reads those tokens uncompressed.

Two ways to attend:

* ``paged_attention=False`` (the reference's behaviour): ``update`` returns
  the full keys/values, the compressed part decompressed by the library's
  kernels, for the model's own attention;
* ``paged_attention=True`` with the attention function registered by
  ``enable_paged_attention(model)``: a decode step (one query token)
  runs the paged TurboQuant decode over the compressed pages and the paged
  float decode over the residual, merged by log-sum-exp, and never
  materialises the keys/values.  Other calls (prefill, masked batches) attend
  over materialised keys/values with PyTorch's SDPA.

Divergence from the reference, on purpose: a token's codes are written once.
The reference re-compresses the decompressed older tokens at every spill
(compress(decompress(old) ++ residual)), which quantises them again.

Takes every compressor setting the TurboQuant pages serve (head_dim 1 ..
256, 1 .. 8 bits per angle, qjl_dim 1 .. 256); a worker-GPU offloader
(core/offloaded_compressor.py) is not supported.
"""
from __future__ import annotations

import math
import os
from typing import Any, Optional, Tuple

import numpy as np
import torch
from transformers.cache_utils import Cache, CacheLayerMixin

from . import _lib, tq_pages
from .kv_quantizer import KVCacheCompressor
from .paged_attention_cuda import combine_attention, decode_workspace, paged_attention_decode
from .turboquant_cuda import CUDATurboQuantOps

__all__ = ["TurboQuantLayer", "TurboQuantCache", "enable_paged_attention", "turbo_paged_attention",
           "ATTENTION_NAME"]

ATTENTION_NAME = "vramancer_turbo"
PAGE = 16


def _int32(host, device):
    return torch.from_numpy(np.ascontiguousarray(host, dtype=np.int32)).to(device)


class TurboQuantLayer(CacheLayerMixin):
    """One layer's cache: a paged residual of recent tokens and TurboQuant
    pages for the rest (core/turboquant_cache.py:78-299)."""

    is_sliding = False

    def __init__(self, compressor: KVCacheCompressor, residual_length: int = 128, offloader: Any = None,
                 layer_idx: int = 0, paged_attention: bool = False):
        super().__init__()
        if offloader is not None:
            raise NotImplementedError("compression on a worker GPU is not supported")
        if residual_length <= 0:
            raise ValueError("residual_length must be positive")
        self.compressor = compressor
        self.residual_length = int(residual_length)
        self.cumulative_length = 0
        self.paged_attention = paged_attention
        self._layer_idx = layer_idx
        self._clear()

    def _clear(self) -> None:
        self._res_pool = None   # [B * rp, 1, 2, KH, 16, D] residual pages, sequence b owns b * rp ..
        self._res_ids = None    # [2, rp * 16, B] int32 page / slot of each residual position
        self._len_rows = None   # [rp * 16 + 1, B] int32, row n all n
        self._len_last = None   # (n, [B] int32 all n) for the compressed count
        self._rp = 0
        self._res_len = 0
        self._tq_pool = None    # [rows, 1, 2, KH, slice] TurboQuant pages, page j of sequence b at j * B + b
        self._n_comp = 0
        self._spill_pending = False
        self._view = (0, 0)     # (compressed, residual) tokens the current step attends
        self._tables = {}
        self._ws = {}

    # -- set-up ----------------------------------------------------------

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        comp = self.compressor
        B, KH, _, D = key_states.shape
        tq_pages._check_compressor(comp)
        if D != comp.head_dim:
            raise RuntimeError(f"key head_dim {D} does not match the compressor's {comp.head_dim}")
        if key_states.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise RuntimeError(f"unsupported key dtype {key_states.dtype}")
        _lib.require_cuda(key_states, value_states)
        self.dtype, self.device = key_states.dtype, key_states.device
        self._B, self._KH, self._D = B, KH, D
        self.keys = torch.tensor([], dtype=self.dtype, device=self.device)
        self.values = torch.tensor([], dtype=self.dtype, device=self.device)
        self._buffers = tq_pages._buffers(comp, self.device)
        self.is_initialized = True

    def _ensure_residual(self, tokens: int) -> None:
        rp = -(-tokens // PAGE)
        if rp <= self._rp:
            return
        rp = max(rp, -(-self.residual_length // PAGE))
        B = self._B
        pool = torch.zeros((B * rp, 1, 2, self._KH, PAGE, self._D), dtype=self.dtype, device=self.device)
        if self._res_pool is not None:
            pool.view(B, rp, -1)[:, :self._rp] = self._res_pool.view(B, self._rp, -1)
        self._res_pool, self._rp = pool, rp
        # page b * rp + t // 16 and slot t % 16 of residual position t of
        # sequence b, token-major ([2, rp * 16, B]): the ids of any run of
        # positions are one contiguous slice
        t = np.arange(rp * PAGE)[:, None]
        self._res_ids = _int32(np.stack(np.broadcast_arrays(np.arange(B)[None, :] * rp + t // PAGE, t % PAGE)),
                               self.device)
        self._tables.clear()

    def _ensure_pages(self, pages_per_seq: int) -> None:
        rows = pages_per_seq * self._B
        have = 0 if self._tq_pool is None else self._tq_pool.shape[0]
        if rows <= have:
            return
        rows = max(rows, 2 * have)
        pool = tq_pages.allocate_pool(rows, 1, self._KH, self.compressor, self.device)
        if have:
            pool[:have] = self._tq_pool
        self._tq_pool = pool
        self._tables.clear()

    # -- writes ------------------------------------------------------------

    def _write_residual(self, key_states, value_states, start: int) -> None:
        """Writes [B, KH, S, D] at residual positions start .. start + S - 1,
        token-major (row t * B + b), with the ids sliced from the residual
        table: no host round trip and no index kernels per step."""
        B, KH, S, D = key_states.shape
        ids = self._res_ids[:, start:start + S].reshape(2, S * B)
        pages, slots = ids[0], ids[1]
        k = key_states.permute(2, 0, 1, 3).reshape(S * B, KH, D).contiguous()
        v = value_states.permute(2, 0, 1, 3).reshape(S * B, KH, D).contiguous()
        pool = self._res_pool
        rc = _lib.load().vrm_kv_write(
            _lib.ptr(k), _lib.ptr(v), _lib.src_dtype_code(k.dtype), _lib.ptr(pages), _lib.ptr(slots), B * S,
            _lib.ptr(pool), _lib.kv_dtype_code(pool.dtype), KH, D, PAGE, 1, pool.shape[0], 0, _lib.stream_of(pool))
        _lib.check(rc, "TurboQuantLayer residual write")

    def _residual_rows(self):
        """Residual K, V as [B, KH, res_len, D] views of the pool's pages."""
        B, KH, D = self._B, self._KH, self._D
        pages = self._res_pool.view(B, self._rp, 2, KH, PAGE, D).permute(0, 2, 3, 1, 4, 5)
        pages = pages.reshape(B, 2, KH, self._rp * PAGE, D)[:, :, :, :self._res_len]
        return pages[:, 0], pages[:, 1]

    def _spill(self) -> None:
        """Moves the residual into TurboQuant pages (tokens n_comp .. on)."""
        n, B, KH, D = self._res_len, self._B, self._KH, self._D
        if n == 0:
            return
        self._ensure_pages(-(-(self._n_comp + n) // PAGE))
        k, v = self._residual_rows()
        k = k.permute(0, 2, 1, 3).reshape(B * n, KH, D).contiguous()
        v = v.permute(0, 2, 1, 3).reshape(B * n, KH, D).contiguous()
        # TurboQuant page (t // 16) * B + b, slot t % 16, sequence-major like k
        # and v; computed on the device (once per residual_length steps)
        t = torch.arange(self._n_comp, self._n_comp + n, dtype=torch.int32, device=self.device)
        pages = ((t // PAGE)[None, :] * B + torch.arange(B, dtype=torch.int32, device=self.device)[:, None])
        pages = pages.reshape(-1).contiguous()
        slots = (t % PAGE)[None, :].expand(B, n).reshape(-1).contiguous()
        signs, jl, lut = self._buffers
        pool = self._tq_pool
        rc = _lib.load().vrm_tq_quant_append(
            _lib.ptr(k), _lib.ptr(v), _lib.src_dtype_code(k.dtype), _lib.ptr(pages), _lib.ptr(slots), B * n,
            _lib.ptr(pool), KH, D, PAGE, 1, pool.shape[0], 0, self.compressor.bits_per_angle, self.compressor.qjl_dim, _lib.ptr(signs),
            _lib.ptr(jl), _lib.ptr(lut), _lib.stream_of(pool))
        _lib.check(rc, "TurboQuantLayer spill")
        self._n_comp += n
        self._res_len = 0

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs
               ) -> Tuple[torch.Tensor, torch.Tensor]:
        """Appends [B, KH, S, D] keys/values.  Returns the full keys/values
        (compressed part decompressed), or, with paged attention, the new
        states tagged for the paged attention function."""
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        if key_states.shape[0] != self._B or key_states.shape[1] != self._KH:
            raise RuntimeError(f"batch/heads changed from {(self._B, self._KH)} to {tuple(key_states.shape[:2])}")
        if self._spill_pending:
            self._spill()
            self._spill_pending = False
        S = key_states.shape[-2]
        self.cumulative_length += S
        self._ensure_residual(self._res_len + S)
        self._write_residual(key_states, value_states, self._res_len)
        self._res_len += S
        self._view = (self._n_comp, self._res_len)
        self._spill_pending = self._res_len >= self.residual_length
        if self.paged_attention:
            key_states._vrm_turbo_layer = self
            return key_states, value_states
        return self.materialize()

    # -- reads -------------------------------------------------------------

    def materialize(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """[B, KH, tokens, D] keys/values of the current view in the model's
        dtype: decompressed TurboQuant tokens, then the residual."""
        n_c, n_r = self._view
        B, KH, D = self._B, self._KH, self._D
        parts_k, parts_v = [], []
        if n_c:
            pj = -(-n_c // PAGE)
            ids = torch.arange(pj * B, dtype=torch.int32, device=self.device)
            codes = tq_pages.read_pages(self._tq_pool, 0, ids, self.compressor)
            comp = self.compressor
            for kv, parts in ((0, parts_k), (1, parts_v)):
                def tokens(name):
                    t = codes[name][:, kv].reshape(pj, B, KH, PAGE, *codes[name].shape[4:])
                    t = t.permute(1, 2, 0, 3, *range(4, t.dim())).reshape(B, KH, pj * PAGE, *t.shape[4:])
                    return t[:, :, :n_c].reshape(B * KH * n_c, *t.shape[3:]).contiguous()

                rows = {"radius": tokens("radius"), "angles": [tokens("angles")], "shape": (B * KH * n_c, D)}
                dec = CUDATurboQuantOps.decompress_gpu(rows, D, comp._padded_dim, comp._n_levels,
                                                       comp.bits_per_angle, comp._hadamard_signs)
                parts.append(dec.reshape(B, KH, n_c, D).to(self.dtype))
        if n_r:
            k, v = self._residual_rows()
            parts_k.append(k)
            parts_v.append(v)
        if not parts_k:
            empty = torch.empty((B, KH, 0, D), dtype=self.dtype, device=self.device)
            return empty, empty
        return torch.cat(parts_k, dim=2), torch.cat(parts_v, dim=2)

    def _table(self, kind: str, pages: int):
        key = (kind, pages)
        t = self._tables.get(key)
        if t is None:
            B = self._B
            j, b = np.arange(pages)[None, :], np.arange(B)[:, None]
            host = j * B + b if kind == "tq" else b * self._rp + j
            t = _int32(host, self.device)
            self._tables[key] = t
        return t

    def _lengths(self, n: int):
        """[B] int32 device array of n: a row of a cached table for residual
        lengths (one table per residual pool size), a cached array otherwise."""
        if n < self._rp * PAGE + 1:
            if self._len_rows is None or self._len_rows.shape[0] != self._rp * PAGE + 1:
                rows = np.broadcast_to(np.arange(self._rp * PAGE + 1)[:, None], (self._rp * PAGE + 1, self._B))
                self._len_rows = _int32(rows, self.device)
            return self._len_rows[n]
        if self._len_last is None or self._len_last[0] != n:  # the compressed count: changes once per spill
            self._len_last = (n, torch.full((self._B,), n, dtype=torch.int32, device=self.device))
        return self._len_last[1]

    def _workspace(self, H: int, pages: int):
        key = (H, pages)
        ws = self._ws.get(key)
        if ws is None:
            ws = decode_workspace(self._B, H, self._KH, self._D, pages, self.device)
            self._ws[key] = ws
        return ws

    def attend_decode(self, query: torch.Tensor, scale: float) -> torch.Tensor:
        """One decode token per sequence, query [B, H, 1, D] -> [B, 1, H, D]:
        paged TurboQuant decode over the compressed tokens (scores against the
        decompressed keys, as the reference's cache hands them to attention:
        no QJL term) and paged float decode over the residual, merged by
        log-sum-exp."""
        B, H, _, D = query.shape
        q = query[:, :, 0, :].float().contiguous()
        n_c, n_r = self._view
        results = []
        if n_c:
            pj = -(-n_c // PAGE)
            ctx = self._lengths(n_c)
            lse = torch.empty((B, H), dtype=torch.float32, device=self.device)
            out = tq_pages.paged_attention_decode_turbo(q, self._tq_pool, self._table("tq", pj), ctx, 0,
                                                        self.compressor, scale=scale,
                                                        workspace=self._workspace(H, pj), lse=lse, qjl=False)
            results.append((out, lse))
        if n_r:
            pr = -(-n_r // PAGE)
            ctx = self._lengths(n_r)
            lse = torch.empty((B, H), dtype=torch.float32, device=self.device)
            out = paged_attention_decode(q, self._res_pool, self._table("res", pr), ctx, 0, scale=scale,
                                         workspace=self._workspace(H, pr), lse=lse)
            results.append((out, lse))
        if not results:
            out = torch.zeros((B, H, D), dtype=torch.float32, device=self.device)
        elif len(results) == 1:
            out = results[0][0]
        else:
            out = combine_attention(results[0][0], results[0][1], results[1][0], results[1][1])
        return out.to(query.dtype).unsqueeze(1)

    # -- bookkeeping (core/turboquant_cache.py:256-299) ----------------------

    def get_seq_length(self) -> int:
        return self.cumulative_length

    def get_max_length(self) -> int:
        return -1

    def get_max_cache_shape(self) -> int:
        return -1

    def get_mask_sizes(self, cache_position) -> Tuple[int, int]:
        query_length = cache_position if isinstance(cache_position, int) else cache_position.shape[0]
        return self.get_seq_length() + query_length, 0

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        """Beam search: sequence b takes the state of sequence beam_idx[b]."""
        if not self.is_initialized:
            return
        idx = beam_idx.to(self.device)
        if self._res_pool is not None:
            view = self._res_pool.view(self._B, self._rp, -1)
            self._res_pool = view.index_select(0, idx).reshape(self._res_pool.shape).contiguous()
        if self._tq_pool is not None:
            rows = self._tq_pool.shape[0]
            view = self._tq_pool.view(rows // self._B, self._B, -1)
            self._tq_pool = view.index_select(1, idx).reshape(self._tq_pool.shape).contiguous()

    def reset(self) -> None:
        self._clear()
        if self.is_initialized:
            self.keys = torch.tensor([], dtype=self.dtype, device=self.device)
            self.values = torch.tensor([], dtype=self.dtype, device=self.device)
        self.cumulative_length = 0


class TurboQuantCache(Cache):
    """Hugging Face cache with TurboQuant-compressed KV
    (core/turboquant_cache.py:306-423): pass as ``past_key_values``."""

    def __init__(self, num_layers: int, head_dim: int, bits_per_angle: int = 3, residual_length: int = 128,
                 device: str = "cuda:0", worker_device: Optional[str] = None, paged_attention: bool = False):
        if worker_device is not None:
            raise NotImplementedError("compression on a worker GPU is not supported")
        # one compressor, hence one rotation, for every layer (the reference's draw order)
        compressor = KVCacheCompressor(head_dim=head_dim, bits_per_angle=bits_per_angle)
        if str(device).startswith("cuda"):
            compressor = compressor.to(device)
        layers = [TurboQuantLayer(compressor, residual_length, None, i, paged_attention) for i in range(num_layers)]
        super().__init__(layers=layers)
        self._head_dim = head_dim
        self._bits_per_angle = bits_per_angle
        self._compressor = compressor

    @classmethod
    def from_model_config(cls, config, bits_per_angle: Optional[int] = None, residual_length: int = 256,
                          device: str = "cuda:0", worker_device: Optional[str] = None,
                          paged_attention: bool = False) -> "TurboQuantCache":
        """Dimensions from a Hugging Face config; bits from VRM_KV_COMPRESSION_BITS
        (core/turboquant_cache.py:376-413)."""
        if hasattr(config, "get_text_config"):
            config = config.get_text_config(decoder=True)
        num_layers = getattr(config, "num_hidden_layers", 12)
        num_heads = getattr(config, "num_attention_heads", 12)
        hidden_size = getattr(config, "hidden_size", 768)
        head_dim = getattr(config, "head_dim", None) or (hidden_size // num_heads)
        if bits_per_angle is None:
            bits_per_angle = int(os.environ.get("VRM_KV_COMPRESSION_BITS", "3"))
        if worker_device is None:
            worker_device = os.environ.get("VRM_TURBOQUANT_WORKER")
        return cls(num_layers=num_layers, head_dim=head_dim, bits_per_angle=bits_per_angle,
                   residual_length=residual_length, device=device, worker_device=worker_device,
                   paged_attention=paged_attention)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        if layer_idx >= len(self.layers):
            return 0
        return self.layers[layer_idx].get_seq_length()

    def get_max_cache_shape(self, layer_idx: int = 0) -> int:
        return -1

    def reorder_cache(self, beam_idx: torch.LongTensor):
        for layer in self.layers:
            layer.reorder_cache(beam_idx)


def _mask_is_open(mask) -> bool:
    if mask is None:
        return True
    if mask.dtype == torch.bool:
        return bool(mask.all())
    return bool((mask == 0).all())


def turbo_paged_attention(module, query, key, value, attention_mask, dropout: float = 0.0,
                          scaling: Optional[float] = None, **kwargs):
    """Attention function for ``attn_implementation="vramancer_turbo"``.

    A decode step (one query token, no masked position, no dropout) over a
    paged ``TurboQuantLayer`` runs the paged decodes; anything else attends
    with SDPA over the materialised keys/values."""
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    layer = getattr(key, "_vrm_turbo_layer", None)
    if scaling is None:
        scaling = 1.0 / math.sqrt(query.shape[-1])
    plain = kwargs.get("softcap") is None and kwargs.get("sliding_window") is None and not dropout
    if layer is not None and query.shape[2] == 1 and plain and _mask_is_open(attention_mask):
        return layer.attend_decode(query, float(scaling)), None
    if layer is not None:
        key, value = layer.materialize()
    return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                  **kwargs)


def enable_paged_attention(model) -> None:
    """Registers ``turbo_paged_attention`` and selects it for ``model``; use
    with ``TurboQuantCache(..., paged_attention=True)``."""
    from transformers import AttentionInterface

    AttentionInterface.register(ATTENTION_NAME, turbo_paged_attention)
    model.set_attn_implementation(ATTENTION_NAME)
