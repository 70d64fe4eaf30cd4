"""Paged KV-cache manager on MI355X: the decode-path part of VRAMancer's
``PagedKVCacheManager`` (core/paged_attention.py:88-1508).

Host side, as in the reference: a free list of physical pages (allocation
pops from its end), one page list and token count per request, reference
counts for forks, and the slot mapping of ``append_token`` (token n of a
request lives in slot n % page_size of its page n // page_size).

Device side, in this library's kernels:

* ``write_kv`` writes a token's K/V rows into the pool with ``vrm_kv_write``
  (float16 / bfloat16 / float32 pools, the reference's raw index-put) or
  quantizes them on append with ``vrm_kv_quant_append`` (int8 / fp8 pools);
  ``write_kv_batch`` does the same for N tokens in one launch;
* ``flush_compression`` compresses every pending row of every layer into the
  TurboQuant pages with one ``vrm_tq_quant_append`` launch (the reference
  builds per-slot dicts, core/paged_attention.py:623-675);
* ``compute_attention_decode`` builds the block table on the device
  (``vrm_build_block_table``) and runs the paged decode;
* ``compute_attention_turbo`` attends the TurboQuant pages in place
  (``vrm_paged_decode_tq``) with the reference's head mapping ``h % n_kv``
  (:1374); pages with no codes for the layer are first compressed from the
  raw pool, as the reference's lazy ``compress_page_bulk`` call does; with
  ``sparse_v_ratio < 1`` each head keeps its top-k softmax weights
  (``vrm_turboquant_score`` + ``vrm_topk_attend``, :1384-1400);
* ``compress_page_bulk`` compresses a page's raw K/V for every layer that has
  no codes yet (``vrm_tq_compress_pool``);
* ``from_hf_cache`` stores a prefilled Hugging Face cache in a request's
  pages with one ``vrm_kv_write`` launch per layer, ``to_hf_cache`` gathers
  it back; ``try_prefix_cache`` shares full pages of a token prefix between
  requests (host bookkeeping, :521-566).

Not built (outside the decode path): multi-GPU pools, the VRAM lending pool,
LRU eviction to other memory tiers (``append_token`` returns ``None`` once
the pool is exhausted, where the reference would try to evict) and parity
engrams.

A manager whose ``device`` is not a GPU keeps the host bookkeeping only: it
allocates no pools, its decode calls return ``None`` (as the reference's do
without a pool) and writes raise ``RuntimeError``.
"""
from __future__ import annotations

import itertools
import math
import os
import threading
import time
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import _lib

__all__ = ["PagedKVConfig", "PhysicalPage", "PageTableEntry", "PagedKVCacheManager", "hf_layers"]

# Pool element types: name -> (torch dtype name, bytes per element).
_POOL_DTYPES = {
    "float16": ("float16", 2), "fp16": ("float16", 2), "half": ("float16", 2),
    "bfloat16": ("bfloat16", 2), "bf16": ("bfloat16", 2),
    "float32": ("float32", 4), "fp32": ("float32", 4), "float": ("float32", 4),
    "int8": ("int8", 1),
    "fp8": ("float8_e4m3fn", 1), "float8_e4m3fn": ("float8_e4m3fn", 1),
}


def _pool_dtype(name: str) -> Tuple[str, int]:
    try:
        return _POOL_DTYPES[name.lower()]
    except KeyError:
        raise ValueError(f"unknown KV dtype {name!r}; expected one of {sorted(_POOL_DTYPES)}") from None


@dataclass
class PagedKVConfig:
    """Configuration of the paged KV cache (core/paged_attention.py:88-146).

    ``dtype`` names the pool's element type: float16 (default), bfloat16,
    float32, or the quantized int8 / fp8 codecs of ``vramancer_amd.kv_quant``.
    """

    page_size: int = 16
    num_layers: int = 12
    num_kv_heads: int = 12
    head_dim: int = 64
    max_pages: int = 4096
    device: str = "cuda:0"
    dtype: str = "float16"
    kv_compression: Optional[str] = None   # None or "turboquant"
    compression_bits: int = 3
    qjl_dim: Optional[int] = None
    sparse_v_ratio: float = 1.0

    @property
    def page_size_bytes(self) -> int:
        """Bytes of one page over all layers: codes of K and V, plus the
        scales of the int8 (per token and head) and fp8 (per head) pools."""
        kind, esize = _pool_dtype(self.dtype)
        per_head = self.page_size * self.head_dim * esize
        if kind == "int8":
            per_head += self.page_size * 4
        elif kind == "float8_e4m3fn":
            per_head += 4
        return 2 * self.num_layers * self.num_kv_heads * per_head

    @property
    def total_memory_bytes(self) -> int:
        return self.page_size_bytes * self.max_pages

    @classmethod
    def from_model(cls, model: Any, max_pages: int = 4096, device: str = "cuda:0") -> "PagedKVConfig":
        """Config from a Hugging Face model's ``config``; compression settings
        from VRM_KV_COMPRESSION, VRM_KV_COMPRESSION_BITS and VRM_SPARSE_V_RATIO
        (core/paged_attention.py:117-146)."""
        kv_comp = os.environ.get("VRM_KV_COMPRESSION", "").lower() or None
        comp_bits = int(os.environ.get("VRM_KV_COMPRESSION_BITS", "3"))
        sparse_v = float(os.environ.get("VRM_SPARSE_V_RATIO", "1.0"))
        config = getattr(model, "config", None)
        if config is None:
            return cls(max_pages=max_pages, device=device, kv_compression=kv_comp, compression_bits=comp_bits,
                       sparse_v_ratio=sparse_v)
        num_layers = getattr(config, "num_hidden_layers", 12)
        num_heads = getattr(config, "num_attention_heads", 12)
        num_kv_heads = getattr(config, "num_key_value_heads", num_heads)
        hidden_size = getattr(config, "hidden_size", 768)
        return cls(num_layers=num_layers, num_kv_heads=num_kv_heads, head_dim=hidden_size // num_heads,
                   max_pages=max_pages, device=device, kv_compression=kv_comp, compression_bits=comp_bits,
                   sparse_v_ratio=sparse_v)


@dataclass
class PhysicalPage:
    """One page of the pool (core/paged_attention.py:152-171)."""

    page_id: int
    ref_count: int = 0
    allocated: bool = False
    last_access: float = field(default_factory=time.time)


@dataclass
class PageTableEntry:
    """A request's physical pages and token count (core/paged_attention.py:178-185)."""

    request_id: str
    pages: List[int] = field(default_factory=list)
    num_tokens: int = 0
    created_at: float = field(default_factory=time.time)


def _is_gpu(device: str) -> bool:
    return str(device).startswith("cuda")


def hf_layers(past_key_values: Any) -> List[Tuple[Any, Any]]:
    """(key, value) per layer of a Hugging Face cache: a ``Cache`` whose
    ``layers`` hold ``keys``/``values``, one with ``key_cache`` /
    ``value_cache`` lists (transformers 4.36-4.x), or a tuple of pairs.  For
    a ``Cache``, the layers up to the first one that holds nothing."""
    layers = getattr(past_key_values, "layers", None)
    if layers is not None:
        filled = itertools.takewhile(lambda l: getattr(l, "keys", None) is not None and l.keys.numel() > 0, layers)
        return [(layer.keys, layer.values) for layer in filled]
    if hasattr(past_key_values, "key_cache"):
        return list(zip(past_key_values.key_cache, past_key_values.value_cache))
    return [(kv[0], kv[1]) for kv in past_key_values]


class PagedKVCacheManager:
    """Block-based KV cache with on-demand page allocation and GPU decode."""

    def __init__(self, config: Optional[PagedKVConfig] = None):
        self.config = cfg = config or PagedKVConfig()
        self._lock = threading.Lock()
        self._pages: List[PhysicalPage] = [PhysicalPage(page_id=i) for i in range(cfg.max_pages)]
        self._free_pages: List[int] = list(range(cfg.max_pages))
        self._page_tables: Dict[str, PageTableEntry] = {}
        self._total_allocations = 0
        self._total_frees = 0
        self._peak_usage = 0
        # Bumped by every change of a page list or token count; keys the
        # device block-table cache of compute_attention_decode.
        self._epoch = 0
        self._table_cache: Optional[dict] = None
        self._workspaces: Dict[tuple, Any] = {}
        # hash(tuple of a full page's token ids) -> page id (:216, :540-558).
        self._prefix_cache: Dict[int, int] = {}
        self._cache_hits = 0

        self._gpu_pool: Any = None
        self._kv_scales: Any = None
        self._tq_pool: Any = None
        self._tq_buffers: Optional[tuple] = None
        # Bit min(s, 63) of _tq_slots[page, layer] is set once slot s of that
        # page and layer holds TurboQuant codes (the reference's
        # _compressed_pages entries, core/paged_attention.py:236-238); only
        # "no bit set" is ever tested.
        self._tq_slots: Optional[np.ndarray] = None
        self._pending_compress: List[tuple] = []
        self._kv_compressor: Any = None
        self._init_kv_compression()
        if _is_gpu(cfg.device):
            self._init_pools()

    # ------------------------------------------------------------------
    # Set-up
    # ------------------------------------------------------------------

    def _init_kv_compression(self) -> None:
        """TurboQuant compressor built as core/paged_attention.py:366-401 does
        (same constructor call, so the same draws of torch's global RNG)."""
        comp = self.config.kv_compression
        if comp is None:
            return
        if comp != "turboquant":
            raise ValueError(f"unknown kv_compression {comp!r}; expected None or 'turboquant'")
        from .kv_quantizer import KVCacheCompressor

        self._kv_compressor = KVCacheCompressor(head_dim=self.config.head_dim,
                                                bits_per_angle=self.config.compression_bits,
                                                qjl_dim=self.config.qjl_dim)

    def _init_pools(self) -> None:
        import torch

        cfg = self.config
        kind, _ = _pool_dtype(cfg.dtype)
        dev = torch.device(cfg.device)
        if kind in ("int8", "float8_e4m3fn"):
            from . import kv_quant

            self._gpu_pool, self._kv_scales = kv_quant.allocate_pool(
                cfg.max_pages, cfg.num_layers, cfg.num_kv_heads, cfg.head_dim,
                "int8" if kind == "int8" else "fp8", cfg.page_size, dev)
        else:
            self._gpu_pool = torch.zeros((cfg.max_pages, cfg.num_layers, 2, cfg.num_kv_heads, cfg.page_size,
                                          cfg.head_dim), dtype=getattr(torch, kind), device=dev)
        if self._kv_compressor is not None:
            from . import tq_pages

            if kind not in ("float16", "bfloat16", "float32"):
                raise RuntimeError("TurboQuant compression needs a float16, bfloat16 or float32 raw pool "
                                   f"(got {cfg.dtype})")
            self._kv_compressor = self._kv_compressor.to(dev)
            self._tq_pool = tq_pages.allocate_pool(cfg.max_pages, cfg.num_layers, cfg.num_kv_heads,
                                                   self._kv_compressor, dev, cfg.page_size)
            self._tq_buffers = tq_pages._buffers(self._kv_compressor, dev)
            self._tq_slots = np.zeros((cfg.max_pages, cfg.num_layers), dtype=np.uint64)

    def _require_pool(self, what: str) -> None:
        if self._gpu_pool is None:
            raise RuntimeError(f"{what} needs a GPU pool (manager device is {self.config.device!r})")

    # ------------------------------------------------------------------
    # Allocation (core/paged_attention.py:403-519, 916-931)
    # ------------------------------------------------------------------

    def _alloc_page(self) -> Optional[int]:
        if not self._free_pages:
            return None
        page_id = self._free_pages.pop()
        page = self._pages[page_id]
        page.allocated = True
        page.ref_count = 1
        page.last_access = time.time()
        self._total_allocations += 1
        return page_id

    def allocate(self, request_id: str, num_tokens: int = 0) -> PageTableEntry:
        """Page list for a new request, with pages for ``num_tokens`` tokens."""
        with self._lock:
            if request_id in self._page_tables:
                return self._page_tables[request_id]
            entry = PageTableEntry(request_id=request_id)
            for _ in range(math.ceil(num_tokens / self.config.page_size) if num_tokens > 0 else 0):
                page_id = self._alloc_page()
                if page_id is None:
                    break
                entry.pages.append(page_id)
            entry.num_tokens = num_tokens
            self._page_tables[request_id] = entry
            self._peak_usage = max(self._peak_usage, self.config.max_pages - len(self._free_pages))
            self._epoch += 1
            return entry

    def _append_locked(self, request_id: str) -> Optional[Tuple[int, int]]:
        entry = self._page_tables.get(request_id)
        if entry is None:
            return None
        slot = entry.num_tokens % self.config.page_size
        page_index = entry.num_tokens // self.config.page_size
        if page_index >= len(entry.pages):
            page_id = self._alloc_page()
            if page_id is None:
                return None
            entry.pages.append(page_id)
            self._peak_usage = max(self._peak_usage, self.config.max_pages - len(self._free_pages))
        physical = entry.pages[page_index]
        entry.num_tokens += 1
        self._pages[physical].last_access = time.time()
        self._epoch += 1
        return physical, slot

    def append_token(self, request_id: str) -> Optional[Tuple[int, int]]:
        """(page_id, slot) for a request's next token, allocating a page when
        the last one is full; ``None`` for an unknown request or a full pool."""
        with self._lock:
            return self._append_locked(request_id)

    def append_tokens(self, request_ids: Sequence[str], strict: bool = False) -> Tuple[Any, Any]:
        """``append_token`` for a batch, as two int32 device tensors [N]
        (page ids, slots) ready for ``write_kv_batch``; a request that gets no
        slot has page -1 and slot -1, which the writers skip.

        With ``strict`` the batch is checked first and nothing changes when
        it fails: an unknown request id raises ``KeyError``; too few free
        pages for the requests whose last page is full, or (fp8 pools)
        requests sharing the page their token goes to, raise
        ``RuntimeError``.  An fp8 append rescales its page, so one launch may
        write a page once only."""
        import torch

        self._require_pool("append_tokens")
        out = np.full((2, len(request_ids)), -1, dtype=np.int32)
        PS = self.config.page_size
        with self._lock:
            if strict:
                entries = [self._page_tables.get(rid) for rid in request_ids]
                missing = [rid for rid, e in zip(request_ids, entries) if e is None]
                if missing:
                    raise KeyError(f"unknown request ids {missing}")
                opening = [rid for rid, e in zip(request_ids, entries) if e.num_tokens // PS >= len(e.pages)]
                if len(opening) > len(self._free_pages):
                    raise RuntimeError(f"no page left for requests {opening[len(self._free_pages):]} "
                                       f"(pool of {self.config.max_pages} pages)")
                if self._gpu_pool.dtype == torch.float8_e4m3fn:
                    tails = [e.pages[e.num_tokens // PS] for e in entries if e.num_tokens // PS < len(e.pages)]
                    if len(set(tails)) < len(tails):
                        raise RuntimeError("requests of an fp8 pool that share the page their next token goes to "
                                           "(forks) cannot append in one launch")
            for i, rid in enumerate(request_ids):
                got = self._append_locked(rid)
                if got is not None:
                    out[0, i], out[1, i] = got
        dev = torch.from_numpy(out).to(self._gpu_pool.device)
        return dev[0], dev[1]

    @property
    def gpu_pool(self) -> Any:
        """The device K/V pool, or ``None`` for a host-only manager."""
        return self._gpu_pool

    def request_ids(self) -> set:
        """Ids of the requests that hold a page table."""
        with self._lock:
            return set(self._page_tables)

    def token_counts(self, request_ids: Sequence[str]) -> np.ndarray:
        """Token count of each request (0 for an unknown id), int64 on the host."""
        with self._lock:
            return np.array([e.num_tokens if (e := self._page_tables.get(rid)) is not None else 0
                             for rid in request_ids], dtype=np.int64)

    def free(self, request_id: str) -> int:
        """Drops a request; returns how many pages went back to the free list."""
        with self._lock:
            entry = self._page_tables.pop(request_id, None)
            if entry is None:
                return 0
            freed = 0
            for page_id in entry.pages:
                page = self._pages[page_id]
                page.ref_count -= 1
                if page.ref_count <= 0:
                    page.allocated = False
                    page.ref_count = 0
                    if self._tq_slots is not None:
                        # its codes belong to the old request: the next owner's
                        # tokens are compressed afresh
                        self._tq_slots[page_id] = 0
                    self._free_pages.append(page_id)
                    freed += 1
                    self._total_frees += 1
            self._epoch += 1
            return freed

    def fork(self, src_request_id: str, dst_request_id: str) -> Optional[PageTableEntry]:
        """New request sharing every page of ``src_request_id`` (ref counts +1)."""
        with self._lock:
            src = self._page_tables.get(src_request_id)
            if src is None:
                return None
            entry = PageTableEntry(request_id=dst_request_id, pages=list(src.pages), num_tokens=src.num_tokens)
            for page_id in entry.pages:
                self._pages[page_id].ref_count += 1
            self._page_tables[dst_request_id] = entry
            self._epoch += 1
            return entry

    def try_prefix_cache(self, request_id: str, token_ids: Sequence[int]) -> int:
        """Prefix caching over full pages (core/paged_attention.py:521-566).

        Walks ``token_ids`` a full page at a time (a trailing partial page is
        not looked at): a page whose token tuple hashes to an entry of the
        prefix cache that is still allocated is shared (ref count + 1) and
        counts ``page_size`` hits; otherwise a new page is allocated and
        registered under that hash, and the hit count restarts at 0 (only a
        run of hits ending at the last full page counts).  The walk stops when
        the pool is empty.  The request's token count becomes pages *
        page_size.  Returns the hit count."""
        PS = self.config.page_size
        with self._lock:
            entry = self._page_tables.get(request_id)
            if entry is None:
                entry = self._page_tables[request_id] = PageTableEntry(request_id=request_id)
            hits = 0
            for start in range(0, len(token_ids) - PS + 1, PS):
                key = hash(tuple(token_ids[start:start + PS]))
                cached = self._prefix_cache.get(key)
                if cached is not None and self._pages[cached].allocated:
                    entry.pages.append(cached)
                    self._pages[cached].ref_count += 1
                    self._pages[cached].last_access = time.time()
                    hits += PS
                    self._cache_hits += 1
                else:
                    page_id = self._alloc_page()
                    if page_id is None:
                        break
                    entry.pages.append(page_id)
                    self._prefix_cache[key] = page_id
                    hits = 0
            entry.num_tokens = len(entry.pages) * PS
            self._peak_usage = max(self._peak_usage, self.config.max_pages - len(self._free_pages))
            self._epoch += 1
            return hits

    # ------------------------------------------------------------------
    # Writes (core/paged_attention.py:568-675)
    # ------------------------------------------------------------------

    def _write_rows(self, layer_idx: int, page_ids, slots, key, value) -> None:
        cfg = self.config
        pool = self._gpu_pool
        KH, D = cfg.num_kv_heads, cfg.head_dim
        if key.dtype != value.dtype:
            raise RuntimeError("key and value must share a dtype")
        if not 0 <= layer_idx < cfg.num_layers:
            raise RuntimeError(f"layer_idx {layer_idx} outside [0, {cfg.num_layers})")
        code = _lib.kv_dtype_code(pool.dtype)
        N = key.shape[0]
        if code in (_lib.VRM_KV_I8, _lib.VRM_KV_FP8E4M3):
            from . import kv_quant

            kv_quant.quantize_append(pool, self._kv_scales, layer_idx, page_ids, slots, key, value)
            return
        rc = _lib.load().vrm_kv_write(
            _lib.ptr(key), _lib.ptr(value), _lib.src_dtype_code(key.dtype), _lib.ptr(page_ids), _lib.ptr(slots), N,
            _lib.ptr(pool), code, KH, D, cfg.page_size, cfg.num_layers, cfg.max_pages, int(layer_idx),
            _lib.stream_of(pool))
        _lib.check(rc, "write_kv")

    def _rows(self, t, n: int, what: str):
        """[n, KH, D] contiguous view of a K or V argument on the pool's device."""
        cfg = self.config
        _lib.require_cuda(t, self._gpu_pool)
        if t.numel() != n * cfg.num_kv_heads * cfg.head_dim:
            raise RuntimeError(f"{what} must hold {n} x {cfg.num_kv_heads} x {cfg.head_dim} values, "
                               f"got shape {tuple(t.shape)}")
        return t.reshape(n, cfg.num_kv_heads, cfg.head_dim).contiguous()

    def write_kv(self, request_id: str, layer_idx: int, page_id: int, slot: int, key: Any, value: Any) -> None:
        """Writes one token's K/V ([num_kv_heads, head_dim]) to (page_id, slot)
        of ``layer_idx``; with TurboQuant compression the rows also wait in
        the queue that ``flush_compression`` empties."""
        import torch

        self._require_pool("write_kv")
        key = self._rows(key, 1, "key")
        value = self._rows(value, 1, "value")
        ids = torch.tensor([[page_id], [slot]], dtype=torch.int32).to(self._gpu_pool.device)
        self._write_rows(layer_idx, ids[0], ids[1], key, value)
        if self._kv_compressor is not None:
            self._pending_compress.append((layer_idx, ids[0], ids[1], key, value, [(int(page_id), int(slot))]))

    def write_kv_batch(self, layer_idx: int, page_ids: Any, slots: Any, key: Any, value: Any,
                       host_slots: Optional[Sequence[Tuple[int, int]]] = None) -> None:
        """Writes N tokens' K/V ([N, num_kv_heads, head_dim]) in one launch;
        ``page_ids`` / ``slots`` are [N] device tensors (``append_tokens``).
        ``host_slots`` optionally lists the same (page, slot) pairs on the host,
        which spares the compression queue a device read-back."""
        import torch

        self._require_pool("write_kv_batch")
        N = int(page_ids.shape[0])
        key = self._rows(key, N, "key")
        value = self._rows(value, N, "value")
        page_ids = page_ids.to(torch.int32).contiguous()
        slots = slots.to(torch.int32).contiguous()
        if tuple(slots.shape) != (N,):
            raise RuntimeError("page_ids and slots must both be [N]")
        self._write_rows(layer_idx, page_ids, slots, key, value)
        if self._kv_compressor is not None:
            self._pending_compress.append((layer_idx, page_ids, slots, key, value,
                                           list(host_slots) if host_slots is not None else None))

    def flush_compression(self) -> None:
        """Compresses every queued row, all layers at once, into the TurboQuant
        pages: one launch per source dtype."""
        import torch

        pending, self._pending_compress = self._pending_compress, []
        if not pending or self._kv_compressor is None:
            return
        cfg = self.config
        L = cfg.num_layers
        groups: Dict[Any, list] = {}
        for item in pending:
            groups.setdefault(item[3].dtype, []).append(item)
        signs, jl, lut = self._tq_buffers
        lib = _lib.load()
        for dtype, items in groups.items():
            # (page, layer) pairs flattened to page * L + layer, so that one
            # launch covers every layer: the pool is viewed as [P * L, 1, ...].
            flat = torch.cat([it[1].to(torch.int64) * L + it[0] for it in items]).to(torch.int32)
            slots = torch.cat([it[2] for it in items])
            key = torch.cat([it[3] for it in items])
            value = torch.cat([it[4] for it in items])
            N = key.shape[0]
            rc = lib.vrm_tq_quant_append(
                _lib.ptr(key), _lib.ptr(value), _lib.src_dtype_code(dtype), _lib.ptr(flat), _lib.ptr(slots), N,
                _lib.ptr(self._tq_pool), cfg.num_kv_heads, cfg.head_dim, cfg.page_size, 1, cfg.max_pages * L, 0,
                cfg.compression_bits, self._kv_compressor.qjl_dim, _lib.ptr(signs), _lib.ptr(jl), _lib.ptr(lut),
                _lib.stream_of(key))
            _lib.check(rc, "flush_compression")
        for layer_idx, pids, slots, _, _, host in pending:
            pairs = host if host is not None else list(zip(pids.tolist(), slots.tolist()))
            for pid, slot in pairs:
                if 0 <= pid < cfg.max_pages and 0 <= slot < cfg.page_size:
                    self._tq_slots[pid, layer_idx] |= np.uint64(1 << min(slot, 63))

    def read_kv(self, request_id: str, layer_idx: int) -> Optional[Tuple[Any, Any]]:
        """(keys, values) of a request for one layer, [num_kv_heads, tokens,
        head_dim] (core/paged_attention.py:677-712); quantized pools are
        dequantized to float32."""
        import torch

        if self._gpu_pool is None:
            return None
        with self._lock:
            entry = self._page_tables.get(request_id)
            if entry is None or not entry.pages:
                return None
            page_ids, tokens = list(entry.pages), entry.num_tokens
        cfg = self.config
        ids = torch.tensor(page_ids, dtype=torch.int32).to(self._gpu_pool.device)
        if self._kv_scales is not None:
            from . import kv_quant

            pages = kv_quant.dequantize_pages(self._gpu_pool, self._kv_scales, layer_idx, ids)
        else:
            pages = self._gpu_pool[ids.long(), layer_idx]
        # [n, 2, KH, PS, D] -> [KH, n * PS, D] per K/V
        keys = pages[:, 0].permute(1, 0, 2, 3).reshape(cfg.num_kv_heads, -1, cfg.head_dim)[:, :tokens]
        values = pages[:, 1].permute(1, 0, 2, 3).reshape(cfg.num_kv_heads, -1, cfg.head_dim)[:, :tokens]
        return keys, values

    # ------------------------------------------------------------------
    # Hugging Face caches (core/paged_attention.py:716-912)
    # ------------------------------------------------------------------

    def from_hf_cache(self, request_id: str, past_key_values: Any) -> None:
        """Stores a prefilled Hugging Face cache in a request's pages
        (core/paged_attention.py:716-805).

        ``past_key_values`` is a ``Cache`` or a tuple of (key, value) pairs,
        keys/values [batch, num_kv_heads, seq_len, head_dim]; batch row 0 is
        stored, as in the reference.  Pages are added until seq_len tokens
        fit (fewer when the pool runs out), the token count becomes seq_len,
        and each of the first num_layers layers is written with one
        ``vrm_kv_write`` launch (for int8 / fp8 pools, one
        ``vrm_kv_quant_pages`` launch over whole pages).  TurboQuant codes are not written here: as in the reference they are
        made when a turbo decode or ``compress_page_bulk`` needs them.  Does
        nothing without a pool."""
        import torch

        if self._gpu_pool is None or past_key_values is None:
            return
        if self._page_tables.get(request_id) is None:
            self.allocate(request_id)
        layers = hf_layers(past_key_values)
        if not layers:
            return
        cfg = self.config
        seq_len = int(layers[0][0].shape[2])
        for k, v in layers[:cfg.num_layers]:
            for t in (k, v):
                if t.dim() != 4 or t.shape[1] != cfg.num_kv_heads or t.shape[2] != seq_len \
                        or t.shape[3] != cfg.head_dim:
                    raise RuntimeError(f"cache states must be [batch, {cfg.num_kv_heads}, {seq_len}, "
                                       f"{cfg.head_dim}], got {tuple(t.shape)}")
        with self._lock:
            entry = self._page_tables[request_id]
            while len(entry.pages) < math.ceil(seq_len / cfg.page_size):
                page_id = self._alloc_page()
                if page_id is None:
                    break
                entry.pages.append(page_id)
            entry.num_tokens = seq_len
            self._peak_usage = max(self._peak_usage, cfg.max_pages - len(self._free_pages))
            self._epoch += 1
            pages = np.asarray(entry.pages, dtype=np.int64)
        PS, KH, D = cfg.page_size, cfg.num_kv_heads, cfg.head_dim
        n = min(seq_len, len(pages) * PS)
        if n == 0:
            return
        dev = self._gpu_pool.device
        nl = min(len(layers), cfg.num_layers)
        if self._kv_scales is not None:
            # Quantized pools take whole pages (the fp8 scale is one per page).
            from . import kv_quant

            NP = -(-n // PS)
            ids = torch.from_numpy(pages[:NP].astype(np.int32)).to(dev)
            n_valid = torch.from_numpy(np.minimum(PS, n - PS * np.arange(NP)).astype(np.int32)).to(dev)

            def page_major(t):  # [1, KH, S, D] -> [NP, KH, PS, D], zero past n
                rows = torch.zeros((KH, NP * PS, D), dtype=t.dtype, device=dev)
                rows[:, :n] = t[0, :, :n]
                return rows.view(KH, NP, PS, D).transpose(0, 1)

            for layer_idx in range(nl):
                k, v = layers[layer_idx]
                _lib.require_cuda(k, v, self._gpu_pool)
                kv_quant.quantize_pages(self._gpu_pool, self._kv_scales, layer_idx, ids, page_major(k),
                                        page_major(v), n_valid)
            return
        t = np.arange(n)
        ids = torch.from_numpy(np.stack([pages[t // PS], t % PS]).astype(np.int32)).to(dev)
        for layer_idx in range(nl):
            k, v = layers[layer_idx]
            key = self._rows(k[0, :, :n].transpose(0, 1), n, "key")
            value = self._rows(v[0, :, :n].transpose(0, 1), n, "value")
            self._write_rows(layer_idx, ids[0], ids[1], key, value)

    def to_hf_cache(self, request_id: str) -> Optional[tuple]:
        """A request's pages as a Hugging Face legacy cache
        (core/paged_attention.py:807-912): a tuple over num_layers of (key,
        value), each [1, num_kv_heads, tokens, head_dim] in the pool's dtype
        (float32 for int8 / fp8 pools, dequantized).  ``None`` without a pool
        or for a request with no page."""
        if self._gpu_pool is None:
            return None
        out = []
        for layer_idx in range(self.config.num_layers):
            got = self.read_kv(request_id, layer_idx)
            if got is None:
                return None
            out.append((got[0].unsqueeze(0), got[1].unsqueeze(0)))
        return tuple(out)

    # ------------------------------------------------------------------
    # Decode (core/paged_attention.py:1193-1418)
    # ------------------------------------------------------------------

    def _block_table(self, request_ids: Sequence[str], device) -> Optional[tuple]:
        """Device (page_table [B, width], context_lens [B]) for a batch of
        requests; ``None`` when no request has a page.

        ``width`` is the longest page list plus headroom (entries past a
        request's pages are -1; the decode reads only ctx's pages).  The
        table is kept for the next call with the same requests: reused as is
        while no page list or token count changed; when the requests only
        grew within the width (decode steps: every count + 1, now and then a
        new page) the new token counts and page ids are uploaded and patched
        in place on the current stream, an upload of O(B) values instead of
        every page id; anything else rebuilds it with
        ``vrm_build_block_table``."""
        import torch

        rids, dev = tuple(request_ids), str(device)
        c = self._table_cache
        if c is not None and c["key"] == (rids, dev) and c["epoch"] == self._epoch:
            return c["result"]
        B = len(rids)
        with self._lock:
            epoch = self._epoch
            entries = [self._page_tables.get(rid) for rid in rids]
            lists = [e.pages if e is not None else [] for e in entries]
            counts = np.fromiter((len(p) for p in lists), dtype=np.int64, count=B)
            ntok = np.fromiter((e.num_tokens if e is not None else 0 for e in entries), dtype=np.int64, count=B)
            max_pp = int(counts.max()) if B else 0
            grow = (c is not None and c["key"] == (rids, dev) and max_pp <= c["width"]
                    and all(a is b for a, b in zip(entries, c["entries"])) and bool((counts >= c["counts"]).all()))
            if grow:
                old = c["counts"]
                new = [(b * c["width"] + j, lists[b][j]) for b in np.flatnonzero(counts > old).tolist()
                       for j in range(int(old[b]), int(counts[b]))]
            elif max_pp:
                total = int(counts.sum())
                flat = np.fromiter(itertools.chain.from_iterable(lists), dtype=np.int32, count=total)
        if max_pp == 0:
            return None
        if grow:
            n = len(new)
            host = np.empty(B + 2 * n, dtype=np.int64)  # token counts, flat table indices, page ids: one upload
            host[:B] = ntok
            if n:
                host[B:] = np.asarray(new, dtype=np.int64).T.reshape(-1)
            buf = torch.from_numpy(host).to(device)
            table, ctx = c["result"]
            ctx.copy_(buf[:B])
            if n:
                table.view(-1).index_copy_(0, buf[B:B + n], buf[B + n:].to(torch.int32))
            c.update(epoch=epoch, counts=counts, ntok=ntok, buf=buf)
            return c["result"]
        width = max_pp + max(16, max_pp // 8)
        host = np.empty(2 * B + 1 + total, dtype=np.int32)  # offsets, token counts, pages: one upload
        host[0] = 0
        np.cumsum(counts, out=host[1:B + 1])
        host[B + 1:2 * B + 1] = ntok
        host[2 * B + 1:] = flat
        buf = torch.from_numpy(host).to(device)
        table = torch.empty((B, width), dtype=torch.int32, device=device)
        ctx = torch.empty((B,), dtype=torch.int32, device=device)
        rc = _lib.load().vrm_build_block_table(
            _lib.ptr(buf[2 * B + 1:]) if total else None, total, _lib.ptr(buf), _lib.ptr(buf[B + 1:]), B, width,
            _lib.ptr(table), _lib.ptr(ctx), _lib.stream_of(table))
        _lib.check(rc, "build_block_table")
        self._table_cache = dict(key=(rids, dev), epoch=epoch, entries=entries, counts=counts, ntok=ntok,
                                 width=width, result=(table, ctx), buf=buf)
        return table, ctx

    def _workspace(self, B: int, H: int, max_pp: int, device):
        from .paged_attention_cuda import decode_workspace

        cfg = self.config
        key = (B, H, max_pp, str(device))
        ws = self._workspaces.get(key)
        if ws is None:
            if len(self._workspaces) > 8:
                self._workspaces.clear()
            ws = decode_workspace(B, H, cfg.num_kv_heads, cfg.head_dim, max_pp, device, cfg.page_size)
            self._workspaces[key] = ws
        return ws

    def compute_attention_decode(self, query: Any, request_ids: list, layer_idx: int,
                                 scale: Optional[float] = None) -> Any:
        """Decode attention of a batch straight from the pool: query [B, H, D]
        -> [B, H, D] float32 (core/paged_attention.py:1193-1253).  Returns
        ``None`` without a pool or when no request has a page."""
        from .paged_attention_cuda import paged_attention_decode

        if self._gpu_pool is None:
            return None
        got = self._block_table(request_ids, query.device)
        if got is None:
            return None
        table, ctx = got
        B, H = query.shape[0], query.shape[1]
        # the host token counts pick the kernel (even batches: the balanced decode)
        ntok = self._table_cache["ntok"] if self._table_cache is not None else None
        return paged_attention_decode(query, self._gpu_pool, table, ctx, layer_idx, scale, kv_scales=self._kv_scales,
                                      workspace=self._workspace(B, H, table.shape[1], query.device),
                                      context_lens_host=ntok)

    def _ensure_compressed(self, page_ids: Sequence[int], layer_idx: int) -> None:
        missing = [p for p in dict.fromkeys(page_ids) if self._tq_slots[p, layer_idx] == 0]
        for pid in missing:
            self.compress_page_bulk(pid)

    def compute_attention_turbo(self, query: Any, request_id: str, layer_idx: int,
                                scale: Optional[float] = None) -> Any:
        """Attention of one request's query [num_heads, head_dim] over its
        TurboQuant pages (core/paged_attention.py:1259-1418): QJL-corrected
        scores of the rotated query, softmax, dense decompressed values, with
        query head h reading kv-head h % num_kv_heads.  Returns [num_heads,
        head_dim] float32, or ``None`` without compression or data."""
        if self._kv_compressor is None:
            return None
        with self._lock:
            entry = self._page_tables.get(request_id)
            if entry is None or not entry.pages:
                return None
            page_ids, num_tokens = list(entry.pages), entry.num_tokens
        if num_tokens <= 0:
            return None
        self._require_pool("compute_attention_turbo")
        self._ensure_compressed(page_ids, layer_idx)
        num_heads = query.shape[0] if query.dim() >= 2 else 1
        q = query.reshape(1, num_heads, self.config.head_dim)
        if self._sparse_k(num_tokens) < num_tokens:
            return self._turbo_sparse(q[0], page_ids, num_tokens, layer_idx, scale)
        return self._turbo_decode(q, [page_ids], [num_tokens], layer_idx, scale)[0]

    def _sparse_k(self, num_tokens: int) -> int:
        """Tokens whose values a head keeps: max(1, ceil(sparse_v_ratio * seq))
        (core/paged_attention.py:1379-1380)."""
        return max(1, int(math.ceil(self.config.sparse_v_ratio * num_tokens)))

    def _turbo_sparse(self, q, page_ids, num_tokens, layer_idx, scale):
        """Sparse V of compute_attention_turbo (core/paged_attention.py:
        1384-1400) for one request: per kv-head, scores of its query heads
        (h % KH), the renormalised top-k softmax and the weighted sum of those
        tokens' values, all in library kernels."""
        import torch

        from . import tq_pages
        from .turboquant_cuda import CUDATurboQuantOps, topk_attend

        cfg = self.config
        KH, D = cfg.num_kv_heads, cfg.head_dim
        H = q.shape[0]
        comp = self._kv_compressor
        dev = self._tq_pool.device
        ids = torch.tensor(page_ids, dtype=torch.int32).to(dev)
        codes = tq_pages.read_pages(self._tq_pool, layer_idx, ids, comp, cfg.page_size)  # [NP, K/V, KH, PS, ...]
        if scale is None:
            scale = 1.0 / math.sqrt(D)
        n = num_tokens
        k = self._sparse_k(n)
        qf = q.to(dev, torch.float32)
        signs, jl = comp._hadamard_signs, comp.jl_matrix
        args = (D, comp._padded_dim, comp._n_levels, comp.bits_per_angle)
        out = torch.empty((H, D), dtype=torch.float32, device=dev)

        def tokens(name, kv, kvh):  # the request's first n tokens of one kv-head, page-major
            t = codes[name][:, kv, kvh]
            return t.reshape(-1, *t.shape[2:])[:n].contiguous()

        for kvh in range(KH):
            group = torch.arange(kvh, H, KH, device=dev)
            keys = {"radius": tokens("radius", 0, kvh), "angles": [tokens("angles", 0, kvh)],
                    "qjl_signs": tokens("qjl_signs", 0, kvh), "qjl_norms": tokens("qjl_norms", 0, kvh)}
            scores = CUDATurboQuantOps.attention_score_gpu(qf[group], keys, *args, signs, jl, comp.qjl_dim,
                                                           scale=scale)
            vals = {"radius": tokens("radius", 1, kvh), "angles": [tokens("angles", 1, kvh)], "shape": (n, D)}
            out[group] = topk_attend(scores, k, CUDATurboQuantOps.decompress_gpu(vals, *args, signs))
        return out

    def compute_attention_turbo_batch(self, query: Any, request_ids: Sequence[str], layer_idx: int,
                                      scale: Optional[float] = None) -> Any:
        """``compute_attention_turbo`` for a batch in one launch: query
        [B, H, D] -> [B, H, D] float32; a request without pages or tokens
        gets zeros."""
        import torch

        if self._kv_compressor is None:
            return None
        self._require_pool("compute_attention_turbo_batch")
        with self._lock:
            lists, ntok = [], []
            for rid in request_ids:
                entry = self._page_tables.get(rid)
                lists.append(list(entry.pages) if entry is not None else [])
                ntok.append(entry.num_tokens if entry is not None else 0)
        for pages, n in zip(lists, ntok):
            if n > 0:
                self._ensure_compressed(pages[:math.ceil(n / self.config.page_size)], layer_idx)
        if not any(lists):
            return torch.zeros(query.shape, dtype=torch.float32, device=query.device)
        out = self._turbo_decode(query, lists, ntok, layer_idx, scale)
        for b, (pages, n) in enumerate(zip(lists, ntok)):
            if n > 0 and pages and self._sparse_k(n) < n:
                out[b] = self._turbo_sparse(query[b], pages, n, layer_idx, scale)
        return out

    def _turbo_decode(self, query, lists, ntok, layer_idx, scale):
        """Paged TurboQuant decode with the reference's h % n_kv head mapping.

        The kernel gives query head j kv-head j // (H / KH); the reference's
        group of kv-head k is heads k, k + KH, k + 2 KH, ..., so query heads
        are permuted into kernel order (j = k * (H / KH) + g for head
        g * KH + k) and the output permuted back."""
        import torch

        cfg = self.config
        KH, D = cfg.num_kv_heads, cfg.head_dim
        B, H = query.shape[0], query.shape[1]
        if H % KH:
            raise RuntimeError(f"num_heads {H} is not a multiple of num_kv_heads {KH}")
        dev = self._tq_pool.device
        ratio = H // KH
        order = torch.arange(H).reshape(ratio, KH).t().reshape(-1)  # kernel head j <- reference head order[j]
        q = query.to(dev, torch.float32)[:, order.to(dev)].contiguous()
        max_pp = max(1, max(len(p) for p in lists))
        table = np.full((B, max_pp + 1), -1, dtype=np.int32)  # last column: context lengths
        for b, pages in enumerate(lists):
            table[b, :len(pages)] = pages
            table[b, max_pp] = ntok[b]
        t = torch.from_numpy(table).to(dev)
        page_table = t[:, :max_pp].contiguous()
        ctx = t[:, max_pp].contiguous()
        if scale is None:
            scale = 1.0 / math.sqrt(D)
        out = torch.empty((B, H, D), dtype=torch.float32, device=dev)
        ws = self._workspace(B, H, max_pp, dev)
        signs, jl, lut = self._tq_buffers
        rc = _lib.load().vrm_paged_decode_tq(
            _lib.ptr(q), _lib.ptr(self._tq_pool), _lib.ptr(page_table), _lib.ptr(ctx), _lib.ptr(out), _lib.ptr(ws),
            ws.numel() * ws.element_size(), B, H, KH, D, cfg.page_size, cfg.num_layers, cfg.max_pages, max_pp,
            int(layer_idx), float(scale), cfg.compression_bits, self._kv_compressor.qjl_dim, _lib.ptr(signs),
            _lib.ptr(jl), _lib.ptr(lut), _lib.stream_of(q))
        _lib.check(rc, "compute_attention_turbo")
        inverse = torch.empty_like(order)
        inverse[order] = torch.arange(H)
        return out[:, inverse.to(dev)]

    def compress_page_bulk(self, page_id: int, num_valid_slots: int = 0) -> bool:
        """Compresses a page's raw K/V into TurboQuant codes for every layer
        that has none yet; slots from ``num_valid_slots`` on (when > 0) get
        zero codes (core/paged_attention.py:1420-1496).  False without
        compression, without a pool or for a free page."""
        import torch

        if self._kv_compressor is None or self._gpu_pool is None:
            return False
        cfg = self.config
        if not 0 <= page_id < cfg.max_pages or not self._pages[page_id].allocated:
            return False
        ps = num_valid_slots if num_valid_slots > 0 else cfg.page_size
        ps = min(ps, cfg.page_size)
        layers = [l for l in range(cfg.num_layers) if self._tq_slots[page_id, l] == 0]
        if not layers:
            return True
        L = cfg.num_layers
        host = np.array([[page_id * L + l for l in layers], [ps] * len(layers)], dtype=np.int32)
        dev = torch.from_numpy(host).to(self._gpu_pool.device)
        signs, jl, lut = self._tq_buffers
        rc = _lib.load().vrm_tq_compress_pool(
            _lib.ptr(self._gpu_pool), _lib.kv_dtype_code(self._gpu_pool.dtype), _lib.ptr(dev[0]), _lib.ptr(dev[1]),
            len(layers), _lib.ptr(self._tq_pool), cfg.num_kv_heads, cfg.head_dim, cfg.page_size, 1,
            cfg.max_pages * L, 0, cfg.compression_bits, self._kv_compressor.qjl_dim, _lib.ptr(signs), _lib.ptr(jl),
            _lib.ptr(lut), _lib.stream_of(self._gpu_pool))
        _lib.check(rc, "compress_page_bulk")
        self._tq_slots[page_id, layers] = np.uint64((1 << min(ps, 64)) - 1)
        return True

    # ------------------------------------------------------------------
    # Introspection
    # ------------------------------------------------------------------

    @property
    def kv_compression_active(self) -> bool:
        return self._kv_compressor is not None

    @property
    def compression_ratio(self) -> float:
        """fp16 bits per dim over the compressor's bits per dim."""
        if self._kv_compressor is None:
            return 1.0
        return 16.0 / self._kv_compressor.bits_per_dim()

    def stats(self) -> Dict[str, Any]:
        used = self.config.max_pages - len(self._free_pages)
        compressed = int(np.count_nonzero(self._tq_slots.any(axis=1))) if self._tq_slots is not None else 0
        return {
            "total_pages": len(self._pages),
            "used_pages": used,
            "free_pages": len(self._free_pages),
            "utilization": used / max(len(self._pages), 1),
            "peak_usage": self._peak_usage,
            "total_allocations": self._total_allocations,
            "total_frees": self._total_frees,
            "active_requests": len(self._page_tables),
            "prefix_cache_entries": len(self._prefix_cache),
            "prefix_cache_hits": self._cache_hits,
            "page_size_tokens": self.config.page_size,
            "memory_mb": self.config.total_memory_bytes / 1e6,
            "devices": [self.config.device],
            "kv_compression": self.config.kv_compression or "none",
            "compressed_pages": compressed,
            "compression_ratio": self.compression_ratio,
        }

    def __repr__(self) -> str:
        s = self.stats()
        return (f"PagedKVCache(pages={s['used_pages']}/{s['total_pages']}, "
                f"requests={s['active_requests']}, mem={s['memory_mb']:.1f}MB)")
