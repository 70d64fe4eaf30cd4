"""Host bookkeeping of the paged cache manager (no GPU needed).

Expected values follow the reference's allocator as written in
core/paged_attention.py: pages are popped from the end of a free list that
starts as [0 .. max_pages), freed pages are appended to it, append_token maps
token n to (pages[n // page_size], n % page_size) and allocates a page when
n reaches the end of the list, fork shares pages with ref counts.
"""
import math

import pytest

from vramancer_amd.paged_attention import PagedKVCacheManager, PagedKVConfig


def _mgr(**kw):
    cfg = dict(page_size=16, num_layers=2, num_kv_heads=2, head_dim=128, max_pages=8, device="cpu")
    cfg.update(kw)
    return PagedKVCacheManager(PagedKVConfig(**cfg))


def test_allocate_pops_from_the_end_of_the_free_list():
    m = _mgr()
    e = m.allocate("a", num_tokens=20)
    assert e.pages == [7, 6] and e.num_tokens == 20
    assert m.allocate("a", num_tokens=99) is e  # an existing request is returned as is
    assert m.allocate("b").pages == []


def test_append_token_slot_mapping_and_page_growth():
    m = _mgr()
    m.allocate("a", num_tokens=20)
    assert m.append_token("a") == (6, 4)
    for n in range(21, 32):
        assert m.append_token("a") == (6, n % 16)
    assert m.append_token("a") == (5, 0)  # token 32 opens the third page
    assert m._page_tables["a"].pages == [7, 6, 5]
    assert m._page_tables["a"].num_tokens == 33
    assert m.append_token("missing") is None


def test_pool_exhaustion_returns_none():
    m = _mgr(max_pages=2)
    m.allocate("a", num_tokens=32)
    assert m.append_token("a") is None
    assert m._page_tables["a"].num_tokens == 32


def test_free_and_reuse_order():
    m = _mgr()
    m.allocate("a", num_tokens=40)  # pages 7, 6, 5
    m.allocate("b", num_tokens=1)   # page 4
    assert m.free("a") == 3
    assert m.free("a") == 0
    # freed pages were appended in list order, so the last freed (5) comes back first
    assert m.allocate("c", num_tokens=48).pages == [5, 6, 7]
    s = m.stats()
    assert s["used_pages"] == 4 and s["total_frees"] == 3 and s["total_allocations"] == 7
    assert s["peak_usage"] == 4


def test_fork_shares_pages_with_ref_counts():
    m = _mgr()
    m.allocate("a", num_tokens=17)
    f = m.fork("a", "b")
    assert f.pages == [7, 6] and f.num_tokens == 17
    assert [m._pages[p].ref_count for p in (7, 6)] == [2, 2]
    assert m.free("a") == 0  # still referenced by the fork
    assert m.free("b") == 2
    assert m.fork("gone", "x") is None


def test_page_size_bytes():
    base = dict(page_size=16, num_layers=48, num_kv_heads=8, head_dim=128)
    # the reference's formula for float pools, core/paged_attention.py:107-111
    assert PagedKVConfig(dtype="float16", **base).page_size_bytes == 2 * 48 * 8 * 128 * 16 * 2 == 3145728
    assert PagedKVConfig(dtype="float32", **base).page_size_bytes == 2 * 48 * 8 * 128 * 16 * 4
    assert PagedKVConfig(dtype="bfloat16", **base).page_size_bytes == 3145728
    # int8: one byte per code plus a float32 scale per token and head
    assert PagedKVConfig(dtype="int8", **base).page_size_bytes == 2 * 48 * 8 * 16 * (128 + 4)
    # fp8: one byte per code plus a float32 scale per page and head
    assert PagedKVConfig(dtype="fp8", **base).page_size_bytes == 2 * 48 * 8 * (16 * 128 + 4)
    cfg = PagedKVConfig(dtype="int8", max_pages=16384, **base)
    assert cfg.total_memory_bytes == cfg.page_size_bytes * 16384
    with pytest.raises(ValueError):
        PagedKVConfig(dtype="int4").page_size_bytes


def test_from_model_reads_model_config_and_env(monkeypatch):
    class FakeModel:
        class config:
            num_hidden_layers = 48
            num_attention_heads = 40
            num_key_value_heads = 8
            hidden_size = 5120

    monkeypatch.setenv("VRM_KV_COMPRESSION", "TurboQuant")
    monkeypatch.setenv("VRM_KV_COMPRESSION_BITS", "4")
    monkeypatch.setenv("VRM_SPARSE_V_RATIO", "0.25")
    cfg = PagedKVConfig.from_model(FakeModel(), max_pages=100, device="cuda:1")
    assert (cfg.num_layers, cfg.num_kv_heads, cfg.head_dim) == (48, 8, 128)
    assert (cfg.kv_compression, cfg.compression_bits, cfg.sparse_v_ratio) == ("turboquant", 4, 0.25)
    assert (cfg.max_pages, cfg.device) == (100, "cuda:1")
    monkeypatch.delenv("VRM_KV_COMPRESSION")
    assert PagedKVConfig.from_model(None).kv_compression is None


def test_host_only_manager_without_gpu():
    m = _mgr(kv_compression="turboquant", compression_bits=3)
    assert m.kv_compression_active
    # 127 * 3 + 16 + 64 + 16 bits per 128 dims (core/kv_quantizer.py:564-572)
    assert m.compression_ratio == pytest.approx(16.0 / ((127 * 3 + 16 + 64 + 16) / 128))
    s = m.stats()
    assert s["kv_compression"] == "turboquant" and s["compressed_pages"] == 0
    m.allocate("a", num_tokens=3)
    assert m.compute_attention_decode(None, ["a"], 0) is None  # no pool, as the reference without one
    assert m.compute_attention_turbo(None, "missing", 0) is None
    assert m.compress_page_bulk(7) is False
    with pytest.raises(RuntimeError, match="GPU pool"):
        m.write_kv("a", 0, 7, 0, None, None)
    with pytest.raises(RuntimeError, match="GPU pool"):
        m.compute_attention_turbo(None, "a", 0)
    assert _mgr().stats()["compression_ratio"] == 1.0


def test_unknown_compression_is_rejected():
    with pytest.raises(ValueError):
        _mgr(kv_compression="zstd")


def test_pages_needed_is_ceil_division():
    for n in (1, 15, 16, 17, 47, 48):
        m = _mgr()
        assert len(m.allocate("a", num_tokens=n).pages) == math.ceil(n / 16)


def test_prefix_cache_miss_then_hit():
    """core/paged_attention.py:521-566: full pages only; a first request
    registers its pages, a second with the same prefix shares them."""
    m = _mgr(page_size=4, max_pages=16)
    tokens = [1, 2, 3, 4, 5, 6, 7, 8, 9, 10]  # two full pages and a partial one
    assert m.try_prefix_cache("a", tokens) == 0
    assert m._page_tables["a"].pages == [15, 14] and m._page_tables["a"].num_tokens == 8
    assert m.try_prefix_cache("b", tokens) == 8
    assert m._page_tables["b"].pages == [15, 14]
    assert [m._pages[p].ref_count for p in (15, 14)] == [2, 2]
    s = m.stats()
    assert s["prefix_cache_entries"] == 2 and s["prefix_cache_hits"] == 2 and s["active_requests"] == 2
    assert m.free("a") == 0 and m.free("b") == 2


def test_prefix_cache_hits_count_only_a_run_to_the_last_page():
    m = _mgr(page_size=4, max_pages=16)
    m.try_prefix_cache("a", [1, 2, 3, 4, 5, 6, 7, 8])
    # first page hits, second misses: the count restarts at the miss
    assert m.try_prefix_cache("b", [1, 2, 3, 4, 0, 0, 0, 0]) == 0
    assert m._page_tables["b"].pages == [15, 13]
    # a miss then a hit counts the hit
    assert m.try_prefix_cache("c", [9, 9, 9, 9, 5, 6, 7, 8]) == 4
    assert m._page_tables["c"].pages == [12, 14]


def test_prefix_cache_skips_freed_pages_and_stops_when_full():
    m = _mgr(page_size=4, max_pages=3)
    m.try_prefix_cache("a", [1, 2, 3, 4])
    m.free("a")
    # the registered page is free again: a miss, which re-registers the page popped
    assert m.try_prefix_cache("b", [1, 2, 3, 4]) == 0
    assert m._page_tables["b"].pages == [2]
    assert m.try_prefix_cache("c", list(range(100, 116))) == 0
    assert m._page_tables["c"].pages == [1, 0] and m._page_tables["c"].num_tokens == 8


def test_hf_conversions_without_a_pool():
    """Without a GPU pool from_hf_cache does nothing and to_hf_cache returns
    None (core/paged_attention.py:728-729, 825-826)."""
    torch = pytest.importorskip("torch")
    m = _mgr()
    m.allocate("a")
    m.from_hf_cache("a", ((torch.zeros(1, 2, 3, 128), torch.zeros(1, 2, 3, 128)),))
    assert m._page_tables["a"].num_tokens == 0 and m.to_hf_cache("a") is None


def test_hf_layers_reads_each_cache_form():
    torch = pytest.importorskip("torch")
    from transformers import DynamicCache

    from vramancer_amd.paged_attention import hf_layers

    k = [torch.full((1, 2, 3, 4), float(i)) for i in range(3)]
    v = [t + 10 for t in k]
    legacy = tuple(zip(k, v))
    dyn = DynamicCache()
    for i in range(3):
        dyn.update(k[i], v[i], i)

    class Old:  # transformers 4.36-4.x attribute form
        key_cache, value_cache = k, v

    for form in (legacy, dyn, Old()):
        got = hf_layers(form)
        assert len(got) == 3
        assert all(torch.equal(a, b) and torch.equal(c, d) for (a, c), b, d in zip(got, k, v))
