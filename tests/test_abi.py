"""The C-ABI library loads on a host without a GPU, exports every function
include/vrm_paged.h declares, and rejects bad arguments on the host (these
paths return before any HIP call, so no device is touched)."""
import ctypes
import os
import re

import pytest

from vramancer_amd import _lib

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
HEADER = os.path.join(ROOT, "include", "vrm_paged.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vrm_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"


def test_abi_version(lib):
    assert lib.vrm_abi_version() == _lib.VRM_ABI_VERSION == 2


def _header_bytes(B):
    return ((16 + 2 * B + 1) * 4 + 255) // 256 * 256


def test_split_geometry_is_host_only(lib):
    # 14B int8 shape: 64 sequences x 8 kv heads; the workspace holds a header
    # (partition size, first work item of each sequence) and the partials of
    # at most B + ceil(2048 / KH) work items
    ns = lib.vrm_paged_decode_num_splits(64, 40, 8, 256, 16)
    assert 64 * ns >= 64 + 2048 // 8
    assert lib.vrm_paged_decode_workspace_bytes(64, 40, 128, ns) == _header_bytes(64) + 64 * 40 * ns * 130 * 4
    # the capacity does not depend on the page-table width (long contexts get longer partitions)
    assert lib.vrm_paged_decode_num_splits(64, 40, 8, 8192, 16) == ns
    assert lib.vrm_paged_decode_num_splits(129, 64, 8, 8192, 16) * 129 >= 129 + 256
    assert lib.vrm_paged_decode_num_splits(1, 3, 2, 4, 16) == 0  # H % KH != 0


# a fake scale pointer far from the fake pool pointers (a plain pool's scales
# must not start inside its codes)
SC = 1 << 40


def _decode(lib, **kw):
    a = dict(q=1, pool=1, sc=None, pt=1, cl=1, out=1, ws=1, wsb=1 << 30, B=2, H=8, KH=2, D=128, PS=16, L=1, P=4,
             max_pp=2, layer=0, scale=0.1, dt=_lib.VRM_KV_BF16)
    a.update(kw)
    return lib.vrm_paged_decode(a["q"], a["pool"], a["sc"], a["pt"], a["cl"], a["out"], a["ws"], a["wsb"], a["B"],
                                a["H"], a["KH"], a["D"], a["PS"], a["L"], a["P"], a["max_pp"], a["layer"],
                                a["scale"], a["dt"], None)


def test_decode_rejects_bad_arguments(lib):
    assert _decode(lib, q=None) == -1 and b"null" in lib.vrm_last_error()
    assert _decode(lib, H=7) == -1 and b"multiple" in lib.vrm_last_error()
    assert _decode(lib, layer=1) == -1 and b"layer_idx" in lib.vrm_last_error()
    assert _decode(lib, D=257) == -2 and b"head_dim" in lib.vrm_last_error()
    assert _decode(lib, D=100, dt=_lib.VRM_KV_I8, sc=SC) == -2 and b"head_dim" in lib.vrm_last_error()
    assert _decode(lib, PS=6, dt=_lib.VRM_KV_FP8E4M3, sc=SC) == -2 and b"page_size" in lib.vrm_last_error()
    assert _decode(lib, dt=99) == -1 and b"kv_dtype" in lib.vrm_last_error()
    assert _decode(lib, dt=_lib.VRM_KV_I8) == -1 and b"kv_scales" in lib.vrm_last_error()
    assert _decode(lib, sc=1) == -1 and b"float pool" in lib.vrm_last_error()
    assert _decode(lib, wsb=16) == -3 and b"workspace" in lib.vrm_last_error()
    assert _decode(lib, scale=float("nan")) == -1


def test_kv_slab_bytes(lib):
    """Bytes per (page, layer): plain layouts 2 KH PS D elements (codes only),
    inline records of PS (2 D + 8) bytes (int8) or 2 PS D + 128 (fp8) per
    kv-head."""
    assert lib.vrm_kv_slab_bytes(_lib.VRM_KV_I8, 8, 16, 128) == 32768
    assert lib.vrm_kv_slab_bytes(_lib.VRM_KV_FP8E4M3, 8, 16, 128) == 32768
    assert lib.vrm_kv_slab_bytes(_lib.VRM_KV_I8_INLINE, 8, 16, 128) == 8 * (16 * 256 + 128) == 33792
    assert lib.vrm_kv_slab_bytes(_lib.VRM_KV_FP8E4M3_INLINE, 8, 16, 128) == 8 * (4096 + 128)
    assert lib.vrm_kv_slab_bytes(_lib.VRM_KV_I8_INLINE, 3, 8, 48) == 3 * 8 * (96 + 8)
    assert lib.vrm_kv_slab_bytes(_lib.VRM_KV_BF16, 4, 16, 128) == 2 * 4 * 16 * 128 * 2
    assert lib.vrm_kv_slab_bytes(_lib.VRM_KV_F32, 12, 16, 64) == 2 * 12 * 16 * 64 * 4
    assert lib.vrm_kv_slab_bytes(_lib.VRM_KV_I8_INLINE, 8, 6, 128) == 0   # page size not a multiple of 4
    assert lib.vrm_kv_slab_bytes(_lib.VRM_KV_I8_INLINE, 8, 16, 100) == 0  # head_dim not a multiple of 16
    assert lib.vrm_kv_slab_bytes(99, 8, 16, 128) == 0


def test_inline_pool_scale_pointer_checks(lib):
    """An inline pool's kv_scales must be kv_pool + 2 PS D; a plain pool's may
    not start inside its codes (an inline buffer passed with the plain dtype).
    Both are refused on the host by the decode, balanced, quantizer and
    dequantizer entries."""
    pool = 1 << 20
    inl = pool + 2 * 16 * 128
    # accepted pointers: the call goes on to the workspace check
    assert _decode(lib, pool=pool, sc=inl, dt=_lib.VRM_KV_I8_INLINE, wsb=16) == -3
    assert _decode(lib, pool=pool, sc=inl, dt=_lib.VRM_KV_FP8E4M3_INLINE, wsb=16) == -3
    assert _decode(lib, pool=pool, sc=inl + 4, dt=_lib.VRM_KV_I8_INLINE) == -1 and b"inline" in lib.vrm_last_error()
    assert _decode(lib, pool=pool, sc=inl, dt=_lib.VRM_KV_I8) == -1 and b"inside" in lib.vrm_last_error()
    assert _decode(lib, pool=pool, sc=inl, dt=_lib.VRM_KV_FP8E4M3) == -1 and b"inside" in lib.vrm_last_error()
    bal = lib.vrm_paged_decode_balanced
    args = [1, pool, inl, 1, 1, 1, None, 2, 8, 2, 128, 16, 1, 4, 2, 0, 0.1, _lib.VRM_KV_I8, None]
    assert bal(*args) == -1 and b"inside" in lib.vrm_last_error()
    args[2] = inl + 16
    args[17] = _lib.VRM_KV_I8_INLINE
    assert bal(*args) == -1 and b"inline" in lib.vrm_last_error()
    q = lib.vrm_kv_quant_append
    assert q(1, 1, _lib.VRM_SRC_BF16, 1, 1, 4, pool, inl, _lib.VRM_KV_I8, 2, 128, 16, 1, 4, 0, None) == -1
    assert b"inside" in lib.vrm_last_error()
    assert q(1, 1, _lib.VRM_SRC_BF16, 1, 1, 0, pool, inl, _lib.VRM_KV_I8_INLINE, 2, 128, 16, 1, 4, 0, None) == 0
    assert q(1, 1, _lib.VRM_SRC_BF16, 1, 1, 0, pool, SC, _lib.VRM_KV_I8_INLINE, 2, 128, 16, 1, 4, 0, None) == -1
    dq = lib.vrm_kv_dequant_pages
    assert dq(pool, inl, _lib.VRM_KV_FP8E4M3, 1, 0, 1, 2, 128, 16, 1, 4, 0, None) == -1
    assert dq(pool, inl, _lib.VRM_KV_FP8E4M3_INLINE, 1, 0, 1, 2, 128, 16, 1, 4, 0, None) == 0


def test_quant_rejects_bad_arguments(lib):
    f = lib.vrm_kv_quant_append
    ok = dict(k=1, v=1, src=_lib.VRM_SRC_BF16, pid=1, sl=1, N=4, pool=1, sc=SC, dt=_lib.VRM_KV_I8, KH=8, D=128, PS=16,
              L=2, P=10, layer=0)

    def call(**kw):
        a = dict(ok)
        a.update(kw)
        return f(a["k"], a["v"], a["src"], a["pid"], a["sl"], a["N"], a["pool"], a["sc"], a["dt"], a["KH"], a["D"],
                 a["PS"], a["L"], a["P"], a["layer"], None)

    assert call(k=None) == -1
    assert call(dt=_lib.VRM_KV_BF16) == -1 and b"quantized" in lib.vrm_last_error()
    assert call(src=7) == -1
    assert call(layer=2) == -1
    assert call(D=100) == -2
    assert call(D=264) == -2
    assert call(PS=6) == -2
    assert call(N=0) == 0  # nothing to do, nothing launched


def test_turboquant_rejects_bad_arguments(lib):
    c = lib.vrm_turboquant_compress
    assert c(1, 0, 4, 128, 128, 6, 3, 64, 1, 1, 1, 1, 1, 1, 1, None) == -1  # levels mismatch
    assert c(1, 0, 4, 128, 128, 7, 9, 64, 1, 1, 1, 1, 1, 1, 1, None) == -1  # bits
    assert c(1, 0, 4, 100, 100, 7, 3, 64, 1, 1, 1, 1, 1, 1, 1, None) == -2  # padded_dim
    assert c(1, 0, 0, 128, 128, 7, 3, 64, 1, 1, 1, 1, 1, 1, 1, None) == 0   # N == 0


def test_manager_and_attend_entries_reject_bad_arguments(lib):
    """Argument checks of the block table, raw write, pool compression, score,
    top-k, pack and merge entries: rejected on the host, nothing launched."""
    bt = lib.vrm_build_block_table
    assert bt(1, 4, 1, 1, -1, 8, 1, 1, None) == -1
    assert bt(1, 4, 1, 1, 70000, 8, 1, 1, None) == -2
    assert bt(1, 4, None, 1, 2, 8, 1, 1, None) == -1 and b"null" in lib.vrm_last_error()
    assert bt(None, 0, None, None, 0, 0, None, None, None) == 0

    w = lib.vrm_kv_write
    args = [1, 1, _lib.VRM_SRC_F32, 1, 1, 2, 1, _lib.VRM_KV_F16, 2, 64, 16, 3, 9, 0, None]

    def kw(i, v):
        a = list(args)
        a[i] = v
        return w(*a)

    assert kw(7, _lib.VRM_KV_I8) == -1 and b"float pool" in lib.vrm_last_error()
    assert kw(2, 7) == -1
    assert kw(13, 3) == -1 and b"layer_idx" in lib.vrm_last_error()
    assert kw(0, None) == -1
    assert kw(5, 0) == 0

    cp = lib.vrm_tq_compress_pool
    assert cp(1, _lib.VRM_KV_I8, 1, 1, 2, 1, 2, 128, 16, 1, 4, 0, 3, 64, 1, 1, 1, None) == -1
    assert cp(1, _lib.VRM_KV_F16, 1, 1, 2, 1, 2, 300, 16, 1, 4, 0, 3, 64, 1, 1, 1, None) == -2
    assert cp(1, _lib.VRM_KV_F16, 1, 1, 2, 1, 2, 96, 16, 1, 4, 0, 9, 64, 1, 1, 1, None) == -2
    assert cp(1, _lib.VRM_KV_F16, 1, 1, 2, 1, 2, 96, 16, 1, 4, 0, 3, 257, 1, 1, 1, None) == -2
    assert cp(1, _lib.VRM_KV_F16, 1, 1, 0, 1, 2, 128, 16, 1, 4, 0, 3, 64, 1, 1, 1, None) == 0

    sb = lib.vrm_turboquant_score_workspace_bytes(5, 128, 64)
    assert sb == 5 * 192 * 4
    sc = lib.vrm_turboquant_score
    assert sc(1, 5, 1, 1, 1, 1, 9, 128, 128, 7, 3, 0, 1, 1, 1, 1.0, 1, sb, 1, None) == -1
    assert sc(1, 5, 1, 1, 1, 1, 9, 128, 128, 7, 3, 64, 1, 1, 1, 1.0, 1, sb - 4, 1, None) == -3
    assert sc(1, 5, 1, 1, 1, 1, 9, 100, 100, 7, 3, 64, 1, 1, 1, 1.0, 1, sb, 1, None) == -2
    assert sc(None, 0, None, None, None, None, 9, 128, 128, 7, 3, 64, None, None, None, 1.0, None, 0, None,
              None) == 0

    tb = lib.vrm_topk_attend_workspace_bytes(3, 10)
    # selection [M][2] u32, indices and weights [M][k], row meta [M] (16-byte
    # aligned), partial sums [M][16 splits][256] f32
    r16 = lambda x: (x + 15) // 16 * 16  # noqa: E731
    assert tb == r16(r16(3 * 8 + 3 * 10 * 8) + 3 * 8) + 3 * 16 * 256 * 4
    tk = lib.vrm_topk_attend
    assert tk(1, 3, 10, 10, 11, 1, 64, 64, 1, 64, 1, tb, None) == -1  # k > N
    assert tk(1, 3, 10, 10, 0, 1, 64, 64, 1, 64, 1, tb, None) == -1   # k < 1
    assert tk(1, 3, 10, 9, 5, 1, 64, 64, 1, 64, 1, tb, None) == -1    # row stride below N
    assert tk(1, 3, 10, 10, 10, 1, 64, 64, 1, 64, 1, tb - 1, None) == -3
    assert tk(1, 0, 10, 10, 5, 1, 64, 64, 1, 64, None, 0, None) == 0

    assert lib.vrm_pack_bits(1, 4, 8, 9, 1, None) == -1
    assert lib.vrm_unpack_bits(None, 4, 8, 3, 1, None) == -1
    assert lib.vrm_pack_bits(None, 0, 8, 3, None, None) == 0

    assert lib.vrm_attn_combine(1, 1, 1, 1, -1, 64, 1, None, None) == -1
    assert lib.vrm_attn_combine(None, 1, 1, 1, 4, 64, 1, None, None) == -1
    assert lib.vrm_attn_combine(None, None, None, None, 0, 64, None, None, None) == 0

    assert lib.vrm_paged_decode_lse(1, 1, None, 1, 1, 1, None, 1, 1 << 30, 2, 8, 8, 64, 16, 1, 4, 4, 0, 0.125,
                                    _lib.VRM_KV_F32, None) == -1
    assert lib.vrm_paged_decode_tq_lse(1, 1, 1, 1, 1, None, 1, 1 << 30, 2, 8, 8, 128, 16, 1, 4, 4, 0, 0.1, 3, 64,
                                       1, 1, 1, 0, None) == -1


def test_tq_slice_sizes():
    """Slice sizes of the two TurboQuant page layouts, from their field
    lists: the tuned one (head_dim 128, qjl_dim 64, 2..4 bits, 16 tokens:
    16 * bits angle bytes, 8 sign bytes, 2 radius and 2 norm bytes a token)
    and the generic one (a token record of ceil((padded_dim - 1) * bits / 32)
    angle dwords, ceil(qjl_dim / 32) sign dwords and two fp16 fields)."""
    lib = _lib.load()
    for bits in (2, 3, 4):
        assert lib.vrm_tq_slice_bytes(128, bits, 64) == 16 * (16 * bits + 8 + 4)
        assert lib.vrm_tq_slice_bytes_ps(128, bits, 64, 16) == 16 * (16 * bits + 8 + 4)
    cases = [  # head_dim, bits, qjl_dim, page_size, padded_dim
        (96, 3, 64, 4, 128), (64, 1, 32, 16, 64), (64, 8, 33, 5, 64), (256, 5, 256, 16, 256),
        (33, 2, 1, 1, 64), (128, 4, 64, 8, 128), (128, 1, 64, 16, 128), (200, 7, 100, 3, 256),
        # head_dims below 33 pad to 32, 16, ..., 2 (the reference's 2^ceil(log2 max(head_dim, 2)))
        (32, 3, 16, 16, 32), (32, 3, 64, 16, 32), (17, 4, 16, 16, 32), (16, 3, 8, 16, 16), (8, 2, 4, 8, 8),
        (5, 4, 4, 16, 8), (3, 3, 2, 16, 4), (2, 3, 1, 16, 2), (1, 8, 1, 4, 2),
    ]
    for hd, bits, qjl, ps, pd in cases:
        rec = 4 * (-(-(pd - 1) * bits // 32)) + 4 * (-(-qjl // 32)) + 4
        assert lib.vrm_tq_slice_bytes_ps(hd, bits, qjl, ps) == ps * rec, (hd, bits, qjl, ps)
    for bad in [(0, 3, 64, 16), (257, 3, 64, 16), (96, 0, 64, 16), (96, 9, 64, 16), (96, 3, 0, 16),
                (96, 3, 257, 16), (96, 3, 64, 0)]:
        assert lib.vrm_tq_slice_bytes_ps(*bad) == 0, bad


def test_python_api_refuses_cpu_tensors():
    import torch
    from vramancer_amd.paged_attention_cuda import paged_attention_decode

    q = torch.randn(1, 4, 64)
    pool = torch.randn(2, 1, 2, 4, 16, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        paged_attention_decode(q, pool, torch.zeros(1, 1, dtype=torch.int32), torch.ones(1, dtype=torch.int32), 0)


def test_decode_wrappers_validate_out_workspace_and_table():
    """The Python wrappers check the tensors the kernels write or index
    through before any pointer reaches the library: out is a contiguous
    float32 [B, H, D] on the query's device, the workspace is contiguous on
    that device, the page table is [B, max_pages] and context_lens [B]."""
    import torch
    from vramancer_amd.paged_attention_cuda import check_outputs

    q = torch.randn(2, 8, 64)
    pt = torch.zeros(2, 3, dtype=torch.int32)
    cl = torch.ones(2, dtype=torch.int32)
    check_outputs(q, torch.empty(2, 8, 64), torch.empty(100, dtype=torch.uint8), pt, cl)
    check_outputs(q, None, None, pt, cl)
    bad = [
        dict(out=torch.empty(2, 8, 64, dtype=torch.float16)),
        dict(out=torch.empty(2, 8, 32)),
        dict(out=torch.empty(2, 64, 8).transpose(1, 2)),
        dict(out=torch.empty(2, 8, 64, device="meta")),
        dict(workspace=torch.empty(64, dtype=torch.uint8)[::2]),
        dict(workspace=torch.empty(64, dtype=torch.uint8, device="meta")),
        dict(page_table=torch.zeros(1, 3, dtype=torch.int32)),
        dict(page_table=torch.zeros(2, dtype=torch.int32)),
        dict(page_table=torch.zeros(2, 0, dtype=torch.int32)),
        dict(context_lens=torch.ones(3, dtype=torch.int32)),
    ]
    for kw in bad:
        a = dict(out=None, workspace=None, page_table=pt, context_lens=cl)
        a.update(kw)
        with pytest.raises(RuntimeError):
            check_outputs(q, a["out"], a["workspace"], a["page_table"], a["context_lens"])


def test_balanced_decode_selection_rule():
    """The balanced decode is chosen only for int8 / fp8 pools, at least 128
    (sequence, kv-head) pairs, and contexts within 10 % of their mean."""
    import torch
    from vramancer_amd.paged_attention_cuda import prefer_balanced

    assert prefer_balanced([4096] * 64, 8, torch.int8)
    assert prefer_balanced([4096] * 64, 8, torch.float8_e4m3fn)
    assert not prefer_balanced([4096] * 64, 8, torch.bfloat16)
    assert not prefer_balanced([4096] * 8, 8, torch.int8)          # 64 pairs: too few workgroups
    assert not prefer_balanced([1024, 8192] * 32, 8, torch.int8)   # ragged
    assert prefer_balanced([4000, 4400] * 32, 8, torch.int8)       # max 4400 <= 1.1 * mean 4200
    assert not prefer_balanced([0] * 64, 8, torch.int8)
    assert not prefer_balanced([], 8, torch.int8)
    assert prefer_balanced(torch.full((64,), 4096, dtype=torch.int32), 8, torch.int8)


def test_balanced_entry_rejects_bad_arguments(lib):
    f = lib.vrm_paged_decode_balanced
    args = [1, 1, SC, 1, 1, 1, None, 2, 8, 2, 128, 16, 1, 4, 2, 0, 0.1, _lib.VRM_KV_I8, None]

    def call(i, v):
        a = list(args)
        a[i] = v
        return f(*a)

    assert call(0, None) == -1
    assert call(2, None) == -1 and b"kv_scales" in lib.vrm_last_error()
    assert call(17, _lib.VRM_KV_BF16) == -2
    assert call(17, 99) == -1
    assert call(10, 256) == -2 and b"head_dim" in lib.vrm_last_error()
    assert call(10, 48) == -2 and b"head_dim" in lib.vrm_last_error()
    assert call(11, 32) == -2 and b"page_size" in lib.vrm_last_error()
    # the measuring build takes the same arguments (no lse) and the same checks
    g = lib.vrm_paged_decode_balanced_loads
    largs = args[:6] + args[7:]
    assert g(*largs[:2], None, *largs[3:]) == -1 and b"kv_scales" in lib.vrm_last_error()
    bad = list(largs)
    bad[9] = 256
    assert g(*bad) == -2 and b"head_dim" in lib.vrm_last_error()
