// Device side of the paged cache manager: block-table build and raw slot
// writes.
//
// PagedKVCacheManager.compute_attention_decode (core/paged_attention.py:
// 1226-1248) fills a -1-padded [B, max_pp] int32 page table element by element
// from each request's page list, then the context lengths.  Here the host
// hands over the lists concatenated (flat_pages, offsets) and one kernel
// scatters them, so a batch costs one copy of sum(pages) ints instead of
// B * max_pp host writes and a B * max_pp upload.
//
// write_kv's raw index-put into a float pool (:611-612,
// pool[page, layer, 0|1, :, slot, :] = key|value) is vrm_kv_write: one
// wavefront per (token, K/V, kv-head) row converts the row to the pool's
// element type, rounding to nearest even as PyTorch's copy does.
#include "vrm_common.h"

namespace vrm {
namespace {

constexpr int kTableThreads = 256;

__global__ void __launch_bounds__(kTableThreads)
    build_table_kernel(const int32_t* flat_pages, int n_flat, const int32_t* offsets, const int32_t* num_tokens,
                       int max_pp, int32_t* page_table, int32_t* context_lens) {
  const int b = blockIdx.y;
  const int p = blockIdx.x * kTableThreads + threadIdx.x;
  const int beg = offsets[b];
  const int end = offsets[b + 1];
  // A malformed list (offsets outside the flat array or decreasing) yields
  // absent pages rather than reads outside flat_pages.
  const bool ok = beg >= 0 && end >= beg && end <= n_flat;
  const int n = ok ? end - beg : 0;
  if (p < max_pp) page_table[(size_t)b * max_pp + p] = p < n ? flat_pages[beg + p] : -1;
  if (p == 0) context_lens[b] = num_tokens[b];
}

template <int SRC>
__device__ __forceinline__ float load_elem(const void* p, size_t i) {
  if constexpr (SRC == VRM_SRC_F32) {
    return static_cast<const float*>(p)[i];
  } else if constexpr (SRC == VRM_SRC_F16) {
    return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else {
    return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
}

// float32 -> bfloat16 bits, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
  const uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

template <int DST>
__device__ __forceinline__ void store_elem(void* p, size_t i, float x) {
  if constexpr (DST == VRM_KV_F32) {
    static_cast<float*>(p)[i] = x;
  } else if constexpr (DST == VRM_KV_F16) {
    static_cast<uint16_t*>(p)[i] = __builtin_bit_cast(unsigned short, (_Float16)x);
  } else {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(x);
  }
}

struct KvWriteArgs {
  const void* key;
  const void* value;
  const int32_t* page_ids;
  const int32_t* slots;
  void* pool;
  int KH, D, PS, L, P, layer;
};

// Row x = (n * 2 + kv) * KH + h; source rows are [N][KH][D].
template <int SRC, int DST>
__global__ void __launch_bounds__(64) kv_write_kernel(KvWriteArgs a) {
  const int x = blockIdx.x;
  const int h = x % a.KH;
  const int kv = (x / a.KH) & 1;
  const int n = x / (2 * a.KH);
  const int pid = a.page_ids[n];
  const int slot = a.slots[n];
  if (pid < 0 || pid >= a.P || slot < 0 || slot >= a.PS) return;  // rows aimed outside the pool are dropped
  const size_t src = ((size_t)n * a.KH + h) * a.D;
  const size_t dst = (((((size_t)pid * a.L + a.layer) * 2 + kv) * a.KH + h) * a.PS + slot) * a.D;
  const void* from = kv ? a.value : a.key;
  for (int d = threadIdx.x; d < a.D; d += 64) store_elem<DST>(a.pool, dst + d, load_elem<SRC>(from, src + d));
}

template <int SRC>
void launch_kv_write(const KvWriteArgs& a, int rows, int kv_dtype, hipStream_t st) {
  switch (kv_dtype) {
    case VRM_KV_F32: hipLaunchKernelGGL((kv_write_kernel<SRC, VRM_KV_F32>), dim3(rows), dim3(64), 0, st, a); break;
    case VRM_KV_F16: hipLaunchKernelGGL((kv_write_kernel<SRC, VRM_KV_F16>), dim3(rows), dim3(64), 0, st, a); break;
    default: hipLaunchKernelGGL((kv_write_kernel<SRC, VRM_KV_BF16>), dim3(rows), dim3(64), 0, st, a); break;
  }
}

}  // namespace
}  // namespace vrm

using namespace vrm;

extern "C" int vrm_build_block_table(const int32_t* flat_pages, int n_flat, const int32_t* offsets,
                                     const int32_t* num_tokens, int B, int max_pp, int32_t* page_table,
                                     int32_t* context_lens, vrm_stream_t stream) {
  const char* who = "vrm_build_block_table";
  if (B < 0 || max_pp < 0 || n_flat < 0) {
    set_error("%s: bad sizes (B=%d max_pp=%d n_flat=%d)", who, B, max_pp, n_flat);
    return VRM_ERR_ARG;
  }
  if (B > 65535) {
    set_error("%s: batch %d above 65535", who, B);
    return VRM_ERR_UNSUPPORTED;
  }
  if (B == 0) {
    clear_error();
    return VRM_OK;
  }
  if (!offsets || !num_tokens || !page_table || !context_lens || (n_flat > 0 && !flat_pages)) {
    set_error("%s: null pointer argument", who);
    return VRM_ERR_ARG;
  }
  const int bx = max_pp > 0 ? (max_pp + kTableThreads - 1) / kTableThreads : 1;
  hipLaunchKernelGGL(build_table_kernel, dim3(bx, B), dim3(kTableThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     flat_pages, n_flat, offsets, num_tokens, max_pp, page_table, context_lens);
  return launch_status(who);
}

extern "C" int vrm_kv_write(const void* key, const void* value, int src_dtype, const int32_t* page_ids,
                            const int32_t* slots, int N, void* kv_pool, int kv_dtype, int KH, int D, int PS, int L,
                            int P, int layer_idx, vrm_stream_t stream) {
  const char* who = "vrm_kv_write";
  if (N < 0 || KH <= 0 || D <= 0 || PS <= 0 || L <= 0 || P <= 0) {
    set_error("%s: bad sizes (N=%d KH=%d D=%d PS=%d L=%d P=%d)", who, N, KH, D, PS, L, P);
    return VRM_ERR_ARG;
  }
  if (layer_idx < 0 || layer_idx >= L) {
    set_error("%s: layer_idx %d outside [0, %d)", who, layer_idx, L);
    return VRM_ERR_ARG;
  }
  if (src_dtype != VRM_SRC_F32 && src_dtype != VRM_SRC_F16 && src_dtype != VRM_SRC_BF16) {
    set_error("%s: unknown source dtype %d", who, src_dtype);
    return VRM_ERR_ARG;
  }
  if (kv_dtype != VRM_KV_F32 && kv_dtype != VRM_KV_F16 && kv_dtype != VRM_KV_BF16) {
    set_error("%s: kv_dtype %d is not a float pool (quantized pools are written by vrm_kv_quant_append)", who,
              kv_dtype);
    return VRM_ERR_ARG;
  }
  if ((long long)N * 2 * KH > 0x7fffffffLL) {
    set_error("%s: too many rows (N=%d KH=%d)", who, N, KH);
    return VRM_ERR_UNSUPPORTED;
  }
  if (N == 0) {
    clear_error();
    return VRM_OK;
  }
  if (!key || !value || !page_ids || !slots || !kv_pool) {
    set_error("%s: null pointer argument", who);
    return VRM_ERR_ARG;
  }
  KvWriteArgs a{key, value, page_ids, slots, kv_pool, KH, D, PS, L, P, layer_idx};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int rows = N * 2 * KH;
  switch (src_dtype) {
    case VRM_SRC_F32: launch_kv_write<VRM_SRC_F32>(a, rows, kv_dtype, st); break;
    case VRM_SRC_F16: launch_kv_write<VRM_SRC_F16>(a, rows, kv_dtype, st); break;
    default: launch_kv_write<VRM_SRC_BF16>(a, rows, kv_dtype, st); break;
  }
  return launch_status(who);
}
