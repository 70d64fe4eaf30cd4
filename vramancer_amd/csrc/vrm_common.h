// Shared helpers for the gfx950 kernels of libvrm_paged.so: error reporting,
// argument checks and the few wave-level primitives the kernels use.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vrm_paged.h"
#include "vrm_e4m3.h"

namespace vrm {

// Stores a printf-formatted message as the thread's last error.
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Converts the launch status of the last kernel into the ABI status.
int launch_status(const char* what);

constexpr int kWave = 64;

// Butterfly exchange across lanes lane ^ mask of a 64-wide wavefront.
// ds_swizzle covers masks below 32 within each 32-lane half; mask 32 crosses
// halves and uses ds_bpermute.
template <int MASK>
__device__ __forceinline__ float xor_shfl(float v) {
  static_assert(MASK > 0 && MASK < 64 && (MASK & (MASK - 1)) == 0, "power-of-two mask");
  if constexpr (MASK < 32) {
    // ds_swizzle bit mode: and_mask = 0x1f, or_mask = 0, xor_mask = MASK.
    constexpr int pattern = 0x1f | (MASK << 10);
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), pattern));
  } else {
    const int lane = __lane_id();
    return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ MASK) << 2, __float_as_int(v)));
  }
}

// Sum over the aligned group of N lanes (N a power of two <= 64) that
// contains this lane; every lane of the group receives the total.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (N >= 2) v += xor_shfl<1>(v);
  if constexpr (N >= 4) v += xor_shfl<2>(v);
  if constexpr (N >= 8) v += xor_shfl<4>(v);
  if constexpr (N >= 16) v += xor_shfl<8>(v);
  if constexpr (N >= 32) v += xor_shfl<16>(v);
  if constexpr (N >= 64) v += xor_shfl<32>(v);
  return v;
}

template <int N>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (N >= 2) v = fmaxf(v, xor_shfl<1>(v));
  if constexpr (N >= 4) v = fmaxf(v, xor_shfl<2>(v));
  if constexpr (N >= 8) v = fmaxf(v, xor_shfl<4>(v));
  if constexpr (N >= 16) v = fmaxf(v, xor_shfl<8>(v));
  if constexpr (N >= 32) v = fmaxf(v, xor_shfl<16>(v));
  if constexpr (N >= 64) v = fmaxf(v, xor_shfl<32>(v));
  return v;
}

// Sum over lanes that share (lane mod STRIDE): butterflies with masks
// STRIDE, 2*STRIDE, ..., 32.
template <int STRIDE>
__device__ __forceinline__ float strided_sum(float v) {
  if constexpr (STRIDE <= 1) v += xor_shfl<1>(v);
  if constexpr (STRIDE <= 2) v += xor_shfl<2>(v);
  if constexpr (STRIDE <= 4) v += xor_shfl<4>(v);
  if constexpr (STRIDE <= 8) v += xor_shfl<8>(v);
  if constexpr (STRIDE <= 16) v += xor_shfl<16>(v);
  if constexpr (STRIDE <= 32) v += xor_shfl<32>(v);
  return v;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}

// OCP e4m3fn byte -> float32 (exact); shared with the host tests.
__device__ __forceinline__ float e4m3fn_to_f32(uint32_t b) { return vrm_e4m3::decode(b); }

// Where a pool keeps the codes and scales of (page, layer, K/V, kv-head):
// the codes of that slice start at pool + page * this->page + layer *
// this->layer + kvh * head + kv * this->kv bytes, its scales at scales + page
// * s_page + layer * s_layer + kvh * s_head + kv * s_kv floats (then one per
// token for int8).  Plain pools are the dense [P][L][2][KH][PS][row] arrays
// (and, for int8 / fp8, a separate dense scale array): a page's slabs of all
// layers lie together.  The inline int8 / fp8 layout keeps a kv-head's codes
// and scales in the (page, layer) slab (inline_scale_offset below), the scale
// pointer then pointing into the first slab, and lays the slabs out layer by
// layer: the P slabs of one layer are one contiguous run.
struct PoolGeom {
  long long slab;     // pool bytes per (page, layer)
  long long head;     // bytes from one kv-head's code slices to the next one's
  long long kv;       // bytes from a kv-head's K codes to its V codes
  long long s_slab;   // scale floats per (page, layer)
  long long s_head;   // scale floats from one kv-head to the next
  long long s_kv;     // scale floats from a kv-head's K scales to its V scales
  long long page;     // bytes from a (page, layer) slab to the next page's of the layer
  long long layer;    // bytes from a (page, layer) slab to the next layer's of the page
  long long s_page;   // the same two strides in scale floats
  long long s_layer;
};

inline bool inline_pool(int kv_dtype) { return kv_dtype == VRM_KV_I8_INLINE || kv_dtype == VRM_KV_FP8E4M3_INLINE; }

// Inline slabs hold per kv-head a record of its K and V codes followed by
// its K and V scales: int8 PS each (PS (2 D + 8) bytes in all), fp8 one each,
// the record padded to 2 PS D + 128 bytes so that every kv-head's codes start
// on a 128-byte line.  The first record's scales are 2 PS D bytes into the
// pool.
inline long long inline_scale_offset(int PS, int D) { return 2LL * PS * D; }

// Geometry of a pool of P pages and L layers of kv_dtype whose token rows
// hold row_bytes bytes (D codes, D / 2 for the 4-bit pool, D elements of a
// float pool).
inline PoolGeom pool_geom(int kv_dtype, int KH, int PS, int D, long long row_bytes, int P, int L) {
  PoolGeom g{};
  const bool fp8 = kv_dtype == VRM_KV_FP8E4M3 || kv_dtype == VRM_KV_FP8E4M3_INLINE;
  const long long slice = (long long)PS * row_bytes;
  if (inline_pool(kv_dtype)) {
    g.kv = slice;
    if (fp8) {
      g.head = 2 * slice + 128;
      g.slab = KH * g.head;
      g.s_head = g.head / 4;
      g.s_kv = 1;
    } else {
      g.head = 2 * slice + 8LL * PS;
      g.slab = KH * g.head;
      g.s_head = g.head / 4;
      g.s_kv = PS;
    }
    g.s_slab = g.slab / 4;
    g.page = g.slab;
    g.layer = (long long)P * g.slab;
    g.s_page = g.s_slab;
    g.s_layer = (long long)P * g.s_slab;
  } else {
    g.head = slice;
    g.kv = KH * slice;
    g.slab = 2 * g.kv;
    const long long per_head = fp8 ? 1 : PS;  // int8: one scale per token; fp8: one per page
    g.s_head = per_head;
    g.s_kv = KH * per_head;
    g.s_slab = 2 * g.s_kv;
    g.page = (long long)L * g.slab;
    g.layer = g.slab;
    g.s_page = (long long)L * g.s_slab;
    g.s_layer = g.s_slab;
  }
  return g;
}

// An inline pool's scales sit inline_scale_offset() bytes past its codes; a
// plain pool's are a separate array (one that starts inside the codes is an
// inline buffer passed with the plain dtype, refused rather than misread or
// overwritten).
inline int check_pool_scales(int kv_dtype, const void* kv_pool, const void* kv_scales, int KH, int PS, int D, int L,
                             int P, const char* who) {
  const char* pool = static_cast<const char*>(kv_pool);
  const char* sc = static_cast<const char*>(kv_scales);
  if (inline_pool(kv_dtype)) {
    const long long off = inline_scale_offset(PS, D);
    if (sc != pool + off) {
      set_error("%s: an inline pool's kv_scales must point %lld bytes past kv_pool", who, off);
      return VRM_ERR_ARG;
    }
  } else if (sc && sc >= pool && sc < pool + (long long)P * L * 2 * KH * PS * D) {
    set_error("%s: kv_scales points inside the codes of a plain pool (an inline pool needs the inline kv_dtype)",
              who);
    return VRM_ERR_ARG;
  }
  return VRM_OK;
}

}  // namespace vrm
