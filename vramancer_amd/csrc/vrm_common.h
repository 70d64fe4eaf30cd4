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

}  // namespace vrm
