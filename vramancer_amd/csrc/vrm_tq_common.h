// Helpers shared by the TurboQuant codec (vrm_turboquant.hip) and the
// generic TurboQuant decode (vrm_decode_tq_generic.hip): IEEE square root,
// fp16 rounding, the per-wavefront LDS ordering point and the in-register
// Walsh-Hadamard transform in the reference's butterfly order.
#pragma once
#include "vrm_common.h"

#include <math.h>

namespace vrm {
namespace {

// IEEE square root.  HIP's __fsqrt_rn is the approximate native v_sqrt_f32 in
// this toolchain; sqrtf lowers to the correctly rounded sequence (hipcc's
// default -fhip-fp32-correctly-rounded-divide-sqrt), as does '/'.
__device__ __forceinline__ float sqrt_rn(float x) { return sqrtf(x); }

template <int SRC>
__device__ __forceinline__ float load_row(const void* p, size_t i) {
  if constexpr (SRC == VRM_SRC_F32) {
    return static_cast<const float*>(p)[i];
  } else if constexpr (SRC == VRM_SRC_F16) {
    return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else {
    return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
  return __builtin_bit_cast(unsigned short, (_Float16)x);  // round to nearest even
}

// Each row of the codec belongs to one wavefront, whose LDS working set no
// other wavefront touches.  A wavefront's LDS operations complete in program
// order, so a wavefront-scope fence is what orders one lane's LDS writes
// before another lane's later reads: no s_barrier, and workgroups can carry
// several rows whose wavefronts never wait for each other.
__device__ __forceinline__ void row_sync() { __syncwarp(); }

// Registers per lane of a PD-element row spread as element e -> (lane e % 64,
// register e / 64); below 64 elements lanes PD .. 63 hold nothing of the row.
constexpr int tq_per_lane(int pd) { return (pd + 63) / 64; }

// In-register Walsh-Hadamard transform of a PD-element row spread as above;
// same butterfly order as the reference.  For PD < 64 the lanes past the row
// exchange among themselves only (lane ^ h < PD for lane < PD), and their
// values are never used.
template <int PD>
__device__ __forceinline__ void fwht(float (&v)[tq_per_lane(PD)], int lane) {
  constexpr int PER = tq_per_lane(PD);
#pragma unroll
  for (int h = 1; h < PD; h <<= 1) {
    if (h < 64) {
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        float other;
        switch (h) {
          case 1: other = xor_shfl<1>(v[k]); break;
          case 2: other = xor_shfl<2>(v[k]); break;
          case 4: other = xor_shfl<4>(v[k]); break;
          case 8: other = xor_shfl<8>(v[k]); break;
          case 16: other = xor_shfl<16>(v[k]); break;
          default: other = xor_shfl<32>(v[k]); break;
        }
        // lower element keeps a + b, upper keeps a - b with a = lower, b = upper
        v[k] = (lane & h) ? __fsub_rn(other, v[k]) : __fadd_rn(v[k], other);
      }
    } else {
      const int rh = h / 64;
      float nv[PER];
#pragma unroll
      for (int k = 0; k < PER; ++k) nv[k] = (k & rh) ? __fsub_rn(v[k ^ rh], v[k]) : __fadd_rn(v[k], v[k ^ rh]);
#pragma unroll
      for (int k = 0; k < PER; ++k) v[k] = nv[k];
    }
  }
}

}  // namespace
}  // namespace vrm
