// TurboQuant codec (randomized Hadamard rotation + PolarQuant angles + QJL
// residual signs) for gfx950.
//
// The contract is the reference's CPU path, KVCacheCompressor.compress /
// decompress (core/kv_quantizer.py:240-324, 391-417, 481-500), evaluated
// operation by operation in IEEE binary32 so that the codes come out
// bit-identical:
//   rotate   x * signs, Walsh-Hadamard butterflies h = 1, 2, 4, ... with
//            (a + b, a - b), then a true division by (float)sqrt(pd);
//   encode   per level r = sqrt((a*a + b*b) + 1e-12f), theta = atan2(b, a)
//            with the C library's float atan2 (see vrm_fdlibm_atan2f.h);
//   bin      trunc(((theta - lo) / (hi - lo)) * 2^bits) clamped;
//   decode   from the fp32 radius with the {cos, sin} of the bin centres
//            (a host-built table, since the reference's values come from
//            PyTorch's CPU sin/cos);
//   QJL      sign(residual . jl_j) accumulated in float64 (the reference's
//            BLAS order is unknown; ties within its rounding are documented);
//            norm with eight interleaved fused accumulators summed in order,
//            which is how PyTorch's CPU 2-norm kernel reduces a 128-float row.
// One 64-lane wavefront per row; the row lives in LDS between stages.
#include "vrm_common.h"
#include "vrm_fdlibm_atan2f.h"

#include <math.h>

namespace vrm {
namespace {

#pragma clang fp contract(off)

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

// In-register Walsh-Hadamard transform of a PD-element row spread as element
// e -> (lane e % 64, register e / 64); same butterfly order as the reference.
template <int PD>
__device__ __forceinline__ void fwht(float (&v)[PD / 64], int lane) {
  constexpr int PER = PD / 64;
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

struct TqArgs {
  const void* kv;
  int N, head_dim, bits, qjl_dim;
  const float* signs;
  const float* jl;
  const float* lut;  // [2 level kinds][cos, sin][2^bits]
  uint16_t* radius;
  uint8_t* angles;
  uint8_t* qjl_signs;
  uint16_t* qjl_norms;
  float* out;        // decompress output
};

// Polar decode of one row into `recon` (LDS, PD floats) from the fp32 radius
// and the level-major bins in `bins`.  Levels run from the top (one angle)
// down to level 0, interleaving (r cos, r sin) pairs.
template <int PD>
__device__ __forceinline__ void polar_decode(float radius, const uint8_t* bins, const float* lut, int nb,
                                             float* bufA, float* bufB, float* recon, int lane) {
  constexpr int NL = __builtin_ctz(PD);
  float* cur = bufA;
  float* nxt = bufB;
  if (lane == 0) cur[0] = radius;
  __syncthreads();
  // level_offset(l) = sum_{i<l} PD >> (i + 1) = PD - (PD >> l)
  for (int level = NL - 1; level >= 0; --level) {
    const int count = PD >> (level + 1);
    const int off = PD - (PD >> level);
    const float* cos_t = lut + (level == 0 ? 0 : 2 * nb);
    const float* sin_t = cos_t + nb;
    float* dst = level == 0 ? recon : nxt;
    for (int i = lane; i < count; i += 64) {
      const int idx = min((int)bins[off + i], nb - 1);  // caller-supplied bins stay inside the table
      const float r = cur[i];
      dst[2 * i] = __fmul_rn(r, cos_t[idx]);
      dst[2 * i + 1] = __fmul_rn(r, sin_t[idx]);
    }
    __syncthreads();
    float* t = cur;
    cur = nxt;
    nxt = t;
  }
}

template <int SRC, int PD>
__global__ void __launch_bounds__(64) tq_compress_kernel(TqArgs a) {
  constexpr int PER = PD / 64;
  constexpr int NL = __builtin_ctz(PD);
  __shared__ float rot[PD];
  __shared__ float bufA[PD / 2];
  __shared__ float bufB[PD / 2];
  __shared__ float recon[PD];
  __shared__ uint8_t bins[PD];
  __shared__ float norm_acc[8];

  const int lane = threadIdx.x;
  const int row = blockIdx.x;
  const int nb = 1 << a.bits;

  // ---- rotate ----
  float v[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int e = k * 64 + lane;
    const float x = e < a.head_dim ? load_row<SRC>(a.kv, (size_t)row * a.head_dim + e) : 0.f;
    v[k] = __fmul_rn(x, a.signs[e]);
  }
  fwht<PD>(v, lane);
  const float root = (float)sqrt((double)PD);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    v[k] = __fdiv_rn(v[k], root);
    rot[k * 64 + lane] = v[k];
  }
  __syncthreads();

  // ---- polar encode + bin ----
  const float lo0 = (float)-3.141592653589793, range0 = (float)6.283185307179586;
  const float range1 = (float)1.5707963267948966;
  const float nbf = (float)nb;
  const float* cur = rot;
  float* nxt = bufA;
  for (int level = 0; level < NL; ++level) {
    const int count = PD >> (level + 1);
    const int off = PD - (PD >> level);
    for (int i = lane; i < count; i += 64) {
      const float x0 = cur[2 * i], x1 = cur[2 * i + 1];
      const float r = sqrt_rn(__fadd_rn(__fadd_rn(__fmul_rn(x0, x0), __fmul_rn(x1, x1)), 1e-12f));
      const float th = vrm_fdlibm::atan2f(x1, x0);
      float nrm = level == 0 ? __fdiv_rn(__fsub_rn(th, lo0), range0) : __fdiv_rn(th, range1);
      int idx = (int)__fmul_rn(nrm, nbf);  // truncation toward zero, as .long()
      idx = min(max(idx, 0), nb - 1);
      bins[off + i] = (uint8_t)idx;
      a.angles[(size_t)row * (PD - 1) + off + i] = (uint8_t)idx;
      nxt[i] = r;
    }
    __syncthreads();
    cur = nxt;
    nxt = (nxt == bufA) ? bufB : bufA;
  }
  const float radius = cur[0];
  if (lane == 0) a.radius[row] = f32_to_f16_bits(radius);

  // ---- reconstruct from the fp32 radius, residual ----
  polar_decode<PD>(radius, bins, a.lut, nb, bufA, bufB, recon, lane);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int e = k * 64 + lane;
    rot[e] = __fsub_rn(v[k], recon[e]);  // rot now holds the residual
  }
  __syncthreads();

  // ---- QJL signs (float64 dot) ----
  for (int j = lane; j < a.qjl_dim; j += 64) {
    const float* jr = a.jl + (size_t)j * PD;
    double s = 0.0;
    for (int e = 0; e < PD; ++e) s = fma((double)rot[e], (double)jr[e], s);
    a.qjl_signs[(size_t)row * a.qjl_dim + j] = s > 0.0 ? 1 : 0;
  }
  // ---- residual norm: 8 interleaved fused accumulators, summed in order ----
  if (lane < 8) {
    float acc = 0.f;
    for (int e = lane; e < PD; e += 8) acc = fmaf(rot[e], rot[e], acc);
    norm_acc[lane] = acc;
  }
  __syncthreads();
  if (lane == 0) {
    float s = norm_acc[0];
#pragma unroll
    for (int k = 1; k < 8; ++k) s = __fadd_rn(s, norm_acc[k]);
    a.qjl_norms[row] = f32_to_f16_bits(sqrt_rn(s));
  }
}

template <int PD>
__global__ void __launch_bounds__(64) tq_decompress_kernel(TqArgs a, int rotated) {
  constexpr int PER = PD / 64;
  __shared__ float bufA[PD / 2];
  __shared__ float bufB[PD / 2];
  __shared__ float recon[PD];
  __shared__ uint8_t bins[PD];
  const int lane = threadIdx.x;
  const int row = blockIdx.x;
  const int nb = 1 << a.bits;
  for (int i = lane; i < PD - 1; i += 64) bins[i] = a.angles[(size_t)row * (PD - 1) + i];
  const float radius = f16_bits_to_f32(a.radius[row]);
  __syncthreads();
  polar_decode<PD>(radius, bins, a.lut, nb, bufA, bufB, recon, lane);
  float v[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) v[k] = recon[k * 64 + lane];
  if (rotated) {
#pragma unroll
    for (int k = 0; k < PER; ++k) a.out[(size_t)row * PD + k * 64 + lane] = v[k];
    return;
  }
  fwht<PD>(v, lane);
  const float root = (float)sqrt((double)PD);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int e = k * 64 + lane;
    const float y = __fmul_rn(__fdiv_rn(v[k], root), a.signs[e]);
    if (e < a.head_dim) a.out[(size_t)row * a.head_dim + e] = y;
  }
}

int check_tq(int N, int head_dim, int padded_dim, int n_levels, int bits, const char* who) {
  if (N < 0 || head_dim <= 0 || head_dim > padded_dim) {
    set_error("%s: bad sizes (N=%d head_dim=%d padded_dim=%d)", who, N, head_dim, padded_dim);
    return VRM_ERR_ARG;
  }
  if (padded_dim != 64 && padded_dim != 128 && padded_dim != 256) {
    set_error("%s: padded_dim %d unsupported (64, 128, 256)", who, padded_dim);
    return VRM_ERR_UNSUPPORTED;
  }
  if ((1 << n_levels) != padded_dim) {
    set_error("%s: n_levels %d does not match padded_dim %d", who, n_levels, padded_dim);
    return VRM_ERR_ARG;
  }
  if (bits < 1 || bits > 8) {
    set_error("%s: bits_per_angle %d outside [1, 8]", who, bits);
    return VRM_ERR_ARG;
  }
  return VRM_OK;
}

}  // namespace
}  // namespace vrm

using namespace vrm;

extern "C" int vrm_turboquant_compress(const void* kv, int src_dtype, int N, int head_dim, int padded_dim,
                                       int n_levels, int bits, int qjl_dim, const float* signs, const float* jl,
                                       const float* angle_lut, uint16_t* radius, uint8_t* angles,
                                       uint8_t* qjl_signs, uint16_t* qjl_norms, vrm_stream_t stream) {
  const char* who = "vrm_turboquant_compress";
  int rc = check_tq(N, head_dim, padded_dim, n_levels, bits, who);
  if (rc) return rc;
  if (qjl_dim <= 0 || qjl_dim > 4 * padded_dim) {
    set_error("%s: qjl_dim %d outside [1, %d]", who, qjl_dim, 4 * padded_dim);
    return VRM_ERR_ARG;
  }
  if (src_dtype != VRM_SRC_F32 && src_dtype != VRM_SRC_F16 && src_dtype != VRM_SRC_BF16) {
    set_error("%s: unknown source dtype %d", who, src_dtype);
    return VRM_ERR_ARG;
  }
  if (N == 0) return VRM_OK;
  if (!kv || !signs || !jl || !angle_lut || !radius || !angles || !qjl_signs || !qjl_norms) {
    set_error("%s: null pointer argument", who);
    return VRM_ERR_ARG;
  }
  TqArgs a{};
  a.kv = kv;
  a.N = N;
  a.head_dim = head_dim;
  a.bits = bits;
  a.qjl_dim = qjl_dim;
  a.signs = signs;
  a.jl = jl;
  a.lut = angle_lut;
  a.radius = radius;
  a.angles = angles;
  a.qjl_signs = qjl_signs;
  a.qjl_norms = qjl_norms;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define VRM_TQ_LAUNCH(SRC, PDV) \
  hipLaunchKernelGGL((tq_compress_kernel<SRC, PDV>), dim3(N), dim3(64), 0, st, a)
#define VRM_TQ_PD(SRC)                                  \
  switch (padded_dim) {                                 \
    case 64: VRM_TQ_LAUNCH(SRC, 64); break;             \
    case 128: VRM_TQ_LAUNCH(SRC, 128); break;           \
    default: VRM_TQ_LAUNCH(SRC, 256); break;            \
  }
  switch (src_dtype) {
    case VRM_SRC_F32: VRM_TQ_PD(VRM_SRC_F32); break;
    case VRM_SRC_F16: VRM_TQ_PD(VRM_SRC_F16); break;
    default: VRM_TQ_PD(VRM_SRC_BF16); break;
  }
#undef VRM_TQ_PD
#undef VRM_TQ_LAUNCH
  return launch_status(who);
}

extern "C" int vrm_turboquant_decompress(const uint16_t* radius, const uint8_t* angles, int N, int head_dim,
                                         int padded_dim, int n_levels, int bits, const float* signs,
                                         const float* angle_lut, float* out, int rotated, vrm_stream_t stream) {
  const char* who = "vrm_turboquant_decompress";
  int rc = check_tq(N, head_dim, padded_dim, n_levels, bits, who);
  if (rc) return rc;
  if (N == 0) return VRM_OK;
  if (!radius || !angles || !signs || !angle_lut || !out) {
    set_error("%s: null pointer argument", who);
    return VRM_ERR_ARG;
  }
  TqArgs a{};
  a.N = N;
  a.head_dim = head_dim;
  a.bits = bits;
  a.signs = signs;
  a.lut = angle_lut;
  a.radius = const_cast<uint16_t*>(radius);
  a.angles = const_cast<uint8_t*>(angles);
  a.out = out;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (padded_dim) {
    case 64: hipLaunchKernelGGL(tq_decompress_kernel<64>, dim3(N), dim3(64), 0, st, a, rotated); break;
    case 128: hipLaunchKernelGGL(tq_decompress_kernel<128>, dim3(N), dim3(64), 0, st, a, rotated); break;
    default: hipLaunchKernelGGL(tq_decompress_kernel<256>, dim3(N), dim3(64), 0, st, a, rotated); break;
  }
  return launch_status(who);
}
