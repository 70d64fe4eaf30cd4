// Quantize-on-append for the int8 and fp8-e4m3 paged pools, bulk page writes
// (prefill) and page dequantization.
//
// The reference writes raw K/V rows with an index-put
// (core/paged_attention.py:611-612, pool[page, layer, 0|1, :, slot, :] = k|v)
// and has no int8/fp8 codec; the codecs here are this library's definitions:
//   int8: per (token, head) scale = amax / 127, code = clamp(rne(x / scale), +-127)
//   fp8 : per (page, head) scale = amax / 448, code = e4m3fn_rne(x / scale)
// Divisions are IEEE round-to-nearest so codes are bit-identical to the same
// formulas evaluated with PyTorch on the CPU.
//
// Layout of a quantized (page, layer, K/V, head) slice of PS x D codes: K is
// token-major (code of token t, dim d at t * D + d, as the reference's pool);
// V is tiled, code of token t, dim d at
//   ((t / 4 * 16 + d % 16) * (D / 16) + d / 16) * 4 + t % 4,
// so that a decode lane finds the 4 tokens of its MFMA k-slice for the dims
// col, col + 16, ... of its operand row in D / 4 consecutive bytes.
#include "vrm_common.h"

#include <math.h>

namespace vrm {
namespace {

bool quant_pool(int kv_dtype) {
  return kv_dtype == VRM_KV_I8 || kv_dtype == VRM_KV_FP8E4M3 || inline_pool(kv_dtype);
}
bool fp8_pool(int kv_dtype) { return kv_dtype == VRM_KV_FP8E4M3 || kv_dtype == VRM_KV_FP8E4M3_INLINE; }


template <int SRC>
__device__ __forceinline__ float load_src(const void* p, size_t i) {
  if constexpr (SRC == VRM_SRC_F32) {
    return static_cast<const float*>(p)[i];
  } else if constexpr (SRC == VRM_SRC_F16) {
    return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else {
    return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
}

__device__ __forceinline__ int8_t int8_code(float x, float scale) {
  if (!(scale > 0.f)) return 0;
  float r = rintf(__fdiv_rn(x, scale));
  r = fminf(fmaxf(r, -127.f), 127.f);
  return (int8_t)(int)r;
}

__device__ __forceinline__ uint8_t fp8_code(float x, float scale) {
  if (!(scale > 0.f)) return 0;
  return vrm_e4m3::encode(__fdiv_rn(x, scale));
}

struct QuantArgs {
  const void* key;
  const void* value;
  const int32_t* page_ids;
  const int32_t* slots;    // append: slot of each token; pages: valid tokens per page
  uint8_t* pool;
  float* scales;
  int KH, L, P, layer;
  int D, PS;               // head_dim (multiple of 16, <= 256) and page size (multiple of 4)
  PoolGeom g;              // plain or inline layout of codes and scales
};

// Codes of the (page, layer, K/V, kv-head) slice and its scales (int8: PS of
// them, one per token; fp8: one).
__device__ __forceinline__ uint8_t* slice_of(const QuantArgs& a, int pid, int kv, int h) {
  return a.pool + (size_t)pid * a.g.page + (size_t)a.layer * a.g.layer + (size_t)h * a.g.head + (size_t)kv * a.g.kv;
}
__device__ __forceinline__ float* scales_of(const QuantArgs& a, int pid, int kv, int h) {
  return a.scales + (size_t)pid * a.g.s_page + (size_t)a.layer * a.g.s_layer + (size_t)h * a.g.s_head +
         (size_t)kv * a.g.s_kv;
}

// Offset of (token t, dim d) inside a slice: K token-major, V tiled.
__device__ __forceinline__ int code_offset(int kv, int t, int d, int D) {
  return kv ? (((t >> 2) * 16 + (d & 15)) * (D >> 4) + (d >> 4)) * 4 + (t & 3) : t * D + d;
}

// int8, one wavefront per (token row, K/V, head).  src rows: [N][KH][D]
// (append) or [NP][KH][PS][D] (pages).  DMAX = 64, 128 or 256 >= D.
template <int SRC, int DMAX, bool PAGES>
__global__ void __launch_bounds__(64) quant_i8_kernel(QuantArgs a) {
  constexpr int PER = DMAX / 64;
  const int D = a.D, PS = a.PS;
  const int lane = threadIdx.x;
  const int kv = blockIdx.x / a.KH, h = blockIdx.x % a.KH;
  const int n = blockIdx.y;
  const int t = PAGES ? blockIdx.z : 0;
  const int pid = a.page_ids[n];
  const int slot = PAGES ? t : a.slots[n];
  if (pid < 0 || pid >= a.P || slot < 0 || slot >= PS) return;
  const bool valid = PAGES ? (t < a.slots[n]) : true;
  const void* src = kv ? a.value : a.key;
  const size_t row = PAGES ? (((size_t)n * a.KH + h) * PS + t) * D : ((size_t)n * a.KH + h) * D;
  float x[PER];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = i * 64 + lane;
    x[i] = (valid && d < D) ? load_src<SRC>(src, row + d) : 0.f;
    amax = fmaxf(amax, fabsf(x[i]));
  }
  amax = group_max<64>(amax);
  const float scale = __fdiv_rn(amax, 127.f);
  int8_t* dst = reinterpret_cast<int8_t*>(slice_of(a, pid, kv, h));
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = i * 64 + lane;
    if (d < D) dst[code_offset(kv, slot, d, D)] = int8_code(x[i], scale);
  }
  if (lane == 0) scales_of(a, pid, kv, h)[slot] = scale;
}

// fp8 whole pages, one 256-thread workgroup per (page, K/V, head): the page
// maximum over its valid tokens, then the codes (the source is read twice).
template <int SRC>
__global__ void __launch_bounds__(256) quant_fp8_pages_kernel(QuantArgs a) {
  const int D = a.D, PS = a.PS;
  const int N = PS * D;
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int kv = blockIdx.x / a.KH, h = blockIdx.x % a.KH;
  const int n = blockIdx.y;
  const int pid = a.page_ids[n];
  if (pid < 0 || pid >= a.P) return;
  const int n_valid = min(max(a.slots[n], 0), PS);
  const void* src = kv ? a.value : a.key;
  const size_t base = ((size_t)n * a.KH + h) * N;
  float amax = 0.f;
  for (int idx = tid; idx < n_valid * D; idx += 256) amax = fmaxf(amax, fabsf(load_src<SRC>(src, base + idx)));
  amax = group_max<64>(amax);
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float scale = __fdiv_rn(amax, 448.f);
  uint8_t* dst = slice_of(a, pid, kv, h);
  for (int idx = tid; idx < N; idx += 256) {
    const int t = idx / D, d = idx - t * D;
    dst[code_offset(kv, t, d, D)] = t < n_valid ? fp8_code(load_src<SRC>(src, base + idx), scale) : (uint8_t)0;
  }
  if (tid == 0) *scales_of(a, pid, kv, h) = scale;
}

// fp8 append, one 256-thread workgroup per (token, K/V, head).  The page
// scale only grows; when it does, the codes already in the page are
// re-encoded against the new scale.
template <int SRC>
__global__ void __launch_bounds__(256) quant_fp8_append_kernel(QuantArgs a) {
  const int D = a.D, PS = a.PS;  // D <= 256: one element per thread
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int kv = blockIdx.x / a.KH, h = blockIdx.x % a.KH;
  const int n = blockIdx.y;
  const int pid = a.page_ids[n];
  const int slot = a.slots[n];
  if (pid < 0 || pid >= a.P || slot < 0 || slot >= PS) return;
  const void* src = kv ? a.value : a.key;
  const size_t row = ((size_t)n * a.KH + h) * D;
  const float x = tid < D ? load_src<SRC>(src, row + tid) : 0.f;
  float amax = group_max<64>(fabsf(x));
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  float* const sp = scales_of(a, pid, kv, h);
  // Every thread reads the old scale before the barrier; thread 0 overwrites it after.
  const float old_scale = slot > 0 ? *sp : 0.f;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float want = __fdiv_rn(amax, 448.f);
  const float scale = fmaxf(old_scale, want);
  uint8_t* page = slice_of(a, pid, kv, h);
  if (slot > 0 && scale > old_scale) {
    for (int idx = tid; idx < slot * D; idx += 256) {
      const int off = code_offset(kv, idx / D, idx % D, D);
      const float y = e4m3fn_to_f32(page[off]) * old_scale;
      page[off] = fp8_code(y, scale);
    }
  }
  if (tid < D) page[code_offset(kv, slot, tid, D)] = fp8_code(x, scale);
  if (tid == 0) *sp = scale;
}

// Dequantize pages: out[n][2][KH][PS][D] float32.
template <bool FP8>
__global__ void __launch_bounds__(256) dequant_pages_kernel(QuantArgs a, float* out, int D) {
  const int kv = blockIdx.x / a.KH, h = blockIdx.x % a.KH;
  const int n = blockIdx.y;
  const int pid = a.page_ids[n];
  const size_t N = (size_t)a.PS * D;
  float* o = out + (((size_t)n * 2 + kv) * a.KH + h) * N;
  if (pid < 0 || pid >= a.P) {
    for (size_t i = threadIdx.x; i < N; i += 256) o[i] = 0.f;
    return;
  }
  const uint8_t* codes = slice_of(a, pid, kv, h);
  const float* sc = scales_of(a, pid, kv, h);
  for (size_t i = threadIdx.x; i < N; i += 256) {
    const int t = (int)(i / D), d = (int)(i % D);
    const uint8_t c = codes[code_offset(kv, t, d, D)];
    if (FP8) {
      o[i] = e4m3fn_to_f32(c) * sc[0];
    } else {
      o[i] = (float)(int8_t)c * sc[t];
    }
  }
}

int check_quant(const void* key, const void* value, int src_dtype, const int32_t* page_ids, const int32_t* slots,
                int n, void* pool, float* scales, int kv_dtype, int KH, int D, int PS, int L, int P, int layer,
                const char* who) {
  if (!key || !value || !page_ids || !slots || !pool || !scales) {
    set_error("%s: null pointer argument", who);
    return VRM_ERR_ARG;
  }
  if (n < 0 || KH <= 0 || D <= 0 || L <= 0 || P <= 0) {
    set_error("%s: bad sizes (N=%d KH=%d D=%d L=%d P=%d)", who, n, KH, D, L, P);
    return VRM_ERR_ARG;
  }
  if (layer < 0 || layer >= L) {
    set_error("%s: layer_idx %d outside [0, %d)", who, layer, L);
    return VRM_ERR_ARG;
  }
  if (src_dtype != VRM_SRC_F32 && src_dtype != VRM_SRC_F16 && src_dtype != VRM_SRC_BF16) {
    set_error("%s: unknown source dtype %d", who, src_dtype);
    return VRM_ERR_ARG;
  }
  if (!quant_pool(kv_dtype)) {
    set_error("%s: kv_dtype %d is not a quantized pool", who, kv_dtype);
    return VRM_ERR_ARG;
  }
  if (PS <= 0 || PS % 4 || PS > 65535) {
    set_error("%s: page_size %d unsupported (a positive multiple of 4)", who, PS);
    return VRM_ERR_UNSUPPORTED;
  }
  if (D % 16 || D > 256) {
    set_error("%s: head_dim %d unsupported (a multiple of 16 up to 256)", who, D);
    return VRM_ERR_UNSUPPORTED;
  }
  if (n > 65535 || 2 * KH > 65535) {
    set_error("%s: too many rows in one call (%d)", who, n);
    return VRM_ERR_UNSUPPORTED;
  }
  return check_pool_scales(kv_dtype, pool, scales, KH, PS, D, L, P, who);
}

template <int SRC, int DMAX>
void launch_quant(const QuantArgs& a, int n, int kv_dtype, bool pages, hipStream_t st) {
  if (!fp8_pool(kv_dtype)) {
    if (pages)
      hipLaunchKernelGGL((quant_i8_kernel<SRC, DMAX, true>), dim3(2 * a.KH, n, a.PS), dim3(64), 0, st, a);
    else
      hipLaunchKernelGGL((quant_i8_kernel<SRC, DMAX, false>), dim3(2 * a.KH, n, 1), dim3(64), 0, st, a);
  } else {
    if (pages)
      hipLaunchKernelGGL((quant_fp8_pages_kernel<SRC>), dim3(2 * a.KH, n), dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((quant_fp8_append_kernel<SRC>), dim3(2 * a.KH, n), dim3(256), 0, st, a);
  }
}

template <int SRC>
void launch_quant_d(const QuantArgs& a, int n, int kv_dtype, bool pages, int D, hipStream_t st) {
  if (D <= 64)
    launch_quant<SRC, 64>(a, n, kv_dtype, pages, st);
  else if (D <= 128)
    launch_quant<SRC, 128>(a, n, kv_dtype, pages, st);
  else
    launch_quant<SRC, 256>(a, n, kv_dtype, pages, st);
}

int run_quant(const void* key, const void* value, int src_dtype, const int32_t* page_ids, const int32_t* slots,
              int n, void* pool, float* scales, int kv_dtype, int KH, int D, int PS, int L, int P, int layer,
              bool pages, vrm_stream_t stream, const char* who) {
  int rc = check_quant(key, value, src_dtype, page_ids, slots, n, pool, scales, kv_dtype, KH, D, PS, L, P, layer, who);
  if (rc) return rc;
  if (n == 0) {
    clear_error();
    return VRM_OK;
  }
  QuantArgs a{key, value, page_ids, slots, static_cast<uint8_t*>(pool), scales, KH, L, P, layer, D, PS,
              pool_geom(kv_dtype, KH, PS, D, D, P, L)};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (src_dtype) {
    case VRM_SRC_F32: launch_quant_d<VRM_SRC_F32>(a, n, kv_dtype, pages, D, st); break;
    case VRM_SRC_F16: launch_quant_d<VRM_SRC_F16>(a, n, kv_dtype, pages, D, st); break;
    default: launch_quant_d<VRM_SRC_BF16>(a, n, kv_dtype, pages, D, st); break;
  }
  return launch_status(who);
}

}  // namespace
}  // namespace vrm

using namespace vrm;

extern "C" int vrm_kv_quant_append(const void* key, const void* value, int src_dtype, const int32_t* page_ids,
                                   const int32_t* slots, int N, void* kv_pool, float* kv_scales, int kv_dtype,
                                   int KH, int D, int PS, int L, int P, int layer_idx, vrm_stream_t stream) {
  return run_quant(key, value, src_dtype, page_ids, slots, N, kv_pool, kv_scales, kv_dtype, KH, D, PS, L, P,
                   layer_idx, false, stream, "vrm_kv_quant_append");
}

extern "C" int vrm_kv_quant_pages(const void* key, const void* value, int src_dtype, const int32_t* page_ids,
                                  const int32_t* n_valid, int NP, void* kv_pool, float* kv_scales, int kv_dtype,
                                  int KH, int D, int PS, int L, int P, int layer_idx, vrm_stream_t stream) {
  return run_quant(key, value, src_dtype, page_ids, n_valid, NP, kv_pool, kv_scales, kv_dtype, KH, D, PS, L, P,
                   layer_idx, true, stream, "vrm_kv_quant_pages");
}

extern "C" int vrm_kv_dequant_pages(const void* kv_pool, const float* kv_scales, int kv_dtype, const int32_t* page_ids,
                                    int NP, float* out, int KH, int D, int PS, int L, int P, int layer_idx,
                                    vrm_stream_t stream) {
  const char* who = "vrm_kv_dequant_pages";
  if (!kv_pool || !kv_scales || !page_ids || !out) {
    set_error("%s: null pointer argument", who);
    return VRM_ERR_ARG;
  }
  if (NP < 0 || NP > 65535 || KH <= 0 || 2 * KH > 65535 || D <= 0 || L <= 0 || P <= 0 || layer_idx < 0 ||
      layer_idx >= L) {
    set_error("%s: bad sizes", who);
    return VRM_ERR_ARG;
  }
  if (PS <= 0 || PS % 4 || D % 16 || D > 256) {
    set_error("%s: page_size %d / head_dim %d unsupported (multiples of 4 / 16)", who, PS, D);
    return VRM_ERR_UNSUPPORTED;
  }
  if (!quant_pool(kv_dtype)) {
    set_error("%s: kv_dtype %d is not a quantized pool", who, kv_dtype);
    return VRM_ERR_ARG;
  }
  const int rc = check_pool_scales(kv_dtype, kv_pool, kv_scales, KH, PS, D, L, P, who);
  if (rc) return rc;
  if (NP == 0) return VRM_OK;
  QuantArgs a{nullptr, nullptr, page_ids, nullptr, const_cast<uint8_t*>(static_cast<const uint8_t*>(kv_pool)),
              const_cast<float*>(kv_scales), KH, L, P, layer_idx, D, PS, pool_geom(kv_dtype, KH, PS, D, D, P, L)};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (fp8_pool(kv_dtype))
    hipLaunchKernelGGL(dequant_pages_kernel<true>, dim3(2 * KH, NP), dim3(256), 0, st, a, out, D);
  else
    hipLaunchKernelGGL(dequant_pages_kernel<false>, dim3(2 * KH, NP), dim3(256), 0, st, a, out, D);
  return launch_status(who);
}
