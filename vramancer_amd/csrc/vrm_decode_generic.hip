// Generic paged decode for gfx950: every pool kind (f32, f16, bf16, int8,
// fp8-e4m3, the reference's 4-bit layout) at any head_dim <= 256 and any page
// size, with D and PS runtime values.
//
// The reference kernel accepts any head_dim up to 256 and takes the page
// size from the pool's shape (csrc/paged_attention_kernel.cu:102-111,
// :460-466); the matrix-core kernels of vrm_decode_mfma.hip are compiled for
// page 16 and head_dim 64 / 128 / 256, and this kernel serves every other
// shape (head_dim 80, 96, 112, ...; pages of 8 or 32 tokens, ...), with the
// same work items, partials and merge.
//
// One wavefront per (work item, kv-head x group of G query heads), over
// chunks of kGenChunk tokens:
//   phase 1  lane = token: the K row is read element-wise (4 elements per
//            load where the row layout allows), dequantized, and dotted with
//            the G pre-scaled query rows staged in LDS; scores to LDS;
//   phase 2  exact chunk maximum, weights 2^(s - m), folded into the running
//            (max, sum, acc) of the partition;
//   phase 3  lane = dims d, d + 64, ...: the V rows of the chunk's tokens,
//            weighted by the LDS weights.
// int8 / fp8 pools keep this library's tiled V (token t, dim d at byte
// ((t / 4 * 16 + d % 16) * (D / 16) + d / 16) * 4 + t % 4 of the slice), so
// they need D % 16 == 0 and PS % 4 == 0; 4-bit pools need D % 32 == 0 (one
// scale and zero point per 32 dims).
#include "vrm_decode.h"

#include <math.h>

namespace vrm {
namespace dec {
namespace {

constexpr int kGenChunk = 256;  // tokens whose scores a wavefront holds in LDS at once
constexpr int kGenDpl = 4;      // dims per lane in the value pass (D <= 256)
constexpr int kGenMaxG = 8;     // query heads per wavefront

template <int KIND>
struct Elem {
  static constexpr int kBytesNum = KIND == K_F32 ? 4 : (KIND == K_F16 || KIND == K_BF16) ? 2 : 1;
  static constexpr int kBytesDen = KIND == K_Q4 ? 2 : 1;  // bytes per element = num / den
};

// Row bytes of D elements.
template <int KIND>
__device__ __forceinline__ int row_bytes(int D) {
  return D * Elem<KIND>::kBytesNum / Elem<KIND>::kBytesDen;
}

// Element d of a row (codes for int8 / fp8, the nibble for 4-bit pools).
template <int KIND>
__device__ __forceinline__ float elem(const uint8_t* row, int d) {
  if constexpr (KIND == K_F32) return reinterpret_cast<const float*>(row)[d];
  else if constexpr (KIND == K_F16) return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(row)[d]);
  else if constexpr (KIND == K_BF16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(row)[d]);
  else if constexpr (KIND == K_I8) return (float)(int8_t)row[d];
  else if constexpr (KIND == K_FP8) return e4m3fn_to_f32(row[d]);
  else return (float)((row[d >> 1] >> ((d & 1) * 4)) & 0xfu);
}

// Elements d .. d + 3 (d % 4 == 0) with one load; valid when D % 4 == 0 (the
// row start is then aligned to the load's width).
template <int KIND>
__device__ __forceinline__ void elem4(const uint8_t* row, int d, float* x) {
  if constexpr (KIND == K_F32) {
    const float4 v = *reinterpret_cast<const float4*>(row + 4 * d);
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
  } else if constexpr (KIND == K_F16 || KIND == K_BF16) {
    const uint2 v = *reinterpret_cast<const uint2*>(row + 2 * d);
    const uint32_t w[2] = {v.x, v.y};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      x[2 * i] = KIND == K_F16 ? f16_bits_to_f32(w[i] & 0xffffu) : bf16_bits_to_f32(w[i] & 0xffffu);
      x[2 * i + 1] = KIND == K_F16 ? f16_bits_to_f32(w[i] >> 16) : bf16_bits_to_f32(w[i] >> 16);
    }
  } else if constexpr (KIND == K_I8 || KIND == K_FP8) {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(row + d);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = (v >> (8 * i)) & 0xffu;
      x[i] = KIND == K_I8 ? (float)(int8_t)c : e4m3fn_to_f32(c);
    }
  } else {
    const uint32_t v = *reinterpret_cast<const uint16_t*>(row + d / 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = (float)((v >> (4 * i)) & 0xfu);
  }
}

template <int KIND, int G>
__global__ void __launch_bounds__(64) decode_generic_kernel(DecodeArgs a, int D, int PS) {
  extern __shared__ float gen_lds[];
  float* q_lds = gen_lds;                       // [G][D]  query * qscale
  float* s_lds = q_lds + G * D;                 // [G][kGenChunk] scores, then weights
  int* pid_lds = reinterpret_cast<int*>(s_lds + G * kGenChunk);  // [kGenChunk] page id (-1: skip)

  const int lane = threadIdx.x;
  const int group = a.H / a.KH;
  const int chunks = group / G;
  const int unit = blockIdx.y;
  const int kvh = unit / chunks;
  const int h0 = kvh * group + (unit % chunks) * G;
  const int item = blockIdx.x;
  WorkItem wi;
  if (!find_item(a.ctx_lens, a.B, a.max_pp, a.target, item, item == 0 && unit == 0, a.header, wi, PS)) return;
  const int b = wi.b;

  const int RB = row_bytes<KIND>(D);
  const int ngrp = D / 32;                           // 4-bit groups per row
  // 4-bit pools: (page, layer, K/V, head) index of the dense scale / zero arrays
  auto head_index = [&](int pid, int kv) { return (((size_t)pid * a.L + a.layer) * 2 + kv) * a.KH + kvh; };
  // codes of a (page, layer, K/V, kv-head) slice and, for int8 / fp8, its scales
  auto slice_of = [&](int pid, int kv) {
    return a.pool + (size_t)pid * a.g.page + (size_t)a.layer * a.g.layer + (size_t)kvh * a.g.head + (size_t)kv * a.g.kv;
  };
  auto scales_of = [&](int pid, int kv) {
    return a.scales + (size_t)pid * a.g.s_page + (size_t)a.layer * a.g.s_layer + (size_t)kvh * a.g.s_head +
           (size_t)kv * a.g.s_kv;
  };
  const bool vec4 = (D & 3) == 0;

  for (int i = lane; i < G * D; i += 64) {
    const int g = i / D;
    q_lds[i] = a.query[((size_t)b * a.H + h0 + g) * D + (i - g * D)] * a.qscale;
  }
  __syncthreads();

  float m_run[G], l_run[G], acc[G][kGenDpl];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.f;
#pragma unroll
    for (int j = 0; j < kGenDpl; ++j) acc[g][j] = 0.f;
  }

  const int32_t* trow = a.page_table + (size_t)b * a.max_pp;
  const int tok0 = wi.p_begin * PS;
  const int ntok = min(wi.n_pages * PS, wi.ctx - tok0);
  for (int c0 = 0; c0 < ntok; c0 += kGenChunk) {
    const int nt = min(kGenChunk, ntok - c0);
    // ---------------- phase 1: scores, one token per lane ----------------
    for (int tl = lane; tl < kGenChunk; tl += 64) {
      float s[G];
#pragma unroll
      for (int g = 0; g < G; ++g) s[g] = 0.f;
      int pid = -1;
      if (tl < nt) {
        const int tok = tok0 + c0 + tl;
        const int pg = tok / PS;
        const int slot = tok - pg * PS;
        pid = trow[pg];
        if (pid >= 0 && pid < a.P) {
          const uint8_t* row = slice_of(pid, 0) + (size_t)slot * RB;
          if constexpr (KIND == K_Q4) {
            const size_t gi = (head_index(pid, 0) * PS + slot) * ngrp;
            for (int c = 0; c < ngrp; ++c) {
              const float sc = f16_bits_to_f32(a.q4_scale[gi + c]);
              const float zp = f16_bits_to_f32(a.q4_zero[gi + c]);
              for (int d = 32 * c; d < 32 * c + 32; d += 4) {
                float x[4];
                elem4<KIND>(row, d, x);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  const float v = (x[e] - zp) * sc;
#pragma unroll
                  for (int g = 0; g < G; ++g) s[g] = fmaf(q_lds[g * D + d + e], v, s[g]);
                }
              }
            }
          } else {
            if (vec4) {
              for (int d = 0; d < D; d += 4) {
                float x[4];
                elem4<KIND>(row, d, x);
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                  for (int g = 0; g < G; ++g) s[g] = fmaf(q_lds[g * D + d + e], x[e], s[g]);
              }
            } else {
              for (int d = 0; d < D; ++d) {
                const float x = elem<KIND>(row, d);
#pragma unroll
                for (int g = 0; g < G; ++g) s[g] = fmaf(q_lds[g * D + d], x, s[g]);
              }
            }
            float ks = 1.f;
            if constexpr (KIND == K_I8) ks = scales_of(pid, 0)[slot];
            if constexpr (KIND == K_FP8) ks = scales_of(pid, 0)[0];
            if constexpr (KIND == K_I8 || KIND == K_FP8) {
#pragma unroll
              for (int g = 0; g < G; ++g) s[g] *= ks;
            }
          }
        } else {
          pid = -1;
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) s_lds[g * kGenChunk + tl] = pid >= 0 ? s[g] : -INFINITY;
      pid_lds[tl] = pid;
    }
    __syncthreads();

    // ---------------- phase 2: exact chunk maximum, folded into the running state ----------------
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = -INFINITY;
      for (int t = lane; t < nt; t += 64) mx = fmaxf(mx, s_lds[g * kGenChunk + t]);
      mx = group_max<64>(mx);
      const float m_new = fmaxf(m_run[g], mx);
      const float keep = (m_run[g] == -INFINITY) ? 0.f : exp2f(m_run[g] - m_new);
      float sum = 0.f;
      for (int t = lane; t < nt; t += 64) {
        const float sv = s_lds[g * kGenChunk + t];
        const float p = (sv == -INFINITY) ? 0.f : exp2f(sv - m_new);
        sum += p;
        s_lds[g * kGenChunk + t] = p;
      }
      l_run[g] = l_run[g] * keep + group_sum<64>(sum);
      m_run[g] = m_new;
#pragma unroll
      for (int j = 0; j < kGenDpl; ++j) acc[g][j] *= keep;
    }
    __syncthreads();

    // ---------------- phase 3: weighted V, lane = dims ----------------
    for (int tl = 0; tl < nt; ++tl) {
      const int pid = pid_lds[tl];
      if (pid < 0) continue;  // absent page (wave-uniform)
      const int tok = tok0 + c0 + tl;
      const int slot = tok % PS;
      const uint8_t* vs = slice_of(pid, 1);
      float w[G];
#pragma unroll
      for (int g = 0; g < G; ++g) w[g] = s_lds[g * kGenChunk + tl];
      if constexpr (KIND == K_I8 || KIND == K_FP8) {
        const float vscale = scales_of(pid, 1)[KIND == K_I8 ? slot : 0];
#pragma unroll
        for (int g = 0; g < G; ++g) w[g] *= vscale;
      }
#pragma unroll
      for (int j = 0; j < kGenDpl; ++j) {
        const int d = lane + 64 * j;
        if (d < D) {
          float v;
          if constexpr (KIND == K_I8 || KIND == K_FP8) {
            const uint8_t c = vs[(((slot >> 2) * 16 + (d & 15)) * (D >> 4) + (d >> 4)) * 4 + (slot & 3)];
            v = KIND == K_I8 ? (float)(int8_t)c : e4m3fn_to_f32(c);
          } else if constexpr (KIND == K_Q4) {
            const size_t gi = (head_index(pid, 1) * PS + slot) * ngrp + (d >> 5);
            v = (elem<KIND>(vs + (size_t)slot * RB, d) - f16_bits_to_f32(a.q4_zero[gi])) *
                f16_bits_to_f32(a.q4_scale[gi]);
          } else {
            v = elem<KIND>(vs + (size_t)slot * RB, d);
          }
#pragma unroll
          for (int g = 0; g < G; ++g) acc[g][j] = fmaf(w[g], v, acc[g][j]);
        }
      }
    }
    __syncthreads();  // the next chunk overwrites the scores
  }

#pragma unroll
  for (int g = 0; g < G; ++g) {
    float* dst = a.part_acc + ((size_t)item * a.H + h0 + g) * D;
#pragma unroll
    for (int j = 0; j < kGenDpl; ++j)
      if (lane + 64 * j < D) dst[lane + 64 * j] = acc[g][j];
  }
  if (lane < G) {
    float m = -INFINITY, l = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (g == lane) {
        m = m_run[g];
        l = l_run[g];
      }
    a.part_ml[((size_t)item * a.H + h0 + lane) * 2] = l > 0.f ? m : -INFINITY;
    a.part_ml[((size_t)item * a.H + h0 + lane) * 2 + 1] = l;
  }
}

template <int KIND, int G>
hipError_t launch_gen(const DecodeArgs& a0, int B, int D, int PS, hipStream_t st) {
  const int units = a0.KH * ((a0.H / a0.KH) / G);
  const size_t lds = ((size_t)G * D + (size_t)G * kGenChunk + kGenChunk) * sizeof(float);
  DecodeArgs a = a0;
  a.target = items_target(reinterpret_cast<const void*>(&decode_generic_kernel<KIND, G>), 1, lds, units);
  hipLaunchKernelGGL((decode_generic_kernel<KIND, G>), dim3(B + 2 * a.target, units, 1), dim3(64), lds, st, a, D,
                     PS);
  return hipGetLastError();
}

template <int KIND>
hipError_t launch_gen_g(const DecodeArgs& a, int B, int D, int PS, hipStream_t st) {
  switch (pick_group_tile(a.H / a.KH, kGenMaxG)) {
    case 1: return launch_gen<KIND, 1>(a, B, D, PS, st);
    case 2: return launch_gen<KIND, 2>(a, B, D, PS, st);
    case 3: return launch_gen<KIND, 3>(a, B, D, PS, st);
    case 4: return launch_gen<KIND, 4>(a, B, D, PS, st);
    case 5: return launch_gen<KIND, 5>(a, B, D, PS, st);
    case 6: return launch_gen<KIND, 6>(a, B, D, PS, st);
    case 7: return launch_gen<KIND, 7>(a, B, D, PS, st);
    default: return launch_gen<KIND, 8>(a, B, D, PS, st);
  }
}

}  // namespace

hipError_t launch_generic(const DecodeArgs& a, int kind, int B, int D, int PS, hipStream_t st) {
  switch (kind) {
    case K_F32: return launch_gen_g<K_F32>(a, B, D, PS, st);
    case K_F16: return launch_gen_g<K_F16>(a, B, D, PS, st);
    case K_BF16: return launch_gen_g<K_BF16>(a, B, D, PS, st);
    case K_I8: return launch_gen_g<K_I8>(a, B, D, PS, st);
    case K_FP8: return launch_gen_g<K_FP8>(a, B, D, PS, st);
    case K_Q4: return launch_gen_g<K_Q4>(a, B, D, PS, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dec
}  // namespace vrm
