// Paged decode over TurboQuant pages in the generic layout (vrm_tq_layout.h,
// GenLayout): head_dim 1 .. 256 (padded to a power of two from 2 to 256), 1 to 8 bits per
// angle, any QJL width up to 256 and any page size.  The tuned layout (head_dim
// 128, 64 QJL rows, 2 to 4 bits, page 16) has its own kernel
// (vrm_decode_tq.hip); this one computes the same attention,
// compute_attention_turbo's with dense values (core/paged_attention.py:
// 1259-1418):
//   score_t = q_rot . k_polar_t + sqrt(pi / 2) / qjl * norm_t * (q_rot JL^T) . (2 s_t - 1)
//   out     = unrotate(sum_t softmax(scale * score)_t v_polar_t), cut to head_dim
// with q_rot = rotate(pad(q)) (core/kv_quantizer.py:502-535) and the polar
// decode of core/kv_quantizer.py:297-309 from the fp16 radius.
//
// One wavefront per (work item, kv-head x group of G query heads), over
// chunks of 64 tokens whose K and V records are staged in LDS:
//   scores   lane = token: its k_polar is rebuilt dim by dim in a depth-first
//            walk of the polar tree (each level's product kept until the walk
//            leaves its node, so about two products per dim, in the reference's
//            order of roundings) and dotted with the G rotated queries;
//   softmax  per head, exact chunk maximum folded into the running state;
//   values   lane = dims e, e + 64, ...: each token's v_polar elements as
//            product chains from the radius, weighted into the accumulators,
//            which stay in the rotated domain; the inverse rotation is linear,
//            so each partition applies it once to its accumulators.
#include "vrm_decode.h"
#include "vrm_tq_common.h"
#include "vrm_tq_layout.h"

#include <math.h>

namespace vrm {
namespace dec {
namespace {

constexpr int kTqgMaxG = 8;    // query heads per wavefront
constexpr int kTqgChunk = 64;  // tokens per chunk: one per lane in the score pass

// Level-major bin b of a record (dwords), bits per angle `bits`.
__device__ __forceinline__ int rec_bin(const uint32_t* rec, int b, int bits, uint32_t mask) {
  const int bit = b * bits, dw = bit >> 5, sh = bit & 31;
  uint32_t x = rec[dw] >> sh;
  if (sh + bits > 32) x |= rec[dw + 1] << (32 - sh);
  return (int)(x & mask);
}

// LDS of the kernel, in floats / dwords.
struct TqgLds {
  int lut, qrot, qproj, sc, krec, vrec, pid, total;
};
__host__ __device__ inline TqgLds tqg_lds(const tq::GenLayout& g) {
  const int rec_dw = g.record_bytes() / 4;
  TqgLds o;
  o.lut = 0;
  o.qrot = o.lut + (4 << g.bits);
  o.qproj = o.qrot + kTqgMaxG * g.pd;
  o.sc = o.qproj + kTqgMaxG * g.qjl;
  o.krec = o.sc + kTqgMaxG * kTqgChunk;
  o.vrec = o.krec + kTqgChunk * rec_dw;
  o.pid = o.vrec + kTqgChunk * rec_dw;
  o.total = o.pid + kTqgChunk;
  return o;
}

template <int PD>
__global__ void __launch_bounds__(64) decode_tq_gen_kernel(DecodeArgs a, TqDecodeArgs tq, tq::GenLayout gl, int D,
                                                           int G) {
  constexpr int NL = __builtin_ctz(PD);
  constexpr int PER = tq_per_lane(PD);  // lanes past a row of fewer than 64 dims hold nothing
  extern __shared__ __align__(16) float tg_lds[];
  const TqgLds lo = tqg_lds(gl);
  const int nb = 1 << gl.bits;
  const uint32_t mask = (uint32_t)nb - 1u;
  const int rec_dw = gl.record_bytes() / 4;
  float* lut = tg_lds + lo.lut;    // cos level 0, sin level 0, cos levels >= 1, sin levels >= 1: [4][nb]
  float* qrot = tg_lds + lo.qrot;  // [G][PD]
  float* qproj = tg_lds + lo.qproj;  // [G][qjl]
  float* sc = tg_lds + lo.sc;      // [G][64] scores, then weights
  uint32_t* krec = reinterpret_cast<uint32_t*>(tg_lds + lo.krec);  // [64][rec_dw]
  uint32_t* vrec = reinterpret_cast<uint32_t*>(tg_lds + lo.vrec);  // [64][rec_dw]
  int* pid_lds = reinterpret_cast<int*>(tg_lds + lo.pid);          // [64]

  const int lane = threadIdx.x;
  const int group = a.H / a.KH;
  const int chunks = group / G;
  const int unit = blockIdx.y;
  const int kvh = unit / chunks;
  const int h0 = kvh * group + (unit % chunks) * G;
  const int item = blockIdx.x;
  const int PS = gl.ps;
  WorkItem wi;
  if (!find_item(a.ctx_lens, a.B, a.max_pp, a.target, item, item == 0 && unit == 0, a.header, wi, PS)) return;
  const int b = wi.b;

  for (int i = lane; i < 4 * nb; i += 64) lut[i] = tq.lut[i];
  // q_rot = rotate(pad(q)) per head (core/kv_quantizer.py:240-252, 516-518)
  const float root = (float)sqrt((double)PD);
  for (int g = 0; g < G; ++g) {
    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int e = k * 64 + lane;
      const float x = e < D ? a.query[((size_t)b * a.H + h0 + g) * D + e] : 0.f;
      v[k] = e < PD ? __fmul_rn(x, tq.signs[e]) : 0.f;
    }
    fwht<PD>(v, lane);
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (k * 64 + lane < PD) qrot[g * PD + k * 64 + lane] = __fdiv_rn(v[k], root);
  }
  __syncthreads();
  // q_proj = q_rot JL^T (core/kv_quantizer.py:319-321)
  for (int g = 0; g < G; ++g)
    for (int j = lane; j < gl.qjl; j += 64) {
      float s = 0.f;
      for (int e = 0; e < PD; ++e) s = fmaf(qrot[g * PD + e], tq.jl[(size_t)j * PD + e], s);
      qproj[g * gl.qjl + j] = s;
    }
  __syncthreads();

  float m_run[kTqgMaxG], l_run[kTqgMaxG], acc[kTqgMaxG][PER];
#pragma unroll
  for (int g = 0; g < kTqgMaxG; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) acc[g][k] = 0.f;
  }

  const size_t slice = gl.slice_bytes();
  const size_t kv_stride = (size_t)a.KH * slice;
  const size_t page_stride = kv_stride * 2 * a.L;
  auto record = [&](int pid, int kv, int slot) {
    return reinterpret_cast<const uint32_t*>(a.pool + (size_t)pid * page_stride + (size_t)a.layer * 2 * kv_stride +
                                             (size_t)kv * kv_stride + (size_t)kvh * slice +
                                             (size_t)slot * gl.record_bytes());
  };
  const int32_t* trow = a.page_table + (size_t)b * a.max_pp;
  const int tok0 = wi.p_begin * PS;
  const int ntok = min(wi.n_pages * PS, wi.ctx - tok0);
  const int rad_dw = gl.angle_dw + gl.sign_dw;  // dword of (radius, norm)

  for (int c0 = 0; c0 < ntok; c0 += kTqgChunk) {
    const int nt = min(kTqgChunk, ntok - c0);
    // ---------------- stage the chunk's K and V records ----------------
    int pid = -1, slot = 0;
    if (lane < nt) {
      const int tok = tok0 + c0 + lane;
      const int pg = tok / PS;
      slot = tok - pg * PS;
      pid = trow[pg];
      if (pid < 0 || pid >= a.P) pid = -1;
    }
    pid_lds[lane] = pid;
    if (pid >= 0) {
      const uint32_t* ks = record(pid, 0, slot);
      const uint32_t* vs = record(pid, 1, slot);
      for (int i = 0; i < rec_dw; ++i) {
        krec[lane * rec_dw + i] = ks[i];
        vrec[lane * rec_dw + i] = vs[i];
      }
    }
    __syncthreads();

    // ---------------- scores, one token per lane ----------------
    float s[kTqgMaxG];
#pragma unroll
    for (int g = 0; g < kTqgMaxG; ++g) s[g] = 0.f;
    if (pid >= 0) {
      const uint32_t* kr = krec + lane * rec_dw;
      const uint32_t rn = kr[rad_dw];
      const float radius = f16_bits_to_f32(rn & 0xffffu);
      const float norm = f16_bits_to_f32(rn >> 16);
      // prod[l]: the product chain down to level l of the current dim's path
      float prod[NL + 1];
      prod[NL] = radius;
#pragma unroll
      for (int d = 0; d < PD; ++d) {
        const int top = d == 0 ? NL - 1 : __builtin_ctz(d);  // levels whose node changes at dim d
#pragma unroll
        for (int l = NL - 1; l >= 0; --l) {
          if (l <= top) {
            const int bin = rec_bin(kr, (PD - (PD >> l)) + (d >> (l + 1)), gl.bits, mask);
            prod[l] = __fmul_rn(prod[l + 1], lut[(l == 0 ? 0 : 2 * nb) + (((d >> l) & 1) ? nb : 0) + bin]);
          }
        }
#pragma unroll
        for (int g = 0; g < kTqgMaxG; ++g)
          if (g < G) s[g] = fmaf(qrot[g * PD + d], prod[0], s[g]);
      }
      if (tq.qjl_coef != 0.f) {
        float c[kTqgMaxG];
#pragma unroll
        for (int g = 0; g < kTqgMaxG; ++g) c[g] = 0.f;
        for (int j = 0; j < gl.qjl; ++j) {
          const float sg = ((kr[gl.angle_dw + (j >> 5)] >> (j & 31)) & 1u) ? 1.f : -1.f;
#pragma unroll
          for (int g = 0; g < kTqgMaxG; ++g)
            if (g < G) c[g] = fmaf(qproj[g * gl.qjl + j], sg, c[g]);
        }
#pragma unroll
        for (int g = 0; g < kTqgMaxG; ++g) s[g] += (c[g] * tq.qjl_coef) * norm;
      }
#pragma unroll
      for (int g = 0; g < kTqgMaxG; ++g) s[g] *= a.qscale;  // log2 domain
    }

    // ---------------- softmax: exact chunk maximum per head ----------------
#pragma unroll
    for (int g = 0; g < kTqgMaxG; ++g) {
      if (g >= G) break;
      const float x = pid >= 0 ? s[g] : -INFINITY;
      const float mx = group_max<64>(x);
      const float m_new = fmaxf(m_run[g], mx);
      const float keep = m_run[g] == -INFINITY ? 0.f : exp2f(m_run[g] - m_new);
      const float p = x == -INFINITY ? 0.f : exp2f(x - m_new);
      l_run[g] = l_run[g] * keep + group_sum<64>(p);
      m_run[g] = m_new;
#pragma unroll
      for (int k = 0; k < PER; ++k) acc[g][k] *= keep;
      sc[g * kTqgChunk + lane] = p;
    }
    __syncthreads();

    // ---------------- values, lane = dims ----------------
    for (int t = 0; t < nt; ++t) {
      if (pid_lds[t] < 0) continue;  // absent page (wave-uniform)
      const uint32_t* vr = vrec + t * rec_dw;
      const float vrad = f16_bits_to_f32(vr[rad_dw] & 0xffffu);
      float w[kTqgMaxG];
#pragma unroll
      for (int g = 0; g < kTqgMaxG; ++g) w[g] = g < G ? sc[g * kTqgChunk + t] : 0.f;
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const int e = k * 64 + lane;
        if (PD < 64 && e >= PD) continue;  // no element of the row
        float r = vrad;
#pragma unroll
        for (int l = NL - 1; l >= 0; --l) {
          const int bin = rec_bin(vr, (PD - (PD >> l)) + (e >> (l + 1)), gl.bits, mask);
          r = __fmul_rn(r, lut[(l == 0 ? 0 : 2 * nb) + (((e >> l) & 1) ? nb : 0) + bin]);
        }
#pragma unroll
        for (int g = 0; g < kTqgMaxG; ++g) acc[g][k] = fmaf(w[g], r, acc[g][k]);
      }
    }
    __syncthreads();  // the next chunk overwrites the records and weights
  }

  // ---------------- unrotate the partition's accumulators, write the partials ----------------
#pragma unroll
  for (int g = 0; g < kTqgMaxG; ++g) {
    if (g >= G) break;
    float y[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) y[k] = acc[g][k];
    fwht<PD>(y, lane);
    float* dst = a.part_acc + ((size_t)item * a.H + h0 + g) * D;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int e = k * 64 + lane;
      if (e < D) dst[e] = __fmul_rn(__fdiv_rn(y[k], root), tq.signs[e]);
    }
  }
  if (lane < G) {
    float m = -INFINITY, l = 0.f;
#pragma unroll
    for (int g = 0; g < kTqgMaxG; ++g)
      if (g == lane) {
        m = m_run[g];
        l = l_run[g];
      }
    a.part_ml[((size_t)item * a.H + h0 + lane) * 2] = l > 0.f ? m : -INFINITY;
    a.part_ml[((size_t)item * a.H + h0 + lane) * 2 + 1] = l;
  }
}

template <int PD>
hipError_t launch_tqg(const DecodeArgs& a0, const TqDecodeArgs& tq, const tq::GenLayout& gl, int B, int D, int G,
                      hipStream_t st) {
  const int units = a0.KH * ((a0.H / a0.KH) / G);
  const size_t lds = (size_t)tqg_lds(gl).total * sizeof(float);
  DecodeArgs a = a0;
  a.target = items_target(reinterpret_cast<const void*>(&decode_tq_gen_kernel<PD>), 1, lds, units);
  hipLaunchKernelGGL(decode_tq_gen_kernel<PD>, dim3(B + 2 * a.target, units, 1), dim3(64), lds, st, a, tq, gl, D, G);
  return hipGetLastError();
}

}  // namespace

size_t tq_generic_lds_bytes(const tq::GenLayout& gl) { return (size_t)tqg_lds(gl).total * sizeof(float); }

hipError_t launch_tq_generic(const DecodeArgs& a, const TqDecodeArgs& tq, const tq::GenLayout& gl, int B, int D,
                             hipStream_t st) {
  const int G = pick_group_tile(a.H / a.KH, kTqgMaxG);
  switch (gl.pd) {
    case 2: return launch_tqg<2>(a, tq, gl, B, D, G, st);
    case 4: return launch_tqg<4>(a, tq, gl, B, D, G, st);
    case 8: return launch_tqg<8>(a, tq, gl, B, D, G, st);
    case 16: return launch_tqg<16>(a, tq, gl, B, D, G, st);
    case 32: return launch_tqg<32>(a, tq, gl, B, D, G, st);
    case 64: return launch_tqg<64>(a, tq, gl, B, D, G, st);
    case 128: return launch_tqg<128>(a, tq, gl, B, D, G, st);
    default: return launch_tqg<256>(a, tq, gl, B, D, G, st);
  }
}

}  // namespace dec
}  // namespace vrm
