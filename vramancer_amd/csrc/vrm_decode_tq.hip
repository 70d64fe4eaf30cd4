// Paged decode over TurboQuant pages (gfx950): the attention of the
// reference's compute_attention_turbo (core/paged_attention.py:1259-1418,
// dense values, head h reading kv-head h / (H / KH)) without decompressing
// anything to memory.
//
// For each (sequence, query head), over the tokens of its pages:
//   score_t = q_rot . k_polar_t + sqrt(pi / 2) / 64 * norm_t * (q_rot JL^T) . (2 s_t - 1)
//   out     = unrotate( sum_t softmax(scale * score)_t v_polar_t )
// with q_rot = H(q * signs) / sqrt(128) and k_polar / v_polar the polar
// reconstructions (rotated domain, from the fp16 radius) of
// KVCacheCompressor.attention_score / decompress (core/kv_quantizer.py:
// 481-535).  The inverse rotation is linear, so it is applied once to the
// weighted sum instead of to every value.
//
// Work split as in the other stream kernels (work items of find_item, one
// wavefront per (kv-head, head chunk), up to 16 query heads in the columns of
// 16x16 MFMA tiles).  Lane (t, g) = (lane % 16, lane / 16) rebuilds dims
// 32 g .. 32 g + 31 of token t of a page from quarter g of the token's angle
// record (vrm_tq_layout.h), multiplying the radius by the {cos, sin} of the
// bin centres level by level (6 down to 0) as the reference does, so the
// reconstruction equals the reference's polar decode bit for bit.
//   S^T   = K Q^T on v_mfma_f32_16x16x32_f16, K and q_rot as hi + lo fp16
//           (k index (chunk c, group g, element e) <-> dim 32 g + 8 c + e);
//   QJL   = S P^T: the sign bits as exact +-1 fp16 against q_rot JL^T
//           (computed on the matrix cores at set-up, hi + lo);
//   V     rounded to fp16, moved to token-per-lane order by an exact one-hot
//         MFMA transpose, then O^T += V^T P^T with P as hi + lo.
#include "vrm_decode.h"
#include "vrm_tq_layout.h"

#include <math.h>

namespace vrm {
namespace dec {
namespace {

namespace T = vrm::tq;

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int kWaves = 4;             // wavefronts per workgroup (at most)
constexpr float kLazyRescale = 3.0f;  // as in vrm_decode_mfma.hip
constexpr float kNoMax = -1.0e30f;

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float f16_to_f32(uint32_t bits) { return (float)__builtin_bit_cast(_Float16, (uint16_t)bits); }

// WIDTH bits at bit `pos` of the little-endian bit stream w[]; pos is a
// constant after unrolling, so the indexing folds to one or two ALU ops.
template <int WIDTH>
__device__ __forceinline__ uint32_t bit_field(const uint32_t* w, int pos) {
  const int dw = pos / 32, sh = pos % 32;
  if (sh + WIDTH <= 32) return __builtin_amdgcn_ubfe(w[dw], sh, WIDTH);
  return __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(w[dw + 1], w[dw], sh), 0, WIDTH);
}

// fp16 pair {fp16(a0 b0), fp16(a1 b1)}, each product rounded once to fp16
// (v_fma_mix with float32 sources).
__device__ __forceinline__ uint32_t mul_f16x2(float a0, float b0, float a1, float b1) {
  uint32_t r;
  asm("v_fma_mixlo_f16 %0, %1, %2, 0\n\tv_fma_mixhi_f16 %0, %3, %4, 0"
      : "=&v"(r)
      : "v"(a0), "v"(b0), "v"(a1), "v"(b1));
  return r;
}

// fp16 pair {fp16(a0 b0 - h.lo), fp16(a1 b1 - h.hi)}: the residuals of the
// products against their fp16 roundings h, each one fused multiply-add.
__device__ __forceinline__ uint32_t residual_f16x2(float a0, float b0, float a1, float b1, uint32_t h) {
  uint32_t r;
  asm("v_fma_mixlo_f16 %0, %1, %2, -%5 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %0, %3, %4, -%5 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
      : "=&v"(r)
      : "v"(a0), "v"(b0), "v"(a1), "v"(b1), "v"(h));
  return r;
}

// In-register Walsh-Hadamard transform of 128 values, element e in lane e % 64,
// register e / 64, in the reference's butterfly order.
__device__ __forceinline__ void fwht128(float (&v)[2], int lane) {
#pragma unroll
  for (int h = 1; h < 64; h <<= 1) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      float other;
      switch (h) {
        case 1: other = xor_shfl<1>(v[k]); break;
        case 2: other = xor_shfl<2>(v[k]); break;
        case 4: other = xor_shfl<4>(v[k]); break;
        case 8: other = xor_shfl<8>(v[k]); break;
        case 16: other = xor_shfl<16>(v[k]); break;
        default: other = xor_shfl<32>(v[k]); break;
      }
      v[k] = (lane & h) ? other - v[k] : v[k] + other;
    }
  }
  const float a = v[0], b = v[1];
  v[0] = a + b;
  v[1] = a - b;
}

template <int BITS>
struct TqSlot {
  uint32_t kq[BITS];  // K angle quarter grp of token col
  uint32_t vq[BITS];  // V angle quarter grp of token col
  uint32_t ktop[2];   // last dword of K quarters 0 and 1 + grp / 2 (level 6 / level 5 spares)
  uint32_t vtop[2];
  uint32_t krad, vrad, knorm;  // fp16 bits
  uint2 ksign;                 // 64 QJL sign bits of token col
  bool ok;                     // page id inside the pool (wave-uniform)
};

template <int BITS>
__global__ void __launch_bounds__(64 * kWaves, 2) decode_tq_kernel(DecodeArgs a, TqDecodeArgs tq, int G) {
  constexpr int NB = 1 << BITS;
  constexpr int RING = 4;
  constexpr int SLICE = T::slice_bytes(BITS);
  constexpr int ABYTES = T::angle_bytes(BITS);
  constexpr int D = T::kPD;

  // {cos, sin} of the bin centres of levels >= 1, singly and, at 4 bits
  // (levels 3 and 2), for two sibling angles at once (index bin_a + NB bin_b)
  __shared__ float2 lut[NB];
  __shared__ float4 lut2[BITS <= 3 ? 1 : NB * NB];
  __shared__ uint2 sign_lut[16];  // 4 sign bits -> 4 fp16 +-1 (bit i -> element i)
  // Two levels per lookup: for a node angle a and the angles b, c of its two
  // children (index a + NB (b + NB c)), the products (cos a cos b, cos a sin b,
  // sin a cos c, sin a sin c); t10 for levels 1/0 (level 0 has its own bin
  // centres) and, at 2 and 3 bits, t32 for levels 3/2.  They share LDS with
  // qbuf (per wave: q_rot rows before the stream, the output columns after
  // it), which is dead while the tables are read.
  constexpr bool kT32 = BITS <= 3;
  constexpr int NT = NB * NB * NB;
  constexpr int QBUF_BYTES = kWaves * 16 * (D + 4) * 4;
  constexpr int TAB_BYTES = (kT32 ? 2 : 1) * NT * 16;
  __shared__ __attribute__((aligned(16))) unsigned char shbuf[QBUF_BYTES > TAB_BYTES ? QBUF_BYTES : TAB_BYTES];
  float(*qbuf)[16][D + 4] = reinterpret_cast<float(*)[16][D + 4]>(shbuf);
  float4* t10 = reinterpret_cast<float4*>(shbuf);
  float4* t32 = t10 + NT;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int group = a.H / a.KH;
  const int chunks = group / G;
  const int unit = blockIdx.y * (blockDim.x >> 6) + wave;
  const int kvh = unit / chunks;
  const int h0 = kvh * group + (unit % chunks) * G;

  for (int i = threadIdx.x; i < NB; i += blockDim.x) lut[i] = make_float2(tq.lut[2 * NB + i], tq.lut[3 * NB + i]);
  if constexpr (BITS > 3) {
    for (int i = threadIdx.x; i < NB * NB; i += blockDim.x) {
      const int ba = i % NB, bb = i / NB;
      lut2[i] = make_float4(tq.lut[2 * NB + ba], tq.lut[3 * NB + ba], tq.lut[2 * NB + bb], tq.lut[3 * NB + bb]);
    }
  }
  if (threadIdx.x < 16) {
    uint32_t h[4];
    for (int e = 0; e < 4; ++e) h[e] = ((threadIdx.x >> e) & 1) ? 0x3c00u : 0xbc00u;  // fp16 +1 / -1
    sign_lut[threadIdx.x] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
  }
  __syncthreads();

  const int item = blockIdx.x;
  WorkItem wi;
  if (!find_item(a.ctx_lens, a.B, a.max_pp, a.target, item, item == 0 && unit == 0, a.header, wi)) return;
  const int b = wi.b;
  const int n_pages = wi.n_pages;
  const int last = n_pages - 1;
  const int tok_end = min(n_pages * kPS, wi.ctx - wi.p_begin * kPS);
  const int32_t* trow = a.page_table + (size_t)b * a.max_pp + wi.p_begin;
  auto ids_at = [&](int first) { return trow[min(first + (lane & (RING - 1)), last)]; };
  float(*qb)[D + 4] = qbuf[wave];

  // ---------------- q_rot of this wave's heads (row r: head min(r, G - 1)) ----------------
  const float root = (float)sqrt(128.0);
#pragma unroll 1
  for (int r = 0; r < 16; ++r) {
    const float* qrow = a.query + ((size_t)b * a.H + h0 + min(r, G - 1)) * D;
    float v[2] = {qrow[lane] * tq.signs[lane], qrow[lane + 64] * tq.signs[lane + 64]};
    fwht128(v, lane);
    qb[r][lane] = v[0] / root;
    qb[r][lane + 64] = v[1] / root;
  }
  wave_sync();
  // B operand of S^T: lane (col, grp) holds q_rot[col][32 grp + 8 c + e] * qscale
  v8h QH[4][2];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = qb[col][32 * grp + 8 * c + e] * a.qscale;
      const _Float16 hi = (_Float16)x;
      QH[c][0][e] = hi;
      QH[c][1][e] = (_Float16)(x - (float)hi);
    }
  // q_proj^T = JL q_rot^T on the matrix cores: tile j (JL rows 16 j ..), result
  // in lane (col, grp) for rows 16 j + 4 grp + r.  The QJL product uses the
  // matching k order: chunk c, element e <-> JL row 16 (2 c + e / 4) + 4 grp + e % 4.
  v8h PJ[2][2];
  {
    float pj[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v8h ah, al, bh, bl;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = tq.jl[(size_t)(16 * j + col) * D + 32 * c + 8 * grp + e];
          ah[e] = (_Float16)x;
          al[e] = (_Float16)(x - (float)ah[e]);
          const float y = qb[col][32 * c + 8 * grp + e];
          bh[e] = (_Float16)y;
          bl[e] = (_Float16)(y - (float)bh[e]);
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, acc, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) pj[j][r] = acc[r];
    }
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = pj[2 * c + e / 4][e % 4];
        const _Float16 hi = (_Float16)x;
        PJ[c][0][e] = hi;
        PJ[c][1][e] = (_Float16)(x - (float)hi);
      }
  }
  // one-hot operands of the V transpose: E_h[8 grp + e][col] = (8 grp + e == 16 h + col)
  v8h onehot[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      onehot[h][e] = (grp == 2 * h + (col >> 3) && e == (col & 7)) ? (_Float16)1.f : (_Float16)0.f;
  const float qjl_scale = a.qscale * tq.qjl_coef;

  // every wave of the workgroup is done with qbuf (all share the work item,
  // so all reach this point): its LDS now holds the two-level tables
  __syncthreads();
  {
    const float* cos1 = tq.lut + 2 * NB;  // levels >= 1
    const float* sin1 = tq.lut + 3 * NB;
    const float* cos0 = tq.lut;           // level 0
    const float* sin0 = tq.lut + NB;
    for (int i = threadIdx.x; i < NT; i += blockDim.x) {
      const int ia = i % NB, ib = (i / NB) % NB, ic = i / (NB * NB);
      t10[i] = make_float4(cos1[ia] * cos0[ib], cos1[ia] * sin0[ib], sin1[ia] * cos0[ic], sin1[ia] * sin0[ic]);
      if constexpr (kT32)
        t32[i] = make_float4(cos1[ia] * cos1[ib], cos1[ia] * sin1[ib], sin1[ia] * cos1[ic], sin1[ia] * sin1[ic]);
    }
  }
  __syncthreads();

  // ---------------- streaming state ----------------
  float m_run = kNoMax, l_run = 0.f;
  // O^T block 2 c + h: row 4 grp + r <-> dim 32 (2 h + (4 grp + r) / 8) + 8 c + (4 grp + r) % 8
  v4f acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};

  const size_t kv_stride = (size_t)a.KH * SLICE;
  const size_t page_stride = kv_stride * 2 * a.L;
  const uint8_t* layer_base = a.pool + (size_t)a.layer * 2 * kv_stride + (size_t)kvh * SLICE;
  auto page_ok = [&](int pid) { return pid >= 0 && pid < a.P; };
  const int top1 = (1 + (grp >> 1)) * BITS + BITS - 1;  // dword of slot 31 of quarter 1 + grp / 2

  auto load_page = [&](TqSlot<BITS>& s, int pid) {
    s.ok = page_ok(pid);
    const uint8_t* ks = layer_base + (size_t)(s.ok ? pid : 0) * page_stride;
    const uint8_t* vs = ks + kv_stride;
    const uint32_t* krec = reinterpret_cast<const uint32_t*>(ks + col * ABYTES);
    const uint32_t* vrec = reinterpret_cast<const uint32_t*>(vs + col * ABYTES);
#pragma unroll
    for (int i = 0; i < BITS; ++i) {
      s.kq[i] = krec[grp * BITS + i];
      s.vq[i] = vrec[grp * BITS + i];
    }
    s.ktop[0] = krec[BITS - 1];
    s.ktop[1] = krec[top1];
    s.vtop[0] = vrec[BITS - 1];
    s.vtop[1] = vrec[top1];
    s.krad = reinterpret_cast<const uint16_t*>(ks + T::radius_offset(BITS))[col];
    s.vrad = reinterpret_cast<const uint16_t*>(vs + T::radius_offset(BITS))[col];
    s.knorm = reinterpret_cast<const uint16_t*>(ks + T::norms_offset(BITS))[col];
    s.ksign = reinterpret_cast<const uint2*>(ks + T::signs_offset(BITS))[col];
  };

  // dims 32 grp .. 32 grp + 31 of one token: the reference's tree of
  // products, two levels per lookup from the product tables below level 4
  // (4 bits: levels 3 and 2 one at a time with sibling angles together), so
  // each value is the reference's within a float32 rounding or two.
  // Leaves the last level's products to the caller: value 4 j + k of the
  // group is y[j] * t[j][k].
  auto rebuild = [&](const uint32_t* q, uint32_t top0, uint32_t topq, float radius, float (&y)[8], float4 (&t)[8]) {
    constexpr int sh31 = (31 * BITS) % 32;  // slot 31 never straddles a dword
    const float2 t6 = lut[(top0 >> sh31) & (NB - 1)];
    const float2 t5 = lut[(topq >> sh31) & (NB - 1)];
    float p = radius;
    p = p * ((grp >> 1) ? t6.y : t6.x);  // bit 6 of the dims
    p = p * ((grp & 1) ? t5.y : t5.x);   // bit 5
    const float2 c4 = lut[bit_field<BITS>(q, (kT32 ? 30 : 0) * BITS)];  // level 4
    const float x3[2] = {p * c4.x, p * c4.y};
    if constexpr (kT32) {
      // levels 3 and 2: node j and its children in slots 24 + 3 j .. 26 + 3 j
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float4 t = t32[bit_field<3 * BITS>(q, (24 + 3 * j) * BITS)];
        y[4 * j] = x3[j] * t.x;
        y[4 * j + 1] = x3[j] * t.y;
        y[4 * j + 2] = x3[j] * t.z;
        y[4 * j + 3] = x3[j] * t.w;
      }
    } else {
      // level 3 (slots 1, 2), then level 2 (slots 3 .. 6), sibling angles together
      const float4 a3 = lut2[bit_field<2 * BITS>(q, 1 * BITS)];
      const float x2[4] = {x3[0] * a3.x, x3[0] * a3.y, x3[1] * a3.z, x3[1] * a3.w};
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const float4 a2 = lut2[bit_field<2 * BITS>(q, (3 + i) * BITS)];
        y[2 * i] = x2[i] * a2.x;
        y[2 * i + 1] = x2[i] * a2.y;
        y[2 * i + 2] = x2[i + 1] * a2.z;
        y[2 * i + 3] = x2[i + 1] * a2.w;
      }
    }
    // levels 1 and 0: node j and its children in slots 3 j .. 3 j + 2 (4 bits:
    // node slot 7 + j, children slots 15 + 2 j, 16 + 2 j)
#pragma unroll
    for (int j = 0; j < 8; ++j)
      t[j] = t10[kT32 ? bit_field<3 * BITS>(q, 3 * j * BITS)
                      : bit_field<BITS>(q, (7 + j) * BITS) + NB * bit_field<2 * BITS>(q, (15 + 2 * j) * BITS)];
  };
  auto comp = [](const float4& v, int k) { return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w; };

  // Scores (log2 domain) of this lane's tokens 4 grp + r of page pi.
  auto page_scores = [&](const TqSlot<BITS>& s, int pi, float* sc) {
    float y[8];
    float4 t[8];
    rebuild(s.kq, s.ktop[0], s.ktop[1], f16_to_f32(s.krad), y, t);
    v4f c4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      // k = y t as hi = fp16(k) and lo = fp16(k - hi)
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const int j = (8 * c + e) >> 2, k = e & 3;
        hw[e / 2] = mul_f16x2(y[j], comp(t[j], k), y[j], comp(t[j], k + 1));
        lw[e / 2] = residual_f16x2(y[j], comp(t[j], k), y[j], comp(t[j], k + 1), hw[e / 2]);
      }
      const v8h kh = __builtin_bit_cast(v8h, make_uint4(hw[0], hw[1], hw[2], hw[3]));
      const v8h kl = __builtin_bit_cast(v8h, make_uint4(lw[0], lw[1], lw[2], lw[3]));
      c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, QH[c][0], c4, 0, 0, 0);
      c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, QH[c][1], c4, 0, 0, 0);
      c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, QH[c][0], c4, 0, 0, 0);
    }
    v4f cq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      // elements e < 4: JL rows 32 c + 4 grp + e; e >= 4: rows 32 c + 16 + 4 grp + e - 4
      const uint32_t word = c == 0 ? s.ksign.x : s.ksign.y;
      const uint2 lo = sign_lut[__builtin_amdgcn_ubfe(word, 4 * grp, 4)];
      const uint2 hi = sign_lut[__builtin_amdgcn_ubfe(word, 16 + 4 * grp, 4)];
      const v8h sg = __builtin_bit_cast(v8h, make_uint4(lo.x, lo.y, hi.x, hi.y));
      cq = __builtin_amdgcn_mfma_f32_16x16x32_f16(sg, PJ[c][0], cq, 0, 0, 0);
      cq = __builtin_amdgcn_mfma_f32_16x16x32_f16(sg, PJ[c][1], cq, 0, 0, 0);
    }
    const float nrm = f16_to_f32(s.knorm);  // norm of token col; row r needs token 4 grp + r
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 4 * grp + r;
      const float nt = __int_as_float(__builtin_amdgcn_ds_bpermute(t << 2, __float_as_int(nrm)));  // lane t holds token t
      sc[r] = (s.ok && pi * kPS + t < tok_end) ? c4[r] + qjl_scale * nt * cq[r] : -INFINITY;
    }
  };

  // V of 16 dims (block 2 c + h) for this lane's 4 tokens of one page, exact
  // fp16 values in token-per-lane order.
  auto v_block = [&](const v8h& vop, int h, float* out4) {
    const v4f t = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, onehot[h], v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r) out4[r] = t[r];
  };
  // Values of this lane's token; absent pages and tokens past the context get
  // radius 0 (whatever the page holds), so they contribute exact zeros.
  auto v_operand = [&](const TqSlot<BITS>& s, int pi, v8h (&vop)[4]) {
    float y[8];
    float4 t[8];
    const bool live = s.ok && pi * kPS + col < tok_end;
    rebuild(s.vq, s.vtop[0], s.vtop[1], live ? f16_to_f32(s.vrad) : 0.f, y, t);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const int j = (8 * c + e) >> 2, k = e & 3;
        w[e / 2] = mul_f16x2(y[j], comp(t[j], k), y[j], comp(t[j], k + 1));
      }
      vop[c] = __builtin_bit_cast(v8h, make_uint4(w[0], w[1], w[2], w[3]));
    }
  };

  auto process_pair = [&](const TqSlot<BITS>& s0, const TqSlot<BITS>& s1, int pi, bool has1) {
    float sc[8];
    page_scores(s0, pi, sc);
    if (has1) {
      page_scores(s1, pi + 1, sc + 4);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[4 + r] = -INFINITY;
    }
    float pm = sc[0];
#pragma unroll
    for (int r = 1; r < 8; ++r) pm = fmaxf(pm, sc[r]);
    pm = fmaxf(pm, xor_shfl<16>(pm));
    pm = fmaxf(pm, xor_shfl<32>(pm));
    if (pm > m_run + kLazyRescale) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - pm);
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] *= alpha;
      m_run = pm;
    }
    v8h Bh, Bl;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = __builtin_amdgcn_exp2f(sc[e] - m_run);
      l_run += p;
      const _Float16 hi = (_Float16)p;
      Bh[e] = hi;
      Bl[e] = (_Float16)(p - (float)hi);
    }
    v8h vop0[4], vop1[4];
    v_operand(s0, pi, vop0);
    v_operand(s1, pi + 1, vop1);  // past the partition: radius 0
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float t[8];
        v_block(vop0[c], h, t);
        v_block(vop1[c], h, t + 4);
        v8h A;
#pragma unroll
        for (int e = 0; e < 8; ++e) A[e] = (_Float16)t[e];  // exact: fp16 values
        acc[2 * c + h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bh, acc[2 * c + h], 0, 0, 0);
        acc[2 * c + h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bl, acc[2 * c + h], 0, 0, 0);
      }
  };

  // ---------------- stream the partition ----------------
  {
    TqSlot<BITS> ring[RING];
    const int ids0 = ids_at(0);
    int ids_next = ids_at(RING);
#pragma unroll
    for (int u = 0; u < RING; ++u) load_page(ring[u], __builtin_amdgcn_readlane(ids0, u));
    for (int base = 0; base < n_pages; base += RING) {
      const int ids_ahead = ids_at(base + 2 * RING);
#pragma unroll
      for (int u = 0; u < RING; u += 2) {
        if (base + u < n_pages) process_pair(ring[u], ring[u + 1], base + u, base + u + 1 < n_pages);
        load_page(ring[u], __builtin_amdgcn_readlane(ids_next, u));
        load_page(ring[u + 1], __builtin_amdgcn_readlane(ids_next, u + 1));
      }
      ids_next = ids_ahead;
    }
  }

  // ---------------- partition result: columns to natural dims, unrotate ----------------
  __syncthreads();  // the tables are dead once every wave has streamed its pages
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 4 * grp + r;
        qb[col][32 * (2 * h + (row >> 3)) + 8 * c + (row & 7)] = acc[2 * c + h][r];
      }
  float l_tot = l_run + xor_shfl<16>(l_run);
  l_tot += xor_shfl<32>(l_tot);
  wave_sync();
  const float s_lo = tq.signs[lane], s_hi = tq.signs[lane + 64];
  for (int hh = 0; hh < G; ++hh) {
    float v[2] = {qb[hh][lane], qb[hh][lane + 64]};
    fwht128(v, lane);
    float* out = a.part_acc + ((size_t)item * a.H + h0 + hh) * D;
    out[lane] = v[0] / root * s_lo;
    out[lane + 64] = v[1] / root * s_hi;
  }
  if (col < G && grp == 0) {
    float* ml = a.part_ml + ((size_t)item * a.H + h0 + col) * 2;
    ml[0] = l_tot > 0.f ? m_run : -INFINITY;
    ml[1] = l_tot;
  }
}

}  // namespace

hipError_t launch_tq_decode(const DecodeArgs& a0, const TqDecodeArgs& tq, int bits, int B, int G, hipStream_t st) {
  const int units = a0.KH * ((a0.H / a0.KH) / G);
  int W = kWaves;
  while (units % W) --W;
  DecodeArgs a = a0;
  const void* fn = bits == 2   ? reinterpret_cast<const void*>(&decode_tq_kernel<2>)
                   : bits == 3 ? reinterpret_cast<const void*>(&decode_tq_kernel<3>)
                               : reinterpret_cast<const void*>(&decode_tq_kernel<4>);
  a.target = items_target(fn, W, 0, units);
  dim3 grid(B + 2 * a.target, units / W, 1);
  dim3 block(64 * W);
  switch (bits) {
    case 2: hipLaunchKernelGGL(decode_tq_kernel<2>, grid, block, 0, st, a, tq, G); break;
    case 3: hipLaunchKernelGGL(decode_tq_kernel<3>, grid, block, 0, st, a, tq, G); break;
    default: hipLaunchKernelGGL(decode_tq_kernel<4>, grid, block, 0, st, a, tq, G); break;
  }
  return hipGetLastError();
}

}  // namespace dec
}  // namespace vrm
