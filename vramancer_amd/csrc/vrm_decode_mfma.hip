// Matrix-core split pass of the paged decode for the quantized pools (gfx950).
//
// Same contract as decode_split_kernel (one wavefront per (sequence, kv-head,
// head group, token partition); partials (max, sum, acc) merged by the
// reduction kernel), but both products run on MFMA instead of the VALU:
//
//  int8:  v_mfma_i32_16x16x64_i8 for QK^T and PV.  The int8 codes are fed to
//         the matrix cores as they sit in memory.  The float32 operand of each
//         product (the query, and the softmax weights times the V scales) is
//         written as three signed 8-bit digits, x ~= s (d1 + d2/254 + d3/254^2)
//         with s = max|x| / 127 per head, so every product is an exact integer
//         dot product and the representation error is below 6.2e-8 * max|x|.
//  fp8:   e4m3fn codes are converted exactly to fp16 (v_cvt_pk_f32_fp8) and
//         multiplied on v_mfma_f32_16x16x32_f16 against a two-term fp16 split
//         (hi + lo) of the float32 operand (about 22 significant bits).
//
// MFMA lane layouts (16x16 tiles, K elements per lane KPL = 16 for i8, 8 for
// f16): A[row][k] sits in lane (row + 16 * (k / KPL)); B[k][col] in lane
// (col + 16 * (k / KPL)); C[row][col] in lane (col + 16 * (row / 4)), register
// row % 4.  Rows are query heads, columns are tokens (QK^T) or head dims (PV).
//
// Memory layout used here (the quantized pools of this library): the K half of
// a (page, layer, head) slice is token-major (16 tokens x D codes), the V half
// is dim-major (D rows of 16 tokens), so a lane's 16-byte load is directly the
// B operand of one MFMA in both products.
#include "vrm_decode.h"

#include <math.h>

namespace vrm {
namespace dec {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr float kInv254 = 1.0f / 254.0f;

// The workgroup is one wavefront, whose LDS accesses execute in order, so a
// compiler-level barrier is all the ordering phases need.  Unlike
// __syncthreads, it does not wait for outstanding global loads, which keeps
// prefetched K/V rows in flight across phase boundaries.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }

__device__ __forceinline__ v4i as_v4i(uint4 u) {
  v4i r;
  r[0] = (int)u.x;
  r[1] = (int)u.y;
  r[2] = (int)u.z;
  r[3] = (int)u.w;
  return r;
}

// Eight e4m3fn codes (two dwords) -> eight fp16 values (exact).
__device__ __forceinline__ v8h fp8x8_to_f16(uint32_t w0, uint32_t w1) {
  const auto a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w0, false);
  const auto b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w0, true);
  const auto c = __builtin_amdgcn_cvt_pk_f32_fp8((int)w1, false);
  const auto d = __builtin_amdgcn_cvt_pk_f32_fp8((int)w1, true);
  v8h r;
  r[0] = (_Float16)a[0];
  r[1] = (_Float16)a[1];
  r[2] = (_Float16)b[0];
  r[3] = (_Float16)b[1];
  r[4] = (_Float16)c[0];
  r[5] = (_Float16)c[1];
  r[6] = (_Float16)d[0];
  r[7] = (_Float16)d[1];
  return r;
}

// Three signed 8-bit digits of u in [-127, 127] (scaled units): u ~= d1 + d2/254 + d3/254^2.
__device__ __forceinline__ void digits3(float u, int& d1, int& d2, int& d3) {
  const float f1 = rintf(u);
  const float r1 = (u - f1) * 254.f;
  const float f2 = rintf(r1);
  const float r2 = (r1 - f2) * 254.f;
  const float f3 = rintf(r2);
  d1 = (int)fminf(fmaxf(f1, -127.f), 127.f);
  d2 = (int)fminf(fmaxf(f2, -127.f), 127.f);
  d3 = (int)fminf(fmaxf(f3, -127.f), 127.f);
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
         ((uint32_t)(d & 0xff) << 24);
}

template <int KIND, int D>
__global__ void __launch_bounds__(64) decode_mfma_kernel(DecodeArgs a, int G) {
  constexpr int KRING = 4;             // pages of K in flight per wavefront
  constexpr int HEAD_BYTES = kPS * D;  // one (page, layer, kv, head) slice of 1-byte codes
  constexpr int NJ = D / 64;           // 16-byte K loads per lane per page
  constexpr int NB = D / 16;           // PV column blocks of 16 head dims
  static_assert(D % 64 == 0, "head_dim must be a multiple of 64");

  const int lane = threadIdx.x;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int split = blockIdx.x;
  const int b = blockIdx.z;
  const int group = a.H / a.KH;
  const int chunks = group / G;
  const int kvh = blockIdx.y / chunks;
  const int h0 = kvh * group + (blockIdx.y % chunks) * G;

  const int ctx = a.ctx_lens[b];
  const int num_pages = ctx > 0 ? min((ctx + kPS - 1) / kPS, a.max_pp) : 0;
  const int p_begin = split * a.pages_per_split;
  const int p_end = min(p_begin + a.pages_per_split, num_pages);
  float* ml_base = a.part_ml + (((size_t)b * a.H + h0) * a.nsplit + split) * 2;
  if (p_begin >= p_end) {
    if (lane < G) {
      ml_base[(size_t)lane * a.nsplit * 2] = -INFINITY;
      ml_base[(size_t)lane * a.nsplit * 2 + 1] = 0.f;
    }
    return;
  }
  const int n_pages = p_end - p_begin;
  const int tok_end = min(p_end * kPS, ctx) - p_begin * kPS;
  const int TS = a.pages_per_split * kPS;  // multiple of 64

  extern __shared__ float lds[];
  float* s_lds = lds;                                        // [G][TS] scores -> operand digits
  float* vs_lds = lds + G * TS;                              // [TS] V dequant factor per token
  int* pid_lds = reinterpret_cast<int*>(vs_lds + TS);        // [pages_per_split]
  float* hstat = reinterpret_cast<float*>(pid_lds + kMaxPagesPerSplit);  // [16][4]: m, l, W

  int my_pid = -1;
  if (lane < n_pages) my_pid = a.page_table[(size_t)b * a.max_pp + p_begin + lane];
  if (lane < a.pages_per_split) pid_lds[lane] = my_pid;
  wave_sync();  // pid_lds is read by other lanes when the V loads are issued

  const size_t kv_stride = (size_t)a.KH * HEAD_BYTES;
  const size_t page_stride = kv_stride * 2 * a.L;
  const uint8_t* layer_base = a.pool + (size_t)a.layer * 2 * kv_stride + (size_t)kvh * HEAD_BYTES;
  auto page_ok = [&](int pid) { return pid >= 0 && pid < a.P; };
  auto head_index = [&](int pid, int kv) { return (((size_t)pid * a.L + a.layer) * 2 + kv) * a.KH + kvh; };

  // ---------------- query operand ----------------
  // This lane's A row is head hq; its k elements are dims j*64 + grp*16 + e.
  const int hq = min(col, G - 1);
  const float* qrow = a.query + ((size_t)b * a.H + h0 + hq) * D;
  float qv[NJ][16];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const float4* src = reinterpret_cast<const float4*>(qrow + j * 64 + grp * 16);
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      const float4 f = src[e4];
      qv[j][4 * e4] = f.x;
      qv[j][4 * e4 + 1] = f.y;
      qv[j][4 * e4 + 2] = f.z;
      qv[j][4 * e4 + 3] = f.w;
    }
  }
  // i8: digit operands QA[j][digit]; f16: hi/lo operands QH[2*j + half][hi|lo]
  v4i QA[KIND == K_I8 ? NJ : 1][3];
  v8h QH[KIND == K_FP8 ? 2 * NJ : 1][2];
  float row_scale[4] = {1.f, 1.f, 1.f, 1.f};  // per C row r: head 4*grp + r
  if constexpr (KIND == K_I8) {
    float qmax = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) qmax = fmaxf(qmax, fabsf(qv[j][e]));
    qmax = fmaxf(qmax, xor_shfl<16>(qmax));
    qmax = fmaxf(qmax, xor_shfl<32>(qmax));
    const float inv = qmax > 0.f ? 127.f / qmax : 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      uint32_t w[3][4];
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        int d[4][3];
#pragma unroll
        for (int i = 0; i < 4; ++i) digits3(qv[j][4 * e4 + i] * inv, d[i][0], d[i][1], d[i][2]);
#pragma unroll
        for (int k = 0; k < 3; ++k) w[k][e4] = pack4(d[0][k], d[1][k], d[2][k], d[3][k]);
      }
#pragma unroll
      for (int k = 0; k < 3; ++k) QA[j][k] = as_v4i(make_uint4(w[k][0], w[k][1], w[k][2], w[k][3]));
    }
    // scale of a digit-1 unit for this lane's head, in the log2 score domain
    const float unit = qmax * (1.f / 127.f) * a.qscale;
#pragma unroll
    for (int r = 0; r < 4; ++r) row_scale[r] = __shfl(unit, 4 * grp + r);
  } else {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = qv[j][half * 8 + e] * a.qscale;
          const _Float16 hi = (_Float16)x;
          QH[2 * j + half][0][e] = hi;
          QH[2 * j + half][1][e] = (_Float16)(x - (float)hi);
        }
  }

  // ---------------- phase 1: scores ----------------
  // Lane (col, grp) loads token col's dims j*64 + grp*16 .. +16 of each page.
  // Pages stream through a ring of KRING register slots so that KRING pages
  // of loads are in flight while one is consumed.
  struct KSlot {
    uint4 k[NJ];
    float ks, vs;
  };
  // Loads are issued unconditionally from a clamped (always valid) address and
  // zeroed afterwards when the page is absent, so every ring slot has the same
  // number of loads in flight and the compiler can wait for the oldest slot
  // only (a branch around a load makes it wait for all of them).
  auto load_k = [&](KSlot& r, int pid) {
    const bool ok = page_ok(pid);
    const int pc = ok ? pid : 0;
    const uint8_t* base = layer_base + (size_t)pc * page_stride + (size_t)col * D + grp * 16;
#pragma unroll
    for (int j = 0; j < NJ; ++j) r.k[j] = ld16(base + j * 64);
    if constexpr (KIND == K_I8) {
      const size_t ts = head_index(pc, 0) * kPS + col;
      r.ks = a.scales[ts];
      r.vs = a.scales[ts + (size_t)a.KH * kPS];
    } else {
      r.ks = a.scales[head_index(pc, 0)];
      r.vs = a.scales[head_index(pc, 1)];
    }
    if (!ok) {
      r.ks = 0.f;
      r.vs = 0.f;
    }
  };
  auto score_page = [&](const KSlot& r, int pi) {
    const int pid = __builtin_amdgcn_readlane(my_pid, pi);
    float sc[4];
    if constexpr (KIND == K_I8) {
      v4i c1 = {0, 0, 0, 0}, c2 = {0, 0, 0, 0}, c3 = {0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const v4i kb = as_v4i(r.k[j]);
        c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(QA[j][0], kb, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(QA[j][1], kb, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(QA[j][2], kb, c3, 0, 0, 0);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        sc[q] = row_scale[q] * r.ks * ((float)c1[q] + ((float)c2[q] + (float)c3[q] * kInv254) * kInv254);
    } else {
      v4f c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const v8h k0 = fp8x8_to_f16(r.k[j].x, r.k[j].y);
        const v8h k1 = fp8x8_to_f16(r.k[j].z, r.k[j].w);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(QH[2 * j][0], k0, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(QH[2 * j][1], k0, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(QH[2 * j + 1][0], k1, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(QH[2 * j + 1][1], k1, c, 0, 0, 0);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) sc[q] = c[q] * r.ks;
    }
    const int t = pi * kPS + col;
    const bool valid = page_ok(pid) && t < tok_end;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int h = 4 * grp + q;
      if (h < G) s_lds[h * TS + t] = valid ? sc[q] : -INFINITY;
    }
    if (grp == 0) vs_lds[t] = valid ? r.vs : 0.f;
  };
  {
    // Ring of KRING pages; slots past the last page reload the last page (an
    // L2 hit) and are never scored.
    KSlot ring[KRING];
    const int last = n_pages - 1;
#pragma unroll
    for (int u = 0; u < KRING; ++u) load_k(ring[u], __builtin_amdgcn_readlane(my_pid, min(u, last)));
    // Fully unrolled over the largest partition (exact trip count, no early
    // exit) so that the wait before each MFMA only covers the oldest slot;
    // pages past n_pages are neither scored nor (beyond the last one) loaded.
#pragma unroll
    for (int pi = 0; pi < kMaxPagesPerSplit; ++pi) {
      if (pi < n_pages) score_page(ring[pi % KRING], pi);
      load_k(ring[pi % KRING], __builtin_amdgcn_readlane(my_pid, min(pi + KRING, last)));
    }
  }

  // The first V loads of phase 3 go out before the softmax phase, which does no
  // global memory traffic of its own.  Phase 3 walks steps s = blk * NCH + ch
  // (column block blk, chunk ch of 4 pages) through a ring of VR slots: slot
  // s % VR holds step s and is refilled with step s + VR.
  constexpr int NCH = kMaxPagesPerSplit / 4;  // chunks of 4 pages per partition, at most
  constexpr int NSTEP = NB * NCH;
  constexpr int VR = 8;                       // 16-byte V rows in flight per lane
  const int nchunks = (n_pages + 3) / 4;
  auto load_v = [&](int step) -> uint4 {
    step = min(step, NSTEP - 1);            // past the end: reload the last row (never used)
    const int blk = step / NCH;
    const int pg = min(step % NCH, nchunks - 1) * 4 + grp;
    const int pid = pg < n_pages ? pid_lds[pg] : -1;
    const bool ok = page_ok(pid);
    const uint4 v = ld16(layer_base + (size_t)(ok ? pid : 0) * page_stride + kv_stride + (size_t)(blk * 16 + col) * kPS);
    return ok ? v : make_uint4(0, 0, 0, 0);
  };
  uint4 vring[VR];
#pragma unroll
  for (int u = 0; u < VR; ++u) vring[u] = load_v(u);
  wave_sync();

  // ---------------- phase 2: softmax statistics and PV operands ----------------
  // For head h: m = max s, p = 2^(s - m), l = sum p, w = p * vscale, W = max w;
  // the A operand of PV is w / W (int8: three digits of 127 w / W; fp8: fp16 hi/lo).
  constexpr int MAXK = kMaxPagesPerSplit * kPS / 64;
  const int nk = TS / 64;
  for (int h = 0; h < G; ++h) {
    float sv[MAXK], wv[MAXK];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
      const int t = lane + 64 * k;
      sv[k] = (k < nk && t < tok_end) ? s_lds[h * TS + t] : -INFINITY;
      mx = fmaxf(mx, sv[k]);
    }
    mx = group_max<64>(mx);
    float sum = 0.f, wmax = 0.f;
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
      const int t = lane + 64 * k;
      const float p = (sv[k] == -INFINITY) ? 0.f : exp2f(sv[k] - mx);
      sum += p;
      wv[k] = (k < nk && t < tok_end) ? p * vs_lds[t] : 0.f;
      wmax = fmaxf(wmax, wv[k]);
    }
    sum = group_sum<64>(sum);
    wmax = group_max<64>(wmax);
    wave_sync();  // every lane has read head h's scores before they are overwritten
    if constexpr (KIND == K_I8) {
      int8_t* dig = reinterpret_cast<int8_t*>(s_lds + h * TS);  // [3][TS]
      const float inv = wmax > 0.f ? 127.f / wmax : 0.f;
#pragma unroll
      for (int k = 0; k < MAXK; ++k) {
        const int t = lane + 64 * k;
        if (k < nk) {
          int d1, d2, d3;
          digits3(wv[k] * inv, d1, d2, d3);
          dig[t] = (int8_t)d1;
          dig[TS + t] = (int8_t)d2;
          dig[2 * TS + t] = (int8_t)d3;
        }
      }
    } else {
      _Float16* ph = reinterpret_cast<_Float16*>(s_lds + h * TS);  // [2][TS]: hi, lo
      const float inv = wmax > 0.f ? 1.f / wmax : 0.f;
#pragma unroll
      for (int k = 0; k < MAXK; ++k) {
        const int t = lane + 64 * k;
        if (k < nk) {
          const float u = wv[k] * inv;
          const _Float16 hi = (_Float16)u;
          ph[t] = hi;
          ph[TS + t] = (_Float16)(u - (float)hi);
        }
      }
    }
    if (lane == 0) {
      hstat[h * 4 + 0] = mx;
      hstat[h * 4 + 1] = sum;
      hstat[h * 4 + 2] = wmax;
    }
  }
  wave_sync();

  // ---------------- phase 3: PV, one 16-dim column block at a time ----------------
  // Step (blk, ch): chunk ch covers pages 4*ch .. 4*ch+3; lane group grp takes
  // page 4*ch + grp, whose 16 tokens of dim (blk*16 + col) are one 16-byte row
  // of the V slice.
  const int hr = min(col, G - 1);
  float* out_base = a.part_acc + ((((size_t)b * a.H + h0) * a.nsplit + split) * D);
  v4i a1 = {0, 0, 0, 0}, a2 = {0, 0, 0, 0}, a3 = {0, 0, 0, 0};
  v4f af = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int blk = 0; blk < NB; ++blk) {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      const int step = blk * NCH + ch;
      const uint4 vc = vring[step % VR];
      vring[step % VR] = load_v(step + VR);
      if (ch < nchunks) {
        if constexpr (KIND == K_I8) {
          const int8_t* dig = reinterpret_cast<const int8_t*>(s_lds + hr * TS) + ch * 64 + grp * 16;
          const v4i p1 = *reinterpret_cast<const v4i*>(dig);
          const v4i p2 = *reinterpret_cast<const v4i*>(dig + TS);
          const v4i p3 = *reinterpret_cast<const v4i*>(dig + 2 * TS);
          const v4i vb = as_v4i(vc);
          a1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(p1, vb, a1, 0, 0, 0);
          a2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(p2, vb, a2, 0, 0, 0);
          a3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(p3, vb, a3, 0, 0, 0);
        } else {
          const _Float16* ph = reinterpret_cast<const _Float16*>(s_lds + hr * TS) + ch * 64 + grp * 16;
          const v8h h0v = *reinterpret_cast<const v8h*>(ph);
          const v8h h1v = *reinterpret_cast<const v8h*>(ph + 8);
          const v8h l0v = *reinterpret_cast<const v8h*>(ph + TS);
          const v8h l1v = *reinterpret_cast<const v8h*>(ph + TS + 8);
          const v8h v0 = fp8x8_to_f16(vc.x, vc.y);  // tokens 0..7 of the page
          const v8h v1 = fp8x8_to_f16(vc.z, vc.w);  // tokens 8..15
          af = __builtin_amdgcn_mfma_f32_16x16x32_f16(h0v, v0, af, 0, 0, 0);
          af = __builtin_amdgcn_mfma_f32_16x16x32_f16(l0v, v0, af, 0, 0, 0);
          af = __builtin_amdgcn_mfma_f32_16x16x32_f16(h1v, v1, af, 0, 0, 0);
          af = __builtin_amdgcn_mfma_f32_16x16x32_f16(l1v, v1, af, 0, 0, 0);
        }
      }
    }
    // column block finished: write it and restart the accumulators
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int h = 4 * grp + q;
      if (h < G) {
        const float W = hstat[h * 4 + 2];
        float val;
        if constexpr (KIND == K_I8)
          val = W * (1.f / 127.f) * ((float)a1[q] + ((float)a2[q] + (float)a3[q] * kInv254) * kInv254);
        else
          val = W * af[q];
        out_base[(size_t)h * a.nsplit * D + blk * 16 + col] = val;
      }
    }
    a1 = v4i{0, 0, 0, 0};
    a2 = v4i{0, 0, 0, 0};
    a3 = v4i{0, 0, 0, 0};
    af = v4f{0.f, 0.f, 0.f, 0.f};
  }
  if (lane < G) {
    ml_base[(size_t)lane * a.nsplit * 2] = hstat[lane * 4 + 0];
    ml_base[(size_t)lane * a.nsplit * 2 + 1] = hstat[lane * 4 + 1];
  }
}

template <int KIND>
hipError_t launch_d(const DecodeArgs& a, int B, int D, int G, hipStream_t st) {
  const int chunks = (a.H / a.KH) / G;
  dim3 grid(a.nsplit, a.KH * chunks, B);
  const int TS = a.pages_per_split * kPS;
  const size_t lds = (size_t)(G + 1) * TS * sizeof(float) + kMaxPagesPerSplit * sizeof(int) + 16 * 4 * sizeof(float);
  switch (D) {
    case 64: hipLaunchKernelGGL((decode_mfma_kernel<KIND, 64>), grid, dim3(64), lds, st, a, G); break;
    case 128: hipLaunchKernelGGL((decode_mfma_kernel<KIND, 128>), grid, dim3(64), lds, st, a, G); break;
    default: hipLaunchKernelGGL((decode_mfma_kernel<KIND, 256>), grid, dim3(64), lds, st, a, G); break;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_quant_mfma(const DecodeArgs& a, int kind, int B, int D, int G, hipStream_t st) {
  if (G < 1 || G > 16 || (a.pages_per_split % 4) != 0 || a.pages_per_split > kMaxPagesPerSplit)
    return hipErrorInvalidValue;
  return kind == K_I8 ? launch_d<K_I8>(a, B, D, G, st) : launch_d<K_FP8>(a, B, D, G, st);
}

}  // namespace dec
}  // namespace vrm
