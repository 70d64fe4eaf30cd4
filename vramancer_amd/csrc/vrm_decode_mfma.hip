// Single-pass matrix-core split kernel of the paged decode for the quantized
// pools (gfx950).
//
// Contract as decode_split_kernel: one wavefront per (sequence, kv-head, head
// group, token partition) leaves (max, sum, unnormalised acc) per query head in
// the workspace and decode_reduce_kernel merges the partitions.
//
// Each page of the partition is streamed once, K and V together, through a
// ring of register slots, with an online softmax:
//   S^T = K Q^T     int8: v_mfma_i32_16x16x64_i8 with the float32 query written
//                   as three signed 8-bit digits q ~= s (d1 + d2/254 + d3/254^2),
//                   s = max|q| / 127 (exact integer dot products; representation
//                   error below 6.2e-8 max|q|);
//                   fp8: e4m3fn -> fp16 (exact) on v_mfma_f32_16x16x32_f16
//                   against a hi + lo fp16 split of the query.
//   O^T += V^T P^T  v_mfma_f32_16x16x32_f16, two pages (32 tokens) per step:
//                   the codes enter as fp16 (exact for int8 and e4m3fn), P is
//                   the softmax weight times the token's (int8) or page's (fp8)
//                   V scale, as a hi + lo fp16 split (about 22 bits).
// The transposed products put one query head in each MFMA column (lane l ->
// head l % 16), so a lane's scores, running maximum, running sum and output
// column all belong to one head and no LDS is needed.
//
// MFMA layouts (16x16 tiles; A[row][k] in lane row + 16 * (k / KPL), B[k][col]
// in lane col + 16 * (k / KPL), C[row][col] in lane col + 16 * (row / 4),
// register row % 4; KPL = 16 for i8, 8 for f16).  Lane (col, grp) =
// (lane % 16, lane / 16).
//
// Pool layout (the quantized pools of this library): in each (page, layer, K/V,
// head) slice K is token-major (as the reference's pool) and V is tiled,
//   V(t, d) at byte ((t / 4 * 16 + d % 16) * (D / 16) + d / 16) * 4 + t % 4,
// so lane (col, grp) finds tokens 4 grp .. 4 grp + 3 of the dims col, col + 16,
// ... (its A operand rows) in D / 4 consecutive bytes.
#include "vrm_decode.h"

#include <math.h>

namespace vrm {
namespace dec {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr float kInv254 = 1.0f / 254.0f;
// The running maximum is raised only when a new score exceeds it by more than
// this (log2 units), so the weights 2^(s - m) stay below 2^kLazyRescale and
// the accumulators are rescaled rarely.
constexpr float kLazyRescale = 3.0f;
// The quantized kernel's PV weights are 2^(s - m - e) * vscale, with e a
// power-of-two exponent of the V scales the stream has seen (vscale < 2^e
// when e was chosen), so the fp16 B operand holds the same relative
// precision whatever the absolute scale of V.  e is raised when a V scale
// reaches 2^(e + kVScaleHeadroom): weights stay below 2^(kLazyRescale +
// kVScaleHeadroom) = 32768 < 65504.
constexpr int kVScaleHeadroom = 12;
// Initial running maximum: finite so that 2^(-inf - m) is 0 for masked tokens.
constexpr float kNoMax = -1.0e30f;

__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }
// 16 bytes at a 4-byte aligned address
__device__ __forceinline__ uint4 ld16_a4(const uint8_t* p) {
  uint4 r;
  __builtin_memcpy(&r, __builtin_assume_aligned(p, 4), 16);
  return r;
}
__device__ __forceinline__ float4 ldf4(const float* p) { return *reinterpret_cast<const float4*>(p); }

__device__ __forceinline__ v4i as_v4i(uint4 u) {
  v4i r;
  r[0] = (int)u.x;
  r[1] = (int)u.y;
  r[2] = (int)u.z;
  r[3] = (int)u.w;
  return r;
}

__device__ __forceinline__ float f4(const float4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

__device__ __forceinline__ uint32_t dword(const uint4& u, int i) { return i == 0 ? u.x : i == 1 ? u.y : i == 2 ? u.z : u.w; }

// Four int8 codes (one dword) -> two dwords of two fp16 each, exact:
// 0x6400 | (c ^ 0x80) is the fp16 value 1152 + c, and 1152 is then subtracted.
__device__ __forceinline__ void i8x4_to_f16(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t u = w ^ 0x80808080u;
  // v_perm_b32: result byte i = byte sel[i] of (src0 << 32 | src1)
  const uint32_t blo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // u0 0x64 u1 0x64
  const uint32_t bhi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // u2 0x64 u3 0x64
  const v2h bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2h, blo) - bias);
  hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2h, bhi) - bias);
}

// Eight e4m3fn codes (two dwords) -> eight fp16 values (exact: every e4m3fn
// value, NaN included, is an fp16 value, and the scale is 1), two codes per
// v_cvt_scalef32_pk_f16_fp8.
__device__ __forceinline__ v8h fp8x8_to_f16(uint32_t w0, uint32_t w1) {
  const v2h a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w0, 1.0f, false);  // bytes 0, 1
  const v2h b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w0, 1.0f, true);   // bytes 2, 3
  const v2h c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w1, 1.0f, false);
  const v2h d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w1, 1.0f, true);
  return v8h{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__device__ __forceinline__ v8h dwords_to_v8h(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return __builtin_bit_cast(v8h, make_uint4(a, b, c, d));
}

// Eight floats w as the float16 pair hi = fp16(w), lo = fp16(w - hi) (the
// residual exact, one rounding): a packed conversion per two values, one
// mixed fused multiply-add per value, a packed conversion per two.  The
// results are matrix-core operands, which may read a VGPR only two wait states
// after a VALU write; the compiler cannot see the writes of an asm statement,
// so the block ends with s_nop 1.
__device__ __forceinline__ void split_hilo8(const float (&w)[8], uint4& hi, uint4& lo) {
  float d[8];
  asm("v_cvt_pk_f16_f32 %0, %16, %17\n\t"
      "v_cvt_pk_f16_f32 %1, %18, %19\n\t"
      "v_cvt_pk_f16_f32 %2, %20, %21\n\t"
      "v_cvt_pk_f16_f32 %3, %22, %23\n\t"
      "v_fma_mix_f32 %8, %0, -1.0, %16 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mix_f32 %9, %0, -1.0, %17 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
      "v_fma_mix_f32 %10, %1, -1.0, %18 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mix_f32 %11, %1, -1.0, %19 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
      "v_fma_mix_f32 %12, %2, -1.0, %20 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mix_f32 %13, %2, -1.0, %21 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
      "v_fma_mix_f32 %14, %3, -1.0, %22 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mix_f32 %15, %3, -1.0, %23 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
      "v_cvt_pk_f16_f32 %4, %8, %9\n\t"
      "v_cvt_pk_f16_f32 %5, %10, %11\n\t"
      "v_cvt_pk_f16_f32 %6, %12, %13\n\t"
      "v_cvt_pk_f16_f32 %7, %14, %15\n\t"
      "s_nop 1"
      : "=&v"(hi.x), "=&v"(hi.y), "=&v"(hi.z), "=&v"(hi.w), "=&v"(lo.x), "=&v"(lo.y), "=&v"(lo.z), "=&v"(lo.w),
        "=&v"(d[0]), "=&v"(d[1]), "=&v"(d[2]), "=&v"(d[3]), "=&v"(d[4]), "=&v"(d[5]), "=&v"(d[6]), "=&v"(d[7])
      : "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]));
}

// Three signed 8-bit digits of u in [-127, 127]: u ~= d1 + d2/254 + d3/254^2.
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

// One page of K and V for this lane, with the scales its tokens need.
template <int D>
struct PageSlot {
  static constexpr int NJ = (D + 63) / 64;
  uint4 k[NJ];  // token col, dims 64 j + 16 grp .. + 15
  uint4 v[NJ];  // tokens 4 grp .. + 3 of dims col + 16 blk, blk = 4 j .. 4 j + 3
  float4 ks;    // int8: K scales of tokens 4 grp .. + 3; fp8: .x = the page's K scale
  float4 vs;    // int8: V scales of the same tokens;      fp8: .x = the page's V scale
  bool ok;      // page id inside the pool (wave-uniform)
};

// Workgroup: W wavefronts for W consecutive (kv-head, head chunk) units of
// one work item (sequence, partition); they stream the neighbouring head slices of
// the same pages (W * 4 KB of K and V per page for int8 D = 128, in one
// contiguous run for a whole page-layer), which keeps DRAM accesses local.
// The wavefronts share nothing and never synchronise.
constexpr int kMaxWaves = 4;
// Balanced mode: one workgroup per (sequence, pair of units), kUnitsPerWg
// units interleaved over its wavefronts (wave w serves unit w % 2), so that
// each unit gets as many older as younger wavefronts: a SIMD issues for its
// oldest wavefront first, and a unit served only by younger wavefronts
// streams about a quarter slower.  The wavefronts of a unit take page pairs
// from an LDS counter, so faster ones take more.

// Balanced-mode epilogue: the partials of the workgroup's wavefronts (max m,
// sum l, unnormalised accumulator; lane (col, grp) holds dims 16 blk + 4 grp +
// r of head col) are merged per unit through LDS with log-sum-exp weights
// 2^(m_w - max m) and written to a.out[b][h0(u) .. h0(u) + G - 1] (and
// a.lse), or, with PARTIAL and not direct, left unnormalised with their
// (max, sum) as work item `item`'s partials for the merge pass.  Every
// wavefront of the workgroup must call it.
template <int D, int NB, bool PARTIAL, int UPW = kUnitsPerWg>
__device__ __forceinline__ void balanced_merge(const DecodeArgs& a, float* lds, int W, int wave, int G, int b,
                                               int item, int unit0, int units, int chunks, const v4f (&acc)[NB],
                                               float m, float l_tot, bool direct = false) {
  const int lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  float* part = lds;
  float* ml = lds + (size_t)W * G * D;
  if (col < G) {
    float* dst = part + ((size_t)wave * G + col) * D;
#pragma unroll
    for (int blk = 0; blk < NB; ++blk)
      *reinterpret_cast<float4*>(dst + blk * 16 + grp * 4) = make_float4(acc[blk][0], acc[blk][1], acc[blk][2], acc[blk][3]);
    if (grp == 0) {
      ml[((size_t)wave * G + col) * 2] = l_tot > 0.f ? m : -INFINITY;
      ml[((size_t)wave * G + col) * 2 + 1] = l_tot;
    }
  }
  __syncthreads();
  // One (unit, head) output row per wavefront at a time: its log-sum-exp
  // weights are computed once (wave-uniform), each lane folds its dims
  // lane + 64 i in the same order as the partials were written.
  const int group = a.H / a.KH;
  constexpr int PER = (D + 63) / 64;
  for (int pr = wave; pr < UPW * G; pr += W) {
    const int ul = pr / G, g = pr - ul * G;
    const int unit = unit0 + ul;
    if (unit >= units) continue;
    float M = -INFINITY;
    for (int w = ul; w < W; w += UPW) M = fmaxf(M, ml[(w * G + g) * 2]);
    float L = 0.f, o[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) o[i] = 0.f;
    if (M != -INFINITY) {
      for (int w = ul; w < W; w += UPW) {
        const float mw = ml[(w * G + g) * 2];
        const float f = mw == -INFINITY ? 0.f : exp2f(mw - M);
        L = fmaf(f, ml[(w * G + g) * 2 + 1], L);
        const float* src = part + ((size_t)w * G + g) * D + lane;
#pragma unroll
        for (int i = 0; i < PER; ++i)
          if (lane + 64 * i < D) o[i] = fmaf(f, src[64 * i], o[i]);
      }
    }
    const int h0 = (unit / chunks) * group + (unit % chunks) * G;
    if (PARTIAL && !direct) {
      const size_t prow = (size_t)item * a.H + h0 + g;
#pragma unroll
      for (int i = 0; i < PER; ++i)
        if (lane + 64 * i < D) a.part_acc[prow * D + lane + 64 * i] = o[i];
      if (lane == 0) {
        a.part_ml[prow * 2] = L > 0.f ? M : -INFINITY;  // o and L are relative to 2^M
        a.part_ml[prow * 2 + 1] = L;
      }
    } else {
      const size_t row = (size_t)b * a.H + h0 + g;
#pragma unroll
      for (int i = 0; i < PER; ++i)
        if (lane + 64 * i < D) a.out[row * D + lane + 64 * i] = L > 0.f ? o[i] * (1.f / L) : 0.f;
      // ln sum_t exp(scale q.k_t) = (max + log2 L) ln 2, the maxima being in the log2 domain
      if (a.lse && lane == 0) a.lse[row] = L > 0.f ? (M + log2f(L)) * 0.6931471805599453f : -INFINITY;
    }
  }
}

// LOADS: a measuring build that issues exactly the kernel's loads (same
// addresses, order, ring and page hand-out) and folds the loaded words into
// a checksum instead of computing: the time of its access pattern alone.
// ITEMS (balanced builds): the workgroup's wavefronts share the pages of one
// work item (a partition of a sequence, sized on the device as for the item
// mode) instead of a whole sequence, and leave the item's merged partials for
// the merge pass: the balanced mode's latency hiding for any batch, with no
// host-side knowledge of the lengths.
//
// stream_item computes work item `item` (balanced: sequence `item`; ITEMS:
// piece `item` of row blockIdx.y) for the unit group wg_units (item mode: the
// units of blockIdx.y).  It returns the number of work items of the batch (1
// in balanced mode, ITEMS: the row's pieces), or 0, having done nothing, when
// there is no such item.
template <int KIND, int D, bool BALANCED, bool LOADS, bool ITEMS, int UPW>
__device__ __forceinline__ int stream_item(const DecodeArgs& a, int G, const int item, const int wg_units) {
  constexpr int RING = D <= 128 ? 4 : 2;  // pages in registers (two being consumed)
  // Pages of 16 << vshift tokens are streamed as 16-token sub-pages: work
  // items, ids and masks count sub-pages, and sub-page v of a sequence is
  // token block v & vmask of its table entry v >> vshift.
  const int vshift = BALANCED ? 0 : a.vshift;  // the balanced mode takes 16-token pages only
  const int vmask = (1 << vshift) - 1;
  constexpr int NJ = (D + 63) / 64;       // 16-byte loads per lane and page, for K and for V
  constexpr int NB = D / 16;              // 16-dim blocks of the output column
  // The last 64-dim chunk holds KPART dims (head_dim 80 / 96 / 112: 16 / 32 /
  // 48): K lanes grp < KPART / 16 and the first KPART / 16 V dwords are real,
  // the rest is zero (never loaded: past the row).
  constexpr int KPART = D - 64 * (NJ - 1);
  static_assert(D % 16 == 0 && D <= 256, "head_dim must be a multiple of 16, at most 256");
  static_assert(RING % 2 == 0, "pages are consumed in pairs");
  // the measuring build leaves its checksum in out, which only the balanced
  // entry sets (item mode writes partials to the workspace)
  static_assert(!LOADS || BALANCED, "the load-only build exists for the balanced mode only");
  static_assert(!ITEMS || (BALANCED && !LOADS), "work items of shared pages are a balanced build that computes");

  // The shared-items pass calls this once per work item in a loop: its lane
  // values are derived afresh per item from an opaque copy of the thread
  // index, since hoisted out of that loop they stay live through the page
  // loop and spill (a lane offset to scratch, compare masks to lanes).
  int tid = threadIdx.x;
  if constexpr (ITEMS) asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int group = a.H / a.KH;
  const int chunks = group / G;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // item mode: the workgroup's waves are W units of one work item; balanced
  // mode: wave w serves unit UPW * wg_units + w % UPW of the
  // item (sequence, or with ITEMS a partition of one)
  const int units = a.KH * chunks;
  const int unit = BALANCED ? wg_units * UPW + wave % UPW : wg_units * (int)(blockDim.x >> 6) + wave;
  const bool unit_ok = !BALANCED || unit < units;
  const int kvh = min(unit, units - 1) / chunks;
  const int h0 = kvh * group + (min(unit, units - 1) % chunks) * G;

  // work item (sequence, partition) of this wave; in item mode the first wave
  // of the launch also records the partition geometry for the merge pass;
  // in balanced mode the item is the whole sequence and the wave takes page
  // pairs of it as it goes
  WorkItem wi;
  int* ids_lds = nullptr;  // balanced mode: the sequence's page ids
  int* pair_ctr = nullptr;
  float* merge_lds = nullptr;
  if constexpr (BALANCED) {
    extern __shared__ __align__(16) int balanced_lds[];
    // the first piece of row r most likely starts sequence r B / rows (it
    // does when the lengths are equal): its page ids are requested together
    // with the lengths, and used if so
    int spec_b = -1, spec_id = 0;
    if constexpr (ITEMS) {
      if (item == 0) {
        spec_b = min((int)((long long)blockIdx.y * a.B / a.target), a.B - 1);
        if (tid < a.max_pp) spec_id = a.page_table[(size_t)spec_b * a.max_pp + tid];
      }
      // every wavefront derives the same item (so the workgroup leaves as a
      // whole, before its first barrier); wave 0 of the first workgroup
      // records the partition geometry for the merge pass
      if (!find_piece(a.ctx_lens, a.B, a.max_pp, a.target, blockIdx.y, item,
                      blockIdx.y == 0 && item == 0 && wg_units == 0 && wave == 0, a.out != nullptr, a.header, wi))
        return 0;
    } else {
      wi.b = item;
      wi.ctx = a.ctx_lens[wi.b];
      wi.p_begin = 0;
      wi.n_pages = seq_pages(wi.ctx, a.max_pp);
      wi.items = 1;
    }
    ids_lds = balanced_lds;
    pair_ctr = balanced_lds + a.max_pp;
    merge_lds = reinterpret_cast<float*>(reinterpret_cast<char*>(balanced_lds) + balanced_merge_offset(a.max_pp));
    const int32_t* row = a.page_table + (size_t)wi.b * a.max_pp + wi.p_begin;  // an item's pages lie in one row
    const bool spec_hit = wi.b == spec_b && wi.p_begin == 0;
    // The item's whole pages are read in ascending order of page id, in
    // kIdBuckets buckets of the id's top bits (a counting sort; the order
    // within a bucket is the LDS atomics').  Over an inline pool a layer's
    // slabs are one run, and workgroups that stream equal lengths then sweep
    // it together: 3.6 % faster than the table's order over a shuffled pool.
    // The online softmax and the merge do not depend on the order; the
    // partial last page keeps its place, where the token bound masks it.
    const int n_whole = min(max(wi.ctx / kPS - wi.p_begin, 0), wi.n_pages);
    if (n_whole >= 4 && n_whole <= (int)blockDim.x) {
      const int t = tid;
      int* const bucket_ctr = pair_ctr + kMaxUnitsPerWg;
      const int shift = max(0, 32 - __clz(max(a.P - 1, 1)) - kIdBucketBits);
      int id = 0, bkt = 0, pos = 0;
      static_assert(kIdBuckets == 64, "one bucket counter per lane of wavefront 0");
      if (wave == 0) bucket_ctr[lane] = 0;
      if (t < n_whole) {
        id = spec_hit ? spec_id : row[t];
        bkt = min(max(id, 0) >> shift, kIdBuckets - 1);  // absent pages: the end buckets
      }
      __syncthreads();
      if (t < n_whole) pos = atomicAdd(&bucket_ctr[bkt], 1);
      __syncthreads();
      if (wave == 0) {
        // exclusive prefix sums of the bucket counts: sums within rows of 16
        // lanes (row_shr 1, 2, 4, 8, zeros shifted in), then the rows'
        // totals (row_bcast 15 into rows 1 and 3, row_bcast 31 into 2 and 3);
        // lane conditions would be hoisted out of the item loop as masks
        const int c = bucket_ctr[lane];
        int x = c;
        x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);
        x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);
        x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);
        x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);
        x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);
        x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);
        bucket_ctr[lane] = x - c;
      }
      __syncthreads();
      if (t < n_whole) ids_lds[bucket_ctr[bkt] + pos] = id;
      for (int i = n_whole + t; i < wi.n_pages; i += blockDim.x) ids_lds[i] = row[i];
    } else {
      for (int i = tid; i < wi.n_pages; i += blockDim.x)
        ids_lds[i] = spec_hit && i == tid ? spec_id : row[i];
    }
    if (tid < UPW) pair_ctr[tid] = 0;
    __syncthreads();
  } else {
    if (!find_item(a.ctx_lens, a.B, a.max_pp << vshift, a.target, item, item == 0 && unit == 0, a.header, wi))
      return 0;
  }
  const int b = wi.b;
  const int batch_items = wi.items;
  const int n_pages = wi.n_pages;
  const int last = n_pages - 1;
  const int tok_end = min(n_pages * kPS, wi.ctx - wi.p_begin * kPS);  // valid tokens of the partition
  // page ids, fetched RING pages ahead of the data: lane u < RING reads the id
  // of page first + u (clamped to the last page)
  const int32_t* prow = a.page_table + (size_t)b * a.max_pp;
  // sub-page id (page << vshift | block), or -1 for an absent page
  auto ids_at = [&](int first) {
    const int v = wi.p_begin + min(first + (lane & (RING - 1)), last);
    const int pid = prow[v >> vshift];
    return pid >= 0 && pid < a.P ? (pid << vshift) | (v & vmask) : -1;
  };

  // (page, layer) slabs and the kv-head's place in them, for codes and scales
  // (the plain and the inline pool layouts differ only in these strides)
  const size_t page_stride = (size_t)a.g.page;
  const uint8_t* layer_base = a.pool + (size_t)a.layer * a.g.layer + (size_t)kvh * a.g.head;
  const size_t s_page_stride = (size_t)a.g.s_page;
  const float* s_layer_base = a.scales + (size_t)a.layer * a.g.s_layer + (size_t)kvh * a.g.s_head;
  auto page_ok = [&](int vpid) { return vpid >= 0 && (vpid >> vshift) < a.P; };

  // Loads are issued unconditionally from a clamped, always valid address and
  // zeroed afterwards for an absent page, so every slot keeps the same loads
  // in flight (a branch around a load makes the compiler wait for all of them).
  // A slot's K half (codes, scales and the page's ok flag) and V half load
  // separately: the balanced mode refills K as soon as a pair's scores are
  // taken and V once its PV product is done.
  auto load_page_part = [&](PageSlot<D>& s, int vpid, bool kpart, bool vpart) {
    const bool ok = page_ok(vpid);
    const int pc = (ok ? vpid : 0) >> vshift;  // page
    const int sub = (ok ? vpid : 0) & vmask;   // its 16-token block
    // K rows and the 4-token V tiles of a block are 16 D bytes past the previous block's
    const uint8_t* pb = layer_base + (size_t)pc * page_stride + sub * (kPS * D);
    const uint8_t* kb = pb + col * D + grp * 16;
    const uint8_t* vb = pb + a.g.kv + (grp * 16 + col) * (D / 4);
    if (kpart) s.ok = ok;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (KPART == 64 || j < NJ - 1) {
        if (kpart) s.k[j] = ld16(kb + j * 64);
        if (vpart) s.v[j] = (D / 4) % 16 == 0 ? ld16(vb + j * 16) : ld16_a4(vb + j * 16);  // V rows of D / 4 bytes
      } else {
        if (kpart) {
          const bool kin = grp < KPART / 16;
          const uint4 kk = ld16(kin ? kb + j * 64 : kb);  // clamped into the row, then dropped
          s.k[j] = kin ? kk : make_uint4(0u, 0u, 0u, 0u);
        }
        if (vpart) {
          const uint32_t* vw = reinterpret_cast<const uint32_t*>(vb + j * 16);
          s.v[j] = make_uint4(vw[0], KPART >= 32 ? vw[1] : 0u, KPART >= 48 ? vw[2] : 0u, 0u);
        }
      }
    }
    const float* sb = s_layer_base + (size_t)pc * s_page_stride;
    if constexpr (KIND == K_I8) {
      const float* ts = sb + sub * kPS + grp * 4;
      if (kpart) s.ks = ldf4(ts);
      if (vpart) s.vs = ldf4(ts + a.g.s_kv);
    } else {
      if (kpart) s.ks = make_float4(sb[0], 0.f, 0.f, 0.f);
      if (vpart) s.vs = make_float4(sb[a.g.s_kv], 0.f, 0.f, 0.f);
    }
    if (vpart && !ok) {
      s.vs = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int j = 0; j < NJ; ++j) s.v[j] = make_uint4(0, 0, 0, 0);
    }
  };
  auto load_page = [&](PageSlot<D>& s, int vpid) { load_page_part(s, vpid, true, true); };

  // balanced mode: take the first page pair and issue its loads before the
  // query set-up, so that the set-up runs under their latency
  const int npairs = (n_pages + 1) / 2;
  int* const pair_next = BALANCED ? pair_ctr + wave % UPW : nullptr;
  auto grab = [&]() {
    int v = 0;
    if constexpr (BALANCED)
      if (lane == 0) v = __hip_atomic_fetch_add(pair_next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return __builtin_amdgcn_readfirstlane(v);
  };
  auto load_pair = [&](PageSlot<D>& s0, PageSlot<D>& s1, int p, bool kpart = true, bool vpart = true) {
    const int pg = 2 * min(p, npairs - 1);
    load_page_part(s0, ids_lds[pg], kpart, vpart);
    load_page_part(s1, ids_lds[min(pg + 1, n_pages - 1)], kpart, vpart);
  };
  PageSlot<D> bring[BALANCED ? 2 : 1];
  int c0 = 0;
  const bool bstream = BALANCED && unit_ok && npairs > 0;
  if constexpr (BALANCED) {
    if (bstream) {
      c0 = grab();
      load_pair(bring[0], bring[1], c0);
    }
  }

  // ---------------- query operand: this lane's head is min(col, G - 1) ----------------
  const float* qrow = a.query + ((size_t)b * a.H + h0 + min(col, G - 1)) * D;
  float qv[NJ][16];  // dims 64 j + 16 grp + e
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      const bool qin = 64 * j + 16 * grp < D;  // 16-dim groups past the head_dim are zero
      const float4 f = qin ? ldf4(qrow + j * 64 + grp * 16 + e4 * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
      qv[j][4 * e4] = f.x;
      qv[j][4 * e4 + 1] = f.y;
      qv[j][4 * e4 + 2] = f.z;
      qv[j][4 * e4 + 3] = f.w;
    }
  v4i QA[KIND == K_I8 ? NJ : 1][3];       // i8: the three digit operands of chunk j
  v8h QH[KIND == K_FP8 ? 2 * NJ : 1][2];  // fp8: hi / lo operands of 32-dim chunk c
  float qunit = 1.f;                      // i8: log2-domain score of one digit-1 unit
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
    qunit = qmax * (1.f / 127.f) * a.qscale;
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

  // ---------------- streaming state ----------------
  float m_run = kNoMax;  // running maximum of this lane's head (equal in its 4 lanes)
  int vexp = 0;          // V-scale exponent e (wave-uniform)
  float vlimit = 0.f;    // 2^(e + kVScaleHeadroom), 0 until the first positive V scale sets e
  float m_eff = kNoMax;  // m_run + e: the weights are 2^(s - m_eff) * vscale
  float l_run = 0.f;     // this lane's share of sum 2^(s - m_eff)
  v4f acc[NB];           // O^T block blk: rows = dims 16 blk + 4 grp + r, column = head
#pragma unroll
  for (int blk = 0; blk < NB; ++blk) acc[blk] = v4f{0.f, 0.f, 0.f, 0.f};

  // Scores (log2 domain) of this lane's 4 tokens 4 grp + r of page pi; -inf
  // for absent pages and tokens past the context.
  auto page_scores = [&](const PageSlot<D>& s, int pi, float* sc) {
    if constexpr (KIND == K_I8) {
      v4i c1 = {0, 0, 0, 0}, c2 = {0, 0, 0, 0}, c3 = {0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const v4i kop = as_v4i(s.k[j]);
        c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop, QA[j][0], c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop, QA[j][1], c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop, QA[j][2], c3, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sc[r] = (qunit * f4(s.ks, r)) * ((float)c1[r] + ((float)c2[r] + (float)c3[r] * kInv254) * kInv254);
    } else {
      v4f c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const v8h k0 = fp8x8_to_f16(s.k[j].x, s.k[j].y);
        const v8h k1 = fp8x8_to_f16(s.k[j].z, s.k[j].w);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, QH[2 * j][0], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, QH[2 * j][1], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, QH[2 * j + 1][0], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, QH[2 * j + 1][1], c, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[r] = c[r] * s.ks.x;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (!(s.ok && pi * kPS + grp * 4 + r < tok_end)) sc[r] = -INFINITY;
  };

  // Pages pi and pi + 1 (the second may lie past the partition).
  uint32_t probe = 0;  // LOADS: checksum of the loaded words
  // after_scores runs once the pair's K half is dead (the balanced mode
  // refills it there).
  auto process_pair = [&](const PageSlot<D>& s0, const PageSlot<D>& s1, int pi, bool has1, auto&& after_scores) {
    if constexpr (LOADS) {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        probe ^= s0.k[j].x ^ s0.k[j].y ^ s0.k[j].z ^ s0.k[j].w ^ s1.k[j].x ^ s1.k[j].y ^ s1.k[j].z ^ s1.k[j].w;
      probe ^= __float_as_uint(s0.ks.x + s0.ks.y + s0.ks.z + s0.ks.w + s1.ks.x + s1.ks.y + s1.ks.z + s1.ks.w);
      after_scores();
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        probe ^= s0.v[j].x ^ s0.v[j].y ^ s0.v[j].z ^ s0.v[j].w ^ s1.v[j].x ^ s1.v[j].y ^ s1.v[j].z ^ s1.v[j].w;
      probe ^= __float_as_uint(s0.vs.x + s0.vs.y + s0.vs.z + s0.vs.w + s1.vs.x + s1.vs.y + s1.vs.z + s1.vs.w);
      (void)pi;
      (void)has1;
      return;
    }
    float sc[8];
    page_scores(s0, pi, sc);
    if (has1) {
      page_scores(s1, pi + 1, sc + 4);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[4 + r] = -INFINITY;
    }
    after_scores();
    // V scales of the pair's tokens (int8: token 4 grp + r % 4 of page
    // pi + r / 4; fp8: vs[0] and vs[4] are the two pages' scales) and V codes.
    float vs[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      vs[r] = KIND == K_I8 ? f4(s0.vs, r) : s0.vs.x;
      vs[4 + r] = has1 ? (KIND == K_I8 ? f4(s1.vs, r) : s1.vs.x) : 0.f;
    }
    uint4 v0[NJ], v1[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      v0[j] = s0.v[j];
      v1[j] = has1 ? s1.v[j] : make_uint4(0u, 0u, 0u, 0u);
    }
    // Only the sequence's last page holds tokens past the context (absent
    // pages were zeroed when loaded).  When the pair reaches it, the scales
    // of those tokens and, for fp8 (whose NaN codes would survive a zero
    // weight), their codes are zeroed, so whatever the pool holds there
    // cannot reach the output.  The test is wave-uniform.
    if ((pi + 2) * kPS > tok_end) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int n_live = min(max(tok_end - (pi + u) * kPS - 4 * grp, 0), 4);  // this lane's live tokens
        if constexpr (KIND == K_I8) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (r >= n_live) vs[4 * u + r] = 0.f;
        } else {
          const uint32_t keep = n_live >= 4 ? 0xffffffffu : (1u << (8 * n_live)) - 1u;  // byte r = token 4 grp + r
          uint4* v = u ? v1 : v0;
#pragma unroll
          for (int j = 0; j < NJ; ++j) v[j] = make_uint4(v[j].x & keep, v[j].y & keep, v[j].z & keep, v[j].w & keep);
        }
      }
    }
    // A V scale at or above 2^(e + kVScaleHeadroom) raises e (wave-uniform);
    // the first positive scale sets it.
    float vm = vs[0];
    if constexpr (KIND == K_I8) {
#pragma unroll
      for (int r = 1; r < 8; ++r) vm = fmaxf(vm, vs[r]);
    } else {
      vm = fmaxf(vm, vs[4]);
    }
    int e_new = vexp;
    if (__builtin_amdgcn_ballot_w64(vm > vlimit) != 0) {
      float wm = fmaxf(vm, xor_shfl<16>(vm));
      wm = fmaxf(wm, xor_shfl<32>(wm));
      if (wm <= 3.0e38f) {  // finite: an inf scale keeps e (its tokens give inf / NaN as in the reference)
        int ex;
        (void)frexpf(wm, &ex);  // wm < 2^ex
        e_new = max(ex, vlimit > 0.f ? vexp : ex);
        vlimit = ldexpf(1.f, e_new + kVScaleHeadroom);
      }
    }
    float pm = sc[0];
#pragma unroll
    for (int r = 1; r < 8; ++r) pm = fmaxf(pm, sc[r]);
    pm = fmaxf(pm, xor_shfl<16>(pm));
    pm = fmaxf(pm, xor_shfl<32>(pm));
    const bool up = pm > m_run + kLazyRescale;
    if (up || e_new != vexp) {
      const float m_new = up ? pm : m_run;
      const float me_new = m_new + (float)e_new;
      const float alpha = __builtin_amdgcn_exp2f(m_eff - me_new);  // 0 while nothing has been accumulated
      l_run *= alpha;
#pragma unroll
      for (int blk = 0; blk < NB; ++blk) acc[blk] *= alpha;
      m_run = m_new;
      m_eff = me_new;
    }
    vexp = e_new;
    // B operand: k = 8 grp + e <-> token 4 grp + e % 4 of page pi + e / 4.
    float w[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const float p = __builtin_amdgcn_exp2f(sc[r] - m_eff);
      l_run += p;
      w[r] = p * (KIND == K_I8 ? vs[r] : vs[r & 4]);
    }
    uint4 bh, bl;
    split_hilo8(w, bh, bl);
    const v8h Bh = __builtin_bit_cast(v8h, bh);
    const v8h Bl = __builtin_bit_cast(v8h, bl);
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      const uint32_t w0 = dword(v0[blk / 4], blk % 4);
      const uint32_t w1 = dword(v1[blk / 4], blk % 4);
      v8h A;
      if constexpr (KIND == K_I8) {
        uint32_t a0, a1, a2, a3;
        i8x4_to_f16(w0, a0, a1);
        i8x4_to_f16(w1, a2, a3);
        A = dwords_to_v8h(a0, a1, a2, a3);
      } else {
        A = fp8x8_to_f16(w0, w1);
      }
      acc[blk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bh, acc[blk], 0, 0, 0);
      acc[blk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bl, acc[blk], 0, 0, 0);
    }
  };

  // ---------------- stream the partition ----------------
  if constexpr (BALANCED) {
    // Page pairs taken from the unit's LDS counter (in increasing order per
    // wave), one pair in registers: its refill is issued once it has been
    // consumed, and the other wavefronts of the SIMD (three per SIMD) keep
    // the memory busy meanwhile.  Fewer bytes in flight than two pairs per
    // wavefront at two per SIMD, and the pool's reads run faster for it.
    // Loads past the last pair reload it (clamped, unconditional).
    if (bstream) {
      while (c0 < npairs) {
        const int n0 = grab();
        process_pair(bring[0], bring[1], 2 * c0, 2 * c0 + 1 < n_pages,
                     [&] { load_pair(bring[0], bring[1], n0, true, false); });
        load_pair(bring[0], bring[1], n0, false, true);
        c0 = n0;
      }
    }
  } else if (n_pages > 0) {
    // Page q sits in slot q % RING.  The refill loads are unconditional (slots
    // past the last page reload it, an L2 hit), so each wait at the top of a
    // pair covers only the slots that pair consumes.
    PageSlot<D> ring[RING];
    const int ids0 = ids_at(0);
    int ids_next = ids_at(RING);
#pragma unroll
    for (int u = 0; u < RING; ++u) load_page(ring[u], __builtin_amdgcn_readlane(ids0, u));
    for (int base = 0; base < n_pages; base += RING) {
      const int ids_ahead = ids_at(base + 2 * RING);
#pragma unroll
      for (int u = 0; u < RING; u += 2) {
        if (base + u < n_pages) process_pair(ring[u], ring[u + 1], base + u, base + u + 1 < n_pages, [] {});
        load_page(ring[u], __builtin_amdgcn_readlane(ids_next, u));
        load_page(ring[u + 1], __builtin_amdgcn_readlane(ids_next, u + 1));
      }
      ids_next = ids_ahead;
    }
  }

  // ---------------- partition result ----------------
  if constexpr (LOADS) {
    a.out[((size_t)b * a.H + h0) * D + lane] = __uint_as_float(probe);  // lane < 64 <= D
    return batch_items;
  }
  float l_tot = l_run + xor_shfl<16>(l_run);
  l_tot += xor_shfl<32>(l_tot);
  if constexpr (BALANCED) {
    // an item that is its whole sequence goes straight to out when the call
    // has one (the merge pass then leaves that sequence alone)
    const bool direct = ITEMS && a.out && wi.p_begin == 0 && wi.n_pages == seq_pages(wi.ctx, a.max_pp);
    balanced_merge<D, NB, ITEMS, UPW>(a, merge_lds, blockDim.x >> 6, wave, G, b, ITEMS ? wi.slot : item,
                                      wg_units * UPW, units, chunks, acc, m_eff, l_tot, direct);
  } else if (col < G) {
    float* out = a.part_acc + ((size_t)item * a.H + h0 + col) * D;
#pragma unroll
    for (int blk = 0; blk < NB; ++blk)
      *reinterpret_cast<float4*>(out + blk * 16 + grp * 4) =
          make_float4(acc[blk][0], acc[blk][1], acc[blk][2], acc[blk][3]);
    if (grp == 0) {
      float* ml_base = a.part_ml + ((size_t)item * a.H + h0) * 2;
      ml_base[col * 2] = l_tot > 0.f ? m_eff : -INFINITY;  // l and acc are relative to 2^m_eff
      ml_base[col * 2 + 1] = l_tot;
    }
  }
  return batch_items;
}

// p, rebuilt as a global-memory pointer (then cast back to a generic one,
// which the compiler's address-space inference follows): its loads and
// stores become global rather than flat ones.
template <typename T>
__device__ __forceinline__ void as_global(T*& p) {
  using G = __attribute__((address_space(1))) T;
  p = (T*)(G*)(uintptr_t)p;
}

// The kernel's DecodeArgs (its first argument), read afresh from the
// kernarg segment through a pointer the compiler cannot follow across the
// iterations of a loop over work: hoisted out of such a loop, the arguments
// stay live in registers through the whole body and cost it spills.  The
// pointers are made global ones again, so that their loads stay global loads.
__device__ __forceinline__ DecodeArgs kernel_args_afresh() {
  using KWord = const __attribute__((address_space(4))) uint32_t;
  KWord* kp = (KWord*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(kp));
  struct Words {
    uint32_t w[sizeof(DecodeArgs) / 4];
  } words;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(DecodeArgs) / 4); ++i) words.w[i] = kp[i];
  DecodeArgs ai = __builtin_bit_cast(DecodeArgs, words);
  as_global(ai.query);
  as_global(ai.pool);
  as_global(ai.scales);
  as_global(ai.page_table);
  as_global(ai.ctx_lens);
  as_global(ai.header);
  as_global(ai.part_acc);
  as_global(ai.part_ml);
  as_global(ai.out);
  as_global(ai.lse);
  return ai;
}

// grid: (work item, unit group), balanced: (sequence, unit group).  ITEMS:
// (unit group, row), one resident round (a.target rows), each workgroup
// taking the pieces of its row (find_piece) in turn: every row carries the
// same number of pages, and no workgroup waits for a CU behind the working
// ones.  Between two pieces every wavefront has passed the first piece's
// merge barrier, so the next piece's page ids and counters overwrite nothing
// still read.
template <int KIND, int D, bool BALANCED, bool LOADS = false, bool ITEMS = false, int UPW = kUnitsPerWg>
__global__ void __launch_bounds__(64 * (BALANCED ? kMaxBalancedWaves : kMaxWaves))
    decode_stream_kernel(DecodeArgs a, int G) {
  static_assert(UPW == kUnitsPerWg || (ITEMS && UPW <= kMaxUnitsPerWg && kMaxBalancedWaves % UPW == 0),
                "only the shared-items pass takes other unit counts");
  if constexpr (ITEMS) {
    for (int item = 0, items = 1; item < items; ++item) {
      const DecodeArgs ai = kernel_args_afresh();
      items = stream_item<KIND, D, BALANCED, LOADS, ITEMS, UPW>(ai, G, item, blockIdx.x);  // 0: no such piece
    }
  } else {
    stream_item<KIND, D, BALANCED, LOADS, ITEMS, UPW>(a, G, blockIdx.x, blockIdx.y);
  }
}


// ---------------------------------------------------------------------------
// Float pools (bf16, f16): the same single-pass stream over the reference's
// token-major pages.
//   S^T = K Q^T     v_mfma_f32_16x16x32_{bf16,f16}: K rows as stored (lane
//                   (t, g) loads dims 32 c + 8 g .. + 7 of token t), the fp32
//                   query as a hi + lo pair of the pool's type.
//   V transpose     the PV product needs each lane to hold tokens, not dims.
//                   One MFMA against a one-hot operand, T = V E_h with
//                   E_h[k][col] = (k == 16 h + col), moves dims 32 c + 16 h +
//                   col of 16 tokens into lane (col, g) as 4 token rows; the
//                   values are copied exactly (one product by 1.0 per output).
//   O^T += V^T P^T  as in the quantized kernel, two pages per step, P as a hi +
//                   lo pair of the pool's type.
// ---------------------------------------------------------------------------
template <int KIND> struct FloatOps;
template <> struct FloatOps<K_BF16> {
  using vec = v8bf;
  using el = __bf16;
  static __device__ __forceinline__ v4f mma(vec a, vec b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static constexpr uint16_t kOne = 0x3f80;
};
template <> struct FloatOps<K_F16> {
  using vec = v8h;
  using el = _Float16;
  static __device__ __forceinline__ v4f mma(vec a, vec b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static constexpr uint16_t kOne = 0x3c00;
};

template <int D>
struct FloatSlot {
  static constexpr int NC = (D + 31) / 32;
  uint4 k[NC];  // token col, dims 32 c + 8 grp .. + 7
  uint4 v[NC];  // same positions of V
  bool ok;      // page id inside the pool (wave-uniform)
};

template <int KIND, int D>
__global__ void __launch_bounds__(64 * kMaxWaves) decode_stream_float_kernel(DecodeArgs a, int G) {
  using Ops = FloatOps<KIND>;
  using vec = typename Ops::vec;
  using el = typename Ops::el;
  // One page pair in registers: its refill is issued when the pair has been
  // consumed.  A float page is twice an int8 one, and four slots per wave put
  // so many bytes in flight that the pool's reads slowed down (bf16, 32
  // sequences of 1k-8k tokens, 28 / 4 heads, D = 128: partition pass 74.5 us
  // with four slots, 72.0 with two).
  constexpr int RING = 2;
  constexpr int ROW = D * 2;              // bytes per token row
  // pages of 16 << vshift tokens streamed as 16-token sub-pages (as in the quantized kernel)
  const int vshift = a.vshift, vmask = (1 << a.vshift) - 1;
  const int head_bytes = (kPS << vshift) * ROW;  // one (page, layer, K/V, head) slice
  constexpr int NC = (D + 31) / 32;       // 32-dim chunks: one 16-byte load per lane each
  constexpr int NB = D / 16;              // 16-dim blocks of the output column
  // head_dim 80 / 112: the last chunk holds 16 dims, lanes grp < 2 (the rest
  // is zero, never loaded: past the row)
  constexpr int CPART = D - 32 * (NC - 1);
  static_assert(D % 16 == 0 && D <= 128, "head_dim must be a multiple of 16, at most 128");

  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int group = a.H / a.KH;
  const int chunks = group / G;
  const int unit = blockIdx.y * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kvh = unit / chunks;
  const int h0 = kvh * group + (unit % chunks) * G;

  // work item (sequence, partition) of this workgroup; the first wave of the
  // launch also records the partition geometry for the merge pass
  const int item = blockIdx.x;
  WorkItem wi;
  if (!find_item(a.ctx_lens, a.B, a.max_pp << vshift, a.target, item, item == 0 && unit == 0, a.header, wi)) return;
  const int b = wi.b;
  const int n_pages = wi.n_pages;
  const int last = n_pages - 1;
  const int tok_end = min(n_pages * kPS, wi.ctx - wi.p_begin * kPS);  // valid tokens of the partition
  // page ids, fetched RING pages ahead of the data: lane u < RING reads the id
  // of page first + u (clamped to the last page)
  const int32_t* prow = a.page_table + (size_t)b * a.max_pp;
  // sub-page id (page << vshift | block), or -1 for an absent page
  auto ids_at = [&](int first) {
    const int v = wi.p_begin + min(first + (lane & (RING - 1)), last);
    const int pid = prow[v >> vshift];
    return pid >= 0 && pid < a.P ? (pid << vshift) | (v & vmask) : -1;
  };
  float* ml_base = a.part_ml + ((size_t)item * a.H + h0) * 2;

  const size_t kv_stride = (size_t)a.KH * head_bytes;
  const size_t page_stride = kv_stride * 2 * a.L;
  const uint8_t* layer_base = a.pool + (size_t)a.layer * 2 * kv_stride + (size_t)kvh * head_bytes;
  auto page_ok = [&](int vpid) { return vpid >= 0 && (vpid >> vshift) < a.P; };

  // query operand (B of S^T): lane (col, grp) holds q[32 c + 8 grp + e] * qscale, hi + lo
  const float* qrow = a.query + ((size_t)b * a.H + h0 + min(col, G - 1)) * D;
  vec QH[NC][2];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const bool qin = 32 * c + 8 * grp < D;
    const float4 f0 = qin ? ldf4(qrow + 32 * c + 8 * grp) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 f1 = qin ? ldf4(qrow + 32 * c + 8 * grp + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float x[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = x[e] * a.qscale;
      const el hi = (el)v;
      QH[c][0][e] = hi;
      QH[c][1][e] = (el)(v - (float)hi);
    }
  }
  // one-hot operands of the V transpose: lane (col, grp), element e is
  // E_h[8 grp + e][col] = (8 grp + e == 16 h + col)
  vec onehot[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      onehot[h][e] = __builtin_bit_cast(el, (uint16_t)((grp == 2 * h + (col >> 3) && e == (col & 7)) ? Ops::kOne : 0));

  float m_run = kNoMax;
  float l_run = 0.f;
  v4f acc[NB];
#pragma unroll
  for (int blk = 0; blk < NB; ++blk) acc[blk] = v4f{0.f, 0.f, 0.f, 0.f};

  auto load_page = [&](FloatSlot<D>& s, int vpid) {
    s.ok = page_ok(vpid);
    const int pc = (s.ok ? vpid : 0) >> vshift;
    const int sub = (s.ok ? vpid : 0) & vmask;
    const uint8_t* kb = layer_base + (size_t)pc * page_stride + (sub * kPS + col) * ROW + grp * 16;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (CPART == 32 || c < NC - 1) {
        s.k[c] = ld16(kb + c * 64);
        s.v[c] = ld16(kb + kv_stride + c * 64);
      } else {
        const bool in = grp < CPART / 8;
        const int off = in ? c * 64 : 0;  // clamped into the row, then dropped
        const uint4 kk = ld16(kb + off), vv = ld16(kb + kv_stride + off);
        s.k[c] = in ? kk : make_uint4(0u, 0u, 0u, 0u);
        s.v[c] = in ? vv : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };

  auto page_scores = [&](const FloatSlot<D>& s, int pi, float* sc) {
    v4f c4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const vec kop = __builtin_bit_cast(vec, s.k[c]);
      c4 = Ops::mma(kop, QH[c][0], c4);
      c4 = Ops::mma(kop, QH[c][1], c4);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[r] = (s.ok && pi * kPS + grp * 4 + r < tok_end) ? c4[r] : -INFINITY;
  };

  // V rows of this lane's token (col) with absent pages and tokens past the
  // context zeroed bitwise, whatever the page holds (NaN included), so that
  // their transposed values are exact zeros; one mask per page, no branch.
  auto v_rows = [&](const FloatSlot<D>& s, int pi, bool page_live, uint4 (&out)[NC]) {
    const uint32_t keep = (page_live && pi * kPS + col < tok_end) ? 0xffffffffu : 0u;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      out[c] = make_uint4(s.v[c].x & keep, s.v[c].y & keep, s.v[c].z & keep, s.v[c].w & keep);
  };
  // V^T of 16 dims (block blk) for this lane's 4 tokens of one page.
  auto v_block = [&](const uint4 (&rows)[NC], int blk, float* out4) {
    const v4f t = Ops::mma(__builtin_bit_cast(vec, rows[blk >> 1]), onehot[blk & 1], v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
    for (int r = 0; r < 4; ++r) out4[r] = t[r];
  };

  auto process_pair = [&](const FloatSlot<D>& s0, const FloatSlot<D>& s1, int pi, bool has1) {
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
      for (int blk = 0; blk < NB; ++blk) acc[blk] *= alpha;
      m_run = pm;
    }
    vec Bh, Bl;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = __builtin_amdgcn_exp2f(sc[e] - m_run);
      l_run += p;
      const el hi = (el)p;
      Bh[e] = hi;
      Bl[e] = (el)(p - (float)hi);
    }
    uint4 rows0[NC], rows1[NC];
    v_rows(s0, pi, s0.ok, rows0);
    v_rows(s1, pi + 1, has1 && s1.ok, rows1);
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      float t[8];
      v_block(rows0, blk, t);
      v_block(rows1, blk, t + 4);
      vec A;
#pragma unroll
      for (int e = 0; e < 8; ++e) A[e] = (el)t[e];  // exact: the values came from the pool
      acc[blk] = Ops::mma(A, Bh, acc[blk]);
      acc[blk] = Ops::mma(A, Bl, acc[blk]);
    }
  };

  {
    FloatSlot<D> ring[RING];
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

  float l_tot = l_run + xor_shfl<16>(l_run);
  l_tot += xor_shfl<32>(l_tot);
  if (col < G) {
    float* out = a.part_acc + ((size_t)item * a.H + h0 + col) * D;
#pragma unroll
    for (int blk = 0; blk < NB; ++blk)
      *reinterpret_cast<float4*>(out + blk * 16 + grp * 4) =
          make_float4(acc[blk][0], acc[blk][1], acc[blk][2], acc[blk][3]);
    if (grp == 0) {
      ml_base[col * 2] = l_tot > 0.f ? m_run : -INFINITY;
      ml_base[col * 2 + 1] = l_tot;
    }
  }
}

// ---------------------------------------------------------------------------
// Q4 pools at head_dim 128: the reference's asymmetric 4-bit layout (per token
// and kv-head D/2 bytes of nibbles, byte j holding dims 2j (low) and 2j + 1
// (high); per 32-dim group a float16 scale and zero point in arrays of their
// own; value = (nibble - zero) * scale), in the same single-pass stream.
//   S^T = K Q^T     per group g, v_mfma_i32_16x16x32_i8 of the nibbles against
//                   the query's three signed 8-bit digits (exact integer dot
//                   products, as in the int8 kernel), then
//                   score = sum_g s_g (q.n_g - z_g sum_{d in g} q_d).
//                   A lane's 8 dims of a group enter as its low nibbles, then
//                   its high nibbles (dims 0 2 4 6 1 3 5 7 of the slice); the
//                   query digits are packed in the same order.
//   V transpose     the one-hot product of the float kernel on the i8 matrix
//                   cores: token col's nibbles move to lane (col, grp) as
//                   tokens 4 grp .. + 3 of one dim, exactly.
//   O^T += V^T P^T  v_mfma_f32_16x16x32_f16 per 16-dim block, the B operand of
//                   the block's group g holding p s_g (hi + lo float16, with
//                   the V-scale exponent of the int8 kernel, so that any fp16
//                   V scale keeps its precision); the zero points' share,
//                   sum_t p s_g z_g per (group, head), is accumulated beside it
//                   and subtracted at the end.
// Scales and zeros (4 x 128 bytes per page and head: K s, K z, V s, V z)
// arrive as one 8-byte load per lane and pass through 1 KB of LDS per wave,
// from which each lane reads the 4 tokens x 4 groups its rows need.
// ---------------------------------------------------------------------------
struct Q4Slot {
  uint32_t k[4];  // token col: dims 32 c + 8 grp .. + 7 (4 bytes of nibbles), group c
  uint32_t v[4];  // the same positions of V
  uint2 sz;       // this lane's 8 bytes of the page's scales / zeros
  bool ok;        // page id inside the pool (wave-uniform)
};

// 8 nibbles (one dword, byte j = dims 2j, 2j + 1) -> i8 operand: low nibbles,
// then high nibbles.
__device__ __forceinline__ long q4_operand(uint32_t w) {
  const uint32_t lo = w & 0x0f0f0f0fu;
  const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;
  return (long)(((uint64_t)hi << 32) | lo);
}

// Dim offset (0 .. 7) inside a lane's 8-dim slice of operand element e.
__device__ __forceinline__ constexpr int q4_dim_of(int e) { return e < 4 ? 2 * e : 2 * (e - 4) + 1; }
// Operand element of dim offset o.
__device__ __forceinline__ constexpr int q4_elem_of(int o) { return (o & 1) ? 4 + (o >> 1) : (o >> 1); }

typedef _Float16 v4h __attribute__((ext_vector_type(4)));

typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

// fp16 bit pattern of 2^k, saturated to infinity above the fp16 range and
// to 0 below its subnormals.
__device__ __forceinline__ uint32_t f16_bits_of_pow2(int k) {
  if (k > 15) return 0x7c00u;
  if (k >= -14) return (uint32_t)(k + 15) << 10;
  return k >= -24 ? 1u << (k + 24) : 0u;
}

// Low halves of two int32 (x, y) as one dword (x in bits 0-15).
__device__ __forceinline__ uint32_t low_halves(int x, int y) {
  return __builtin_amdgcn_perm((uint32_t)y, (uint32_t)x, 0x05040100u);
}

__global__ void __launch_bounds__(64 * kMaxWaves) decode_stream_q4_kernel(DecodeArgs a, int G) {
  constexpr int D = 128;
  constexpr int RING = 4;
  constexpr int ROW = D / 2;             // nibble bytes per token row
  constexpr int HEAD_BYTES = kPS * ROW;  // one (page, layer, K/V, head) slice of codes
  constexpr int NG = D / 32;             // 32-dim groups
  constexpr int NB = D / 16;             // 16-dim blocks of the output column
  constexpr int SZH = kPS * NG * 2;      // bytes of one (page, layer, K/V, head) slice of scales (or zeros)
  static_assert(SZH == 16 * 8, "16 lanes load one slice, 8 bytes each");
  __shared__ __align__(16) uint2 sz_lds[kMaxWaves][2][64];  // [wave][page of the pair][array * 16 + token]

  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int group = a.H / a.KH;
  const int chunks = group / G;
  const int unit = blockIdx.y * (blockDim.x >> 6) + wave;
  const int kvh = unit / chunks;
  const int h0 = kvh * group + (unit % chunks) * G;

  const int item = blockIdx.x;
  WorkItem wi;
  if (!find_item(a.ctx_lens, a.B, a.max_pp, a.target, item, item == 0 && unit == 0, a.header, wi)) return;
  const int b = wi.b;
  const int n_pages = wi.n_pages;
  const int last = n_pages - 1;
  const int tok_end = min(n_pages * kPS, wi.ctx - wi.p_begin * kPS);
  const int32_t* trow = a.page_table + (size_t)b * a.max_pp + wi.p_begin;
  auto ids_at = [&](int first) { return trow[min(first + (lane & (RING - 1)), last)]; };
  float* ml_base = a.part_ml + ((size_t)item * a.H + h0) * 2;

  const size_t kv_stride = (size_t)a.KH * HEAD_BYTES;
  const size_t page_stride = kv_stride * 2 * a.L;
  const uint8_t* layer_base = a.pool + (size_t)a.layer * 2 * kv_stride + (size_t)kvh * HEAD_BYTES;
  auto page_ok = [&](int pid) { return pid >= 0 && pid < a.P; };
  // lane (col, grp) fetches token col of array grp: K scales, K zeros, V scales, V zeros
  // (slice index ((page L + layer) 2 + K/V) KH + kv-head: the page's part is
  // wave-uniform, the K/V part a per-lane offset)
  const uint8_t* sz_base = reinterpret_cast<const uint8_t*>((grp & 1) ? a.q4_zero : a.q4_scale) + col * 8 +
                           (size_t)((grp >> 1) * a.KH + kvh) * SZH;
  const int code_off = col * ROW + grp * 4;  // this lane's bytes in a (page, layer, K/V, head) slice

  // ---------------- query: digits per group, group sums ----------------
  const float* qrow = a.query + ((size_t)b * a.H + h0 + min(col, G - 1)) * D;
  float qv[NG][8];  // dims 32 c + 8 grp + o
#pragma unroll
  for (int c = 0; c < NG; ++c) {
    const float4 f0 = ldf4(qrow + 32 * c + 8 * grp);
    const float4 f1 = ldf4(qrow + 32 * c + 8 * grp + 4);
    qv[c][0] = f0.x; qv[c][1] = f0.y; qv[c][2] = f0.z; qv[c][3] = f0.w;
    qv[c][4] = f1.x; qv[c][5] = f1.y; qv[c][6] = f1.z; qv[c][7] = f1.w;
  }
  float qmax = 0.f;
  float qsum[NG];  // sum over the group of q * qscale (this head)
#pragma unroll
  for (int c = 0; c < NG; ++c) {
    float s = 0.f;
#pragma unroll
    for (int o = 0; o < 8; ++o) {
      qmax = fmaxf(qmax, fabsf(qv[c][o]));
      s += qv[c][o] * a.qscale;
    }
    s += xor_shfl<16>(s);
    s += xor_shfl<32>(s);
    qsum[c] = s;
  }
  qmax = fmaxf(qmax, xor_shfl<16>(qmax));
  qmax = fmaxf(qmax, xor_shfl<32>(qmax));
  const float inv = qmax > 0.f ? 127.f / qmax : 0.f;
  const float qunit = qmax * (1.f / 127.f) * a.qscale * kInv254;  // per unit of 254 d1 + d2 + d3 / 254
  // the zero points' share in the same units: -sum_{d in g} q_d / qunit
  float nqsum[NG];
#pragma unroll
  for (int c = 0; c < NG; ++c) nqsum[c] = qunit > 0.f ? -qsum[c] / qunit : 0.f;
  long QA[NG][3];
#pragma unroll
  for (int c = 0; c < NG; ++c) {
    int d[8][3];
#pragma unroll
    for (int e = 0; e < 8; ++e) digits3(qv[c][q4_dim_of(e)] * inv, d[e][0], d[e][1], d[e][2]);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const uint32_t lo = pack4(d[0][k], d[1][k], d[2][k], d[3][k]);
      const uint32_t hi = pack4(d[4][k], d[5][k], d[6][k], d[7][k]);
      QA[c][k] = (long)(((uint64_t)hi << 32) | lo);
    }
  }
  // one-hot operands of the V transpose: element e of lane (col, grp) is
  // E_h[8 grp + e][col] = 1 when operand row 8 grp + e carries dim 16 h + col
  long onehot[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int e1 = grp == 2 * h + (col >> 3) ? q4_elem_of(col & 7) : -1;
    uint64_t bits = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) bits |= (uint64_t)(e == e1 ? 1 : 0) << (8 * e);
    onehot[h] = (long)bits;
  }

  float m_run = kNoMax;  // running maximum of this lane's head
  int vexp = 0;              // V-scale exponent e (wave-uniform)
  uint32_t vlimit_bits = 0;  // fp16 bits of 2^(e + kVScaleHeadroom), 0 until the first positive V scale sets e
  float m_eff = kNoMax;      // m_run + e: the weights are 2^(s - m_eff) * vscale
  float l_run = 0.f;
  float corr[NG];  // this lane's share of sum_t p s_g z_g for its head, per group
  v4f acc[NB];
#pragma unroll
  for (int g = 0; g < NG; ++g) corr[g] = 0.f;
#pragma unroll
  for (int blk = 0; blk < NB; ++blk) acc[blk] = v4f{0.f, 0.f, 0.f, 0.f};

  auto load_page = [&](Q4Slot& s, int pid) {
    s.ok = page_ok(pid);
    const int pc = s.ok ? pid : 0;
    const uint8_t* kb = layer_base + (size_t)pc * page_stride;  // wave-uniform
#pragma unroll
    for (int c = 0; c < NG; ++c) {
      s.k[c] = *reinterpret_cast<const uint32_t*>(kb + code_off + c * 16);
      s.v[c] = *reinterpret_cast<const uint32_t*>(kb + kv_stride + code_off + c * 16);
    }
    const uint8_t* sb = sz_base + ((size_t)pc * a.L + a.layer) * 2 * a.KH * SZH;  // the page's slices
    s.sz = *reinterpret_cast<const uint2*>(sb);
  };

  // scales / zeros of this lane's tokens 4 grp .. + 3 of one staged page:
  // arr[r][g] = group g of token 4 grp + r
  auto staged = [&](int u, int array, v4h (&arr)[4]) {
    const uint4* p = reinterpret_cast<const uint4*>(&sz_lds[wave][u][array * 16 + 4 * grp]);
    const uint4 x = p[0], y = p[1];
    arr[0] = __builtin_bit_cast(v4h, make_uint2(x.x, x.y));
    arr[1] = __builtin_bit_cast(v4h, make_uint2(x.z, x.w));
    arr[2] = __builtin_bit_cast(v4h, make_uint2(y.x, y.y));
    arr[3] = __builtin_bit_cast(v4h, make_uint2(y.z, y.w));
  };

  auto page_scores = [&](const Q4Slot& s, int u, int pi, float* sc) {
    v4h ks[4], kz[4];
    staged(u, 0, ks);
    staged(u, 1, kz);
    // in units of qunit: sum_g s_g (q.n_g / qunit - z_g sum_{d in g} q_d / qunit)
    float tot[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NG; ++c) {
      const long kop = q4_operand(s.k[c]);
      v4i c1 = {0, 0, 0, 0}, c2 = {0, 0, 0, 0}, c3 = {0, 0, 0, 0};
      c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(kop, QA[c][0], c1, 0, 0, 0);
      c2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(kop, QA[c][1], c2, 0, 0, 0);
      c3 = __builtin_amdgcn_mfma_i32_16x16x32_i8(kop, QA[c][2], c3, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // |c1| <= 15 * 127 * 32 fits 24 bits, and |254 c1 + c2| < 2^24 is
        // exact as a float
        const float d12 = (float)(__mul24(c1[r], 254) + c2[r]);
        const float dot = fmaf((float)c3[r], kInv254, d12);
        tot[r] = fmaf((float)ks[r][c], fmaf((float)kz[r][c], nqsum[c], dot), tot[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[r] = (s.ok && pi * kPS + grp * 4 + r < tok_end) ? tot[r] * qunit : -INFINITY;
  };

  // V^T of 16 dims (block blk) for this lane's 4 tokens of one page, as two
  // dwords of fp16 pairs, exact: the product starts from 0x6400 (fp16 1024),
  // so each 32-bit result holds 0x6400 + nibble, whose low half is the fp16
  // value 1024 + nibble; 1024 is then subtracted (exact).
  const v4i kF16Bias = {0x6400, 0x6400, 0x6400, 0x6400};
  auto v_block = [&](const Q4Slot& s, int blk, uint32_t& d0, uint32_t& d1) {
    const v4i t = __builtin_amdgcn_mfma_i32_16x16x32_i8(q4_operand(s.v[blk >> 1]), onehot[blk & 1], kF16Bias, 0, 0, 0);
    const v2h k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    d0 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2h, low_halves(t[0], t[1])) - k1024);
    d1 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2h, low_halves(t[2], t[3])) - k1024);
  };

  auto process_pair = [&](const Q4Slot& s0, const Q4Slot& s1, int pi, bool has1) {
    // stage both pages' scales / zeros, zeroed for tokens past the context
    // and absent pages (whatever they hold), so that their weights and zero
    // points are exact zeros; the wave's LDS operations complete in order,
    // and the previous pair's reads came before these writes
    const bool live0 = s0.ok && pi * kPS + col < tok_end;
    const bool live1 = has1 && s1.ok && (pi + 1) * kPS + col < tok_end;
    const uint2 z0 = live0 ? s0.sz : make_uint2(0u, 0u), z1 = live1 ? s1.sz : make_uint2(0u, 0u);
    sz_lds[wave][0][lane] = z0;
    sz_lds[wave][1][lane] = z1;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // The V scales of the pair (lanes grp 2 hold token col's four group
    // scales of V): one at or above 2^(e + kVScaleHeadroom) raises e
    // (wave-uniform), the first positive one sets it.  The test compares raw
    // fp16 bits (ordered as the values for non-negative scales; a negative
    // scale's sign bit only sends the pair to the exact path below).
    uint32_t vb;
    {
      const v2u16 a = __builtin_elementwise_max(__builtin_bit_cast(v2u16, z0.x), __builtin_bit_cast(v2u16, z0.y));
      const v2u16 c = __builtin_elementwise_max(__builtin_bit_cast(v2u16, z1.x), __builtin_bit_cast(v2u16, z1.y));
      const v2u16 m = __builtin_elementwise_max(a, c);
      vb = grp == 2 ? max((uint32_t)m[0], (uint32_t)m[1]) : 0u;
    }
    int e_new = vexp;
    if (__builtin_amdgcn_ballot_w64(vb > vlimit_bits) != 0) {
      float vm = 0.f;  // the largest magnitude, exactly
      if (grp == 2) {
        const uint32_t w[4] = {z0.x, z0.y, z1.x, z1.y};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const v2h h = __builtin_bit_cast(v2h, w[i] & 0x7fff7fffu);
          vm = fmaxf(vm, fmaxf((float)h[0], (float)h[1]));
        }
      }
      float wm = fmaxf(vm, xor_shfl<1>(vm));
      wm = fmaxf(wm, xor_shfl<2>(wm));
      wm = fmaxf(wm, xor_shfl<4>(wm));
      wm = fmaxf(wm, xor_shfl<8>(wm));
      wm = fmaxf(wm, xor_shfl<16>(wm));
      wm = fmaxf(wm, xor_shfl<32>(wm));
      if (wm <= 65504.f) {  // finite: an inf scale keeps e (its tokens give inf / NaN as in the reference)
        int ex;
        (void)frexpf(wm, &ex);  // wm < 2^ex
        e_new = max(ex, vlimit_bits > 0u ? vexp : ex);
        vlimit_bits = f16_bits_of_pow2(e_new + kVScaleHeadroom);
      }
    }
    float sc[8];
    page_scores(s0, 0, pi, sc);
    if (has1) {
      page_scores(s1, 1, pi + 1, sc + 4);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[4 + r] = -INFINITY;
    }
    float pm = sc[0];
#pragma unroll
    for (int r = 1; r < 8; ++r) pm = fmaxf(pm, sc[r]);
    pm = fmaxf(pm, xor_shfl<16>(pm));
    pm = fmaxf(pm, xor_shfl<32>(pm));
    const bool up = pm > m_run + kLazyRescale;
    if (up || e_new != vexp) {
      const float m_new = up ? pm : m_run;
      const float me_new = m_new + (float)e_new;
      const float alpha = __builtin_amdgcn_exp2f(m_eff - me_new);  // 0 while nothing has been accumulated
      l_run *= alpha;
#pragma unroll
      for (int g = 0; g < NG; ++g) corr[g] *= alpha;
#pragma unroll
      for (int blk = 0; blk < NB; ++blk) acc[blk] *= alpha;
      m_run = m_new;
      m_eff = me_new;
    }
    vexp = e_new;
    v4h vs[2][4], vz[2][4];
    staged(0, 2, vs[0]);
    staged(0, 3, vz[0]);
    staged(1, 2, vs[1]);
    staged(1, 3, vz[1]);
    // B operands per group: element e <-> token 4 grp + e % 4 of page pi + e / 4
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = __builtin_amdgcn_exp2f(sc[e] - m_eff);
      l_run += p[e];
    }
    v8h Bh[NG], Bl[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      float w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        w[e] = p[e] * (float)vs[e >> 2][e & 3][g];  // 0 for dead tokens (staged zero scale)
        corr[g] = fmaf(w[e], (float)vz[e >> 2][e & 3][g], corr[g]);
      }
      uint4 hw, lw;
      split_hilo8(w, hw, lw);
      Bh[g] = __builtin_bit_cast(v8h, hw);
      Bl[g] = __builtin_bit_cast(v8h, lw);
    }
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      uint32_t a0, a1, a2, a3;
      v_block(s0, blk, a0, a1);
      v_block(s1, blk, a2, a3);
      const v8h A = dwords_to_v8h(a0, a1, a2, a3);  // nibbles: exact
      acc[blk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bh[blk >> 1], acc[blk], 0, 0, 0);
      acc[blk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bl[blk >> 1], acc[blk], 0, 0, 0);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // staged reads before the next pair's writes
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  {
    Q4Slot ring[RING];
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

  float l_tot = l_run + xor_shfl<16>(l_run);
  l_tot += xor_shfl<32>(l_tot);
  float corr_tot[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    corr_tot[g] = corr[g] + xor_shfl<16>(corr[g]);
    corr_tot[g] += xor_shfl<32>(corr_tot[g]);
  }
  if (col < G) {
    float* out = a.part_acc + ((size_t)item * a.H + h0 + col) * D;
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      const float z = corr_tot[blk >> 1];
      *reinterpret_cast<float4*>(out + blk * 16 + grp * 4) =
          make_float4(acc[blk][0] - z, acc[blk][1] - z, acc[blk][2] - z, acc[blk][3] - z);
    }
    if (grp == 0) {
      ml_base[col * 2] = l_tot > 0.f ? m_eff : -INFINITY;  // l and acc are relative to 2^m_eff
      ml_base[col * 2 + 1] = l_tot;
    }
  }
}

template <int KIND, int D>
void launch_kernel(const DecodeArgs& a0, int B, int units, int W, int G, hipStream_t st) {
  const void* fn;
  if constexpr (KIND == K_I8 || KIND == K_FP8)
    fn = reinterpret_cast<const void*>(&decode_stream_kernel<KIND, D, false>);
  else if constexpr (KIND == K_Q4)
    fn = reinterpret_cast<const void*>(&decode_stream_q4_kernel);
  else
    fn = reinterpret_cast<const void*>(&decode_stream_float_kernel<KIND, D <= 128 ? D : 128>);
  DecodeArgs a = a0;
  a.target = items_target(fn, W, 0, units);
  dim3 grid(B + 2 * a.target, units / W, 1);  // at most B + 2 target work items
  dim3 block(64 * W);
  if constexpr (KIND == K_I8 || KIND == K_FP8)
    hipLaunchKernelGGL((decode_stream_kernel<KIND, D, false>), grid, block, 0, st, a, G);
  else if constexpr (KIND == K_Q4)
    hipLaunchKernelGGL(decode_stream_q4_kernel, grid, block, 0, st, a, G);
  else if constexpr (D <= 128)
    hipLaunchKernelGGL((decode_stream_float_kernel<KIND, D>), grid, block, 0, st, a, G);
}

template <int KIND>
hipError_t launch_d(const DecodeArgs& a, int B, int D, int G, hipStream_t st) {
  const int units = a.KH * ((a.H / a.KH) / G);  // (kv-head, head chunk) units per sequence
  int W = kMaxWaves;
  while (units % W) --W;
  switch (D) {
    case 64: launch_kernel<KIND, 64>(a, B, units, W, G, st); break;
    case 80: launch_kernel<KIND, 80>(a, B, units, W, G, st); break;
    case 96: launch_kernel<KIND, 96>(a, B, units, W, G, st); break;
    case 112: launch_kernel<KIND, 112>(a, B, units, W, G, st); break;
    case 128: launch_kernel<KIND, 128>(a, B, units, W, G, st); break;
    default: launch_kernel<KIND, 256>(a, B, units, W, G, st); break;
  }
  return hipGetLastError();
}

// Balanced mode: workgroups of kUnitsPerWg units x WPU wavefronts per unit,
// WPU the largest of 6, 4, 2, 1 whose launch fits one resident round of waves
// and 64 KB of LDS.  Returns hipErrorInvalidValue when even WPU = 1 does not
// fit (page tables too wide for the LDS copy of the ids).
template <int KIND, int D, bool LOADS>
hipError_t launch_balanced_d(const DecodeArgs& a, int B, int G, hipStream_t st) {
  const int units = a.KH * ((a.H / a.KH) / G);
  const int wgs_y = (units + kUnitsPerWg - 1) / kUnitsPerWg;
  // the launch shape of the decode itself, for both builds
  const void* fn = reinterpret_cast<const void*>(&decode_stream_kernel<KIND, D, true, false>);
  const int resident = items_target(fn, kMaxBalancedWaves, 0, 1);  // resident waves (capped)
  for (int wpu = 6; wpu >= 1; wpu = wpu == 6 ? 4 : wpu / 2) {
    const int W = kUnitsPerWg * wpu;
    const size_t lds = balanced_lds_bytes(a.max_pp, W, G, D);
    if (lds > kMaxBalancedLds) continue;
    if (wpu > 1 && (long)B * wgs_y * W > resident) continue;
    hipLaunchKernelGGL((decode_stream_kernel<KIND, D, true, LOADS>), dim3(B, wgs_y, 1), dim3(64 * W), lds, st, a,
                       G);
    return hipGetLastError();
  }
  return hipErrorInvalidValue;
}

// The shared-items pass: 12-wavefront workgroups of UPW units, one resident
// round of rows (a.target) per unit group, each workgroup looping over its
// row's pieces; the merge pass follows.  Four units per workgroup (3
// wavefronts each) when the batch has more sequences than a round has rows of
// two-unit workgroups: twice the rows, so fewer pieces per row, each of which
// drains and refills the wavefronts' page pipeline (c5: 129 sequences over 64
// rows, 244.4 -> 239.8 us); otherwise two (a row is then often one sequence,
// written out directly: c3).
template <int KIND, int D, int UPW>
hipError_t launch_shared_items_upw(const DecodeArgs& a0, int G, size_t lds, hipStream_t st) {
  const int units = a0.KH * ((a0.H / a0.KH) / G);
  const int wgs_y = (units + UPW - 1) / UPW;
  const int W = kMaxBalancedWaves;
  const void* fn = reinterpret_cast<const void*>(&decode_stream_kernel<KIND, D, true, false, true, UPW>);
  if (lds > kMaxBalancedLds) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  DecodeArgs a = a0;
  a.target = items_target(fn, W, lds, wgs_y * W);  // rows: one resident round
  hipLaunchKernelGGL((decode_stream_kernel<KIND, D, true, false, true, UPW>), dim3(wgs_y, a.target, 1), dim3(64 * W),
                     lds, st, a, G);
  return hipGetLastError();
}

template <int KIND, int D>
hipError_t launch_shared_items_d(const DecodeArgs& a0, int B, int G, hipStream_t st) {
  const int units = a0.KH * ((a0.H / a0.KH) / G);
  const size_t lds = balanced_lds_bytes(a0.max_pp, kMaxBalancedWaves, G, D);
  if (lds > shared_items_max_lds()) return hipErrorInvalidValue;
  const void* fn2 = reinterpret_cast<const void*>(&decode_stream_kernel<KIND, D, true, false, true, 2>);
  const int wgs2 = (units + 1) / 2;
  const int rows2 = items_target(fn2, kMaxBalancedWaves, lds, wgs2 * kMaxBalancedWaves);
  if (units >= 4 && B > rows2) return launch_shared_items_upw<KIND, D, 4>(a0, G, lds, st);
  return launch_shared_items_upw<KIND, D, 2>(a0, G, lds, st);
}

template <int KIND>
hipError_t launch_shared_items_kind(const DecodeArgs& a, int B, int D, int G, hipStream_t st) {
  switch (D) {
    case 64: return launch_shared_items_d<KIND, 64>(a, B, G, st);
    case 80: return launch_shared_items_d<KIND, 80>(a, B, G, st);
    case 96: return launch_shared_items_d<KIND, 96>(a, B, G, st);
    case 112: return launch_shared_items_d<KIND, 112>(a, B, G, st);
    case 128: return launch_shared_items_d<KIND, 128>(a, B, G, st);
    default: return hipErrorInvalidValue;
  }
}

template <int KIND, bool LOADS>
hipError_t launch_balanced_kind(const DecodeArgs& a, int B, int D, int G, hipStream_t st) {
  switch (D) {
    case 64: return launch_balanced_d<KIND, 64, LOADS>(a, B, G, st);
    case 80: return launch_balanced_d<KIND, 80, LOADS>(a, B, G, st);
    case 96: return launch_balanced_d<KIND, 96, LOADS>(a, B, G, st);
    case 112: return launch_balanced_d<KIND, 112, LOADS>(a, B, G, st);
    case 128: return launch_balanced_d<KIND, 128, LOADS>(a, B, G, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_q4(const DecodeArgs& a, int B, int G, hipStream_t st) {
  const int units = a.KH * ((a.H / a.KH) / G);
  int W = kMaxWaves;
  while (units % W) --W;
  launch_kernel<K_Q4, 128>(a, B, units, W, G, st);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_stream_balanced(const DecodeArgs& a, int kind, int B, int D, int G, hipStream_t st,
                                  bool loads_only) {
  if (G < 1 || G > 16) return hipErrorInvalidValue;
  switch (kind) {
    case K_I8:
      return loads_only ? launch_balanced_kind<K_I8, true>(a, B, D, G, st)
                        : launch_balanced_kind<K_I8, false>(a, B, D, G, st);
    case K_FP8:
      return loads_only ? launch_balanced_kind<K_FP8, true>(a, B, D, G, st)
                        : launch_balanced_kind<K_FP8, false>(a, B, D, G, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_stream_shared_items(const DecodeArgs& a, int kind, int B, int D, int G, hipStream_t st) {
  if (G < 1 || G > 16) return hipErrorInvalidValue;
  switch (kind) {
    case K_I8: return launch_shared_items_kind<K_I8>(a, B, D, G, st);
    case K_FP8: return launch_shared_items_kind<K_FP8>(a, B, D, G, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_stream_mfma(const DecodeArgs& a, int kind, int B, int D, int G, hipStream_t st) {
  if (G < 1 || G > 16) return hipErrorInvalidValue;
  switch (kind) {
    case K_I8: return launch_d<K_I8>(a, B, D, G, st);
    case K_FP8: return launch_d<K_FP8>(a, B, D, G, st);
    case K_BF16: return D <= 128 ? launch_d<K_BF16>(a, B, D, G, st) : hipErrorInvalidValue;
    case K_F16: return D <= 128 ? launch_d<K_F16>(a, B, D, G, st) : hipErrorInvalidValue;
    case K_Q4: return D == 128 ? launch_q4(a, B, G, st) : hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dec
}  // namespace vrm
