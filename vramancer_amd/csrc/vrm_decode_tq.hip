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
// weighted sum instead of to every value.  (The formulas are written for
// padded dim PD = 128 and 64 QJL rows; the kernel also serves PD = 64 with 32
// rows, where each lane owns 16 dims instead of 32.)
//
// Work split as in the other stream kernels (work items of find_item, one
// wavefront per (kv-head, head chunk), up to 16 query heads in the columns of
// 16x16 MFMA tiles).  Lane (t, g) = (lane % 16, lane / 16) rebuilds dims
// Q g .. Q g + Q - 1 (Q = PD / 4) of token t of a page from quarter g of the
// token's angle record (vrm_tq_layout.h), multiplying the radius by the
// {cos, sin} of the bin centres level by level (top down to 0) as the
// reference does, so the reconstruction equals the reference's polar decode
// bit for bit.
//   S^T   = K Q^T on v_mfma_f32_16x16x32_f16, K and q_rot as hi + lo fp16
//           (k index (chunk c, group g, element e) <-> dim 32 g + 8 c + e);
//   QJL   = S P^T: the sign bits as exact +-1 fp16 against q_rot JL^T
//           (computed on the matrix cores at set-up, hi + lo);
//   V     rounded to fp16, moved to token-per-lane order by an exact one-hot
//         MFMA transpose, then O^T += V^T P^T with P as hi + lo.
#include "vrm_decode.h"
#include "vrm_tq_layout.h"

#include <math.h>

#include <type_traits>

namespace vrm {
namespace dec {
namespace {

namespace T = vrm::tq;

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;             // wavefronts per workgroup (at most)
constexpr int kWideWaves = 8;         // the wide build: one workgroup per CU sharing a 128 KB table
constexpr int kMaxHeads = 8;          // query heads per wave (hi / lo column halves)
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

// Byte offset (field << LOG2) of the WIDTH-bit field at bit `pos` of the
// little-endian bit stream w[], for a table of 2^LOG2-byte entries: one
// right shift (or a funnel shift where the field straddles two dwords) and
// one mask, the pair gfx950 issues fastest.
template <int WIDTH, int LOG2>
__device__ __forceinline__ uint32_t field_off(const uint32_t* w, int pos) {
  const int dw = pos / 32, sh = pos % 32;
  constexpr uint32_t mask = ((1u << WIDTH) - 1) << LOG2;
  if (sh + WIDTH > 32) return __builtin_amdgcn_alignbit(w[dw + 1], w[dw], sh - LOG2) & mask;
  if (sh >= LOG2) return (w[dw] >> (sh - LOG2)) & mask;
  return (w[dw] << (LOG2 - sh)) & mask;
}

template <typename T>
__device__ __forceinline__ T lds_at(const T* base, uint32_t off) {
  return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + off);
}

// Products of the last polar level rounded to fp16, eight per call: value
// 4 j + k (j = 0, 1; k = 0..3) is y_j t_j.k.  hi gets fp16 of the float32
// product; split8 also gives lo = fp16(y t - hi), the residual of the exact
// product by one mixed-precision fused multiply-add against the fp16 hi.
// (v_fma_mix{lo,hi}_f16 would round each product straight to fp16 in one
// instruction, but on gfx950 each issues at half the rate of a multiply and
// a packed conversion together; measured, this order is 10 % faster.)  The
// results feed matrix-core instructions, which may read a VGPR only two wait
// states after a VALU instruction wrote it.  The compiler pads its own code
// for that but cannot see the writes inside an asm statement, so each block
// ends with s_nop 1 (two wait states).
__device__ __forceinline__ void round8(float y0, const float4& t0, float y1, const float4& t1, uint4& hi) {
  float k[8];
  asm("v_mul_f32 %4, %12, %14\n\t"
      "v_mul_f32 %5, %12, %15\n\t"
      "v_mul_f32 %6, %12, %16\n\t"
      "v_mul_f32 %7, %12, %17\n\t"
      "v_mul_f32 %8, %13, %18\n\t"
      "v_mul_f32 %9, %13, %19\n\t"
      "v_mul_f32 %10, %13, %20\n\t"
      "v_mul_f32 %11, %13, %21\n\t"
      "v_cvt_pk_f16_f32 %0, %4, %5\n\t"
      "v_cvt_pk_f16_f32 %1, %6, %7\n\t"
      "v_cvt_pk_f16_f32 %2, %8, %9\n\t"
      "v_cvt_pk_f16_f32 %3, %10, %11\n\t"
      "s_nop 1"
      : "=&v"(hi.x), "=&v"(hi.y), "=&v"(hi.z), "=&v"(hi.w), "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]),
        "=&v"(k[4]), "=&v"(k[5]), "=&v"(k[6]), "=&v"(k[7])
      : "v"(y0), "v"(y1), "v"(t0.x), "v"(t0.y), "v"(t0.z), "v"(t0.w), "v"(t1.x), "v"(t1.y), "v"(t1.z),
        "v"(t1.w));
}

__device__ __forceinline__ void split8(float y0, const float4& t0, float y1, const float4& t1, uint4& hi, uint4& lo) {
  float k[8];
  asm("v_mul_f32 %8, %16, %18\n\t"
      "v_mul_f32 %9, %16, %19\n\t"
      "v_mul_f32 %10, %16, %20\n\t"
      "v_mul_f32 %11, %16, %21\n\t"
      "v_mul_f32 %12, %17, %22\n\t"
      "v_mul_f32 %13, %17, %23\n\t"
      "v_mul_f32 %14, %17, %24\n\t"
      "v_mul_f32 %15, %17, %25\n\t"
      "v_cvt_pk_f16_f32 %0, %8, %9\n\t"
      "v_cvt_pk_f16_f32 %1, %10, %11\n\t"
      "v_cvt_pk_f16_f32 %2, %12, %13\n\t"
      "v_cvt_pk_f16_f32 %3, %14, %15\n\t"
      "v_fma_mix_f32 %8, %16, %18, -%0 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mix_f32 %9, %16, %19, -%0 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "v_fma_mix_f32 %10, %16, %20, -%1 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mix_f32 %11, %16, %21, -%1 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "v_fma_mix_f32 %12, %17, %22, -%2 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mix_f32 %13, %17, %23, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "v_fma_mix_f32 %14, %17, %24, -%3 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mix_f32 %15, %17, %25, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "v_cvt_pk_f16_f32 %4, %8, %9\n\t"
      "v_cvt_pk_f16_f32 %5, %10, %11\n\t"
      "v_cvt_pk_f16_f32 %6, %12, %13\n\t"
      "v_cvt_pk_f16_f32 %7, %14, %15\n\t"
      "s_nop 1"
      : "=&v"(hi.x), "=&v"(hi.y), "=&v"(hi.z), "=&v"(hi.w), "=&v"(lo.x), "=&v"(lo.y), "=&v"(lo.z), "=&v"(lo.w),
        "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(k[4]), "=&v"(k[5]), "=&v"(k[6]), "=&v"(k[7])
      : "v"(y0), "v"(y1), "v"(t0.x), "v"(t0.y), "v"(t0.z), "v"(t0.w), "v"(t1.x), "v"(t1.y), "v"(t1.z),
        "v"(t1.w));
}

// split8 for tables that also carry fp16 copies of their entries (h0, h1:
// the fp16 t_j.k as two packed pairs each).  hi is the fp16 product of the
// fp16 factors, fp16(y_j) * fp16(t_j.k) by one packed multiply per two values
// (within two units in the last place of fp16(y t)), and lo = fp16(y t - hi)
// is the residual of the exact product as in split8, so hi + lo carries y t
// to the same 22 bits.  Ends with s_nop 1 (its results are MFMA operands).
__device__ __forceinline__ void split8p(float y0, const float4& t0, uint2 h0, float y1, const float4& t1, uint2 h1,
                                        uint4& hi, uint4& lo) {
  float k[8];
  uint32_t yh;
  asm("v_cvt_pk_f16_f32 %16, %17, %18\n\t"
      "v_pk_mul_f16 %0, %27, %16 op_sel_hi:[1,0]\n\t"
      "v_pk_mul_f16 %1, %28, %16 op_sel_hi:[1,0]\n\t"
      "v_pk_mul_f16 %2, %29, %16 op_sel:[0,1] op_sel_hi:[1,1]\n\t"
      "v_pk_mul_f16 %3, %30, %16 op_sel:[0,1] op_sel_hi:[1,1]\n\t"
      "v_fma_mix_f32 %8, %17, %19, -%0 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mix_f32 %9, %17, %20, -%0 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "v_fma_mix_f32 %10, %17, %21, -%1 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mix_f32 %11, %17, %22, -%1 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "v_fma_mix_f32 %12, %18, %23, -%2 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mix_f32 %13, %18, %24, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "v_fma_mix_f32 %14, %18, %25, -%3 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mix_f32 %15, %18, %26, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "v_cvt_pk_f16_f32 %4, %8, %9\n\t"
      "v_cvt_pk_f16_f32 %5, %10, %11\n\t"
      "v_cvt_pk_f16_f32 %6, %12, %13\n\t"
      "v_cvt_pk_f16_f32 %7, %14, %15\n\t"
      "s_nop 1"
      : "=&v"(hi.x), "=&v"(hi.y), "=&v"(hi.z), "=&v"(hi.w), "=&v"(lo.x), "=&v"(lo.y), "=&v"(lo.z), "=&v"(lo.w),
        "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(k[4]), "=&v"(k[5]), "=&v"(k[6]), "=&v"(k[7]),
        "=&v"(yh)
      : "v"(y0), "v"(y1), "v"(t0.x), "v"(t0.y), "v"(t0.z), "v"(t0.w), "v"(t1.x), "v"(t1.y), "v"(t1.z),
        "v"(t1.w), "v"(h0.x), "v"(h0.y), "v"(h1.x), "v"(h1.y));
}

// The P^T operand of eight weights p (float32): fp16(p) where neg_sel is -0
// (hi columns), fp16(p - fp16(p)) where it is -1 (lo columns), as one packed
// conversion per two values, one mixed fused multiply-add per value
// (p + neg_sel * fp16(p), exact) and one packed conversion per two.  The
// result feeds a matrix-core instruction: the block ends with s_nop 1.
__device__ __forceinline__ uint4 weights8(const float (&p)[8], float neg_sel) {
  uint4 out;
  uint32_t h[4];
  float d[8];
  asm("v_cvt_pk_f16_f32 %4, %16, %17\n\t"
      "v_cvt_pk_f16_f32 %5, %18, %19\n\t"
      "v_cvt_pk_f16_f32 %6, %20, %21\n\t"
      "v_cvt_pk_f16_f32 %7, %22, %23\n\t"
      "v_fma_mix_f32 %8, %4, %24, %16 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mix_f32 %9, %4, %24, %17 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
      "v_fma_mix_f32 %10, %5, %24, %18 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mix_f32 %11, %5, %24, %19 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
      "v_fma_mix_f32 %12, %6, %24, %20 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mix_f32 %13, %6, %24, %21 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
      "v_fma_mix_f32 %14, %7, %24, %22 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mix_f32 %15, %7, %24, %23 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
      "v_cvt_pk_f16_f32 %0, %8, %9\n\t"
      "v_cvt_pk_f16_f32 %1, %10, %11\n\t"
      "v_cvt_pk_f16_f32 %2, %12, %13\n\t"
      "v_cvt_pk_f16_f32 %3, %14, %15\n\t"
      "s_nop 1"
      : "=&v"(out.x), "=&v"(out.y), "=&v"(out.z), "=&v"(out.w), "=&v"(h[0]), "=&v"(h[1]), "=&v"(h[2]), "=&v"(h[3]),
        "=&v"(d[0]), "=&v"(d[1]), "=&v"(d[2]), "=&v"(d[3]), "=&v"(d[4]), "=&v"(d[5]), "=&v"(d[6]), "=&v"(d[7])
      : "v"(p[0]), "v"(p[1]), "v"(p[2]), "v"(p[3]), "v"(p[4]), "v"(p[5]), "v"(p[6]), "v"(p[7]), "v"(neg_sel));
  return out;
}

// Maximum over lanes lane % 16 + {0, 16, 32, 48} (the four rows of a
// column), by the VALU lane swaps of gfx950 instead of LDS round trips.
__device__ __forceinline__ float max_rows4(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float m = __builtin_amdgcn_fmed3f(__uint_as_float(a[0]), __uint_as_float(a[1]), INFINITY);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  return __builtin_amdgcn_fmed3f(__uint_as_float(b[0]), __uint_as_float(b[1]), INFINITY);
}

// Value of lane (lane + 8) % 16 of the same row of 16 lanes (DPP row_ror:8).
__device__ __forceinline__ float row_swap8(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xf, 0xf, false));
}

// In-register Walsh-Hadamard transform of PD = 64 or 128 values, element e in
// lane e % 64, register e / 64, in the reference's butterfly order.
template <int PD>
__device__ __forceinline__ void fwht_pd(float (&v)[PD / 64], int lane) {
#pragma unroll
  for (int h = 1; h < 64; h <<= 1) {
#pragma unroll
    for (int k = 0; k < PD / 64; ++k) {
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
  if constexpr (PD == 128) {
    const float a = v[0], b = v[1];
    v[0] = a + b;
    v[1] = a - b;
  }
}

// Dwords of a lane's angle quarter as loaded: quarter grp of a record starts
// at bit grp * PD / 4 * BITS, a dword boundary except at PD 64 and 3 bits,
// where odd quarters start at bit 16 of a dword and take two.
template <int BITS, int PD>
struct QuarterWords {
  static constexpr bool kSplit = (PD / 4 * BITS) % 32 != 0;
  static constexpr int kN = kSplit ? 2 : PD / 4 * BITS / 32;
};

template <int BITS, int PD>
struct TqSlot {
  static constexpr int QW = QuarterWords<BITS, PD>::kN;
  uint32_t kq[QW];    // K angle quarter grp of token col (as loaded)
  uint32_t vq[QW];    // V angle quarter grp of token col
  uint32_t ktop[2];   // dwords of K holding the spares of quarters 0 and 1 + grp / 2 (the top two levels)
  uint32_t vtop[2];
  uint32_t krad, vrad, knorm;  // fp16 bits
  uint32_t ksign[PD / 64];     // PD / 2 QJL sign bits of token col
  bool ok;                     // page id inside the pool (wave-uniform)
};

// WIDE (4 bits at padded dim 128): workgroups of up to kWideWaves
// wavefronts, one per CU, so that its t10 fits in LDS with the fp16 copy
// K's packed hi parts read (128 KB).
template <int BITS, int PD, bool WIDE>
__global__ void __launch_bounds__(64 * (WIDE ? kWideWaves : kWaves), WIDE ? 1 : 2)
    decode_tq_kernel(DecodeArgs a, TqDecodeArgs tq, int G, int hd) {
  constexpr int WAVES = WIDE ? kWideWaves : kWaves;
  constexpr int NB = 1 << BITS;
  constexpr int RING = 4;
  constexpr int SLICE = T::slice_bytes(PD, BITS);
  constexpr int ABYTES = T::angle_bytes(PD, BITS);
  constexpr int D = PD;
  constexpr int QS = T::quarter_slots(PD);  // slots of a quarter = dims a lane rebuilds (32 or 16)
  constexpr int NC = PD / 32;               // 8-dim chunks of a lane's dims
  constexpr int NY = PD / 16;               // level-1 nodes of a lane's dims
  constexpr int NQJ = PD / 64;              // dwords of QJL sign bits per token
  constexpr int PER = PD / 64;              // Hadamard elements per lane
  using QWords = QuarterWords<BITS, PD>;
  using Slot = TqSlot<BITS, PD>;

  // {cos, sin} of the bin centres of levels >= 1, singly and, at 4 bits
  // (levels 3 and 2), for two sibling angles at once (index bin_a + NB bin_b)
  __shared__ float2 lut[NB];
  __shared__ float4 lut2[BITS <= 3 ? 1 : NB * NB];
  __shared__ uint2 sign_mask[16];  // 4 sign bits -> 4 fp16 sign masks (bit i clear: element i negated)
  // Two levels per lookup: for a node angle a and the angles b, c of its two
  // children (index a + NB (b + NB c)), the products (cos a cos b, cos a sin b,
  // sin a cos c, sin a sin c); t10 for levels 1/0 (level 0 has its own bin
  // centres) and, at 2 and 3 bits, t32 for levels 3/2.  They share LDS with
  // qbuf (per wave: q_rot rows before the stream, the output columns after
  // it), which is dead while the tables are read.  At 2 and 3 bits t10 is
  // followed by t10h, the same products as fp16 pairs (the factors of K's
  // packed hi parts, split8p) at the same 16-byte stride, so one address
  // serves both lookups (at 4 bits in the wide build only: 64 KB each).
  constexpr bool kT32 = BITS <= 3;
  // K's hi parts by split8p (at padded dim 64 its extra registers cost the
  // third wavefront per SIMD, measured slower)
  constexpr bool kPackedHi = PD == 128 && (kT32 || WIDE);
  constexpr int NT = NB * NB * NB;
  constexpr int QBUF_BYTES = WAVES * 16 * (D + 4) * 4;
  constexpr int TAB_BYTES = ((kPackedHi ? 2 : 1) + (kT32 ? 1 : 0)) * NT * 16;
  __shared__ __attribute__((aligned(16))) unsigned char shbuf[QBUF_BYTES > TAB_BYTES ? QBUF_BYTES : TAB_BYTES];
  float(*qbuf)[16][D + 4] = reinterpret_cast<float(*)[16][D + 4]>(shbuf);
  float4* t10 = reinterpret_cast<float4*>(shbuf);
  float4* t32 = t10 + (kPackedHi ? 2 : 1) * NT;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int grp = lane >> 4;
  // Matrix-core columns: column n < 8 carries the hi part of head n of the
  // wave's G <= 8 heads, column n + 8 its lo part (columns of heads >= G
  // repeat head G - 1).  A score or output is the sum of columns n and n + 8.
  const int hcol = col & 7;
  const bool lo_col = col >= 8;
  const float neg_sel = lo_col ? -1.f : -0.f;  // P^T: hi columns fp16(p), lo columns fp16(p - fp16(p))
  // byte offset of the cos (+0) or sin (+4) half of a {cos, sin} entry for
  // the top two levels of this lane's dims
  const uint32_t sel6 = (uint32_t)(grp >> 1) << 2, sel5 = (uint32_t)(grp & 1) << 2;
  const int group = a.H / a.KH;
  const int chunks = group / G;
  const int unit = blockIdx.y * (blockDim.x >> 6) + wave;
  const int kvh = unit / chunks;
  const int h0 = kvh * group + (unit % chunks) * G;

  for (int i = threadIdx.x; i < NB; i += blockDim.x) lut[i] = make_float2(tq.lut[2 * NB + i], tq.lut[3 * NB + i]);
  const float* lutf = reinterpret_cast<const float*>(lut);
  if constexpr (BITS > 3) {
    for (int i = threadIdx.x; i < NB * NB; i += blockDim.x) {
      const int ba = i % NB, bb = i / NB;
      lut2[i] = make_float4(tq.lut[2 * NB + ba], tq.lut[3 * NB + ba], tq.lut[2 * NB + bb], tq.lut[3 * NB + bb]);
    }
  }
  if (threadIdx.x < 16) {
    uint32_t h[4];
    for (int e = 0; e < 4; ++e) h[e] = ((threadIdx.x >> e) & 1) ? 0u : 0x8000u;
    sign_mask[threadIdx.x] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
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
  const float root = (float)sqrt((double)PD);
#pragma unroll 1
  for (int r = 0; r < 8; ++r) {
    // the query padded with zeros to the padded dim, as the compressor pads keys
    const float* qrow = a.query + ((size_t)b * a.H + h0 + min(r, G - 1)) * hd;
    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) v[k] = lane + 64 * k < hd ? qrow[lane + 64 * k] * tq.signs[lane + 64 * k] : 0.f;
    fwht_pd<PD>(v, lane);
#pragma unroll
    for (int k = 0; k < PER; ++k) qb[r][lane + 64 * k] = v[k] / root;
  }
  wave_sync();
  // B operand of S^T: x = q_rot[hcol][Q grp + 8 c + e] * qscale as hi
  // (columns < 8) + lo (columns >= 8); against K hi and K lo this sums
  // (Kh + Kl)(qh + ql) over the two column halves.
  v8h QB[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = qb[hcol][QS * grp + 8 * c + e] * a.qscale;
      const _Float16 hi = (_Float16)x;
      const _Float16 lo = (_Float16)(x - (float)hi);
      QB[c][e] = lo_col ? lo : hi;
    }
  // q_proj^T = JL q_rot^T on the matrix cores: tile j (JL rows 16 j ..), result
  // in lane (col, grp) for rows 16 j + 4 grp + r.  The QJL product uses the
  // matching k order: chunk c, element e <-> JL row 16 (2 c + e / 4) + 4 grp + e % 4.
  // PJ carries q_proj times the QJL scale, hi / lo by column half like QB.
  const float qjl_scale = a.qscale * tq.qjl_coef;
  v8h PJ[NQJ];
  {
    float pj[2 * NQJ][4];
#pragma unroll
    for (int j = 0; j < 2 * NQJ; ++j) {
      v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        v8h ah, al, bh, bl;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = tq.jl[(size_t)(16 * j + col) * D + 32 * c + 8 * grp + e];
          ah[e] = (_Float16)x;
          al[e] = (_Float16)(x - (float)ah[e]);
          const float y = qb[hcol][32 * c + 8 * grp + e];
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
    for (int c = 0; c < NQJ; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = pj[2 * c + e / 4][e % 4] * qjl_scale;
        const _Float16 hi = (_Float16)x;
        PJ[c][e] = lo_col ? (_Float16)(x - (float)hi) : hi;
      }
  }
  // one-hot operands of the V transpose: E_h[8 grp + e][col] = (8 grp + e == 16 h + col)
  v8h onehot[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      onehot[h][e] = (grp == 2 * h + (col >> 3) && e == (col & 7)) ? (_Float16)1.f : (_Float16)0.f;

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
      const float4 e = make_float4(cos1[ia] * cos0[ib], cos1[ia] * sin0[ib], sin1[ia] * cos0[ic], sin1[ia] * sin0[ic]);
      t10[i] = e;
      if constexpr (kPackedHi) {
        const uint32_t h01 = __builtin_bit_cast(uint32_t, v2h{(_Float16)e.x, (_Float16)e.y});
        const uint32_t h23 = __builtin_bit_cast(uint32_t, v2h{(_Float16)e.z, (_Float16)e.w});
        t10[NT + i] = make_float4(__uint_as_float(h01), __uint_as_float(h23), 0.f, 0.f);
      }
      if constexpr (kT32)
        t32[i] = make_float4(cos1[ia] * cos1[ib], cos1[ia] * sin1[ib], sin1[ia] * cos1[ic], sin1[ia] * sin1[ic]);
    }
  }
  __syncthreads();

  // ---------------- streaming state ----------------
  float m_run = kNoMax, l_run = 0.f;
  // O^T block 2 c + h: row 4 grp + r <-> dim Q (2 h + (4 grp + r) / 8) + 8 c + (4 grp + r) % 8
  v4f acc[2 * NC];
#pragma unroll
  for (int i = 0; i < 2 * NC; ++i) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};

  const size_t kv_stride = (size_t)a.KH * SLICE;
  const size_t page_stride = kv_stride * 2 * a.L;
  const uint8_t* layer_base = a.pool + (size_t)a.layer * 2 * kv_stride + (size_t)kvh * SLICE;
  auto page_ok = [&](int pid) { return pid >= 0 && pid < a.P; };
  // quarter grp: first dword and bit offset in it (0, or 16 for odd quarters at PD 64 and 3 bits)
  const int q_dw = grp * QS * BITS / 32;
  const uint32_t q_sh = (grp * QS * BITS) % 32;
  // the spare slot QS - 1 of quarter 0 (the root angle) and of quarter
  // 1 + grp / 2 (the next level): dwords, and the spare's bit in them, which
  // is top_sh for every quarter except the odd one at PD 64 and 3 bits (16
  // bits higher, shifted down before use by top1_sh)
  constexpr int top_bit = (QS - 1) * BITS;
  constexpr int top0_dw = top_bit / 32;
  constexpr int top_sh = top_bit % 32;  // a spare never straddles a dword
  const int top1_bit = (1 + (grp >> 1)) * QS * BITS + top_bit;
  const int top1_dw = top1_bit / 32;
  const uint32_t top1_sh = top1_bit % 32 - top_sh;

  auto load_page = [&](Slot& s, int pid) {
    s.ok = page_ok(pid);
    const uint8_t* ks = layer_base + (size_t)(s.ok ? pid : 0) * page_stride;
    const uint8_t* vs = ks + kv_stride;
    const uint32_t* krec = reinterpret_cast<const uint32_t*>(ks + col * ABYTES);
    const uint32_t* vrec = reinterpret_cast<const uint32_t*>(vs + col * ABYTES);
#pragma unroll
    for (int i = 0; i < QWords::kN; ++i) {
      s.kq[i] = krec[q_dw + i];
      s.vq[i] = vrec[q_dw + i];
    }
    s.ktop[0] = krec[top0_dw];
    s.ktop[1] = krec[top1_dw];
    s.vtop[0] = vrec[top0_dw];
    s.vtop[1] = vrec[top1_dw];
    s.krad = reinterpret_cast<const uint16_t*>(ks + T::radius_offset(PD, BITS))[col];
    s.vrad = reinterpret_cast<const uint16_t*>(vs + T::radius_offset(PD, BITS))[col];
    s.knorm = reinterpret_cast<const uint16_t*>(ks + T::norms_offset(PD, BITS))[col];
    if constexpr (NQJ == 2) {
      const uint2 w = reinterpret_cast<const uint2*>(ks + T::signs_offset(PD, BITS))[col];
      s.ksign[0] = w.x;
      s.ksign[NQJ - 1] = w.y;
    } else {
      s.ksign[0] = reinterpret_cast<const uint32_t*>(ks + T::signs_offset(PD, BITS))[col];
    }
  };

  // dims Q grp .. Q grp + Q - 1 of one token: the reference's tree of
  // products, two levels per lookup from the product tables below level 4
  // (4 bits: levels 3 and 2 one at a time with sibling angles together), so
  // each value is the reference's within a float32 rounding or two.
  // Leaves the last level's products to the caller: value 4 j + k of the
  // group is y[j] * t[j][k].  The quarter's words are aligned here, at the
  // point of use, so that the ring's loads stay in flight until then.
  // with_fp16 (std::true_type, tables of 2 and 3 bits): also th[j], the fp16
  // copy of t[j] (split8p's factors).
  auto rebuild = [&](auto with_fp16, const uint32_t* qw, uint32_t top0, uint32_t topq, float radius,
                     float (&y)[NY], float4 (&t)[NY], uint2 (&th)[NY]) {
    uint32_t q[QWords::kN];
    if constexpr (QWords::kSplit) {
      q[0] = __builtin_amdgcn_alignbit(qw[1], qw[0], q_sh);
      q[1] = qw[1] >> q_sh;
      topq >>= top1_sh;
    } else {
#pragma unroll
      for (int i = 0; i < QWords::kN; ++i) q[i] = qw[i];
    }
    // the {cos, sin} entry's component this lane's dims take: cos where the
    // top bit of the dims (bit 6 at PD 128) is clear, sin where set; then
    // the same for the next bit
    const float t6 = lds_at(lutf, field_off<BITS, 3>(&top0, top_sh) | sel6);
    const float t5 = lds_at(lutf, field_off<BITS, 3>(&topq, top_sh) | sel5);
    float p = radius;
    p = p * t6;
    p = p * t5;
    if constexpr (PD == 64) {
      // levels 3 and 2: the quarter's root and its children
      if constexpr (kT32) {
        const float4 t3 = lds_at(t32, field_off<3 * BITS, 4>(q, 12 * BITS));
        y[0] = p * t3.x;
        y[1] = p * t3.y;
        y[2] = p * t3.z;
        y[3] = p * t3.w;
      } else {
        const float2 c3 = lds_at(lut, field_off<BITS, 3>(q, 0));
        const float x2[2] = {p * c3.x, p * c3.y};
        const float4 a2 = lds_at(lut2, field_off<2 * BITS, 4>(q, 1 * BITS));
        y[0] = x2[0] * a2.x;
        y[1] = x2[0] * a2.y;
        y[2] = x2[1] * a2.z;
        y[3] = x2[1] * a2.w;
      }
    } else {
    const float2 c4 = lds_at(lut, field_off<BITS, 3>(q, (kT32 ? 30 : 0) * BITS));  // level 4
    const float x3[2] = {p * c4.x, p * c4.y};
    if constexpr (kT32) {
      // levels 3 and 2: node j and its children in slots 24 + 3 j .. 26 + 3 j
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float4 t = lds_at(t32, field_off<3 * BITS, 4>(q, (24 + 3 * j) * BITS));
        y[4 * j] = x3[j] * t.x;
        y[4 * j + 1] = x3[j] * t.y;
        y[4 * j + 2] = x3[j] * t.z;
        y[4 * j + 3] = x3[j] * t.w;
      }
    } else {
      // level 3 (slots 1, 2), then level 2 (slots 3 .. 6), sibling angles together
      const float4 a3 = lds_at(lut2, field_off<2 * BITS, 4>(q, 1 * BITS));
      const float x2[4] = {x3[0] * a3.x, x3[0] * a3.y, x3[1] * a3.z, x3[1] * a3.w};
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const float4 a2 = lds_at(lut2, field_off<2 * BITS, 4>(q, (3 + i) * BITS));
        y[2 * i] = x2[i] * a2.x;
        y[2 * i + 1] = x2[i] * a2.y;
        y[2 * i + 2] = x2[i + 1] * a2.z;
        y[2 * i + 3] = x2[i + 1] * a2.w;
      }
    }
    }
    // levels 1 and 0: node j and its children in slots 3 j .. 3 j + 2 (4 bits:
    // node slot NY - 1 + j, children slots 2 NY - 1 + 2 j, 2 NY + 2 j)
#pragma unroll
    for (int j = 0; j < NY; ++j) {
      const uint32_t off = kT32 ? field_off<3 * BITS, 4>(q, 3 * j * BITS)
                                : field_off<BITS, 4>(q, (NY - 1 + j) * BITS) |
                                      field_off<2 * BITS, 4 + BITS>(q, (2 * NY - 1 + 2 * j) * BITS);
      t[j] = lds_at(t10, off);
      if constexpr (decltype(with_fp16)::value) th[j] = lds_at(reinterpret_cast<const uint2*>(t10 + NT), off);
    }
  };

  // Scores (log2 domain) of this lane's tokens 4 grp + r of page pi, for
  // head hcol (both column halves hold the same sums).  Unless the pair is
  // full (a present page, every token inside the context), tokens of absent
  // pages and past the context score -inf.
  auto page_scores = [&](const Slot& s, int pi, bool full, float* sc) {
    float y[NY];
    float4 t[NY];
    uint2 th[NY];
    rebuild(std::integral_constant<bool, kPackedHi>{}, s.kq, s.ktop[0], s.ktop[1], f16_to_f32(s.krad), y, t, th);
    v4f c4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      // k = y t as hi (fp16 near k) and lo = fp16(k - hi)
      uint4 hw, lw;
      if constexpr (kPackedHi)
        split8p(y[2 * c], t[2 * c], th[2 * c], y[2 * c + 1], t[2 * c + 1], th[2 * c + 1], hw, lw);
      else
        split8(y[2 * c], t[2 * c], y[2 * c + 1], t[2 * c + 1], hw, lw);
      c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, hw), QB[c], c4, 0, 0, 0);
      c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, lw), QB[c], c4, 0, 0, 0);
    }
    {
      // The QJL term on the same accumulator: row operand +-norm of token col
      // (the fp16 norm with its sign bit flipped where the sign bit is clear;
      // exact), against PJ (zero for scores without the term, whose norms are
      // still finite; tokens past the context are masked below).
      const uint32_t nn = s.knorm | (s.knorm << 16);
#pragma unroll
      for (int c = 0; c < NQJ; ++c) {
        // elements e < 4: JL rows 32 c + 4 grp + e; e >= 4: rows 32 c + 16 + 4 grp + e - 4
        const uint32_t word = s.ksign[c];
        const uint2 lo = sign_mask[__builtin_amdgcn_ubfe(word, 4 * grp, 4)];
        const uint2 hi = sign_mask[__builtin_amdgcn_ubfe(word, 16 + 4 * grp, 4)];
        const v8h sn = __builtin_bit_cast(v8h, make_uint4(nn ^ lo.x, nn ^ lo.y, nn ^ hi.x, nn ^ hi.y));
        c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(sn, PJ[c], c4, 0, 0, 0);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[r] = c4[r] + row_swap8(c4[r]);
    if (!full) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (!(s.ok && pi * kPS + 4 * grp + r < tok_end)) sc[r] = -INFINITY;
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
  auto v_operand = [&](const Slot& s, int pi, bool full, v8h (&vop)[NC]) {
    float y[NY];
    float4 t[NY];
    float radius = f16_to_f32(s.vrad);
    if (!full && !(s.ok && pi * kPS + col < tok_end)) radius = 0.f;
    uint2 th[NY];
    rebuild(std::false_type{}, s.vq, s.vtop[0], s.vtop[1], radius, y, t, th);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      uint4 w;
      round8(y[2 * c], t[2 * c], y[2 * c + 1], t[2 * c + 1], w);
      vop[c] = __builtin_bit_cast(v8h, w);
    }
  };

  auto process_pair = [&](const Slot& s0, const Slot& s1, int pi) {
    // wave-uniform: both pages present and every token inside the context
    const bool full = s0.ok && s1.ok && (pi + 2) * kPS <= tok_end;
    float sc[8];
    page_scores(s0, pi, full, sc);
    page_scores(s1, pi + 1, full, sc + 4);
    float pm = sc[0];
#pragma unroll
    for (int r = 1; r < 8; ++r) pm = fmaxf(pm, sc[r]);
    pm = max_rows4(pm);
    if (pm > m_run + kLazyRescale) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - pm);
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < 2 * NC; ++i) acc[i] *= alpha;
      m_run = pm;
    }
    // P^T as hi (columns < 8) and lo (columns >= 8)
    float pw[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pw[e] = __builtin_amdgcn_exp2f(sc[e] - m_run);
      l_run += pw[e];
    }
    const v8h Bp = __builtin_bit_cast(v8h, weights8(pw, neg_sel));
    v8h vop0[NC], vop1[NC];
    v_operand(s0, pi, full, vop0);
    v_operand(s1, pi + 1, full, vop1);  // past the partition: radius 0
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float t[8];
        v_block(vop0[c], h, t);
        v_block(vop1[c], h, t + 4);
        v8h A;
#pragma unroll
        for (int e = 0; e < 8; ++e) A[e] = (_Float16)t[e];  // exact: fp16 values
        acc[2 * c + h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bp, acc[2 * c + h], 0, 0, 0);
      }
  };

  // ---------------- stream the partition ----------------
  {
    Slot ring[RING];
    const int ids0 = ids_at(0);
    int ids_next = ids_at(RING);
#pragma unroll
    for (int u = 0; u < RING; ++u) load_page(ring[u], __builtin_amdgcn_readlane(ids0, u));
    for (int base = 0; base < n_pages; base += RING) {
      const int ids_ahead = ids_at(base + 2 * RING);
#pragma unroll
      for (int u = 0; u < RING; u += 2) {
        // pages past the partition repeat its last page id; their tokens are
        // past tok_end, so they score -inf and carry radius 0
        process_pair(ring[u], ring[u + 1], base + u);
        load_page(ring[u], __builtin_amdgcn_readlane(ids_next, u));
        load_page(ring[u + 1], __builtin_amdgcn_readlane(ids_next, u + 1));
      }
      ids_next = ids_ahead;
    }
  }

  // ---------------- partition result: columns to natural dims, unrotate ----------------
  __syncthreads();  // the tables are dead once every wave has streamed its pages
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 4 * grp + r;
        // hi column + lo column of head hcol
        qb[col][QS * (2 * h + (row >> 3)) + 8 * c + (row & 7)] = acc[2 * c + h][r] + row_swap8(acc[2 * c + h][r]);
      }
  float l_tot = l_run + xor_shfl<16>(l_run);
  l_tot += xor_shfl<32>(l_tot);
  wave_sync();
  float sg[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) sg[k] = tq.signs[lane + 64 * k];
  for (int hh = 0; hh < G; ++hh) {
    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) v[k] = qb[hh][lane + 64 * k];
    fwht_pd<PD>(v, lane);
    // unrotated, then cut to the head_dim
    float* out = a.part_acc + ((size_t)item * a.H + h0 + hh) * hd;
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (lane + 64 * k < hd) out[lane + 64 * k] = v[k] / root * sg[k];
  }
  if (col < G && grp == 0) {
    float* ml = a.part_ml + ((size_t)item * a.H + h0 + col) * 2;
    ml[0] = l_tot > 0.f ? m_run : -INFINITY;
    ml[1] = l_tot;
  }
}

}  // namespace

template <int PD>
hipError_t launch_tq_pd(const DecodeArgs& a0, const TqDecodeArgs& tq, int bits, int B, int hd, hipStream_t st) {
  const int G = pick_group_tile(a0.H / a0.KH, kMaxHeads);
  const int units = a0.KH * ((a0.H / a0.KH) / G);
  // 4 bits at padded dim 128 take the wide build when its workgroups are full
  const bool wide = bits == 4 && PD == 128 && units % kWideWaves == 0;
  int W = wide ? kWideWaves : kWaves;
  while (units % W) --W;
  DecodeArgs a = a0;
  constexpr bool kHasWide = PD == 128;
  const void* fn = bits == 2   ? reinterpret_cast<const void*>(&decode_tq_kernel<2, PD, false>)
                   : bits == 3 ? reinterpret_cast<const void*>(&decode_tq_kernel<3, PD, false>)
                   : wide      ? reinterpret_cast<const void*>(&decode_tq_kernel<4, PD, kHasWide>)
                               : reinterpret_cast<const void*>(&decode_tq_kernel<4, PD, false>);
  a.target = items_target(fn, W, 0, units);
  dim3 grid(B + 2 * a.target, units / W, 1);
  dim3 block(64 * W);
  switch (bits) {
    case 2: hipLaunchKernelGGL((decode_tq_kernel<2, PD, false>), grid, block, 0, st, a, tq, G, hd); break;
    case 3: hipLaunchKernelGGL((decode_tq_kernel<3, PD, false>), grid, block, 0, st, a, tq, G, hd); break;
    default:
      if (wide)
        hipLaunchKernelGGL((decode_tq_kernel<4, PD, kHasWide>), grid, block, 0, st, a, tq, G, hd);
      else
        hipLaunchKernelGGL((decode_tq_kernel<4, PD, false>), grid, block, 0, st, a, tq, G, hd);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_tq_decode(const DecodeArgs& a0, const TqDecodeArgs& tq, int bits, int B, int hd, hipStream_t st) {
  return hd <= 64 ? launch_tq_pd<64>(a0, tq, bits, B, hd, st) : launch_tq_pd<128>(a0, tq, bits, B, hd, st);
}

}  // namespace dec
}  // namespace vrm
