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
#include "vrm_tq_common.h"
#include "vrm_tq_layout.h"

#include <math.h>

namespace vrm {
namespace {

#pragma clang fp contract(off)

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

// Element e of the polar decode of one row from the fp32 radius and the
// level-major bins (level l at offset PD - (PD >> l)).  The reference decodes
// level by level from the top, each value r of level l becoming the pair
// (r cos, r sin) of level l - 1; element e is therefore the product chain
//   ((radius * f_{NL-1}) * f_{NL-2}) ... * f_0,
// f_l the cos (bit l of e clear) or sin (set) of angle e >> (l + 1) of level
// l, the same roundings in the same order, with no exchange between lanes.
template <int PD>
__device__ __forceinline__ float polar_element(float radius, const uint8_t* bins, const float* lut, int nb, int e) {
  constexpr int NL = __builtin_ctz(PD);
  float r = radius;
#pragma unroll
  for (int l = NL - 1; l >= 0; --l) {
    const int idx = min((int)bins[PD - (PD >> l) + (e >> (l + 1))], nb - 1);  // caller-supplied bins stay in the table
    r = __fmul_rn(r, lut[(l == 0 ? 0 : 2 * nb) + (((e >> l) & 1) ? nb : 0) + idx]);
  }
  return r;
}

// Polar decode of one row into `recon` (LDS, PD floats); bins may have been
// written by any lane before the call, recon is visible to every lane after.
template <int PD>
__device__ __forceinline__ void polar_decode(float radius, const uint8_t* bins, const float* lut, int nb,
                                             float* recon, int lane) {
  row_sync();
#pragma unroll
  for (int k = 0; k < tq_per_lane(PD); ++k)
    if (k * 64 + lane < PD) recon[k * 64 + lane] = polar_element<PD>(radius, bins, lut, nb, k * 64 + lane);
  row_sync();
}

// LDS working set of one row.
template <int PD>
struct RowLds {
  float rot[PD];               // rotated row
  float rad[PD];               // radius of each polar node, level-major like the bins
  alignas(16) double res[PD];  // QJL residual, widened once by the lane that owns it
  uint8_t bins[PD];
  float norm_acc[8];
};

// Rotation and polar encoding of one row (source element e at src[e] for
// e < head_dim, zero padding above): leaves the level-major bins in w.bins,
// the rotated row in v (element e in lane e % 64, register e / 64; lanes past
// a row of fewer than 64 elements hold zeros) and in w.rot, and returns the
// fp32 final radius.
template <int SRC, int PD>
__device__ __forceinline__ float encode_row(const void* src, size_t first, int head_dim, const float* signs, int bits,
                                            float (&v)[tq_per_lane(PD)], RowLds<PD>& w, int lane) {
  constexpr int PER = tq_per_lane(PD);
  constexpr int NL = __builtin_ctz(PD);
  const int nb = 1 << bits;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int e = k * 64 + lane;
    const float x = e < head_dim ? load_row<SRC>(src, first + e) : 0.f;
    v[k] = e < PD ? __fmul_rn(x, signs[e]) : 0.f;
  }
  fwht<PD>(v, lane);
  const float root = (float)sqrt((double)PD);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    v[k] = __fdiv_rn(v[k], root);
    if (k * 64 + lane < PD) w.rot[k * 64 + lane] = v[k];
  }
  row_sync();

  // The radii only need square roots, level after level: node i of level l
  // (w.rad[PD - (PD >> l) + i]) over children 2 i, 2 i + 1 of level l - 1
  // (the rotated row below level 0).
  for (int level = 0; level < NL; ++level) {
    const float* child = level == 0 ? w.rot : w.rad + (PD - (PD >> (level - 1)));
    float* rad = w.rad + (PD - (PD >> level));
    for (int i = lane; i < (PD >> (level + 1)); i += 64) {
      const float x0 = child[2 * i], x1 = child[2 * i + 1];
      rad[i] = sqrt_rn(__fadd_rn(__fadd_rn(__fmul_rn(x0, x0), __fmul_rn(x1, x1)), 1e-12f));
    }
    row_sync();
  }
  // With every child known, the angles of all levels are independent: lane
  // takes bins b = lane, lane + 64, ... of the level-major order.
  const float lo0 = (float)-3.141592653589793, range0 = (float)6.283185307179586;
  const float range1 = (float)1.5707963267948966;
  const float nbf = (float)nb;
  for (int b = lane; b < PD - 1; b += 64) {
    const int level = NL - 1 - (31 - __builtin_clz(PD - b - 1));  // PD >> (level + 1) < PD - b <= PD >> level
    const int i = b - (PD - (PD >> level));
    const float* child = level == 0 ? w.rot : w.rad + (PD - (PD >> (level - 1)));
    const float x0 = child[2 * i], x1 = child[2 * i + 1];
    const float th = vrm_fdlibm::atan2f(x1, x0);
    const float nrm = level == 0 ? __fdiv_rn(__fsub_rn(th, lo0), range0) : __fdiv_rn(th, range1);
    int idx = (int)__fmul_rn(nrm, nbf);  // truncation toward zero, as .long()
    idx = min(max(idx, 0), nb - 1);
    w.bins[b] = (uint8_t)idx;
  }
  row_sync();
  return w.rad[PD - 2];
}

// Residual against the reconstruction from the fp32 radius, its QJL signs
// (float64 dot products; sign(j) is handed to put_sign) and the residual norm
// as PyTorch's CPU 2-norm reduces a row: eight interleaved fused accumulators
// summed in order for rows of 4 floats or more, one fused chain for a row of
// 2 (measured against torch.norm at 2 .. 256 floats).  Returns the norm.
template <int PD, typename PutSign>
__device__ __forceinline__ float qjl_row(const float (&v)[tq_per_lane(PD)], float radius, const float* lut, int bits,
                                         const float* jl, int qjl_dim, RowLds<PD>& w, int lane, PutSign put_sign) {
  constexpr int PER = tq_per_lane(PD);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int e = k * 64 + lane;
    if (e < PD) w.res[e] = (double)__fsub_rn(v[k], polar_element<PD>(radius, w.bins, lut, 1 << bits, e));
  }
  row_sync();
  // Lane j walks row j of the JL matrix.  With a 16-byte aligned matrix (every
  // row is then aligned, PD being a multiple of 4) it reads four floats per
  // load; the residual comes as doubles, two per LDS broadcast.  The
  // accumulation order is the element order either way.
  const bool vec = PD >= 4 && (reinterpret_cast<uintptr_t>(jl) & 15) == 0;
  const double2* r2 = reinterpret_cast<const double2*>(w.res);
  for (int j = lane; j < qjl_dim; j += 64) {
    const float* jr = jl + (size_t)j * PD;
    double s = 0.0;
    if (vec) {
      const float4* jr4 = reinterpret_cast<const float4*>(jr);
#pragma unroll 8
      for (int m = 0; m < PD / 4; ++m) {
        const float4 x = jr4[m];
        const double2 ra = r2[2 * m], rb = r2[2 * m + 1];
        s = fma(ra.x, (double)x.x, s);
        s = fma(ra.y, (double)x.y, s);
        s = fma(rb.x, (double)x.z, s);
        s = fma(rb.y, (double)x.w, s);
      }
    } else {
      for (int e = 0; e < PD; ++e) s = fma(w.res[e], (double)jr[e], s);
    }
    put_sign(j, s > 0.0);
  }
  if constexpr (PD == 2) {
    const float x0 = (float)w.res[0], x1 = (float)w.res[1];  // exact: widened from floats
    return sqrt_rn(fmaf(x1, x1, __fmul_rn(x0, x0)));
  }
  if (lane < 8) {
    float acc = 0.f;
#pragma unroll
    for (int m = 0; m < (PD + 7) / 8; ++m) {
      if (lane + 8 * m < PD) {
        const float x = (float)w.res[lane + 8 * m];  // exact: widened from a float
        acc = fmaf(x, x, acc);
      }
    }
    w.norm_acc[lane] = acc;
  }
  row_sync();
  float s = w.norm_acc[0];
#pragma unroll
  for (int k = 1; k < 8; ++k) s = __fadd_rn(s, w.norm_acc[k]);
  return sqrt_rn(s);
}

// Launch shape of the row kernels: a launch of at least kBulkMinRows rows
// packs kBulkRows rows (one wavefront each) per workgroup, so a compute unit
// holds more rows at once than its workgroup slots allow at one row each;
// smaller launches keep one row per workgroup, spread over more units.
constexpr int kBulkRows = 4;
constexpr int kBulkMinRows = 4096;

// LUT_LDS: the angle table (4 x 2^bits floats, bits <= 4) is read from LDS.
template <int SRC, int PD, int ROWS, bool LUT_LDS>
__global__ void __launch_bounds__(64 * ROWS) tq_compress_kernel(TqArgs a) {
  __shared__ RowLds<PD> rows_lds[ROWS];
  __shared__ float lut_lds[LUT_LDS ? 64 : 1];
  const int lane = threadIdx.x & 63;
  if constexpr (LUT_LDS) {
    if (threadIdx.x < (4 << a.bits)) lut_lds[threadIdx.x] = a.lut[threadIdx.x];
    __syncthreads();  // the workgroup's only barrier, before any wavefront leaves
  }
  const int row = blockIdx.x * ROWS + (int)(threadIdx.x >> 6);
  if (row >= a.N) return;
  RowLds<PD>& w = rows_lds[threadIdx.x >> 6];
  float v[tq_per_lane(PD)];
  const float radius = encode_row<SRC, PD>(a.kv, (size_t)row * a.head_dim, a.head_dim, a.signs, a.bits, v, w, lane);
  for (int i = lane; i < PD - 1; i += 64) a.angles[(size_t)row * (PD - 1) + i] = w.bins[i];
  if (lane == 0) a.radius[row] = f32_to_f16_bits(radius);
  const float* lut = LUT_LDS ? lut_lds : a.lut;
  const float norm = qjl_row<PD>(v, radius, lut, a.bits, a.jl, a.qjl_dim, w, lane, [&](int j, bool pos) {
    a.qjl_signs[(size_t)row * a.qjl_dim + j] = pos ? 1 : 0;
  });
  if (lane == 0) a.qjl_norms[row] = f32_to_f16_bits(norm);
}

// ---------------------------------------------------------------------------
// Writes TurboQuant codes straight into the pages of a TurboQuant pool
// (layout in vrm_tq_layout.h).  One wavefront per (row, K/V): the codes are
// those of tq_compress_kernel; V rows skip the QJL stage, whose output the
// attention never reads for values.
// ---------------------------------------------------------------------------
struct TqPoolArgs {
  const void* key;
  const void* value;
  const int32_t* page_ids;
  const int32_t* slots;    // append: slot of each token; pages: nullptr
  const int32_t* n_valid;  // pages: valid tokens of each page; append: nullptr
  uint8_t* pool;
  int rows;  // rows of one K/V side: tokens * KH (append) or pages * KH * 16 (pages)
  int KH, L, P, layer, bits, head_dim;
  int from_pool;  // pages: key/value are a float pool [P][L][2][KH][16][head_dim] read at (page_ids[n], layer)
  const float* signs;
  const float* jl;
  const float* lut;
};

template <int SRC, int BITS, int ROWS, int PD>
__global__ void __launch_bounds__(64 * ROWS) tq_pool_write_kernel(TqPoolArgs a) {
  namespace L = vrm::tq;
  constexpr int QJL = L::tuned_qjl(PD);
  constexpr int SLICE = L::slice_bytes(PD, BITS);
  __shared__ RowLds<PD> rows_lds[ROWS];
  __shared__ uint32_t rows_signs[ROWS][QJL / 32];
  __shared__ float lut_lds[4 << BITS];  // the angle table ({level 0, levels >= 1} x {cos, sin} x 2^BITS)
  const int lane = threadIdx.x & 63;
  if (threadIdx.x < (4 << BITS)) lut_lds[threadIdx.x] = a.lut[threadIdx.x];
  __syncthreads();  // the workgroup's only barrier, before any wavefront leaves
  const int x = blockIdx.x * ROWS + (int)(threadIdx.x >> 6);
  if (x >= a.rows) return;
  RowLds<PD>& w = rows_lds[threadIdx.x >> 6];
  uint32_t* sign_bits = rows_signs[threadIdx.x >> 6];
  const int kv = blockIdx.y;
  // append: x = n * KH + h (token n); pages: x = (np * KH + h) * 16 + t
  int n, h, t;
  size_t src_first;
  bool live = true;
  if (a.slots) {
    n = x / a.KH;
    h = x % a.KH;
    t = a.slots[n];
    src_first = (size_t)x * a.head_dim;
  } else {
    t = x % L::kTokens;
    h = (x / L::kTokens) % a.KH;
    n = x / (L::kTokens * a.KH);
    live = t < a.n_valid[n];
    src_first = (size_t)x * a.head_dim;
  }
  const int pid = a.page_ids[n];
  if (pid < 0 || pid >= a.P || t < 0 || t >= L::kTokens) return;  // rows aimed outside the pool are dropped
  if (a.from_pool) src_first = (((((size_t)pid * a.L + a.layer) * 2 + kv) * a.KH + h) * L::kTokens + t) * a.head_dim;
  uint8_t* slice = a.pool + ((((size_t)pid * a.L + a.layer) * 2 + kv) * a.KH + h) * SLICE;
  constexpr int abytes = L::angle_bytes(PD, BITS);
  constexpr int sbytes = L::sign_bytes(PD);
  uint8_t* rec = slice + (size_t)t * abytes;
  uint16_t* radius_out = reinterpret_cast<uint16_t*>(slice + L::radius_offset(PD, BITS)) + t;
  if (!live) {  // slots past the page's valid tokens hold zero records
    for (int i = lane; i < abytes; i += 64) rec[i] = 0;
    if (lane == 0) *radius_out = 0;
    if (kv == 0) {
      if (lane < sbytes) slice[L::signs_offset(PD, BITS) + t * sbytes + lane] = 0;
      if (lane == 0) reinterpret_cast<uint16_t*>(slice + L::norms_offset(PD, BITS))[t] = 0;
    }
    return;
  }
  float v[tq_per_lane(PD)];
  const void* src = kv ? a.value : a.key;
  const float radius = encode_row<SRC, PD>(src, src_first, a.head_dim, a.signs, BITS, v, w, lane);
  // angle record: the PD slots (4 quarters of PD / 4) as one bit stream, so
  // dword k covers slots from the one holding bit 32 k, at most 32 / BITS + 2
  if (lane < abytes / 4) {
    const int k = lane;
    const int s0 = (32 * k) / BITS;
    uint32_t word = 0;
#pragma unroll
    for (int m = 0; m < 32 / BITS + 2; ++m) {
      const int gs = s0 + m;  // slot gs % (PD / 4) of quarter gs / (PD / 4)
      const int bi = gs < PD && gs * BITS < 32 * k + 32
                         ? L::bin_index_of(PD, gs / L::quarter_slots(PD), gs % L::quarter_slots(PD), BITS)
                         : -1;
      if (bi >= 0) {
        const int shift = gs * BITS - 32 * k;  // negative for a slot straddling the dword start
        const uint32_t val = w.bins[bi];
        word |= shift >= 0 ? (val << shift) : (val >> -shift);
      }
    }
    reinterpret_cast<uint32_t*>(rec)[lane] = word;
  }
  if (lane == 0) *radius_out = f32_to_f16_bits(radius);
  if (kv == 1) return;
  if (lane < QJL / 32) sign_bits[lane] = 0;
  row_sync();
  const float norm = qjl_row<PD>(v, radius, lut_lds, BITS, a.jl, QJL, w, lane, [&](int j, bool pos) {
    if (pos) atomicOr(&sign_bits[j >> 5], 1u << (j & 31));
  });
  row_sync();
  if (lane < QJL / 32)
    reinterpret_cast<uint32_t*>(slice + L::signs_offset(PD, BITS) + t * sbytes)[lane] = sign_bits[lane];
  if (lane == 0) reinterpret_cast<uint16_t*>(slice + L::norms_offset(PD, BITS))[t] = f32_to_f16_bits(norm);
}

// Writer of the generic page layout (vrm_tq_layout.h, GenLayout): every
// compressor setting the tuned layout does not cover, any page size.  One
// wavefront per (row, K/V), one row per workgroup; the codes are those of
// tq_compress_kernel.
template <int SRC, int PD>
__global__ void __launch_bounds__(64) tq_pool_write_gen_kernel(TqPoolArgs a, tq::GenLayout g) {
  __shared__ RowLds<PD> w;
  __shared__ uint32_t sign_words[8];  // qjl <= 256
  const int lane = threadIdx.x;
  const int x = blockIdx.x;
  const int kv = blockIdx.y;
  // append: x = n * KH + h (token n); pages: x = (np * KH + h) * PS + t
  int n, h, t;
  bool live = true;
  if (a.slots) {
    n = x / a.KH;
    h = x % a.KH;
    t = a.slots[n];
  } else {
    t = x % g.ps;
    h = (x / g.ps) % a.KH;
    n = x / (g.ps * a.KH);
    live = t < a.n_valid[n];
  }
  size_t src_first = (size_t)x * a.head_dim;
  const int pid = a.page_ids[n];
  if (pid < 0 || pid >= a.P || t < 0 || t >= g.ps) return;  // rows aimed outside the pool are dropped
  if (a.from_pool) src_first = (((((size_t)pid * a.L + a.layer) * 2 + kv) * a.KH + h) * g.ps + t) * a.head_dim;
  uint8_t* rec = a.pool + ((((size_t)pid * a.L + a.layer) * 2 + kv) * a.KH + h) * g.slice_bytes() +
                 (size_t)t * g.record_bytes();
  uint32_t* rec32 = reinterpret_cast<uint32_t*>(rec);
  uint16_t* rad16 = reinterpret_cast<uint16_t*>(rec + g.radius_offset());
  if (!live) {  // slots past the page's valid tokens hold zero records
    for (int i = lane; i < g.record_bytes() / 4; i += 64) rec32[i] = 0;
    return;
  }
  float v[tq_per_lane(PD)];
  const void* src = kv ? a.value : a.key;
  const float radius = encode_row<SRC, PD>(src, src_first, a.head_dim, a.signs, g.bits, v, w, lane);
  // angle dword k covers record bits [32 k, 32 k + 32): bins from the one holding bit 32 k
  for (int k = lane; k < g.angle_dw; k += 64) {
    uint32_t word = 0;
    for (int b = (32 * k) / g.bits; b < PD - 1 && b * g.bits < 32 * k + 32; ++b) {
      const int shift = b * g.bits - 32 * k;  // negative for a bin straddling the dword start
      const uint32_t val = w.bins[b];
      word |= shift >= 0 ? (val << shift) : (val >> -shift);
    }
    rec32[k] = word;
  }
  if (lane == 0) rad16[0] = f32_to_f16_bits(radius);
  if (kv == 1) {  // values carry no QJL fields
    if (lane < g.sign_dw) rec32[g.angle_dw + lane] = 0;
    if (lane == 0) rad16[1] = 0;
    return;
  }
  if (lane < 8) sign_words[lane] = 0;
  row_sync();
  const float norm = qjl_row<PD>(v, radius, a.lut, g.bits, a.jl, g.qjl, w, lane, [&](int j, bool pos) {
    if (pos) atomicOr(&sign_words[j >> 5], 1u << (j & 31));
  });
  row_sync();
  if (lane < g.sign_dw) rec32[g.angle_dw + lane] = sign_words[lane];
  if (lane == 0) rad16[1] = f32_to_f16_bits(norm);
}

// Reads a generic-layout pool back into the reference's raw code format:
// row ((n * 2 + kv) * KH + h) * PS + t gets radius, level-major bins
// [pd - 1], sign bytes [qjl] and norm.  V rows get zero signs and norms.
__global__ void __launch_bounds__(64) tq_pool_read_gen_kernel(const uint8_t* pool, const int32_t* page_ids, int KH,
                                                              int L_, int P, int layer, tq::GenLayout g,
                                                              uint16_t* radius, uint8_t* angles, uint8_t* qjl_signs,
                                                              uint16_t* norms) {
  const int lane = threadIdx.x;
  const int row = blockIdx.x;
  const int t = row % g.ps;
  const int h = (row / g.ps) % KH;
  const int kv = (row / (g.ps * KH)) % 2;
  const int n = row / (g.ps * KH * 2);
  const int pid = page_ids[n];
  const int na = g.pd - 1;
  if (pid < 0 || pid >= P) {  // absent page: zero codes
    for (int i = lane; i < na; i += 64) angles[(size_t)row * na + i] = 0;
    for (int j = lane; j < g.qjl; j += 64) qjl_signs[(size_t)row * g.qjl + j] = 0;
    if (lane == 0) radius[row] = norms[row] = 0;
    return;
  }
  const uint8_t* rec = pool + ((((size_t)pid * L_ + layer) * 2 + kv) * KH + h) * g.slice_bytes() +
                       (size_t)t * g.record_bytes();
  const uint32_t* rec32 = reinterpret_cast<const uint32_t*>(rec);
  const uint32_t mask = (1u << g.bits) - 1u;
  for (int i = lane; i < na; i += 64) {
    const int bit = i * g.bits, dw = bit >> 5, sh = bit & 31;
    uint32_t x = rec32[dw] >> sh;
    if (sh + g.bits > 32) x |= rec32[dw + 1] << (32 - sh);
    angles[(size_t)row * na + i] = (uint8_t)(x & mask);
  }
  const uint16_t* rad16 = reinterpret_cast<const uint16_t*>(rec + g.radius_offset());
  if (lane == 0) radius[row] = rad16[0];
  for (int j = lane; j < g.qjl; j += 64)
    qjl_signs[(size_t)row * g.qjl + j] = kv == 0 ? (uint8_t)((rec32[g.angle_dw + (j >> 5)] >> (j & 31)) & 1u) : 0;
  if (lane == 0) norms[row] = kv == 0 ? rad16[1] : 0;
}

// Reads a TurboQuant pool back into the reference's raw code format, for
// inspection and for the codec tests: for page n, kv, head h, token t (row
// ((n * 2 + kv) * KH + h) * 16 + t), radius, level-major bins, sign bytes and
// norm.  V rows get zero signs and norms.
__global__ void __launch_bounds__(64) tq_pool_read_kernel(const uint8_t* pool, const int32_t* page_ids, int KH,
                                                          int L_, int P, int layer, int pd, int bits,
                                                          uint16_t* radius, uint8_t* angles, uint8_t* qjl_signs,
                                                          uint16_t* norms) {
  namespace L = vrm::tq;
  const int lane = threadIdx.x;
  const int row = blockIdx.x;
  const int t = row % L::kTokens;
  const int h = (row / L::kTokens) % KH;
  const int kv = (row / (L::kTokens * KH)) % 2;
  const int n = row / (L::kTokens * KH * 2);
  const int pid = page_ids[n];
  const int na = pd - 1, qjl = L::tuned_qjl(pd);
  if (pid < 0 || pid >= P) {  // absent page: zero codes
    for (int i = lane; i < na; i += 64) angles[(size_t)row * na + i] = 0;
    if (lane < qjl) qjl_signs[(size_t)row * qjl + lane] = 0;
    if (lane == 0) radius[row] = norms[row] = 0;
    return;
  }
  const uint8_t* slice = pool + ((((size_t)pid * L_ + layer) * 2 + kv) * KH + h) * L::slice_bytes(pd, bits);
  const int abytes = L::angle_bytes(pd, bits);
  const uint8_t* rec = slice + (size_t)t * abytes;
  for (int i = lane; i < na; i += 64) {
    // find (quarter, slot) of level-major bin i
    int l = 0;
    while (i >= L::level_offset(pd, l + 1)) ++l;
    int g, s;
    L::slot_of(pd, l, i - L::level_offset(pd, l), bits, g, s);
    const int bit = (g * L::quarter_slots(pd) + s) * bits;
    uint32_t x = rec[bit / 8] | ((bit / 8 + 1 < abytes) ? (uint32_t)rec[bit / 8 + 1] << 8 : 0u);
    angles[(size_t)row * na + i] = (uint8_t)((x >> (bit % 8)) & ((1u << bits) - 1));
  }
  if (lane == 0) radius[row] = reinterpret_cast<const uint16_t*>(slice + L::radius_offset(pd, bits))[t];
  if (lane < qjl) {
    const uint8_t byte = kv == 0 ? slice[L::signs_offset(pd, bits) + t * L::sign_bytes(pd) + lane / 8] : 0;
    qjl_signs[(size_t)row * qjl + lane] = (byte >> (lane % 8)) & 1;
  }
  if (lane == 0) norms[row] = kv == 0 ? reinterpret_cast<const uint16_t*>(slice + L::norms_offset(pd, bits))[t] : 0;
}

template <int PD, int ROWS>
__global__ void __launch_bounds__(64 * ROWS) tq_decompress_kernel(TqArgs a, int rotated) {
  constexpr int PER = tq_per_lane(PD);
  __shared__ uint8_t bins_rows[ROWS][PD];
  __shared__ float lut_lds[64];  // the angle table for up to 4 bits (4 x 16 entries)
  const int lane = threadIdx.x & 63;
  const int nb = 1 << a.bits;
  const bool lut_in_lds = nb <= 16;
  if (lut_in_lds && threadIdx.x < 4 * nb) lut_lds[threadIdx.x] = a.lut[threadIdx.x];
  __syncthreads();  // the workgroup's only barrier, before any wavefront leaves
  const int row = blockIdx.x * ROWS + (int)(threadIdx.x >> 6);
  if (row >= a.N) return;
  uint8_t* bins = bins_rows[threadIdx.x >> 6];
  for (int i = lane; i < PD - 1; i += 64) bins[i] = a.angles[(size_t)row * (PD - 1) + i];
  const float radius = f16_bits_to_f32(a.radius[row]);
  row_sync();
  float v[PER];
  // lanes past a row of fewer than 64 elements decode nothing (their bins
  // would lie past the row's)
  if (lut_in_lds) {  // two copies of the loop, each with the table's address space known
#pragma unroll
    for (int k = 0; k < PER; ++k)
      v[k] = k * 64 + lane < PD ? polar_element<PD>(radius, bins, lut_lds, nb, k * 64 + lane) : 0.f;
  } else {
#pragma unroll
    for (int k = 0; k < PER; ++k)
      v[k] = k * 64 + lane < PD ? polar_element<PD>(radius, bins, a.lut, nb, k * 64 + lane) : 0.f;
  }
  if (rotated) {
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (k * 64 + lane < PD) a.out[(size_t)row * PD + k * 64 + lane] = v[k];
    return;
  }
  fwht<PD>(v, lane);
  const float root = (float)sqrt((double)PD);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int e = k * 64 + lane;
    if (e < a.head_dim) a.out[(size_t)row * a.head_dim + e] = __fmul_rn(__fdiv_rn(v[k], root), a.signs[e]);
  }
}

// Query side of KVCacheCompressor.attention_score (core/kv_quantizer.py:
// 516-521, 319-321): q_rot = rotate(pad(q)) and q_proj = q_rot JL^T.  One
// wavefront per query row m; ws row m holds [q_rot (PD) | q_proj (qjl_dim)].
template <int PD>
__global__ void __launch_bounds__(64) tq_query_kernel(const float* q, int head_dim, const float* signs,
                                                      const float* jl, int qjl_dim, float* ws, int permuted) {
  constexpr int PER = tq_per_lane(PD);
  __shared__ float rot[PD];
  const int lane = threadIdx.x;
  const int m = blockIdx.x;
  float v[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int e = k * 64 + lane;
    const float x = e < head_dim ? q[(size_t)m * head_dim + e] : 0.f;
    v[k] = e < PD ? __fmul_rn(x, signs[e]) : 0.f;
  }
  fwht<PD>(v, lane);
  const float root = (float)sqrt((double)PD);
  float* out = ws + (size_t)m * (PD + qjl_dim);
  // feature f at f, or (matrix-core scores) at (f % 4) * F / 4 + f / 4
  const int F4 = (PD + qjl_dim) / 4;
  auto at = [&](int f) { return permuted ? (f & 3) * F4 + (f >> 2) : f; };
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    v[k] = __fdiv_rn(v[k], root);
    if (k * 64 + lane < PD) {
      rot[k * 64 + lane] = v[k];
      out[at(k * 64 + lane)] = v[k];
    }
  }
  __syncthreads();
  for (int j = lane; j < qjl_dim; j += 64) {
    const float* row = jl + (size_t)j * PD;
    float acc = 0.f;
    for (int e = 0; e < PD; ++e) acc = __fadd_rn(acc, __fmul_rn(rot[e], row[e]));
    out[at(PD + j)] = acc;
  }
}

// Key side: one wavefront per compressed key n rebuilds k_polar (the polar
// decode from the fp16 radius, as attention_score does), then each lane
// scores query rows m = lane, lane + 64, ...:
//   scores[m][n] = out_scale * (q_rot[m] . k_polar[n] + (q_proj[m] . (2 s_n - 1)) * coef * norm_n)
// with coef = sqrt(pi / 2) / qjl_dim (core/kv_quantizer.py:523-535).
template <int PD>
__global__ void __launch_bounds__(64) tq_score_kernel(const float* ws, int M, int qjl_dim, const uint16_t* radius,
                                                      const uint8_t* angles, const uint8_t* qjl_signs,
                                                      const uint16_t* qjl_norms, int N, const float* lut, int bits,
                                                      float coef, float out_scale, float* scores) {
  __shared__ float recon[PD];
  __shared__ uint8_t bins[PD];
  __shared__ float sgn[4 * PD];
  const int lane = threadIdx.x;
  const int n = blockIdx.x;
  for (int i = lane; i < PD - 1; i += 64) bins[i] = angles[(size_t)n * (PD - 1) + i];
  for (int j = lane; j < qjl_dim; j += 64)
    sgn[j] = __fsub_rn(__fmul_rn((float)qjl_signs[(size_t)n * qjl_dim + j], 2.f), 1.f);
  const float r = f16_bits_to_f32(radius[n]);
  const float norm = f16_bits_to_f32(qjl_norms[n]);
  __syncthreads();
  polar_decode<PD>(r, bins, lut, 1 << bits, recon, lane);
  for (int m = lane; m < M; m += 64) {
    const float* qr = ws + (size_t)m * (PD + qjl_dim);
    float dot = 0.f;
    for (int e = 0; e < PD; ++e) dot = __fadd_rn(dot, __fmul_rn(qr[e], recon[e]));
    float raw = 0.f;
    for (int j = 0; j < qjl_dim; ++j) raw = __fadd_rn(raw, __fmul_rn(qr[PD + j], sgn[j]));
    const float corr = __fmul_rn(__fmul_rn(raw, coef), norm);
    scores[(size_t)m * N + n] = __fmul_rn(__fadd_rn(dot, corr), out_scale);
  }
}


// Scores on the matrix cores, for the page format (padded_dim 128, qjl_dim
// 64): scores = out_scale * [k_polar | coef norm (2 s - 1)] . [q_rot | q_proj],
// a [keys x 192] x [192 x queries] product on v_mfma_f32_16x16x4_f32, 16
// keys per wavefront against every 16-query tile in turn.  Lane (key, g)
// holds key features f = 4 j + g (A[key][f] of MFMA step j):
//   * dims 4 j + g of k_polar: the radii top-down to the level-1 angles (the
//     reference's products in its order, so each dim is the value polar
//     decode gives), then the level-1 and level-0 factors of the dim;
//   * QJL features 4 j + g: (2 s - 1) coef norm.
// The query kernel writes row m of the workspace feature-permuted (feature f
// at (f % 4) * 48 + f / 4), so a lane's 48 query features are contiguous.
// Sums run in the matrix cores' order; the result is float32 all through.
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kMfmaKeys = 16;   // keys per wavefront
constexpr int kMfmaWaves = 4;   // wavefronts per workgroup

__global__ void __launch_bounds__(64 * kMfmaWaves) tq_score_mfma_kernel(const float* ws, int M, const uint16_t* radius,
                                                                      const uint8_t* angles, const uint8_t* qjl_signs,
                                                                      const uint16_t* qjl_norms, int N,
                                                                      const float* lut, int bits, float coef,
                                                                      float out_scale, float* scores) {
  constexpr int PD = 128, QJ = 64, F = PD + QJ, J = F / 4, NP = PD / 4;  // 48 steps, 32 of them polar
  constexpr int ROWB = PD - 1;  // angle bytes per key
  __shared__ __align__(16) uint8_t bins_lds[kMfmaWaves][kMfmaKeys * ROWB + 16];
  __shared__ float lut_lds[64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = lane & 15;
  const int g = lane >> 4;
  const int nb = 1 << bits;
  if (threadIdx.x < 4 * nb) lut_lds[threadIdx.x] = lut[threadIdx.x];
  __syncthreads();  // the workgroup's only barrier, before any wavefront leaves
  const int n0 = (blockIdx.x * kMfmaWaves + wave) * kMfmaKeys;
  if (n0 >= N) return;
  const int nk = min(kMfmaKeys, N - n0);

  // this wavefront's keys' angle bytes into LDS (n0 * 127 is a multiple of 16)
  {
    const int total = nk * ROWB;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(angles + (size_t)n0 * ROWB);
    uint32_t* dst = reinterpret_cast<uint32_t*>(bins_lds[wave]);
    for (int i = lane; i < total / 4; i += 64) dst[i] = src[i];
    if (lane < (total & 3)) bins_lds[wave][(total & ~3) + lane] = angles[(size_t)n0 * ROWB + (total & ~3) + lane];
  }
  row_sync();

  const bool valid = row < nk;
  const int kr = min(row, nk - 1);
  const int key = n0 + kr;
  const uint8_t* kb = bins_lds[wave] + kr * ROWB;
  auto factor = [&](int level, int angle, int sine) {
    const int b = min((int)kb[PD - (PD >> level) + angle], nb - 1);
    return lut_lds[(level == 0 ? 0 : 2 * nb) + (sine ? nb : 0) + b];
  };
  float A[J];
  {
    // radii top-down: after level l the value of node i is r * f_6 * ... * f_l
    float cur[NP];
    cur[0] = f16_bits_to_f32(radius[key]);
#pragma unroll
    for (int level = 6, cnt = 1; level >= 2; --level, cnt *= 2) {
#pragma unroll
      for (int i = cnt - 1; i >= 0; --i) {  // downwards, so cur[i] is read before cur[2 i], cur[2 i + 1] are written
        const float r = cur[i];
        cur[2 * i] = __fmul_rn(r, factor(level, i, 0));
        cur[2 * i + 1] = __fmul_rn(r, factor(level, i, 1));
      }
    }
#pragma unroll
    for (int j = 0; j < NP; ++j) {  // dim 4 j + g
      const float r0 = __fmul_rn(cur[j], factor(1, j, g >> 1));
      A[j] = valid ? __fmul_rn(r0, factor(0, 2 * j + (g >> 1), g & 1)) : 0.f;
    }
  }
  {
    const float cn = valid ? coef * f16_bits_to_f32(qjl_norms[key]) : 0.f;
    const uint4* sg = reinterpret_cast<const uint4*>(qjl_signs + (size_t)key * QJ);
#pragma unroll
    for (int t = 0; t < QJ / 16; ++t) {
      const uint4 w = sg[t];  // sign bytes 16 t .. 16 t + 15
      const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {  // feature 4 (4 t + u) + g: byte g of dword u
        const float s = (float)((d[u] >> (8 * g)) & 0xffu);
        A[NP + 4 * t + u] = __fmul_rn(__fsub_rn(__fmul_rn(s, 2.f), 1.f), cn);
      }
    }
  }

  for (int m0 = 0; m0 < M; m0 += 16) {
    const int m = min(m0 + row, M - 1);
    const float4* qb = reinterpret_cast<const float4*>(ws + (size_t)m * F + g * J);
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < J / 4; ++t) {
      const float4 b = qb[t];
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[4 * t], b.x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[4 * t + 1], b.y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[4 * t + 2], b.z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[4 * t + 3], b.w, acc, 0, 0, 0);
    }
    // C[key 4 g + r][query row]
    if (m0 + row < M) {
      float* out = scores + (size_t)(m0 + row) * N + n0 + 4 * g;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (4 * g + r < nk) out[r] = __fmul_rn(acc[r], out_scale);
    }
  }
}

// The same scores, for up to kScoreMaxLds bytes of staged queries: one
// wavefront per kScoreKeys keys, the query rows (q_rot, q_proj) staged in LDS
// once (row stride PD + qjl_dim + 1 floats, so lane m reads a bank of its
// own), kScoreBatch keys rebuilt at a time and scored together; each score
// is summed in the same order as tq_score_kernel's.
constexpr int kScoreKeys = 16;
constexpr int kScoreBatch = 4;
constexpr int kScoreMaxLds = 60 * 1024;

template <int PD>
__global__ void __launch_bounds__(64) tq_score_lds_kernel(const float* ws, int M, int qjl_dim,
                                                          const uint16_t* radius, const uint8_t* angles,
                                                          const uint8_t* qjl_signs, const uint16_t* qjl_norms, int N,
                                                          const float* lut, int bits, float coef, float out_scale,
                                                          float* scores) {
  extern __shared__ float dyn[];  // [M][W] queries, then [kScoreBatch][qjl_dim] signs
  __shared__ float recon[kScoreBatch][PD];
  __shared__ uint8_t bins[PD];
  const int lane = threadIdx.x;
  const int W = PD + qjl_dim + 1;
  float* qs = dyn;
  float* sgn = dyn + (size_t)M * W;
  for (int i = lane; i < M * (PD + qjl_dim); i += 64) {
    const int m = i / (PD + qjl_dim), e = i - m * (PD + qjl_dim);
    qs[m * W + e] = ws[i];
  }
  const int first = blockIdx.x * kScoreKeys;
  const int last = min(N, first + kScoreKeys);
  for (int n0 = first; n0 < last; n0 += kScoreBatch) {
    const int nb = min(kScoreBatch, last - n0);
    float norm[kScoreBatch];
    for (int kb = 0; kb < nb; ++kb) {
      const int n = n0 + kb;
      for (int i = lane; i < PD - 1; i += 64) bins[i] = angles[(size_t)n * (PD - 1) + i];
      for (int j = lane; j < qjl_dim; j += 64)
        sgn[kb * qjl_dim + j] = __fsub_rn(__fmul_rn((float)qjl_signs[(size_t)n * qjl_dim + j], 2.f), 1.f);
      norm[kb] = f16_bits_to_f32(qjl_norms[n]);
      polar_decode<PD>(f16_bits_to_f32(radius[n]), bins, lut, 1 << bits, recon[kb], lane);
    }
    for (int m = lane; m < M; m += 64) {
      const float* qr = qs + m * W;
      float dot[kScoreBatch], raw[kScoreBatch];
#pragma unroll
      for (int kb = 0; kb < kScoreBatch; ++kb) dot[kb] = raw[kb] = 0.f;
      for (int e = 0; e < PD; ++e) {
        const float qv = qr[e];
#pragma unroll
        for (int kb = 0; kb < kScoreBatch; ++kb) dot[kb] = __fadd_rn(dot[kb], __fmul_rn(qv, recon[kb][e]));
      }
      for (int j = 0; j < qjl_dim; ++j) {
        const float qv = qr[PD + j];
#pragma unroll
        for (int kb = 0; kb < kScoreBatch; ++kb) raw[kb] = __fadd_rn(raw[kb], __fmul_rn(qv, sgn[kb * qjl_dim + j]));
      }
#pragma unroll
      for (int kb = 0; kb < kScoreBatch; ++kb) {
        if (kb < nb) {
          const float corr = __fmul_rn(__fmul_rn(raw[kb], coef), norm[kb]);
          scores[(size_t)m * N + n0 + kb] = __fmul_rn(__fadd_rn(dot[kb], corr), out_scale);
        }
      }
    }
    __syncthreads();  // recon / sgn / bins are rewritten for the next keys
  }
}

int check_tq(int N, int head_dim, int padded_dim, int n_levels, int bits, const char* who) {
  if (N < 0 || head_dim <= 0 || head_dim > padded_dim) {
    set_error("%s: bad sizes (N=%d head_dim=%d padded_dim=%d)", who, N, head_dim, padded_dim);
    return VRM_ERR_ARG;
  }
  if (padded_dim < 2 || padded_dim > 256 || (padded_dim & (padded_dim - 1))) {
    set_error("%s: padded_dim %d unsupported (a power of two from 2 to 256)", who, padded_dim);
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
  const bool bulk = N >= kBulkMinRows;
  const bool lut_lds = bits <= 4;
#define VRM_TQ_LAUNCH(SRC, PDV)                                                                                     \
  if (bulk && lut_lds)                                                                                              \
    hipLaunchKernelGGL((tq_compress_kernel<SRC, PDV, kBulkRows, true>), dim3((N + kBulkRows - 1) / kBulkRows),      \
                       dim3(64 * kBulkRows), 0, st, a);                                                             \
  else if (bulk)                                                                                                    \
    hipLaunchKernelGGL((tq_compress_kernel<SRC, PDV, kBulkRows, false>), dim3((N + kBulkRows - 1) / kBulkRows),     \
                       dim3(64 * kBulkRows), 0, st, a);                                                             \
  else                                                                                                              \
    hipLaunchKernelGGL((tq_compress_kernel<SRC, PDV, 1, false>), dim3(N), dim3(64), 0, st, a)
#define VRM_TQ_PD(SRC)                                  \
  switch (padded_dim) {                                 \
    case 2: VRM_TQ_LAUNCH(SRC, 2); break;               \
    case 4: VRM_TQ_LAUNCH(SRC, 4); break;               \
    case 8: VRM_TQ_LAUNCH(SRC, 8); break;               \
    case 16: VRM_TQ_LAUNCH(SRC, 16); break;             \
    case 32: VRM_TQ_LAUNCH(SRC, 32); break;             \
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
  const bool bulk = N >= kBulkMinRows;
#define VRM_TQ_DECOMP(PDV)                                                                                   \
  if (bulk)                                                                                                  \
    hipLaunchKernelGGL((tq_decompress_kernel<PDV, kBulkRows>), dim3((N + kBulkRows - 1) / kBulkRows),        \
                       dim3(64 * kBulkRows), 0, st, a, rotated);                                             \
  else                                                                                                       \
    hipLaunchKernelGGL((tq_decompress_kernel<PDV, 1>), dim3(N), dim3(64), 0, st, a, rotated)
  switch (padded_dim) {
    case 2: VRM_TQ_DECOMP(2); break;
    case 4: VRM_TQ_DECOMP(4); break;
    case 8: VRM_TQ_DECOMP(8); break;
    case 16: VRM_TQ_DECOMP(16); break;
    case 32: VRM_TQ_DECOMP(32); break;
    case 64: VRM_TQ_DECOMP(64); break;
    case 128: VRM_TQ_DECOMP(128); break;
    default: VRM_TQ_DECOMP(256); break;
  }
#undef VRM_TQ_DECOMP
  return launch_status(who);
}

namespace {
int check_tq_pool(int KH, int D, int PS, int L, int P, int layer_idx, int bits, int qjl_dim, const char* who) {
  if (KH <= 0 || L <= 0 || P <= 0 || layer_idx < 0 || layer_idx >= L) {
    set_error("%s: bad sizes (KH=%d L=%d P=%d layer=%d)", who, KH, L, P, layer_idx);
    return VRM_ERR_ARG;
  }
  if (!tq::tuned_layout(D, bits, qjl_dim, PS) && !tq::generic_ok(D, bits, qjl_dim, PS)) {
    set_error("%s: TurboQuant pages take head_dim 1 .. 256, 1 .. 8 bits per angle, qjl_dim 1 .. 256 and a "
              "positive page size (got %d, %d, %d, %d)", who, D, bits, qjl_dim, PS);
    return VRM_ERR_UNSUPPORTED;
  }
  return VRM_OK;
}

int tq_pool_write(const void* key, const void* value, int src_dtype, const int32_t* page_ids, const int32_t* slots,
                  const int32_t* n_valid, int rows, uint8_t* tq_pool, int KH, int D, int PS, int L, int P,
                  int layer_idx, int bits, int qjl_dim, const float* signs, const float* jl, const float* angle_lut,
                  vrm_stream_t stream, const char* who, bool from_pool = false) {
  int rc = check_tq_pool(KH, D, PS, L, P, layer_idx, bits, qjl_dim, who);
  if (rc) return rc;
  if (rows < 0) {
    set_error("%s: negative count", who);
    return VRM_ERR_ARG;
  }
  if (src_dtype != VRM_SRC_F32 && src_dtype != VRM_SRC_F16 && src_dtype != VRM_SRC_BF16) {
    set_error("%s: unknown source dtype %d", who, src_dtype);
    return VRM_ERR_ARG;
  }
  if (rows == 0) return VRM_OK;
  if (!key || !value || !page_ids || !tq_pool || !signs || !jl || !angle_lut || (!slots && !n_valid)) {
    set_error("%s: null pointer argument", who);
    return VRM_ERR_ARG;
  }
  if (rows > 0x7fffffff / 2) {
    set_error("%s: too many rows", who);
    return VRM_ERR_UNSUPPORTED;
  }
  TqPoolArgs a{};
  a.key = key;
  a.value = value;
  a.page_ids = page_ids;
  a.slots = slots;
  a.n_valid = n_valid;
  a.pool = tq_pool;
  a.rows = rows;
  a.KH = KH;
  a.L = L;
  a.P = P;
  a.layer = layer_idx;
  a.bits = bits;
  a.head_dim = D;
  a.from_pool = from_pool ? 1 : 0;
  a.signs = signs;
  a.jl = jl;
  a.lut = angle_lut;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int pd = tq::tuned_pd(D, bits, qjl_dim, PS);
  if (!pd) {
    const tq::GenLayout g = tq::gen_layout(D, bits, qjl_dim, PS);
    const dim3 grid(rows, 2);
#define VRM_TQ_WRITE_GEN_PD(SRC, PDV) \
  hipLaunchKernelGGL((tq_pool_write_gen_kernel<SRC, PDV>), grid, dim3(64), 0, st, a, g)
#define VRM_TQ_WRITE_GEN(SRC)                                       \
  switch (g.pd) {                                                   \
    case 2: VRM_TQ_WRITE_GEN_PD(SRC, 2); break;                     \
    case 4: VRM_TQ_WRITE_GEN_PD(SRC, 4); break;                     \
    case 8: VRM_TQ_WRITE_GEN_PD(SRC, 8); break;                     \
    case 16: VRM_TQ_WRITE_GEN_PD(SRC, 16); break;                   \
    case 32: VRM_TQ_WRITE_GEN_PD(SRC, 32); break;                   \
    case 64: VRM_TQ_WRITE_GEN_PD(SRC, 64); break;                   \
    case 128: VRM_TQ_WRITE_GEN_PD(SRC, 128); break;                 \
    default: VRM_TQ_WRITE_GEN_PD(SRC, 256); break;                  \
  }
    switch (src_dtype) {
      case VRM_SRC_F32: VRM_TQ_WRITE_GEN(VRM_SRC_F32); break;
      case VRM_SRC_F16: VRM_TQ_WRITE_GEN(VRM_SRC_F16); break;
      default: VRM_TQ_WRITE_GEN(VRM_SRC_BF16); break;
    }
#undef VRM_TQ_WRITE_GEN
#undef VRM_TQ_WRITE_GEN_PD
    return launch_status(who);
  }
  // bulk writes pack kBulkRows rows (wavefronts) per workgroup, small ones one
  const bool bulk = rows >= kBulkMinRows;
  const dim3 grid(bulk ? (rows + kBulkRows - 1) / kBulkRows : rows, 2);
#define VRM_TQ_WRITE_RP(SRC, B, PDV)                                                                         \
  if (bulk)                                                                                                  \
    hipLaunchKernelGGL((tq_pool_write_kernel<SRC, B, kBulkRows, PDV>), grid, dim3(64 * kBulkRows), 0, st, a); \
  else                                                                                                       \
    hipLaunchKernelGGL((tq_pool_write_kernel<SRC, B, 1, PDV>), grid, dim3(64), 0, st, a);
#define VRM_TQ_WRITE_R(SRC, B)          \
  if (pd == 64)                         \
    VRM_TQ_WRITE_RP(SRC, B, 64)         \
  else                                  \
    VRM_TQ_WRITE_RP(SRC, B, 128)
#define VRM_TQ_WRITE(SRC)                          \
  switch (bits) {                                  \
    case 2: VRM_TQ_WRITE_R(SRC, 2); break;         \
    case 3: VRM_TQ_WRITE_R(SRC, 3); break;         \
    default: VRM_TQ_WRITE_R(SRC, 4); break;        \
  }
  switch (src_dtype) {
    case VRM_SRC_F32: VRM_TQ_WRITE(VRM_SRC_F32); break;
    case VRM_SRC_F16: VRM_TQ_WRITE(VRM_SRC_F16); break;
    default: VRM_TQ_WRITE(VRM_SRC_BF16); break;
  }
#undef VRM_TQ_WRITE
#undef VRM_TQ_WRITE_R
#undef VRM_TQ_WRITE_RP
  return launch_status(who);
}
}  // namespace

extern "C" size_t vrm_tq_slice_bytes_ps(int head_dim, int bits, int qjl_dim, int page_size) {
  if (const int pd = tq::tuned_pd(head_dim, bits, qjl_dim, page_size)) return (size_t)tq::slice_bytes(pd, bits);
  if (tq::generic_ok(head_dim, bits, qjl_dim, page_size))
    return tq::gen_layout(head_dim, bits, qjl_dim, page_size).slice_bytes();
  return 0;
}

extern "C" size_t vrm_tq_slice_bytes(int head_dim, int bits, int qjl_dim) {
  return vrm_tq_slice_bytes_ps(head_dim, bits, qjl_dim, tq::kTokens);
}

extern "C" int vrm_tq_quant_append(const void* key, const void* value, int src_dtype, const int32_t* page_ids,
                                   const int32_t* slots, int N, uint8_t* tq_pool, int KH, int D, int PS, int L,
                                   int P, int layer_idx, int bits, int qjl_dim, const float* signs, const float* jl,
                                   const float* angle_lut, vrm_stream_t stream) {
  const char* who = "vrm_tq_quant_append";
  if (N < 0 || KH <= 0 || (long)N * KH > 0x3fffffff) {
    set_error("%s: bad sizes (N=%d KH=%d)", who, N, KH);
    return VRM_ERR_ARG;
  }
  if (N > 0 && !slots) {
    set_error("%s: null slots", who);
    return VRM_ERR_ARG;
  }
  return tq_pool_write(key, value, src_dtype, page_ids, slots, nullptr, N * KH, tq_pool, KH, D, PS, L, P, layer_idx,
                       bits, qjl_dim, signs, jl, angle_lut, stream, who);
}

extern "C" int vrm_tq_quant_pages(const void* key, const void* value, int src_dtype, const int32_t* page_ids,
                                  const int32_t* n_valid, int NP, uint8_t* tq_pool, int KH, int D, int PS, int L,
                                  int P, int layer_idx, int bits, int qjl_dim, const float* signs, const float* jl,
                                  const float* angle_lut, vrm_stream_t stream) {
  const char* who = "vrm_tq_quant_pages";
  if (NP < 0 || KH <= 0 || PS <= 0 || (long)NP * KH * PS > 0x3fffffff) {
    set_error("%s: bad sizes (NP=%d KH=%d PS=%d)", who, NP, KH, PS);
    return VRM_ERR_ARG;
  }
  if (NP > 0 && !n_valid) {
    set_error("%s: null n_valid", who);
    return VRM_ERR_ARG;
  }
  return tq_pool_write(key, value, src_dtype, page_ids, nullptr, n_valid, NP * KH * PS, tq_pool, KH, D, PS, L, P,
                       layer_idx, bits, qjl_dim, signs, jl, angle_lut, stream, who);
}

extern "C" size_t vrm_turboquant_score_workspace_bytes(int M, int padded_dim, int qjl_dim) {
  if (M < 0 || padded_dim <= 0 || qjl_dim < 0) return 0;
  return (size_t)M * (size_t)(padded_dim + qjl_dim) * sizeof(float);
}

extern "C" int vrm_turboquant_score(const float* q, int M, const uint16_t* radius, const uint8_t* angles,
                                    const uint8_t* qjl_signs, const uint16_t* qjl_norms, int N, int head_dim,
                                    int padded_dim, int n_levels, int bits, int qjl_dim, const float* signs,
                                    const float* jl, const float* angle_lut, float out_scale, float* workspace,
                                    size_t workspace_bytes, float* scores, vrm_stream_t stream) {
  const char* who = "vrm_turboquant_score";
  int rc = check_tq(N, head_dim, padded_dim, n_levels, bits, who);
  if (rc) return rc;
  if (M < 0 || M > 65535 || N > 0x7fffffff / 2) {
    set_error("%s: bad sizes (M=%d N=%d)", who, M, N);
    return VRM_ERR_ARG;
  }
  if (qjl_dim <= 0 || qjl_dim > 4 * padded_dim) {
    set_error("%s: qjl_dim %d outside [1, %d]", who, qjl_dim, 4 * padded_dim);
    return VRM_ERR_ARG;
  }
  if (workspace_bytes < vrm_turboquant_score_workspace_bytes(M, padded_dim, qjl_dim)) {
    set_error("%s: workspace of %zu bytes, need %zu", who, workspace_bytes,
              vrm_turboquant_score_workspace_bytes(M, padded_dim, qjl_dim));
    return VRM_ERR_WORKSPACE;
  }
  if (M == 0 || N == 0) {
    clear_error();
    return VRM_OK;
  }
  if (!q || !radius || !angles || !qjl_signs || !qjl_norms || !signs || !jl || !angle_lut || !workspace ||
      !scores) {
    set_error("%s: null pointer argument", who);
    return VRM_ERR_ARG;
  }
  const float coef = (float)(sqrt(M_PI / 2.0) / qjl_dim);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // the matrix-core kernel: page format (its angle table holds 4 x 2^bits
  // <= 64 entries), with its code arrays and the workspace aligned for its 4-
  // and 16-byte loads
  const bool mfma = padded_dim == 128 && qjl_dim == 64 && bits <= 4 &&
                    ((reinterpret_cast<uintptr_t>(angles) & 3) | (reinterpret_cast<uintptr_t>(qjl_signs) & 15) |
                     (reinterpret_cast<uintptr_t>(workspace) & 15)) == 0;
  if (mfma) {
    hipLaunchKernelGGL(tq_query_kernel<128>, dim3(M), dim3(64), 0, st, q, head_dim, signs, jl, qjl_dim, workspace, 1);
    hipLaunchKernelGGL(tq_score_mfma_kernel, dim3((N + kMfmaWaves * kMfmaKeys - 1) / (kMfmaWaves * kMfmaKeys)),
                       dim3(64 * kMfmaWaves), 0, st, workspace, M, radius, angles, qjl_signs, qjl_norms, N,
                       angle_lut, bits, coef, out_scale, scores);
    return launch_status(who);
  }
  const size_t lds = ((size_t)M * (padded_dim + qjl_dim + 1) + (size_t)kScoreBatch * qjl_dim) * sizeof(float);
  const bool staged = lds <= (size_t)kScoreMaxLds;
#define VRM_TQ_SCORE(PDV)                                                                                      \
  hipLaunchKernelGGL(tq_query_kernel<PDV>, dim3(M), dim3(64), 0, st, q, head_dim, signs, jl, qjl_dim, workspace, 0); \
  if (staged)                                                                                                  \
    hipLaunchKernelGGL(tq_score_lds_kernel<PDV>, dim3((N + kScoreKeys - 1) / kScoreKeys), dim3(64), lds, st,   \
                       workspace, M, qjl_dim, radius, angles, qjl_signs, qjl_norms, N, angle_lut, bits, coef,   \
                       out_scale, scores);                                                                     \
  else                                                                                                         \
    hipLaunchKernelGGL(tq_score_kernel<PDV>, dim3(N), dim3(64), 0, st, workspace, M, qjl_dim, radius, angles,     \
                       qjl_signs, qjl_norms, N, angle_lut, bits, coef, out_scale, scores)
  switch (padded_dim) {
    case 2: VRM_TQ_SCORE(2); break;
    case 4: VRM_TQ_SCORE(4); break;
    case 8: VRM_TQ_SCORE(8); break;
    case 16: VRM_TQ_SCORE(16); break;
    case 32: VRM_TQ_SCORE(32); break;
    case 64: VRM_TQ_SCORE(64); break;
    case 128: VRM_TQ_SCORE(128); break;
    default: VRM_TQ_SCORE(256); break;
  }
#undef VRM_TQ_SCORE
  return launch_status(who);
}

extern "C" int vrm_tq_compress_pool(const void* kv_pool, int kv_dtype, const int32_t* page_ids,
                                    const int32_t* n_valid, int NP, uint8_t* tq_pool, int KH, int D, int PS, int L,
                                    int P, int layer_idx, int bits, int qjl_dim, const float* signs, const float* jl,
                                    const float* angle_lut, vrm_stream_t stream) {
  const char* who = "vrm_tq_compress_pool";
  if (NP < 0 || KH <= 0 || PS <= 0 || (long)NP * KH * PS > 0x3fffffff) {
    set_error("%s: bad sizes (NP=%d KH=%d PS=%d)", who, NP, KH, PS);
    return VRM_ERR_ARG;
  }
  int src_dtype;
  switch (kv_dtype) {
    case VRM_KV_F32: src_dtype = VRM_SRC_F32; break;
    case VRM_KV_F16: src_dtype = VRM_SRC_F16; break;
    case VRM_KV_BF16: src_dtype = VRM_SRC_BF16; break;
    default:
      set_error("%s: kv_dtype %d is not a float pool", who, kv_dtype);
      return VRM_ERR_ARG;
  }
  if (NP > 0 && !n_valid) {
    set_error("%s: null n_valid", who);
    return VRM_ERR_ARG;
  }
  return tq_pool_write(kv_pool, kv_pool, src_dtype, page_ids, nullptr, n_valid, NP * KH * PS, tq_pool, KH, D, PS, L,
                       P, layer_idx, bits, qjl_dim, signs, jl, angle_lut, stream, who, true);
}

extern "C" int vrm_tq_read_pages(const uint8_t* tq_pool, const int32_t* page_ids, int NP, int KH, int D, int PS,
                                 int L, int P, int layer_idx, int bits, int qjl_dim, uint16_t* radius,
                                 uint8_t* angles, uint8_t* qjl_signs, uint16_t* qjl_norms, vrm_stream_t stream) {
  const char* who = "vrm_tq_read_pages";
  int rc = check_tq_pool(KH, D, PS, L, P, layer_idx, bits, qjl_dim, who);
  if (rc) return rc;
  if (NP < 0 || (long)NP * 2 * KH * PS > 0x7fffffff) {
    set_error("%s: bad count %d", who, NP);
    return VRM_ERR_ARG;
  }
  if (NP == 0) return VRM_OK;
  if (!tq_pool || !page_ids || !radius || !angles || !qjl_signs || !qjl_norms) {
    set_error("%s: null pointer argument", who);
    return VRM_ERR_ARG;
  }
  const int pd = tq::tuned_pd(D, bits, qjl_dim, PS);
  if (!pd) {
    hipLaunchKernelGGL(tq_pool_read_gen_kernel, dim3(NP * 2 * KH * PS), dim3(64), 0,
                       reinterpret_cast<hipStream_t>(stream), tq_pool, page_ids, KH, L, P, layer_idx,
                       tq::gen_layout(D, bits, qjl_dim, PS), radius, angles, qjl_signs, qjl_norms);
    return launch_status(who);
  }
  hipLaunchKernelGGL(tq_pool_read_kernel, dim3(NP * 2 * KH * tq::kTokens), dim3(64), 0,
                     reinterpret_cast<hipStream_t>(stream), tq_pool, page_ids, KH, L, P, layer_idx, pd, bits, radius,
                     angles, qjl_signs, qjl_norms);
  return launch_status(who);
}
