// Top-k ("sparse V") attention over explicit scores.
//
// The reference keeps, per query row, the k largest softmax weights,
// renormalises them and takes their weighted sum of values
// (KVCacheCompressor.sparse_v_attend, core/kv_quantizer.py:537-562, and
// compute_attention_turbo with sparse_v_ratio < 1, core/paged_attention.py:
// 1384-1400).  Softmax is monotonic, so the kept tokens are the k largest
// scores, and the renormalised weights are the softmax over the kept tokens
// alone:
//   out[m] = sum_{n in S_m} e^(s_mn - max) v_n / sum_{n in S_m} e^(s_mn - max).
// With k = N this is the dense softmax(s) V of the reference's k >= seq_len
// branch.
//
// Selection (topk_select_kernel): the k-th largest score T of each row by a
// radix select, four passes of 8 bits over an order-preserving integer key,
// one workgroup per row.  S_m is every score above T plus, of the scores equal
// to T, the lowest-indexed ones up to k in total (the reference's topk leaves
// the choice among equal weights unspecified).  topk_attend_kernel compacts
// S_m in index order, then computes the weights and the weighted sum.
#include "vrm_common.h"

#include <math.h>

namespace vrm {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
// The row kernels (select, compaction) give each row one workgroup of
// kRowThreads: the passes over a row are chains of dependent steps, and with
// tens of rows per call the wider workgroup is what keeps the units busy.
constexpr int kRowThreads = 1024;
constexpr int kRowWaves = kRowThreads / 64;
constexpr int kSelLoads = 8;  // scores per thread per load round of the radix select

// Ascending float order <-> ascending unsigned order.
__device__ __forceinline__ uint32_t order_key(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ void __launch_bounds__(kRowThreads) topk_select_kernel(const float* scores, int N, long long ld, int k,
                                                               uint32_t* sel) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_prefix, s_remaining;
  const int tid = threadIdx.x;
  const float* row = scores + (size_t)blockIdx.x * ld;
  uint32_t prefix = 0, mask = 0, remaining = (uint32_t)k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    // kSelLoads scores per thread are loaded before any histogram update, so
    // the loads of a pass are not serialised behind the LDS atomics.
    for (int base = 0; base < N; base += kRowThreads * kSelLoads) {
      float x[kSelLoads];
#pragma unroll
      for (int e = 0; e < kSelLoads; ++e) {
        const int n = base + e * kRowThreads + tid;
        x[e] = n < N ? row[n] : 0.f;
      }
#pragma unroll
      for (int e = 0; e < kSelLoads; ++e) {
        const uint32_t key = order_key(x[e]);
        if (base + e * kRowThreads + tid < N && (key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
      }
    }
    __syncthreads();
    if (tid == 0) {
      // walk the bins from the largest keys down until the k-th is inside
      uint32_t r = remaining;
      int b = 255;
      for (; b > 0 && r > hist[b]; --b) r -= hist[b];
      s_prefix = prefix | ((uint32_t)b << shift);
      s_remaining = r;
    }
    __syncthreads();
    prefix = s_prefix;
    remaining = s_remaining;
    mask |= 255u << shift;
    __syncthreads();
  }
  if (tid == 0) {
    sel[2 * blockIdx.x] = prefix;        // key of T
    sel[2 * blockIdx.x + 1] = remaining;  // scores equal to T that are kept
  }
}

// Exclusive prefix sum over the workgroup; `total` gets the sum.
template <int W>
__device__ __forceinline__ int block_exclusive_scan(int v, int& total, int* lds) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int t = __builtin_amdgcn_ds_bpermute(max(lane - d, 0) << 2, inc);
    if (lane >= d) inc += t;
  }
  if (lane == 63) lds[w] = inc;
  __syncthreads();
  int base = 0;
  total = 0;
#pragma unroll
  for (int i = 0; i < W; ++i) {
    const int c = lds[i];
    base += i < w ? c : 0;
    total += c;
  }
  __syncthreads();
  return base + inc - v;
}

template <int W>
__device__ __forceinline__ float block_max(float v, float* lds) {
  v = group_max<64>(v);
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = lds[0];
#pragma unroll
  for (int i = 1; i < W; ++i) r = fmaxf(r, lds[i]);
  __syncthreads();
  return r;
}

template <int W>
__device__ __forceinline__ float block_sum(float v, float* lds) {
  v = group_sum<64>(v);
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < W; ++i) r += lds[i];
  __syncthreads();
  return r;
}

// One workgroup per row.  idx_ws / w_ws: [rows][k] scratch (indices, weights).
// Compaction reads kElems consecutive scores per thread per pass, so one pass
// (two workgroup scans) covers kRowThreads * kElems scores in index order.  For
// D <= kMaxFastD the weighted sum is left to topk_pv_kernel (meta gets the
// row's kept count and weight sum); wider rows are summed here, one thread
// per value dimension.
constexpr int kElems = 4;
constexpr int kMaxFastD = 256;
constexpr int kSplits = 16;  // workgroups per row in the weighted sum

struct RowMeta {
  int count;
  float l;
};

__global__ void __launch_bounds__(kRowThreads) topk_attend_kernel(const float* scores, int N, long long ld, int k,
                                                               const uint32_t* sel, const float* values, int D,
                                                               long long ldv, int32_t* idx_ws, float* w_ws,
                                                               RowMeta* meta, float* out, long long ldo) {
  __shared__ int scan_lds[kRowWaves];
  __shared__ float red_lds[kRowWaves];
  const int tid = threadIdx.x;
  const int m = blockIdx.x;
  const float* row = scores + (size_t)m * ld;
  const uint32_t t_key = sel[2 * m];
  const int ties = (int)sel[2 * m + 1];
  int32_t* idx = idx_ws + (size_t)m * k;
  float* wts = w_ws + (size_t)m * k;
  int count = 0, ties_seen = 0;
  float mx = -INFINITY;
  for (int base = 0; base < N; base += kRowThreads * kElems) {
    const int n0 = base + tid * kElems;
    float s[kElems];
    bool gt[kElems], eq[kElems];
    int n_eq = 0;
#pragma unroll
    for (int e = 0; e < kElems; ++e) {
      const int n = n0 + e;
      s[e] = n < N ? row[n] : 0.f;
      const uint32_t key = order_key(s[e]);
      gt[e] = n < N && key > t_key;
      eq[e] = n < N && key == t_key;
      n_eq += eq[e] ? 1 : 0;
    }
    int eq_total;
    int eq_rank = block_exclusive_scan<kRowWaves>(n_eq, eq_total, scan_lds) + ties_seen;
    bool take[kElems];
    int n_take = 0;
#pragma unroll
    for (int e = 0; e < kElems; ++e) {
      take[e] = gt[e] || (eq[e] && eq_rank < ties);
      eq_rank += eq[e] ? 1 : 0;
      n_take += take[e] ? 1 : 0;
    }
    int take_total;
    int pos = block_exclusive_scan<kRowWaves>(n_take, take_total, scan_lds) + count;
#pragma unroll
    for (int e = 0; e < kElems; ++e) {
      if (take[e]) {
        if (pos < k) {
          idx[pos] = n0 + e;
          mx = fmaxf(mx, s[e]);
        }
        ++pos;
      }
    }
    ties_seen += eq_total;
    count += take_total;
  }
  count = min(count, k);
  mx = block_max<kRowWaves>(mx, red_lds);
  float part = 0.f;
  for (int i = tid; i < count; i += kRowThreads) {
    const float w = expf(row[idx[i]] - mx);
    wts[i] = w;
    part += w;
  }
  const float l = block_sum<kRowWaves>(part, red_lds);  // its barriers also publish idx / wts to the workgroup
  if (D <= kMaxFastD) {
    if (tid == 0) meta[m] = RowMeta{count, l};
    return;
  }
  for (int d = tid; d < D; d += kRowThreads) {
    float acc = 0.f;
    for (int i = 0; i < count; ++i) acc = fmaf(wts[i], values[(size_t)idx[i] * ldv + d], acc);
    out[(size_t)m * ldo + d] = acc / l;
  }
}

// Weighted sum of the kept values of row m = blockIdx.x, split s = blockIdx.y
// of kSplits: the split's tokens (a contiguous range of the kept list) are
// dealt to the wavefronts in turn, 8 tokens' loads issued together; each lane
// holds dims lane, lane + 64, ... of its wavefront's sum, and the wavefronts'
// sums are added through LDS into part[m][s][:].
__global__ void __launch_bounds__(kThreads) topk_pv_kernel(const int32_t* idx_ws, const float* w_ws,
                                                           const RowMeta* meta, int k, const float* values, int D,
                                                           long long ldv, float* part) {
  __shared__ float part_lds[kWaves][kMaxFastD];
  const int m = blockIdx.x, sp = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int count = meta[m].count;
  const int chunk = (count + kSplits - 1) / kSplits;
  const int lo = min(sp * chunk, count), hi = min(lo + chunk, count);
  const int32_t* idx = idx_ws + (size_t)m * k;
  const float* wts = w_ws + (size_t)m * k;
  float acc[kMaxFastD / 64];
#pragma unroll
  for (int c = 0; c < kMaxFastD / 64; ++c) acc[c] = 0.f;
  constexpr int U = 8;  // tokens whose loads are issued together
  int i = lo + wave;
  for (; i + (U - 1) * kWaves < hi; i += U * kWaves) {
    float wt[U], v[U][kMaxFastD / 64];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      wt[u] = wts[i + u * kWaves];
      const float* vr = values + (size_t)idx[i + u * kWaves] * ldv;
#pragma unroll
      for (int c = 0; c < kMaxFastD / 64; ++c) v[u][c] = c * 64 + lane < D ? vr[c * 64 + lane] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int c = 0; c < kMaxFastD / 64; ++c) acc[c] = fmaf(wt[u], v[u][c], acc[c]);
  }
  for (; i < hi; i += kWaves) {
    const float wt = wts[i];
    const float* vr = values + (size_t)idx[i] * ldv;
#pragma unroll
    for (int c = 0; c < kMaxFastD / 64; ++c)
      if (c * 64 + lane < D) acc[c] = fmaf(wt, vr[c * 64 + lane], acc[c]);
  }
#pragma unroll
  for (int c = 0; c < kMaxFastD / 64; ++c) part_lds[wave][c * 64 + lane] = acc[c];
  __syncthreads();
  float* dst = part + ((size_t)m * kSplits + sp) * kMaxFastD;
  for (int d = threadIdx.x; d < D; d += kThreads) {
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) sum += part_lds[w][d];
    dst[d] = sum;
  }
}

// out[m][:] = (sum over the splits of part[m][s][:]) / l_m, splits in order.
__global__ void __launch_bounds__(kThreads) topk_combine_kernel(const float* part, const RowMeta* meta, int D,
                                                                float* out, long long ldo) {
  const int m = blockIdx.x;
  const float l = meta[m].l;
  for (int d = threadIdx.x; d < D; d += kThreads) {
    float sum = 0.f;
    for (int sp = 0; sp < kSplits; ++sp) sum += part[((size_t)m * kSplits + sp) * kMaxFastD + d];
    out[(size_t)m * ldo + d] = sum / l;
  }
}

}  // namespace
}  // namespace vrm

using namespace vrm;

// Workspace: sel [M][2] u32, idx [M][k] i32, weights [M][k] f32, row meta
// [M], weighted-sum partials [M][kSplits][kMaxFastD] f32.
static size_t topk_ws_offsets(int M, int k, size_t* idx_off, size_t* w_off, size_t* meta_off, size_t* part_off) {
  size_t o = (size_t)M * 2 * sizeof(uint32_t);
  *idx_off = o;
  o += (size_t)M * (size_t)k * sizeof(int32_t);
  *w_off = o;
  o += (size_t)M * (size_t)k * sizeof(float);
  o = (o + 15) / 16 * 16;
  *meta_off = o;
  o += (size_t)M * sizeof(RowMeta);
  o = (o + 15) / 16 * 16;
  *part_off = o;
  return o + (size_t)M * kSplits * kMaxFastD * sizeof(float);
}

extern "C" size_t vrm_topk_attend_workspace_bytes(int M, int k) {
  if (M < 0 || k < 0) return 0;
  size_t a, b, c, d;
  return topk_ws_offsets(M, k, &a, &b, &c, &d);
}

extern "C" int vrm_topk_attend(const float* scores, int M, int N, long long ld_scores, int k, const float* values,
                               int D, long long ld_values, float* out, long long ld_out, void* workspace,
                               size_t workspace_bytes, vrm_stream_t stream) {
  const char* who = "vrm_topk_attend";
  if (M < 0 || N <= 0 || D <= 0 || k < 1 || k > N || ld_scores < N || ld_values < D || ld_out < D) {
    set_error("%s: bad sizes (M=%d N=%d k=%d D=%d ld=%lld/%lld/%lld)", who, M, N, k, D, ld_scores, ld_values,
              ld_out);
    return VRM_ERR_ARG;
  }
  if (M > 0x7fffffff / 2) {
    set_error("%s: too many rows (%d)", who, M);
    return VRM_ERR_UNSUPPORTED;
  }
  if (workspace_bytes < vrm_topk_attend_workspace_bytes(M, k)) {
    set_error("%s: workspace of %zu bytes, need %zu", who, workspace_bytes, vrm_topk_attend_workspace_bytes(M, k));
    return VRM_ERR_WORKSPACE;
  }
  if (M == 0) {
    clear_error();
    return VRM_OK;
  }
  if (!scores || !values || !out || !workspace) {
    set_error("%s: null pointer argument", who);
    return VRM_ERR_ARG;
  }
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  size_t idx_off, w_off, meta_off, part_off;
  topk_ws_offsets(M, k, &idx_off, &w_off, &meta_off, &part_off);
  uint32_t* sel = reinterpret_cast<uint32_t*>(ws);
  int32_t* idx = reinterpret_cast<int32_t*>(ws + idx_off);
  float* wts = reinterpret_cast<float*>(ws + w_off);
  RowMeta* meta = reinterpret_cast<RowMeta*>(ws + meta_off);
  float* part = reinterpret_cast<float*>(ws + part_off);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(topk_select_kernel, dim3(M), dim3(kRowThreads), 0, st, scores, N, ld_scores, k, sel);
  hipLaunchKernelGGL(topk_attend_kernel, dim3(M), dim3(kRowThreads), 0, st, scores, N, ld_scores, k, sel, values, D,
                     ld_values, idx, wts, meta, out, ld_out);
  if (D <= kMaxFastD) {
    hipLaunchKernelGGL(topk_pv_kernel, dim3(M, kSplits), dim3(kThreads), 0, st, idx, wts, meta, k, values, D,
                       ld_values, part);
    hipLaunchKernelGGL(topk_combine_kernel, dim3(M), dim3(kThreads), 0, st, part, meta, D, out, ld_out);
  }
  return launch_status(who);
}
