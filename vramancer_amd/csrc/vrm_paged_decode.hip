// Split-K paged decode attention for gfx950.
//
// Semantics follow the reference's decode path (core/paged_attention_cuda.py:
// 187-231 and csrc/paged_attention_kernel.cu:61-174): per sequence b and query
// head h, out = softmax(scale * q . K^T) V over the first context_lens[b]
// tokens of the sequence's pages, with GQA head h reading kv-head h / (H/KH).
//
// Design (MI355X-first, not the reference's one-warp-per-head loop):
//  * one 64-lane wavefront per (sequence, kv-head, head group, token
//    partition); the query heads that share a kv-head are packed into the same
//    wavefront, so every K/V byte is read from HBM once per partition instead
//    of once per query head;
//  * each lane issues 16-byte loads of the contiguous [PS][D] page slice; the
//    page ids of a partition are fetched with one vector load up front and the
//    next page is loaded while the current one is consumed;
//  * this VALU kernel serves the float32 pool and the 4-bit pool (dequantized
//    in registers as (nibble - zero) * scale); the bf16, f16, int8 and fp8
//    pools go to the single-pass matrix-core kernels of vrm_decode_mfma.hip;
//  * phase 1 writes all scores of the partition to LDS, phase 2 takes the
//    exact partition maximum, phase 3 streams V once with fixed weights, so no
//    running rescale of the accumulators is needed;
//  * partitions leave (max, sum, unnormalised acc) in the workspace and a
//    second kernel merges them with log-sum-exp weights.
#include "vrm_decode.h"

#include <math.h>

#include <map>
#include <mutex>
#include <tuple>
#include <utility>

namespace vrm {
namespace dec {

// Work items one resident round of `kernel` holds: resident wavefronts (CU
// count x workgroups per CU from the occupancy query, capped at
// kMaxTargetWaves) over the wavefronts of one item.  Cached per (device,
// kernel, workgroup size, LDS bytes): the generic kernels' LDS depends on the
// call's head_dim or TurboQuant setting, and with it their occupancy.
int items_target(const void* kernel, int waves_per_block, size_t lds_bytes, int units) {
  using Key = std::tuple<int, const void*, int, size_t>;
  static std::mutex mu;
  static std::map<Key, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  const Key key{dev, kernel, waves_per_block, lds_bytes};
  int waves = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) waves = it->second;
  }
  if (waves == 0) {
    int cus = 0, blocks = 0;
    if (dev < 0 || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, 64 * waves_per_block, lds_bytes) != hipSuccess ||
        blocks <= 0)
      blocks = 1;
    waves = cus * blocks * waves_per_block;
    std::lock_guard<std::mutex> lock(mu);
    cache[key] = waves;
  }
  return std::max(1, std::min(waves, kMaxTargetWaves) / units);
}

size_t shared_items_max_lds() {
  static std::mutex mu;
  static std::map<int, size_t> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return kMaxBalancedLds;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int bytes = 0;
  size_t lim = kMaxBalancedLds;
  if (hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && bytes > 0)
    lim = std::max(kMaxBalancedLds, std::min<size_t>((size_t)bytes, 160 * 1024));
  cache[dev] = lim;
  return lim;
}

namespace {

template <int KIND>
__device__ __forceinline__ void unpack16(const uint4 r, float* x) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
  if constexpr (KIND == K_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = __uint_as_float(w[i]);
  } else if constexpr (KIND == K_F16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
      x[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
    }
  } else if constexpr (KIND == K_BF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {  // K_Q4: raw nibbles; byte j holds d = 2j (low) and 2j + 1 (high)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t byte = (w[i] >> (8 * j)) & 0xffu;
        x[8 * i + 2 * j] = (float)(byte & 0xfu);
        x[8 * i + 2 * j + 1] = (float)(byte >> 4);
      }
    }
  }
}



// Registers holding one page of K or V for this lane, plus its dequant factors.
template <int KIND, int LPP>
struct PageRegs {
  uint4 data[LPP];
  float s0[LPP];  // q4: group scale of the lane's chunk
  float s1[LPP];  // q4: group zero point
};

// One wavefront per (work item, kv head x head chunk).  A partition longer
// than kChunkPages pages is walked in chunks; each chunk runs the three
// phases below with its own exact maximum and is folded into the running
// (max, sum, acc) of the partition.
constexpr int kChunkPages = 64;

template <int KIND, int D, int G>
__global__ void __launch_bounds__(64) decode_split_kernel(DecodeArgs a) {
  constexpr int E = Kv<KIND>::kElems;         // elements per 16-byte lane chunk
  constexpr int RB = D * 16 / E;              // bytes per token row
  constexpr int LPT = RB / 16;                // lanes per token
  constexpr int TPL = 64 / LPT;               // tokens per wave load
  constexpr int LPP = (kPS + TPL - 1) / TPL;  // wave loads per page
  constexpr int HEAD_BYTES = kPS * RB;        // one (page, layer, kv, head) slice
  constexpr int Q4G = D / 32;                 // 4-bit groups per row
  constexpr int TS = kChunkPages * kPS;       // tokens per chunk
  static_assert(LPT >= 1 && LPT <= 64 && (64 % LPT) == 0, "lane mapping");
  static_assert(TPL <= kPS || (TPL % kPS) == 0, "page mapping");
  static_assert(LPP * TPL * RB == (TPL <= kPS ? HEAD_BYTES : TPL * RB), "load coverage");

  extern __shared__ float lds[];
  float* s_lds = lds;  // [G][TS] scores, then softmax weights

  const int lane = threadIdx.x;
  const int group = a.H / a.KH;
  const int chunks = group / G;
  const int unit = blockIdx.y;
  const int kvh = unit / chunks;
  const int h0 = kvh * group + (unit % chunks) * G;
  const int item = blockIdx.x;
  WorkItem wi;
  if (!find_item(a.ctx_lens, a.B, a.max_pp, a.target, item, item == 0 && unit == 0, a.header, wi)) return;
  const int b = wi.b;

  const int c = lane % LPT;   // which 16-byte chunk of a token row
  const int tl = lane / LPT;  // which token of a wave load
  const bool lane_live = (TPL <= kPS) || (tl < kPS);

  const size_t kv_stride = (size_t)a.KH * HEAD_BYTES;
  const size_t page_stride = kv_stride * 2 * a.L;
  const uint8_t* layer_base = a.pool + (size_t)a.layer * 2 * kv_stride + (size_t)kvh * HEAD_BYTES;

  auto page_ok = [&](int pid) { return pid >= 0 && pid < a.P; };
  // Index of (page, layer, kv, kvh) in units of heads.
  auto head_index = [&](int pid, int kv) { return (((size_t)pid * a.L + a.layer) * 2 + kv) * a.KH + kvh; };

  // Loads page `pid` of K (kv = 0) or V (kv = 1) and the factors this lane needs.
  auto load_page = [&](PageRegs<KIND, LPP>& r, int pid, int kv) {
    const bool ok = page_ok(pid);
    const uint8_t* base = layer_base + (size_t)(ok ? pid : 0) * page_stride + (size_t)kv * kv_stride;
#pragma unroll
    for (int j = 0; j < LPP; ++j) {
      const int tp = j * TPL + tl;
      const bool live = ok && lane_live;
      r.data[j] = live ? *reinterpret_cast<const uint4*>(base + (size_t)j * 1024 + (size_t)lane * 16)
                       : make_uint4(0, 0, 0, 0);
      r.s0[j] = 1.f;
      r.s1[j] = 0.f;
      if constexpr (KIND == K_Q4) {
        if (live) {
          const size_t rs = (head_index(pid, kv) * kPS + tp) * Q4G + c;  // lane chunk c == group c
          r.s0[j] = f16_bits_to_f32(a.q4_scale[rs]);
          r.s1[j] = f16_bits_to_f32(a.q4_zero[rs]);
        }
      }
    }
  };

  // Query chunk of every head of the group, pre-scaled into the log2 domain.
  float qr[G][E];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float* qh = a.query + ((size_t)b * a.H + h0 + g) * D;
#pragma unroll
    for (int e = 0; e < E; ++e) qr[g][e] = qh[c * E + e] * a.qscale;
  }

  float m_run[G], l_run[G], acc[G][E];  // running softmax state of the partition
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[g][e] = 0.f;
  }

  for (int c0 = 0; c0 < wi.n_pages; c0 += kChunkPages) {
  const int n_pages = min(kChunkPages, wi.n_pages - c0);
  const int tok_end = min(n_pages * kPS, wi.ctx - (wi.p_begin + c0) * kPS);  // valid tokens in the chunk
  // Page ids of this chunk: lane i holds logical page p_begin + c0 + i.
  int my_pid = -1;
  if (lane < n_pages) my_pid = a.page_table[(size_t)b * a.max_pp + wi.p_begin + c0 + lane];

  // ---------------- phase 1: scores ----------------
  {
    PageRegs<KIND, LPP> cur;
    int pid_cur = __builtin_amdgcn_readlane(my_pid, 0);
    load_page(cur, pid_cur, 0);
    for (int pi = 0; pi < n_pages; ++pi) {
      PageRegs<KIND, LPP> nxt;
      const int pid_nxt = (pi + 1 < n_pages) ? __builtin_amdgcn_readlane(my_pid, pi + 1) : -1;
      if (pi + 1 < n_pages) load_page(nxt, pid_nxt, 0);
      const bool ok = page_ok(pid_cur);
#pragma unroll
      for (int j = 0; j < LPP; ++j) {
        const int tp = j * TPL + tl;  // token within page
        const int t = pi * kPS + tp;  // token within split
        const bool valid = ok && lane_live && tp < kPS && t < tok_end;
        float x[E];
        unpack16<KIND>(cur.data[j], x);
        if constexpr (KIND == K_Q4) {
#pragma unroll
          for (int e = 0; e < E; ++e) x[e] = (x[e] - cur.s1[j]) * cur.s0[j];
        }
        float part[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float s = 0.f;
#pragma unroll
          for (int e = 0; e < E; ++e) s = fmaf(qr[g][e], x[e], s);
          part[g] = group_sum<LPT>(s);
        }
        if (c == 0 && lane_live && tp < kPS && t < TS) {
#pragma unroll
          for (int g = 0; g < G; ++g) s_lds[g * TS + t] = valid ? part[g] : -INFINITY;
        }
      }
      cur = nxt;
      pid_cur = pid_nxt;
    }
  }
  __syncthreads();

  // ---------------- phase 2: exact chunk maximum, folded into the running state ----------------
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mx = -INFINITY;
    for (int t = lane; t < tok_end; t += 64) mx = fmaxf(mx, s_lds[g * TS + t]);
    mx = group_max<64>(mx);
    const float m_new = fmaxf(m_run[g], mx);
    const float keep = (m_run[g] == -INFINITY) ? 0.f : exp2f(m_run[g] - m_new);
    float sum = 0.f;
    for (int t = lane; t < tok_end; t += 64) {
      const float s = s_lds[g * TS + t];
      const float p = (s == -INFINITY) ? 0.f : exp2f(s - m_new);
      sum += p;
      s_lds[g * TS + t] = p;
    }
    l_run[g] = l_run[g] * keep + group_sum<64>(sum);
    m_run[g] = m_new;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[g][e] *= keep;
  }
  __syncthreads();

  // ---------------- phase 3: weighted V ----------------
  {
    PageRegs<KIND, LPP> cur;
    int pid_cur = __builtin_amdgcn_readlane(my_pid, 0);
    load_page(cur, pid_cur, 1);
    for (int pi = 0; pi < n_pages; ++pi) {
      PageRegs<KIND, LPP> nxt;
      const int pid_nxt = (pi + 1 < n_pages) ? __builtin_amdgcn_readlane(my_pid, pi + 1) : -1;
      if (pi + 1 < n_pages) load_page(nxt, pid_nxt, 1);
      const bool ok = page_ok(pid_cur);
#pragma unroll
      for (int j = 0; j < LPP; ++j) {
        const int tp = j * TPL + tl;
        const int t = pi * kPS + tp;
        const bool valid = ok && lane_live && tp < kPS && t < tok_end;
        if (valid) {
          float x[E];
          unpack16<KIND>(cur.data[j], x);
          if constexpr (KIND == K_Q4) {
#pragma unroll
            for (int e = 0; e < E; ++e) x[e] = (x[e] - cur.s1[j]) * cur.s0[j];
          }
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const float w = s_lds[g * TS + t];
#pragma unroll
            for (int e = 0; e < E; ++e) acc[g][e] = fmaf(w, x[e], acc[g][e]);
          }
        }
      }
      cur = nxt;
      pid_cur = pid_nxt;
    }
  }

  __syncthreads();  // the next chunk overwrites the scores
  }  // chunk loop

  // Lanes that hold the same chunk c (different tokens) sum their partials.
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < E; ++e) acc[g][e] = strided_sum<LPT>(acc[g][e]);

  if (tl == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float* dst = a.part_acc + ((size_t)item * a.H + h0 + g) * D + c * E;
#pragma unroll
      for (int e = 0; e < E; ++e) dst[e] = acc[g][e];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      a.part_ml[((size_t)item * a.H + h0 + g) * 2] = m_run[g];
      a.part_ml[((size_t)item * a.H + h0 + g) * 2 + 1] = l_run[g];
    }
  }
}

// Merges the partitions of one (sequence, head): out = sum_s w_s acc_s / sum_s w_s l_s
// with w_s = 2^(m_s - max_s m_s).  The items of sequence b are its full
// partitions first_b .. first_{b+1} - 1 and its tail item, as recorded in the
// header by the partition pass.  Four wavefronts each fold every fourth
// partial, BATCH at a time with all loads issued together (clamped,
// unconditional), and the four results are combined through LDS.
template <int DMAX>
__global__ void __launch_bounds__(256) decode_reduce_kernel(const float* __restrict__ part_acc,
                                                            const float* __restrict__ part_ml,
                                                            const int32_t* __restrict__ header,
                                                            float* __restrict__ out, float* __restrict__ lse, int H,
                                                            int B, int D) {
  constexpr int PER = DMAX / 64;  // dims per lane; lanes past D idle
  constexpr int BATCH = 4;
  constexpr int WAVES = 4;
  __shared__ float sh_m[WAVES], sh_l[WAVES];
  __shared__ float sh_res[WAVES][DMAX];
  // Workgroups start in blockIdx order: the sequence with the most partials
  // (the longest fold) takes row 0, so that its merge overlaps the others'.
  // The entries of sequence blockIdx.y load together with header[3] and
  // header[4]; only the two swapped rows load theirs again.
  const int y = blockIdx.y;
  const int big = min(max(header[3], 0), B - 1);
  const bool direct = header[4] != 0;
  int first = header[kHeaderInts + y];
  int next = header[kHeaderInts + y + 1];
  int tail = header[kHeaderInts + B + 1 + y];
  const int h = blockIdx.x, b = y == 0 ? big : (y == big ? 0 : y);
  if (b != y) {
    first = header[kHeaderInts + b];
    next = header[kHeaderInts + b + 1];
    tail = header[kHeaderInts + B + 1 + b];
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nf = next - first;
  const int nact = nf + (tail >= 0 ? 1 : 0);
  if (nact == 1 && direct) return;  // the partition pass wrote this sequence's rows
  auto item_of = [&](int s) { return s < nf ? first + s : tail; };
  float M = -INFINITY, Lsum = 0.f;
  float res[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) res[i] = 0.f;
  // Two register batches: the loads of batch k + 1 are in flight while batch k
  // is folded, so a long sequence costs one memory latency, not one per batch.
  float m[2][BATCH], l[2][BATCH], x[2][BATCH][PER];
  auto load_batch = [&](int buf, int s0) {
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const int s = s0 + k * WAVES;
      const size_t it = (size_t)item_of(min(s, nact - 1)) * H + h;
      m[buf][k] = part_ml[it * 2];
      l[buf][k] = part_ml[it * 2 + 1];
#pragma unroll
      for (int i = 0; i < PER; ++i) x[buf][k][i] = i * 64 + lane < D ? part_acc[it * D + i * 64 + lane] : 0.f;
    }
  };
  auto fold_batch = [&](int buf, int s0) {
    float cm = M;
#pragma unroll
    for (int k = 0; k < BATCH; ++k)
      if (s0 + k * WAVES < nact) cm = fmaxf(cm, m[buf][k]);
    if (cm == -INFINITY) return;
    const float keep = (M == -INFINITY) ? 0.f : exp2f(M - cm);
    Lsum *= keep;
#pragma unroll
    for (int i = 0; i < PER; ++i) res[i] *= keep;
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const bool live = s0 + k * WAVES < nact && m[buf][k] != -INFINITY;
      const float w = live ? exp2f(m[buf][k] - cm) : 0.f;
      Lsum = fmaf(w, l[buf][k], Lsum);
#pragma unroll
      for (int i = 0; i < PER; ++i) res[i] = fmaf(w, x[buf][k][i], res[i]);
    }
    M = cm;
  };
  constexpr int STEP = WAVES * BATCH;
  if (wave < nact) {
    load_batch(0, wave);
    int s0 = wave;
    for (; s0 + STEP < nact; s0 += 2 * STEP) {
      load_batch(1, s0 + STEP);
      fold_batch(0, s0);
      load_batch(0, s0 + 2 * STEP);  // unconditional (clamped): a branch would make the compiler wait for all loads
      fold_batch(1, s0 + STEP);
    }
    if (s0 < nact) fold_batch(0, s0);
  }
  if (lane == 0) {
    sh_m[wave] = M;
    sh_l[wave] = Lsum;
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) sh_res[wave][i * 64 + lane] = res[i];
  __syncthreads();
  if (wave == 0) {
    float gm = -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) gm = fmaxf(gm, sh_m[w]);
    float L = 0.f, o[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) o[i] = 0.f;
    if (gm != -INFINITY) {
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        const float f = sh_m[w] == -INFINITY ? 0.f : exp2f(sh_m[w] - gm);
        L = fmaf(f, sh_l[w], L);
#pragma unroll
        for (int i = 0; i < PER; ++i) o[i] = fmaf(f, sh_res[w][i * 64 + lane], o[i]);
      }
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    float* dst = out + ((size_t)b * H + h) * D;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (i * 64 + lane < D) dst[i * 64 + lane] = o[i] * inv;
    // ln sum_t exp(scale q.k_t) = (max + log2 L) ln 2, the maxima being in the log2 domain
    if (lse && lane == 0) lse[(size_t)b * H + h] = L > 0.f ? (gm + log2f(L)) * 0.6931471805599453f : -INFINITY;
  }
}

// The same merge with one wavefront per (sequence, head) and the four heads
// blockIdx.x * 4 .. + 3 of one sequence per workgroup: each wavefront folds
// every partial of its head, BATCH at a time from two register batches, and
// writes the row itself.  A quarter of the workgroups of
// decode_reduce_kernel, for batches where most sequences need no merge or
// few partials.
template <int DMAX>
__global__ void __launch_bounds__(256) decode_reduce_rows_kernel(const float* __restrict__ part_acc,
                                                                 const float* __restrict__ part_ml,
                                                                 const int32_t* __restrict__ header,
                                                                 float* __restrict__ out, float* __restrict__ lse,
                                                                 int H, int B, int D) {
  constexpr int PER = DMAX / 64;
  constexpr int BATCH = 4;
  const int y = blockIdx.y;
  const int big = min(max(header[3], 0), B - 1);
  const bool direct = header[4] != 0;
  int first = header[kHeaderInts + y];
  int next = header[kHeaderInts + y + 1];
  int tail = header[kHeaderInts + B + 1 + y];
  const int b = y == 0 ? big : (y == big ? 0 : y);
  if (b != y) {
    first = header[kHeaderInts + b];
    next = header[kHeaderInts + b + 1];
    tail = header[kHeaderInts + B + 1 + b];
  }
  const int nf = next - first;
  const int nact = nf + (tail >= 0 ? 1 : 0);
  if (nact == 1 && direct) return;  // the partition pass wrote this sequence's rows
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = blockIdx.x * 4 + wave;
  if (h >= H) return;
  auto item_of = [&](int s) { return s < nf ? first + s : tail; };
  float M = -INFINITY, Lsum = 0.f;
  float res[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) res[i] = 0.f;
  float m[2][BATCH], l[2][BATCH], x[2][BATCH][PER];
  auto load_batch = [&](int buf, int s0) {
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const size_t it = (size_t)item_of(min(s0 + k, nact - 1)) * H + h;
      m[buf][k] = part_ml[it * 2];
      l[buf][k] = part_ml[it * 2 + 1];
#pragma unroll
      for (int i = 0; i < PER; ++i) x[buf][k][i] = i * 64 + lane < D ? part_acc[it * D + i * 64 + lane] : 0.f;
    }
  };
  auto fold_batch = [&](int buf, int s0) {
    float cm = M;
#pragma unroll
    for (int k = 0; k < BATCH; ++k)
      if (s0 + k < nact) cm = fmaxf(cm, m[buf][k]);
    if (cm == -INFINITY) return;
    const float keep = (M == -INFINITY) ? 0.f : exp2f(M - cm);
    Lsum *= keep;
#pragma unroll
    for (int i = 0; i < PER; ++i) res[i] *= keep;
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const bool live = s0 + k < nact && m[buf][k] != -INFINITY;
      const float w = live ? exp2f(m[buf][k] - cm) : 0.f;
      Lsum = fmaf(w, l[buf][k], Lsum);
#pragma unroll
      for (int i = 0; i < PER; ++i) res[i] = fmaf(w, x[buf][k][i], res[i]);
    }
    M = cm;
  };
  if (nact > 0) {
    load_batch(0, 0);
    int s0 = 0;
    for (; s0 + BATCH < nact; s0 += 2 * BATCH) {
      load_batch(1, s0 + BATCH);
      fold_batch(0, s0);
      load_batch(0, s0 + 2 * BATCH);  // unconditional (clamped), as above
      fold_batch(1, s0 + BATCH);
    }
    if (s0 < nact) fold_batch(0, s0);
  }
  const float inv = Lsum > 0.f ? 1.f / Lsum : 0.f;
  float* dst = out + ((size_t)b * H + h) * D;
#pragma unroll
  for (int i = 0; i < PER; ++i)
    if (i * 64 + lane < D) dst[i * 64 + lane] = res[i] * inv;
  if (lse && lane == 0) lse[(size_t)b * H + h] = Lsum > 0.f ? (M + log2f(Lsum)) * 0.6931471805599453f : -INFINITY;
}

// out = (e^(lse1 - m) o1 + e^(lse2 - m) o2) / (e^(lse1 - m) + e^(lse2 - m)),
// m = max(lse1, lse2): two attentions over disjoint token sets merged into
// the attention over their union; lse_out (optional) gets the union's lse.
__global__ void __launch_bounds__(256) attn_combine_kernel(const float* __restrict__ o1, const float* __restrict__ lse1,
                                                           const float* __restrict__ o2, const float* __restrict__ lse2,
                                                           long long rows, int D, float* __restrict__ out,
                                                           float* __restrict__ lse_out) {
  const long long x = (long long)blockIdx.x * 256 + threadIdx.x;
  if (x >= rows * D) return;
  const long long r = x / D;
  const float a = lse1[r], c = lse2[r];
  const float m = fmaxf(a, c);
  float w1 = 0.f, w2 = 0.f;
  if (m != -INFINITY) {
    w1 = a == -INFINITY ? 0.f : expf(a - m);
    w2 = c == -INFINITY ? 0.f : expf(c - m);
  }
  const float den = w1 + w2;
  out[x] = den > 0.f ? (w1 * o1[x] + w2 * o2[x]) / den : 0.f;
  if (lse_out && x % D == 0) lse_out[r] = den > 0.f ? m + logf(den) : -INFINITY;
}

template <int KIND, int D, int G>
hipError_t launch_split(const DecodeArgs& a0, int B, hipStream_t st) {
  const int units = a0.KH * ((a0.H / a0.KH) / G);
  const size_t lds = (size_t)G * kChunkPages * kPS * sizeof(float);
  DecodeArgs a = a0;
  a.target = items_target(reinterpret_cast<const void*>(&decode_split_kernel<KIND, D, G>), 1, lds, units);
  dim3 grid(B + 2 * a.target, units, 1);  // at most B + 2 target work items
  hipLaunchKernelGGL((decode_split_kernel<KIND, D, G>), grid, dim3(64), lds, st, a);
  return hipGetLastError();
}

template <int KIND, int D>
hipError_t dispatch_g(const DecodeArgs& a, int B, int G, hipStream_t st) {
  if constexpr (KIND == K_Q4) {  // 32 elements per lane chunk: at most 6 heads per wave (7 spill at D = 128)
    switch (G) {
      case 1: return launch_split<KIND, D, 1>(a, B, st);
      case 2: return launch_split<KIND, D, 2>(a, B, st);
      case 3: return launch_split<KIND, D, 3>(a, B, st);
      case 4: return launch_split<KIND, D, 4>(a, B, st);
      case 5: return launch_split<KIND, D, 5>(a, B, st);
      default: return launch_split<KIND, D, 6>(a, B, st);
    }
  } else {
    switch (G) {
      case 1: return launch_split<KIND, D, 1>(a, B, st);
      case 2: return launch_split<KIND, D, 2>(a, B, st);
      case 3: return launch_split<KIND, D, 3>(a, B, st);
      case 4: return launch_split<KIND, D, 4>(a, B, st);
      case 5: return launch_split<KIND, D, 5>(a, B, st);
      case 6: return launch_split<KIND, D, 6>(a, B, st);
      case 7: return launch_split<KIND, D, 7>(a, B, st);
      default: return launch_split<KIND, D, 8>(a, B, st);
    }
  }
}

template <int KIND>
hipError_t dispatch_d(const DecodeArgs& a, int B, int D, int G, hipStream_t st) {
  switch (D) {
    case 64: return dispatch_g<KIND, 64>(a, B, G, st);
    case 128: return dispatch_g<KIND, 128>(a, B, G, st);
    default: return dispatch_g<KIND, 256>(a, B, G, st);
  }
}

// rows: one wavefront per (sequence, head) (decode_reduce_rows_kernel), for
// the shared-items pass, whose sequences mostly need no merge or a few
// partials (c3's reference-signature call: 98.6 -> 97.7 us); otherwise four
// per (sequence, head), for the work items' 14-16 partials per sequence
// (c2 / c4: 0.3-1.7 us faster than one).
hipError_t launch_reduce(const DecodeArgs& a, float* out, int B, int D, hipStream_t st, bool rows = false) {
  const dim3 block(256);
  if (rows) {
    const dim3 grid((a.H + 3) / 4, B);
    if (D <= 64)
      hipLaunchKernelGGL(decode_reduce_rows_kernel<64>, grid, block, 0, st, a.part_acc, a.part_ml, a.header, out,
                         a.lse, a.H, B, D);
    else if (D <= 128)
      hipLaunchKernelGGL(decode_reduce_rows_kernel<128>, grid, block, 0, st, a.part_acc, a.part_ml, a.header, out,
                         a.lse, a.H, B, D);
    else
      hipLaunchKernelGGL(decode_reduce_rows_kernel<256>, grid, block, 0, st, a.part_acc, a.part_ml, a.header, out,
                         a.lse, a.H, B, D);
    return hipGetLastError();
  }
  const dim3 grid(a.H, B);
  if (D <= 64)
    hipLaunchKernelGGL(decode_reduce_kernel<64>, grid, block, 0, st, a.part_acc, a.part_ml, a.header, out, a.lse,
                       a.H, B, D);
  else if (D <= 128)
    hipLaunchKernelGGL(decode_reduce_kernel<128>, grid, block, 0, st, a.part_acc, a.part_ml, a.header, out, a.lse,
                       a.H, B, D);
  else
    hipLaunchKernelGGL(decode_reduce_kernel<256>, grid, block, 0, st, a.part_acc, a.part_ml, a.header, out, a.lse,
                       a.H, B, D);
  return hipGetLastError();
}

// Work-item capacity of the workspace: a call has at most B + 2 target items
// and target <= kMaxTargetWaves / units with units >= KH wavefronts per item.
long items_capacity(int B, int KH) { return (long)B + 2L * ((kMaxTargetWaves + KH - 1) / KH); }

int check_common(const float* query, const void* pool, const int32_t* page_table, const int32_t* ctx, float* out,
                 int B, int H, int KH, int D, int PS, int L, int P, int max_pp, int layer_idx, float scale) {
  if (!query || !pool || !page_table || !ctx || !out) {
    set_error("vrm_paged_decode: null pointer argument");
    return VRM_ERR_ARG;
  }
  if (B <= 0 || H <= 0 || KH <= 0 || D <= 0 || PS <= 0 || L <= 0 || P <= 0 || max_pp <= 0) {
    set_error("vrm_paged_decode: sizes must be positive (B=%d H=%d KH=%d D=%d PS=%d L=%d P=%d max_pp=%d)", B, H, KH,
              D, PS, L, P, max_pp);
    return VRM_ERR_ARG;
  }
  if (H % KH != 0) {
    set_error("vrm_paged_decode: num_heads %d is not a multiple of num_kv_heads %d", H, KH);
    return VRM_ERR_ARG;
  }
  if (layer_idx < 0 || layer_idx >= L) {
    set_error("vrm_paged_decode: layer_idx %d outside [0, %d)", layer_idx, L);
    return VRM_ERR_ARG;
  }
  if (!(scale == scale)) {
    set_error("vrm_paged_decode: scale is NaN");
    return VRM_ERR_ARG;
  }
  if (D > kMaxHeadDim) {
    set_error("vrm_paged_decode: head_dim %d above %d", D, kMaxHeadDim);
    return VRM_ERR_UNSUPPORTED;
  }
  if (B > 65535 || (long)B * H > 65535L * 65535L) {
    set_error("vrm_paged_decode: batch too large");
    return VRM_ERR_UNSUPPORTED;
  }
  return VRM_OK;
}

// Which passes run_decode enqueues.
enum Passes { kBoth = 3, kPartitionsOnly = 1, kMergeOnly = 2 };

// Shape limits of the pool kinds (VRM_ERR_UNSUPPORTED outside them): the
// int8 / fp8 pools' tiled V needs D % 16 and PS % 4, the 4-bit pool's groups
// D % 32.
int check_kind_shape(int kind, int D, int PS, const char* who) {
  if ((kind == K_I8 || kind == K_FP8) && (D % 16 || PS % 4)) {
    set_error("%s: int8 / fp8 pools need head_dim %% 16 == 0 and page_size %% 4 == 0 (got %d, %d)", who, D, PS);
    return VRM_ERR_UNSUPPORTED;
  }
  if (kind == K_Q4 && D % 32) {
    set_error("%s: head_dim %d is not a multiple of the group size 32", who, D);
    return VRM_ERR_UNSUPPORTED;
  }
  return VRM_OK;
}

int run_decode(DecodeArgs a, int kind, float* out, void* workspace, size_t workspace_bytes, int B, int D, int PS,
               float scale, hipStream_t st, int passes) {
  // The matrix-core stream kernels take the int8 / fp8 pools at every
  // head_dim, the 16-bit float pools at D <= 128 (at D = 256 their registers
  // spill) and the Q4 pool at D = 128 when its codes are 4-byte and its scales
  // and zeros 8-byte aligned (the widths of their loads); the rest runs on
  // the VALU kernel.
  const bool q4_aligned = ((reinterpret_cast<uintptr_t>(a.pool) & 3) | (reinterpret_cast<uintptr_t>(a.q4_scale) & 7) |
                           (reinterpret_cast<uintptr_t>(a.q4_zero) & 7)) == 0;
  // The tuned kernels are compiled for page 16: the matrix-core stream at
  // head_dim 64 / 80 / 96 / 112 / 128 (and 256 for int8 / fp8), the VALU split
  // kernel at 64 / 128 / 256; every other shape runs on the generic kernel
  // (vrm_decode_generic.hip).
  // The int8 / fp8 / bf16 / f16 stream kernels also take pages of 32, 64, ...
  // tokens (16 << vshift), which they stream as 16-token sub-pages.
  const bool stream_d = D == 64 || D == 80 || D == 96 || D == 112 || D == 128 || D == 256;
  const bool split_d = D == 64 || D == 128 || D == 256;
  int vshift = 0;
  while ((kPS << vshift) < PS && vshift < 6) ++vshift;
  const bool sub_pages = (kPS << vshift) == PS;  // PS = 16, 32, 64, ... 1024
  const bool mfma = (PS == kPS && kind == K_Q4 && D == 128 && q4_aligned) ||
                    (sub_pages && (((kind == K_I8 || kind == K_FP8) && stream_d) ||
                                   ((kind == K_BF16 || kind == K_F16) && stream_d && D <= 128)));
  const bool tuned = mfma || (PS == kPS && split_d);
  a.vshift = mfma ? vshift : 0;
  const int max_tile = mfma ? 16 : kind == K_Q4 ? 6 : 8;
  const int G = pick_group_tile(a.H / a.KH, max_tile);
  // int8 / fp8 at page 16 and head_dim 64 .. 128: the work items' pages are
  // shared by balanced workgroups (12 wavefronts, page pairs handed out in
  // LDS), when the page table fits their LDS copy
  const bool shared = (kind == K_I8 || kind == K_FP8) && PS == kPS && D >= 64 && D <= 128 && D % 16 == 0 &&
                      balanced_lds_bytes(a.max_pp, kMaxBalancedWaves, G, D) <= shared_items_max_lds();
  const int units = a.KH * ((a.H / a.KH) / G);  // wavefronts per work item
  (void)units;
  a.B = B;
  const long cap = items_capacity(B, a.KH);
  const size_t need = header_bytes(B) + (size_t)cap * a.H * (D + 2) * sizeof(float);
  if (!workspace || workspace_bytes < need) {
    set_error("vrm_paged_decode: workspace of %zu bytes is smaller than the %zu required", workspace_bytes, need);
    return VRM_ERR_WORKSPACE;
  }
  a.header = reinterpret_cast<int32_t*>(workspace);
  a.part_acc = reinterpret_cast<float*>(static_cast<char*>(workspace) + header_bytes(B));
  a.part_ml = a.part_acc + (size_t)cap * a.H * D;
  a.qscale = scale * kLog2e;
  // with both passes in the call, the shared-items pass writes sequences of
  // one piece to out itself
  a.out = passes == kBoth && shared ? out : nullptr;
  hipError_t e = hipSuccess;
  if ((passes & kPartitionsOnly) && !tuned) {
    e = launch_generic(a, kind, B, D, PS, st);
    if (e != hipSuccess) {
      set_error("vrm_paged_decode: partition kernel launch failed: %s", hipGetErrorString(e));
      return (int)e;
    }
  } else if (passes & kPartitionsOnly) {
    switch (kind) {
      case K_F32: e = dispatch_d<K_F32>(a, B, D, G, st); break;
      case K_F16: e = mfma ? launch_stream_mfma(a, kind, B, D, G, st) : dispatch_d<K_F16>(a, B, D, G, st); break;
      case K_BF16: e = mfma ? launch_stream_mfma(a, kind, B, D, G, st) : dispatch_d<K_BF16>(a, B, D, G, st); break;
      case K_I8:
      case K_FP8:
        e = shared ? launch_stream_shared_items(a, kind, B, D, G, st) : launch_stream_mfma(a, kind, B, D, G, st);
        break;
      default: e = mfma ? launch_stream_mfma(a, kind, B, D, G, st) : dispatch_d<K_Q4>(a, B, D, G, st); break;
    }
    if (e != hipSuccess) {
      set_error("vrm_paged_decode: partition kernel launch failed: %s", hipGetErrorString(e));
      return (int)e;
    }
  }
  if (passes & kMergeOnly) {
    e = launch_reduce(a, out, B, D, st, shared);
    if (e != hipSuccess) {
      set_error("vrm_paged_decode: merge kernel launch failed: %s", hipGetErrorString(e));
      return (int)e;
    }
  }
  clear_error();
  return VRM_OK;
}

// Partition pass over TurboQuant pages, then the shared merge.  gl is the
// generic layout's geometry, or null for the tuned layout.
int run_tq_decode(DecodeArgs a, const TqDecodeArgs& tq, int bits, const tq::GenLayout* gl, float* out,
                  void* workspace, size_t workspace_bytes, int B, int D, float scale, hipStream_t st) {
  a.B = B;
  const long cap = items_capacity(B, a.KH);
  const size_t need = header_bytes(B) + (size_t)cap * a.H * (D + 2) * sizeof(float);
  if (!workspace || workspace_bytes < need) {
    set_error("vrm_paged_decode_tq: workspace of %zu bytes is smaller than the %zu required", workspace_bytes, need);
    return VRM_ERR_WORKSPACE;
  }
  a.header = reinterpret_cast<int32_t*>(workspace);
  a.part_acc = reinterpret_cast<float*>(static_cast<char*>(workspace) + header_bytes(B));
  a.part_ml = a.part_acc + (size_t)cap * a.H * D;
  a.qscale = scale * kLog2e;
  hipError_t e = gl ? launch_tq_generic(a, tq, *gl, B, D, st) : launch_tq_decode(a, tq, bits, B, D, st);
  if (e != hipSuccess) {
    set_error("vrm_paged_decode_tq: partition kernel launch failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  e = launch_reduce(a, out, B, D, st);
  if (e != hipSuccess) {
    set_error("vrm_paged_decode_tq: merge kernel launch failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  clear_error();
  return VRM_OK;
}

int kind_of(int kv_dtype) {
  switch (kv_dtype) {
    case VRM_KV_F32: return K_F32;
    case VRM_KV_F16: return K_F16;
    case VRM_KV_BF16: return K_BF16;
    case VRM_KV_I8:
    case VRM_KV_I8_INLINE: return K_I8;
    case VRM_KV_FP8E4M3:
    case VRM_KV_FP8E4M3_INLINE: return K_FP8;
    default: return -1;
  }
}

// Pool geometry of a decode call (kv_dtype selects the plain or inline layout).
PoolGeom geom_of(int kv_dtype, int kind, int KH, int PS, int D, int P, int L) {
  const long long row = kind == K_F32 ? 4LL * D : (kind == K_F16 || kind == K_BF16) ? 2LL * D : kind == K_Q4 ? D / 2 : D;
  return pool_geom(kv_dtype, KH, PS, D, row, P, L);
}


int decode_entry(const float* query, const void* kv_pool, const float* kv_scales, const int32_t* page_table,
                 const int32_t* context_lens, float* out, void* workspace, size_t workspace_bytes, int B, int H,
                 int KH, int D, int PS, int L, int P, int max_pp, int layer_idx, float scale, int kv_dtype,
                 vrm_stream_t stream, int passes, float* lse = nullptr) {
  int rc = check_common(query, kv_pool, page_table, context_lens, out, B, H, KH, D, PS, L, P, max_pp, layer_idx,
                        scale);
  if (rc) return rc;
  const int kind = kind_of(kv_dtype);
  if (kind < 0) {
    set_error("vrm_paged_decode: unknown kv_dtype %d", kv_dtype);
    return VRM_ERR_ARG;
  }
  if ((kind == K_I8 || kind == K_FP8) && !kv_scales) {
    set_error("vrm_paged_decode: quantized pool needs kv_scales");
    return VRM_ERR_ARG;
  }
  if ((kind != K_I8 && kind != K_FP8) && kv_scales) {
    set_error("vrm_paged_decode: kv_scales given for a float pool");
    return VRM_ERR_ARG;
  }
  rc = check_pool_scales(kv_dtype, kv_pool, kv_scales, KH, PS, D, L, P, "vrm_paged_decode");
  if (rc) return rc;
  DecodeArgs a{};
  a.query = query;
  a.pool = static_cast<const uint8_t*>(kv_pool);
  a.scales = kv_scales;
  a.page_table = page_table;
  a.ctx_lens = context_lens;
  a.H = H;
  a.KH = KH;
  a.L = L;
  a.P = P;
  a.max_pp = max_pp;
  a.layer = layer_idx;
  a.lse = lse;
  a.g = geom_of(kv_dtype, kind, KH, PS, D, P, L);
  rc = check_kind_shape(kind, D, PS, "vrm_paged_decode");
  if (rc) return rc;
  return run_decode(a, kind, out, workspace, workspace_bytes, B, D, PS, scale, reinterpret_cast<hipStream_t>(stream),
                    passes);
}

constexpr float kQjlCoef = (float)(1.2533141373155003 / 64.0);  // sqrt(pi / 2) / qjl_dim

int tq_entry(const float* query, const uint8_t* tq_pool, const int32_t* page_table, const int32_t* context_lens,
             float* out, void* workspace, size_t workspace_bytes, int B, int H, int KH, int D, int PS, int L, int P,
             int max_pp, int layer_idx, float scale, int bits, int qjl_dim, const float* signs, const float* jl,
             const float* angle_lut, float* lse, float qjl_coef, vrm_stream_t stream) {
  int rc = check_common(query, tq_pool, page_table, context_lens, out, B, H, KH, D, PS, L, P, max_pp, layer_idx,
                        scale);
  if (rc) return rc;
  const bool tuned = tq::tuned_layout(D, bits, qjl_dim, PS);
  if (!tuned && !tq::generic_ok(D, bits, qjl_dim, PS)) {
    set_error("vrm_paged_decode_tq: TurboQuant pages take head_dim 33 .. 256, 1 .. 8 bits per angle, qjl_dim "
              "1 .. 256 and a positive page size (got %d, %d, %d, %d)", D, bits, qjl_dim, PS);
    return VRM_ERR_UNSUPPORTED;
  }
  const tq::GenLayout gl = tq::gen_layout(D, bits, qjl_dim, PS);
  if (!tuned && tq_generic_lds_bytes(gl) > 64 * 1024) {
    set_error("vrm_paged_decode_tq: setting needs %zu bytes of LDS", tq_generic_lds_bytes(gl));
    return VRM_ERR_UNSUPPORTED;
  }
  if (!signs || !jl || !angle_lut) {
    set_error("vrm_paged_decode_tq: null compressor buffer");
    return VRM_ERR_ARG;
  }
  DecodeArgs a{};
  a.query = query;
  a.pool = tq_pool;
  a.page_table = page_table;
  a.ctx_lens = context_lens;
  a.H = H;
  a.KH = KH;
  a.L = L;
  a.P = P;
  a.max_pp = max_pp;
  a.layer = layer_idx;
  a.lse = lse;
  // the QJL coefficient sqrt(pi / 2) / qjl_dim, or 0 for scores without the term
  TqDecodeArgs tq{signs, jl, angle_lut, qjl_coef != 0.f ? (float)(1.2533141373155003 / qjl_dim) : 0.f};
  return run_tq_decode(a, tq, bits, tuned ? nullptr : &gl, out, workspace, workspace_bytes, B, D, scale,
                       reinterpret_cast<hipStream_t>(stream));
}

}  // namespace
}  // namespace dec
}  // namespace vrm

using namespace vrm;
using namespace vrm::dec;

extern "C" int vrm_paged_decode_num_splits(int B, int H, int KH, int max_pp, int page_size) {
  (void)page_size;
  if (B <= 0 || H <= 0 || KH <= 0 || max_pp <= 0 || H % KH) return 0;
  // partition slots per sequence: B * nsplit >= the work-item capacity
  return (int)((items_capacity(B, KH) + B - 1) / B);
}

extern "C" size_t vrm_paged_decode_workspace_bytes(int B, int H, int D, int nsplit) {
  if (B <= 0 || H <= 0 || D <= 0 || nsplit <= 0) return 0;
  return header_bytes(B) + (size_t)B * H * nsplit * (D + 2) * sizeof(float);
}

extern "C" int vrm_paged_decode(const float* query, const void* kv_pool, const float* kv_scales,
                                const int32_t* page_table, const int32_t* context_lens, float* out, void* workspace,
                                size_t workspace_bytes, int B, int H, int KH, int D, int PS, int L, int P, int max_pp,
                                int layer_idx, float scale, int kv_dtype, vrm_stream_t stream) {
  return decode_entry(query, kv_pool, kv_scales, page_table, context_lens, out, workspace, workspace_bytes, B, H, KH,
                      D, PS, L, P, max_pp, layer_idx, scale, kv_dtype, stream, kBoth);
}

// ---------------------------------------------------------------------------
// Decode without a caller workspace: the split-K partials live in a fixed
// device array of this file, one copy per GPU, which the library looks up
// once per device (hipGetSymbolAddress, with that device current) and then
// addresses only through the returned pointer.  Nothing is allocated per
// call.  Every call on one GPU uses that GPU's array and leaves it holding its
// partials; nothing in it needs clearing (the partition pass writes the
// header and every partial the merge reads), and calls that overlap on one
// GPU race on it.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = VRM_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace vrm {
namespace dec {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// Device address of `scratch` on the device of `st`.
int scratch_of(hipStream_t st, void** ptr) {
  int dev = 0, cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e == hipSuccess) e = hipStreamGetDevice(st, &dev);
  if (e != hipSuccess) {
    set_error("vrm_paged_decode_noalloc: cannot identify the stream's device: %s", hipGetErrorString(e));
    return (int)e;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("vrm_paged_decode_noalloc: device %d outside [0, %d)", dev, kMaxDevices);
    return VRM_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    if (dev != cur) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess) e = e2;
    }
    if (e != hipSuccess || !p) {
      set_error("vrm_paged_decode_noalloc: hipGetSymbolAddress of the scratch array failed: %s",
                hipGetErrorString(e));
      return e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
    }
    g_scratch[dev] = p;
  }
  *ptr = g_scratch[dev];
  return VRM_OK;
}

}  // namespace
}  // namespace dec
}  // namespace vrm

extern "C" int vrm_paged_decode_noalloc(const float* query, const void* kv_pool, const float* kv_scales,
                                        const int32_t* page_table, const int32_t* context_lens, float* out, int B,
                                        int H, int KH, int D, int PS, int L, int P, int max_pp, int layer_idx,
                                        float scale, int kv_dtype, vrm_stream_t stream) {
  int rc = check_common(query, kv_pool, page_table, context_lens, out, B, H, KH, D, PS, L, P, max_pp, layer_idx,
                        scale);
  if (rc) return rc;
  const size_t need = header_bytes(B) + (size_t)items_capacity(B, KH) * H * (D + 2) * sizeof(float);
  if (need > kNoAllocScratchBytes) {
    set_error("vrm_paged_decode_noalloc: B=%d H=%d KH=%d D=%d needs %zu bytes of split-K scratch, above the "
              "fixed %zu-byte array; use vrm_paged_decode with a workspace",
              B, H, KH, D, need, kNoAllocScratchBytes);
    return VRM_ERR_WORKSPACE;
  }
  void* ws = nullptr;
  rc = scratch_of(reinterpret_cast<hipStream_t>(stream), &ws);
  if (rc) return rc;
  return decode_entry(query, kv_pool, kv_scales, page_table, context_lens, out, ws, kNoAllocScratchBytes, B, H, KH,
                      D, PS, L, P, max_pp, layer_idx, scale, kv_dtype, stream, kBoth);
}

namespace {
int balanced_entry(const float* query, const void* kv_pool, const float* kv_scales, const int32_t* page_table,
                   const int32_t* context_lens, float* out, float* lse, int B, int H, int KH, int D, int PS, int L,
                   int P, int max_pp, int layer_idx, float scale, int kv_dtype, vrm_stream_t stream, bool loads_only,
                   const char* who) {
  int rc = check_common(query, kv_pool, page_table, context_lens, out, B, H, KH, D, PS, L, P, max_pp, layer_idx,
                        scale);
  if (rc) return rc;
  const int kind = kind_of(kv_dtype);
  if (kind != K_I8 && kind != K_FP8) {
    set_error("%s: kv_dtype %d unsupported (int8 and fp8 pools)", who, kv_dtype);
    return kind < 0 ? VRM_ERR_ARG : VRM_ERR_UNSUPPORTED;
  }
  if (!kv_scales) {
    set_error("%s: quantized pool needs kv_scales", who);
    return VRM_ERR_ARG;
  }
  rc = check_pool_scales(kv_dtype, kv_pool, kv_scales, KH, PS, D, L, P, who);
  if (rc) return rc;
  if ((D != 64 && D != 80 && D != 96 && D != 112 && D != 128) || PS != kPS) {
    // at D = 256 two page pairs per wave do not fit in registers
    set_error("%s: head_dim %d / page_size %d unsupported (64, 80, 96, 112 or 128, page 16)", who, D, PS);
    return VRM_ERR_UNSUPPORTED;
  }
  const int G = pick_group_tile(H / KH, 16);
  if (balanced_lds_bytes(max_pp, kUnitsPerWg, G, D) > kMaxBalancedLds) {
    set_error("%s: a page table of width %d does not fit the workgroup's LDS copy; use vrm_paged_decode", who,
              max_pp);
    return VRM_ERR_UNSUPPORTED;
  }
  DecodeArgs a{};
  a.query = query;
  a.pool = static_cast<const uint8_t*>(kv_pool);
  a.scales = kv_scales;
  a.page_table = page_table;
  a.ctx_lens = context_lens;
  a.B = B;
  a.H = H;
  a.KH = KH;
  a.L = L;
  a.P = P;
  a.max_pp = max_pp;
  a.layer = layer_idx;
  a.lse = lse;
  a.out = out;
  a.qscale = scale * kLog2e;
  a.g = geom_of(kv_dtype, kind, KH, PS, D, P, L);
  const hipError_t e = launch_stream_balanced(a, kind, B, D, G, reinterpret_cast<hipStream_t>(stream), loads_only);
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", who, hipGetErrorString(e));
    return (int)e;
  }
  clear_error();
  return VRM_OK;
}
}  // namespace

extern "C" int vrm_paged_decode_balanced(const float* query, const void* kv_pool, const float* kv_scales,
                                         const int32_t* page_table, const int32_t* context_lens, float* out,
                                         float* lse, int B, int H, int KH, int D, int PS, int L, int P, int max_pp,
                                         int layer_idx, float scale, int kv_dtype, vrm_stream_t stream) {
  return balanced_entry(query, kv_pool, kv_scales, page_table, context_lens, out, lse, B, H, KH, D, PS, L, P, max_pp,
                        layer_idx, scale, kv_dtype, stream, false, "vrm_paged_decode_balanced");
}

extern "C" int vrm_paged_decode_balanced_loads(const float* query, const void* kv_pool, const float* kv_scales,
                                               const int32_t* page_table, const int32_t* context_lens, float* out,
                                               int B, int H, int KH, int D, int PS, int L, int P, int max_pp,
                                               int layer_idx, float scale, int kv_dtype, vrm_stream_t stream) {
  return balanced_entry(query, kv_pool, kv_scales, page_table, context_lens, out, nullptr, B, H, KH, D, PS, L, P,
                        max_pp, layer_idx, scale, kv_dtype, stream, true, "vrm_paged_decode_balanced_loads");
}

extern "C" int vrm_paged_decode_partitions(const float* query, const void* kv_pool, const float* kv_scales,
                                           const int32_t* page_table, const int32_t* context_lens, void* workspace,
                                           size_t workspace_bytes, int B, int H, int KH, int D, int PS, int L, int P,
                                           int max_pp, int layer_idx, float scale, int kv_dtype,
                                           vrm_stream_t stream) {
  // `out` is not touched by the partition pass; pass a non-null placeholder for the checks.
  return decode_entry(query, kv_pool, kv_scales, page_table, context_lens, reinterpret_cast<float*>(workspace),
                      workspace, workspace_bytes, B, H, KH, D, PS, L, P, max_pp, layer_idx, scale, kv_dtype, stream,
                      kPartitionsOnly);
}

extern "C" int vrm_paged_decode_merge(const int32_t* context_lens, float* out, const void* workspace,
                                      size_t workspace_bytes, int B, int H, int KH, int D, int PS, int max_pp,
                                      vrm_stream_t stream) {
  if (!context_lens || !out || !workspace) {
    set_error("vrm_paged_decode_merge: null pointer argument");
    return VRM_ERR_ARG;
  }
  if (B <= 0 || H <= 0 || KH <= 0 || H % KH || max_pp <= 0) {
    set_error("vrm_paged_decode_merge: bad sizes");
    return VRM_ERR_ARG;
  }
  if (PS <= 0 || D <= 0 || D > kMaxHeadDim) {
    set_error("vrm_paged_decode_merge: unsupported page_size %d / head_dim %d", PS, D);
    return VRM_ERR_UNSUPPORTED;
  }
  DecodeArgs a{};
  a.ctx_lens = context_lens;
  a.H = H;
  a.KH = KH;
  a.max_pp = max_pp;
  a.L = 1;
  a.P = 1;
  // The merge reads the partition geometry the partition pass left in the
  // workspace header; the dtype below only selects the workspace layout,
  // which is the same for every pool.
  return run_decode(a, K_I8, out, const_cast<void*>(workspace), workspace_bytes, B, D, PS, 1.f,
                    reinterpret_cast<hipStream_t>(stream), kMergeOnly);
}

extern "C" int vrm_paged_decode_q4(const float* query, const uint8_t* kv_pool_q4, const uint16_t* kv_scales,
                                   const uint16_t* kv_zeros, const int32_t* page_table, const int32_t* context_lens,
                                   float* out, void* workspace, size_t workspace_bytes, int B, int H, int KH, int D,
                                   int PS, int L, int P, int max_pp, int layer_idx, float scale,
                                   vrm_stream_t stream) {
  int rc = check_common(query, kv_pool_q4, page_table, context_lens, out, B, H, KH, D, PS, L, P, max_pp, layer_idx,
                        scale);
  if (rc) return rc;
  if (!kv_scales || !kv_zeros) {
    set_error("vrm_paged_decode_q4: null scales/zeros");
    return VRM_ERR_ARG;
  }
  if (D % 32) {
    set_error("vrm_paged_decode_q4: head_dim %d is not a multiple of the group size 32", D);
    return VRM_ERR_UNSUPPORTED;
  }
  DecodeArgs a{};
  a.query = query;
  a.pool = kv_pool_q4;
  a.q4_scale = kv_scales;
  a.q4_zero = kv_zeros;
  a.page_table = page_table;
  a.ctx_lens = context_lens;
  a.H = H;
  a.KH = KH;
  a.L = L;
  a.P = P;
  a.max_pp = max_pp;
  a.layer = layer_idx;
  a.g = geom_of(VRM_KV_I8, K_Q4, KH, PS, D, P, L);  // plain layout of D / 2 bytes per row
  return run_decode(a, K_Q4, out, workspace, workspace_bytes, B, D, PS, scale, reinterpret_cast<hipStream_t>(stream),
                    kBoth);
}

extern "C" int vrm_paged_decode_tq(const float* query, const uint8_t* tq_pool, const int32_t* page_table,
                                   const int32_t* context_lens, float* out, void* workspace, size_t workspace_bytes,
                                   int B, int H, int KH, int D, int PS, int L, int P, int max_pp, int layer_idx,
                                   float scale, int bits, int qjl_dim, const float* signs, const float* jl,
                                   const float* angle_lut, vrm_stream_t stream) {
  return tq_entry(query, tq_pool, page_table, context_lens, out, workspace, workspace_bytes, B, H, KH, D, PS, L, P,
                  max_pp, layer_idx, scale, bits, qjl_dim, signs, jl, angle_lut, nullptr, kQjlCoef, stream);
}

extern "C" int vrm_paged_decode_tq_lse(const float* query, const uint8_t* tq_pool, const int32_t* page_table,
                                       const int32_t* context_lens, float* out, float* lse, void* workspace,
                                       size_t workspace_bytes, int B, int H, int KH, int D, int PS, int L, int P,
                                       int max_pp, int layer_idx, float scale, int bits, int qjl_dim,
                                       const float* signs, const float* jl, const float* angle_lut, int with_qjl,
                                       vrm_stream_t stream) {
  if (!lse) {
    set_error("vrm_paged_decode_tq_lse: null lse");
    return VRM_ERR_ARG;
  }
  // without the QJL term the scores are q_rot . k_polar = q . decompress(k)
  return tq_entry(query, tq_pool, page_table, context_lens, out, workspace, workspace_bytes, B, H, KH, D, PS, L, P,
                  max_pp, layer_idx, scale, bits, qjl_dim, signs, jl, angle_lut, lse, with_qjl ? kQjlCoef : 0.f,
                  stream);
}

extern "C" int vrm_paged_decode_lse(const float* query, const void* kv_pool, const float* kv_scales,
                                    const int32_t* page_table, const int32_t* context_lens, float* out, float* lse,
                                    void* workspace, size_t workspace_bytes, int B, int H, int KH, int D, int PS,
                                    int L, int P, int max_pp, int layer_idx, float scale, int kv_dtype,
                                    vrm_stream_t stream) {
  if (!lse) {
    set_error("vrm_paged_decode_lse: null lse");
    return VRM_ERR_ARG;
  }
  return decode_entry(query, kv_pool, kv_scales, page_table, context_lens, out, workspace, workspace_bytes, B, H, KH,
                      D, PS, L, P, max_pp, layer_idx, scale, kv_dtype, stream, kBoth, lse);
}

extern "C" int vrm_attn_combine(const float* out1, const float* lse1, const float* out2, const float* lse2,
                                long long rows, int D, float* out, float* lse_out, vrm_stream_t stream) {
  const char* who = "vrm_attn_combine";
  if (rows < 0 || D <= 0 || rows * D / 256 > 0x7fffffffLL) {
    set_error("%s: bad sizes (rows=%lld D=%d)", who, rows, D);
    return VRM_ERR_ARG;
  }
  if (rows == 0) {
    clear_error();
    return VRM_OK;
  }
  if (!out1 || !lse1 || !out2 || !lse2 || !out) {
    set_error("%s: null pointer argument", who);
    return VRM_ERR_ARG;
  }
  const long long n = rows * D;
  hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), out1, lse1, out2, lse2, rows, D, out, lse_out);
  return launch_status(who);
}
