// Types shared by the decode kernels of libvrm_paged.so.
#pragma once
#include "vrm_common.h"
#include "vrm_tq_layout.h"

namespace vrm {
namespace dec {

constexpr int kPS = 16;               // tokens per page (the reference's default; the tuned kernels' page)
constexpr int kMaxHeadDim = 256;      // the reference kernel's limit (csrc/paged_attention_kernel.cu:460)
constexpr float kLog2e = 1.4426950408889634f;

enum KvKind { K_F32 = 0, K_F16 = 1, K_BF16 = 2, K_I8 = 3, K_FP8 = 4, K_Q4 = 5 };

template <int KIND> struct Kv;
template <> struct Kv<K_F32> { static constexpr int kElems = 4; };   // elements per 16 B
template <> struct Kv<K_F16> { static constexpr int kElems = 8; };
template <> struct Kv<K_BF16> { static constexpr int kElems = 8; };
template <> struct Kv<K_I8> { static constexpr int kElems = 16; };
template <> struct Kv<K_FP8> { static constexpr int kElems = 16; };
template <> struct Kv<K_Q4> { static constexpr int kElems = 32; };


struct DecodeArgs {
  const float* query;
  const uint8_t* pool;
  const float* scales;        // int8 / fp8 scale arrays
  const uint16_t* q4_scale;   // 4-bit pool group scales (fp16 bits)
  const uint16_t* q4_zero;    // 4-bit pool group zeros (fp16 bits)
  const int32_t* page_table;
  const int32_t* ctx_lens;
  int32_t* header;            // workspace header (see work items below)
  float* part_acc;            // [items][H][D]
  float* part_ml;             // [items][H][2]
  int B, H, KH, L, P, max_pp, layer;
  float qscale;               // scale * log2(e): scores live in the log2 domain
  int target;                 // work items the partition size aims for
  float* lse;                 // optional [B][H] natural-log sum of exp(scale * q.k), written by the merge
  float* out;                 // [B][H][D]: written directly by the balanced (one workgroup per sequence) mode
  int vshift;                 // stream kernels: pages hold 16 << vshift tokens (0: 16-token pages)
  PoolGeom g;                 // where the pool keeps each (page, layer, K/V, kv-head) slice and its scales
};

// ---------------------------------------------------------------------------
// Work items (length-aware split-K).
//
// All sequences' pages are cut into partitions of pps pages.  The host passes
// `target`, the work items the chip holds at once (resident wavefronts of the
// kernel / wavefronts per item).  On the device, from the batch's total page
// count S: pps = max(4, roundup4(ceil(S / target))), so one resident round of
// equal partitions covers the batch; when the shorter tail partitions this
// leaves (one per sequence whose page count pps does not divide) exceed an
// eighth of the round, pps is halved (from S / (2 target)) so that the
// remainders spread over more, smaller items.  Sequence b has
// nf_b = floor(pages_b / pps) full partitions and at most one tail.  Work
// items enumerate every full partition first (sequence-major; they all cost
// the same), then the tails, so the dispatcher starts the equal-sized work
// before the small remainders.  Since S / pps <= 2 target, a batch has at
// most B + 2 target items, a bound the host knows without reading the
// context lengths.
//
// Workspace header (int32), written by the partition pass for the merge:
//   [0] pps   [1] number of items   [2] number of full items
//   [3] the sequence with the most partitions (the merge starts it first)
//   [4] 1 when the partition pass wrote the sequences of one item to out
//       itself (the merge pass skips them), else 0
//   [kHeaderInts + b],         b = 0 .. B : first full item of sequence b
//                                           (entry B = number of full items)
//   [kHeaderInts + B + 1 + b], b < B      : tail item of sequence b, or -1
// ---------------------------------------------------------------------------
constexpr int kMaxTargetWaves = 4096;  // cap on the resident wavefronts a target counts
constexpr int kHeaderInts = 16;

inline size_t header_bytes(int B) { return ((size_t)(kHeaderInts + 2 * B + 1) * 4 + 255) / 256 * 256; }

struct WorkItem {
  int b;        // sequence
  int p_begin;  // first logical page of the partition
  int n_pages;  // pages in the partition (>= 1)
  int ctx;      // context length of the sequence
  int items;    // work items of the whole batch (find_piece: pieces of the row)
  int slot;     // find_piece: the workspace row of the piece's partials
};

// Pages of a sequence of ctx tokens (pages of ps tokens), capped by the table width.
__device__ __forceinline__ int seq_pages(int ctx, int max_pp, int ps = kPS) {
  return ctx > 0 ? min((ctx + ps - 1) / ps, max_pp) : 0;
}

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __builtin_amdgcn_ds_bpermute((__lane_id() ^ m) << 2, v);
  return v;
}

__device__ __forceinline__ int wave_max_int(int v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v = max(v, __builtin_amdgcn_ds_bpermute((__lane_id() ^ m) << 2, v));
  return v;
}

__device__ __forceinline__ int wave_inclusive_scan(int v) {
  const int lane = __lane_id();
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int t = __builtin_amdgcn_ds_bpermute(max(lane - d, 0) << 2, v);
    if (lane >= d) v += t;
  }
  return v;
}

// Finds work item `item` of the batch.  Every wave of a launch derives the
// same geometry from the context lengths; when `writer` is set the wave also
// stores it in the header (with `direct` as header[4]).  Returns false when
// `item` lies past the last item.
__device__ __forceinline__ bool find_item(const int32_t* __restrict__ ctx_lens, int B, int max_pp, int target,
                                          int item, bool writer, int32_t* __restrict__ header, WorkItem& w,
                                          int ps = kPS, bool direct = false) {
  const int lane = __lane_id();
  int S = 0;
  for (int c = 0; c < B; c += 64) {
    const int b = c + lane;
    S += b < B ? seq_pages(ctx_lens[b], max_pp, ps) : 0;
  }
  S = wave_sum_int(S);
  auto roundup4 = [](int v) { return max(4, (v + 3) / 4 * 4); };
  // both candidate partition sizes in one pass (three independent sums, so
  // that their lane exchanges overlap)
  const int pps1 = roundup4((S + target - 1) / target);
  const int pps2 = roundup4((S + 2 * target - 1) / (2 * target));
  int tails = 0, full1 = 0, full2 = 0;
  for (int c = 0; c < B; c += 64) {
    const int b = c + lane;
    const int pages = b < B ? seq_pages(ctx_lens[b], max_pp, ps) : 0;
    tails += (pages % pps1) != 0 ? 1 : 0;
    full1 += pages / pps1;
    full2 += pages / pps2;
  }
  tails = wave_sum_int(tails);
  full1 = wave_sum_int(full1);
  full2 = wave_sum_int(full2);
  const bool halve = tails * 8 > target;
  const int pps = halve ? pps2 : pps1;
  const int n_full = halve ? full2 : full1;
  bool found = false;
  int carry_f = 0, carry_t = n_full;
  for (int c = 0; c < B; c += 64) {
    const int b = c + lane;
    const int ctx = b < B ? ctx_lens[b] : 0;
    const int pages = seq_pages(ctx, max_pp, ps);
    const int nf = pages / pps;
    const int nt = pages - nf * pps > 0 ? 1 : 0;
    const int incl_f = wave_inclusive_scan(nf) + carry_f;
    const int incl_t = wave_inclusive_scan(nt) + carry_t;
    const int excl_f = incl_f - nf;
    const int excl_t = incl_t - nt;
    if (writer && b < B) {
      header[kHeaderInts + b] = excl_f;
      header[kHeaderInts + B + 1 + b] = nt ? excl_t : -1;
    }
    if (!found) {
      const bool in_full = item >= excl_f && item < incl_f;
      const bool in_tail = nt && item == excl_t;
      const unsigned long long hit = __ballot(in_full || in_tail);
      if (hit) {
        const int l = __builtin_ffsll(hit) - 1;
        const bool full = __builtin_amdgcn_readlane(in_full ? 1 : 0, l);
        const int pg = __builtin_amdgcn_readlane(pages, l);
        w.b = c + l;
        w.p_begin = full ? (item - __builtin_amdgcn_readlane(excl_f, l)) * pps : (pg / pps) * pps;
        w.n_pages = full ? pps : pg - w.p_begin;
        w.ctx = __builtin_amdgcn_readlane(ctx, l);
        found = true;
      }
    }
    carry_f = __builtin_amdgcn_readlane(incl_f, 63);
    carry_t = __builtin_amdgcn_readlane(incl_t, 63);
  }
  w.items = carry_t;
  if (writer) {
    // the sequence with the most partitions (first of equals), in a pass of
    // its own so that the other waves' path stays as it is
    int most = -1, most_b = 0;
    for (int c = 0; c < B; c += 64) {
      const int b = c + lane;
      const int pages = b < B ? seq_pages(ctx_lens[b], max_pp, ps) : 0;
      const int cnt = b < B ? pages / pps + (pages % pps != 0 ? 1 : 0) : -1;
      const int cmax = wave_max_int(cnt);
      if (cmax > most) {
        most = cmax;
        most_b = c + __builtin_ffsll(__ballot(cnt == cmax)) - 1;
      }
    }
    if (lane == 0) {
      header[0] = pps;
      header[1] = carry_t;
      header[2] = n_full;
      header[3] = most_b;
      header[4] = direct ? 1 : 0;
      header[kHeaderInts + B] = n_full;
    }
  }
  return found;
}

// Pieces (the shared-items pass).  The batch's pages laid end to end,
// sequence after sequence (S in all), are cut into `rows` runs of C =
// max(kMinPiecePages, roundup4(ceil(S / rows))) pages: row r holds pages
// [r C, (r + 1) C), so that every row carries the same work whatever the
// lengths.  A row's pieces are its runs within each sequence it meets, in
// sequence order.  Sequence b (P_b pages before it, pages_b its own) meets
// rows P_b / C .. (P_b + pages_b - 1) / C, k_b of them; its pieces' partials
// take workspace rows base_b .. base_b + k_b - 1 (base: the exclusive sum of
// k), the piece of row r taking base_b + r - P_b / C.  The header takes the
// work-item form with every piece a full item and no tails, so the merge
// pass reads it unchanged: [kHeaderInts + b] = base_b, [kHeaderInts + B] =
// the number of pieces, tails -1, [0] = C.
constexpr int kMinPiecePages = 16;

__device__ __forceinline__ int lane_rank(unsigned long long m) {  // set bits of m below this lane
  return __builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0));
}

// Finds piece j of row `row` (of `rows`); every wave of the launch derives
// the same geometry, and the `writer` wave stores it in the header (with
// `direct` as header[4]) whether or not the piece exists.  Returns false when
// the row has no piece j; w.items is the row's piece count either way.
__device__ __forceinline__ bool find_piece(const int32_t* __restrict__ ctx_lens, int B, int max_pp, int rows, int row,
                                           int j, bool writer, bool direct, int32_t* __restrict__ header,
                                           WorkItem& w) {
  const int lane = __lane_id();
  int S = 0;
  for (int c = 0; c < B; c += 64) {
    const int b = c + lane;
    S += b < B ? seq_pages(ctx_lens[b], max_pp) : 0;
  }
  S = wave_sum_int(S);
  const int C = max(kMinPiecePages, ((S + rows - 1) / rows + 3) / 4 * 4);
  const long long lo = (long long)row * C;
  const long long hi = min((long long)S, lo + C);
  int carry_p = 0, carry_k = 0, seen = 0, most = -1, most_b = 0;
  bool found = false;
  for (int c = 0; c < B; c += 64) {
    const int b = c + lane;
    const int ctx = b < B ? ctx_lens[b] : 0;
    const int pages = b < B ? seq_pages(ctx, max_pp) : 0;
    const int incl_p = wave_inclusive_scan(pages) + carry_p;
    const int P = incl_p - pages;
    const int k = pages > 0 ? (P + pages - 1) / C - P / C + 1 : 0;
    const int incl_k = wave_inclusive_scan(k) + carry_k;
    const int base = incl_k - k;
    if (writer && b < B) {
      header[kHeaderInts + b] = base;
      header[kHeaderInts + B + 1 + b] = -1;
    }
    const bool meets = pages > 0 && P < hi && P + pages > lo;
    const unsigned long long m = __ballot(meets);
    const int cnt = __popcll(m);
    if (!found && j >= seen && j < seen + cnt) {
      const unsigned long long hit = __ballot(meets && lane_rank(m) == j - seen);
      const int l = __builtin_ffsll(hit) - 1;
      const int pl = __builtin_amdgcn_readlane(P, l);
      const int nl = __builtin_amdgcn_readlane(pages, l);
      const int first = max((int)lo, pl);
      const int end = min((int)hi, pl + nl);
      w.b = c + l;
      w.p_begin = first - pl;
      w.n_pages = end - first;
      w.ctx = __builtin_amdgcn_readlane(ctx, l);
      w.slot = __builtin_amdgcn_readlane(base, l) + row - pl / C;
      found = true;
    }
    seen += cnt;
    if (writer) {
      const int kmax = wave_max_int(b < B ? k : -1);
      if (kmax > most) {
        most = kmax;
        most_b = c + __builtin_ffsll(__ballot(b < B && k == kmax)) - 1;
      }
    }
    carry_p = __builtin_amdgcn_readlane(incl_p, 63);
    carry_k = __builtin_amdgcn_readlane(incl_k, 63);
  }
  w.items = seen;
  if (writer && lane == 0) {
    header[0] = C;
    header[1] = carry_k;
    header[2] = carry_k;
    header[3] = most_b;
    header[4] = direct ? 1 : 0;
    header[kHeaderInts + B] = carry_k;
  }
  return found;
}

// Work items one resident round of `kernel` holds (see work items above).
int items_target(const void* kernel, int waves_per_block, size_t lds_bytes, int units);

// Generic VALU partition pass for every pool kind at any head_dim <= 256 and
// any page size (vrm_decode_generic.hip): the shapes the tuned kernels do
// not compile for.  D and PS are runtime values; int8 / fp8 pools need
// D % 16 == 0 and PS % 4 == 0 (their tiled V), Q4 pools D % 32 == 0.
hipError_t launch_generic(const DecodeArgs& a, int kind, int B, int D, int PS, hipStream_t st);

// Single-pass matrix-core (MFMA) split pass; kind is K_I8, K_FP8, K_BF16 or
// K_F16, D the head dimension, G the query heads per wavefront (<= 16).
hipError_t launch_stream_mfma(const DecodeArgs& a, int kind, int B, int D, int G, hipStream_t st);

// Balanced mode geometry: workgroups of kUnitsPerWg units x (1, 2, 4 or 6)
// wavefronts per unit.  LDS: the sequence's page ids [max_pp], the units'
// page-pair counters [kMaxUnitsPerWg], the page-id buckets' counters
// [kIdBuckets], then (16-byte aligned) the merge area, [W][G][D]
// accumulators and [W][G][2] (m, l); at most kMaxBalancedLds.
constexpr int kMaxBalancedWaves = 12;
constexpr int kUnitsPerWg = 2;     // the balanced mode; the shared-items pass takes 2 or 4
constexpr int kMaxUnitsPerWg = 4;  // page-pair counters the LDS layout leaves room for
constexpr int kIdBucketBits = 6;   // a work item's pages are read in 2^6 buckets of ascending page id
constexpr int kIdBuckets = 1 << kIdBucketBits;
constexpr size_t kMaxBalancedLds = 64 * 1024;
// LDS one workgroup of the shared-items pass may take on the current device
// (its 12-wavefront workgroups hold a CU each, so beyond 64 KB costs no
// occupancy): the device's per-workgroup limit, at most 160 KB.
size_t shared_items_max_lds();
__host__ __device__ inline size_t balanced_merge_offset(int max_pp) {
  return ((size_t)max_pp * 4 + kMaxUnitsPerWg * 4 + kIdBuckets * 4 + 15) / 16 * 16;
}
inline size_t balanced_lds_bytes(int max_pp, int W, int G, int D) {
  return balanced_merge_offset(max_pp) + (size_t)W * G * (D + 2) * sizeof(float);
}

// Balanced-batch decode: one workgroup per (sequence, kUnitsPerWg units)
// whose wavefronts take the sequence's page pairs from LDS counters and merge
// their partials in LDS, writing a.out (and a.lse) directly: no work items,
// no workspace, no merge launch.  Correct for any context lengths; its time follows the
// longest sequence, so it suits batches of about equal lengths.  kind is
// K_I8 or K_FP8, D a multiple of 16 from 64 to 128.
// loads_only: the measuring build that issues the same loads and computes
// nothing (a checksum of the words goes to out).
hipError_t launch_stream_balanced(const DecodeArgs& a, int kind, int B, int D, int G, hipStream_t st,
                                  bool loads_only = false);

// The shared-items partition pass: balanced workgroups of 12 wavefronts (2
// units x 6, or 4 x 3 when the batch has more sequences than a resident round
// has rows of 2-unit workgroups) take the pieces of their row (find_piece),
// sharing each piece's pages through LDS counters, and leave its merged
// partials in the workspace (the merge pass follows) or, for a one-piece
// sequence in a call with out, the output.  kind K_I8 or K_FP8, D a multiple
// of 16 from 64 to 128, 16-token pages; hipErrorInvalidValue when the page
// table is too wide for the LDS copy.
hipError_t launch_stream_shared_items(const DecodeArgs& a, int kind, int B, int D, int G, hipStream_t st);

// Paged decode over TurboQuant pages (vrm_decode_tq.hip).
struct TqDecodeArgs {
  const float* signs;  // [padded_dim] Hadamard signs
  const float* jl;     // [qjl][padded_dim] JL matrix
  const float* lut;    // [cos level 0, sin level 0, cos levels >= 1, sin levels >= 1][2^bits]
  float qjl_coef;      // sqrt(pi / 2) / qjl, or 0 for scores without the QJL term
};
// hd: the head_dim (33 .. 64 or 65 .. 128: the tuned layouts' padded dims 64 and 128).
hipError_t launch_tq_decode(const DecodeArgs& a, const TqDecodeArgs& tq, int bits, int B, int hd, hipStream_t st);

// Paged decode over TurboQuant pages in the generic layout (vrm_decode_tq_generic.hip):
// every compressor setting and page size the tuned kernel above does not
// serve.  tq.lut holds 4 << bits floats, tq.signs padded_dim, tq.jl
// [qjl][padded_dim]; D is the head_dim (<= padded_dim).
hipError_t launch_tq_generic(const DecodeArgs& a, const TqDecodeArgs& tq, const tq::GenLayout& gl, int B, int D,
                             hipStream_t st);
size_t tq_generic_lds_bytes(const tq::GenLayout& gl);

// Largest divisor of the GQA group size that is <= max_tile.
inline int pick_group_tile(int group, int max_tile) {
  for (int g = max_tile; g >= 1; --g)
    if (group % g == 0) return g;
  return 1;
}

}  // namespace dec
}  // namespace vrm
