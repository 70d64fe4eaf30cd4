// Tuned layout of a TurboQuant KV page of this library, for padded dim PD =
// 128 (head_dim 65 .. 128: 7 polar levels, 127 angles, 64 QJL signs) and PD =
// 64 (head_dim 33 .. 64: 6 levels, 63 angles, 32 QJL signs), the compressor's
// default qjl_dim PD / 2 and 16-token pages.
//
// The pool keeps the reference's addressing, tq_pool[P][L][2][KH][slice],
// one slice of slice_bytes(PD, bits) bytes per (page, layer, K/V, kv-head)
// with the 16 tokens of the page:
//   angles  [16][PD / 8 * bits]   bytes 0 ..       (token t at t * PD / 8 * bits)
//   signs   [16][PD / 16]         QJL sign bits (K only; bit j = residual . jl_j > 0)
//   radius  [16]                  fp16 final polar radius
//   norms   [16]                  fp16 residual norm (K only)
// V slices use the angles and radius fields only (same offsets).
//
// Angle record of one token: four quarters of Q = PD / 4 slots of `bits`
// bits.  Quarter g holds the Q - 1 angles of the subtree over dims
// Q g .. Q g + Q - 1 (levels 0 .. LQ, LQ = log2(PD) - 3: 4 at PD 128, 3 at PD
// 64) plus one spare slot that carries a top-level angle, so that a decode
// lane owning those dims reads one short run of bits.  For bits <= 3 a node's
// angle is followed by its two children's, so that the index of a two-level
// product table (node bin + NB * child-0 bin + NB^2 * child-1 bin, NB =
// 2^bits) is one contiguous 3 * bits-bit field; with N1 = PD / 16 level-1
// angles and N3 = N1 / 4 level-3 angles per quarter:
//   slots 3 j, 3 j + 1, 3 j + 2       (j < N1) level 1 angle N1 g + j, then
//                                     level 0 angles 2 N1 g + 2 j, 2 N1 g + 2 j + 1
//   slots 3 N1 + 3 j .. 3 N1 + 3 j + 2
//                                     (j < N3) level 3 angle N3 g + j, then
//                                     level 2 angles 2 N3 g + 2 j, 2 N3 g + 2 j + 1
//   slot 3 N1 + 3 N3 (PD 128 only)    level 4 angle g
// For bits == 4 the levels are in order (the decode reads siblings in pairs):
//   slots 2^m - 1 .. 2^(m + 1) - 2 hold the 2^m angles of level LQ - m of
//   the quarter, in order.
// For every bits, the spare slot Q - 1 holds, in quarter 0, the root angle
// (level LQ + 2), in quarters 1 and 2 the level LQ + 1 angles 0 and 1, and in
// quarter 3 zero.
// Slot s of quarter g occupies bits [(Q g + s) bits, (Q g + s + 1) bits) of
// the record, bit i of the record being bit i % 8 of its byte i / 8
// (little-endian).  The record has exactly the (PD - 1) * bits bits of the
// reference's packed angles, plus `bits` padding bits.  Angle levels and
// indices are those of the reference's level-major bins (core/kv_quantizer.py:
// 262-287): level l holds PD / 2 >> l angles and angle i of level l pairs
// elements 2 i, 2 i + 1 of level l - 1.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace vrm {
namespace tq {

constexpr int kTokens = 16;  // tokens per page of the tuned layout

__host__ __device__ constexpr int log2_pd(int pd) { return pd == 64 ? 6 : pd == 128 ? 7 : 8; }
__host__ __device__ constexpr int quarter_slots(int pd) { return pd / 4; }
__host__ __device__ constexpr int quarter_top(int pd) { return log2_pd(pd) - 3; }  // level of a quarter's root
__host__ __device__ constexpr int tuned_qjl(int pd) { return pd / 2; }
__host__ __device__ constexpr int angle_bytes(int pd, int bits) { return pd / 8 * bits; }  // per token
__host__ __device__ constexpr int sign_bytes(int pd) { return tuned_qjl(pd) / 8; }         // per token
__host__ __device__ constexpr int signs_offset(int pd, int bits) { return kTokens * angle_bytes(pd, bits); }
__host__ __device__ constexpr int radius_offset(int pd, int bits) {
  return signs_offset(pd, bits) + kTokens * sign_bytes(pd);
}
__host__ __device__ constexpr int norms_offset(int pd, int bits) { return radius_offset(pd, bits) + kTokens * 2; }
__host__ __device__ constexpr int slice_bytes(int pd, int bits) { return norms_offset(pd, bits) + kTokens * 2; }

// Offset of level l in the reference's level-major bin array: sum_{i<l} (pd / 2) >> i.
__host__ __device__ constexpr int level_offset(int pd, int l) { return pd - (pd >> l); }

// (quarter, slot) of angle i of level l.
__host__ __device__ inline void slot_of(int pd, int l, int i, int bits, int& quarter, int& slot) {
  const int lq = quarter_top(pd), spare = quarter_slots(pd) - 1;
  const int n1 = pd / 16, n3 = n1 / 4;
  if (l <= lq) {
    const int per = 1 << (lq - l);  // angles of level l per quarter
    quarter = i / per;
    const int a = i % per;  // angle within the quarter
    if (bits == 4) {
      slot = (per - 1) + a;
      return;
    }
    switch (l) {
      case 0: slot = 3 * (a >> 1) + 1 + (a & 1); break;
      case 1: slot = 3 * a; break;
      case 2: slot = 3 * n1 + 3 * (a >> 1) + 1 + (a & 1); break;
      case 3: slot = 3 * n1 + 3 * a; break;
      default: slot = 3 * n1 + 3 * n3; break;
    }
  } else if (l == lq + 1) {
    quarter = 1 + i;
    slot = spare;
  } else {
    quarter = 0;
    slot = spare;
  }
}

// Level-major bin index (reference order) of slot s of quarter g, or -1 for
// the unused spare of quarter 3.
__host__ __device__ inline int bin_index_of(int pd, int g, int s, int bits) {
  const int lq = quarter_top(pd), spare = quarter_slots(pd) - 1;
  const int n1 = pd / 16, n3 = n1 / 4;
  if (s == spare) return g == 0 ? level_offset(pd, lq + 2) : (g <= 2 ? level_offset(pd, lq + 1) + (g - 1) : -1);
  if (bits == 4) {  // slots 2^m - 1 .. 2^(m+1) - 2 hold the 2^m angles of level lq - m
    int m = 0;
    while ((2 << m) <= s + 1) ++m;
    return level_offset(pd, lq - m) + g * (1 << m) + (s + 1 - (1 << m));
  }
  if (s == 3 * n1 + 3 * n3) return level_offset(pd, 4) + g;  // padded dim 128: level 4
  if (s >= 3 * n1) {
    const int k = (s - 3 * n1) / 3, r = (s - 3 * n1) % 3;
    return r == 0 ? level_offset(pd, 3) + n3 * g + k : level_offset(pd, 2) + 2 * n3 * g + 2 * k + (r - 1);
  }
  const int j = s / 3, r = s % 3;
  return r == 0 ? level_offset(pd, 1) + n1 * g + j : level_offset(pd, 0) + 2 * n1 * g + 2 * j + (r - 1);
}

// ---------------------------------------------------------------------------
// Generic page layout: every other setting of the compressor (head_dim 1 ..
// 256, i.e. padded_dim 2, 4, ..., 256, 1 to 8 bits per angle, qjl_dim 1 ..
// 256) and any page size.  A slice holds the page's PS tokens as records of
// record_bytes(), in token order:
//   angle bits   [angle_dw dwords]   level-major bin b at bits
//                                    [b * bits, (b + 1) * bits), bit i of the
//                                    record being bit i % 32 of dword i / 32
//   sign bits    [sign_dw dwords]    QJL sign j at bit j (K only; V: zero)
//   radius       fp16                final polar radius
//   norm         fp16                residual norm (K only; V: zero)
// ---------------------------------------------------------------------------
struct GenLayout {
  int pd;        // padded dim (2, 4, ..., 256)
  int levels;    // log2(pd)
  int bits;      // bits per angle (1 .. 8)
  int qjl;       // QJL rows
  int ps;        // tokens per page
  int angle_dw;  // dwords of angle bits per record
  int sign_dw;   // dwords of sign bits per record
  __host__ __device__ int record_bytes() const { return 4 * (angle_dw + sign_dw) + 4; }
  __host__ __device__ int radius_offset() const { return 4 * (angle_dw + sign_dw); }
  __host__ __device__ size_t slice_bytes() const { return (size_t)ps * record_bytes(); }
};

// Padded dim of a head_dim: the next power of two, at least 2 (the
// reference's 2^ceil(log2 max(head_dim, 2)), core/kv_quantizer.py:225), or 0
// outside 1 .. 256.
__host__ __device__ inline int padded_dim_of(int head_dim) {
  if (head_dim < 1 || head_dim > 256) return 0;
  int pd = 2;
  while (pd < head_dim) pd <<= 1;
  return pd;
}

__host__ __device__ inline GenLayout gen_layout(int head_dim, int bits, int qjl, int ps) {
  GenLayout g{};
  g.pd = padded_dim_of(head_dim);
  g.levels = 0;
  while ((2 << g.levels) <= g.pd) ++g.levels;  // log2(pd)
  g.bits = bits;
  g.qjl = qjl;
  g.ps = ps;
  g.angle_dw = ((g.pd - 1) * bits + 31) / 32;
  g.sign_dw = (qjl + 31) / 32;
  return g;
}

// Padded dim of the tuned layout for a setting, or 0 where it does not apply:
// padded dim 64 or 128 (head_dim 33 .. 128, zero-padded before the rotation
// as the compressor pads), the default PD / 2 QJL rows, 16-token pages, 2 to
// 4 bits.
__host__ __device__ inline int tuned_pd(int head_dim, int bits, int qjl, int ps) {
  const int pd = padded_dim_of(head_dim);
  return (pd == 64 || pd == 128) && qjl == tuned_qjl(pd) && ps == kTokens && bits >= 2 && bits <= 4 ? pd : 0;
}
__host__ __device__ inline bool tuned_layout(int head_dim, int bits, int qjl, int ps) {
  return tuned_pd(head_dim, bits, qjl, ps) != 0;
}

// True for settings the generic layout serves.
__host__ __device__ inline bool generic_ok(int head_dim, int bits, int qjl, int ps) {
  return padded_dim_of(head_dim) != 0 && bits >= 1 && bits <= 8 && qjl >= 1 && qjl <= 256 && ps >= 1;
}

}  // namespace tq
}  // namespace vrm
