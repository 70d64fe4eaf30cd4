// Layout of a TurboQuant KV page of this library (head_dim 65 .. 128:
// padded_dim 128, 7 polar levels, 127 angles, 64 QJL signs).
//
// The pool keeps the reference's addressing, tq_pool[P][L][2][KH][slice],
// one slice of kTqSliceBytes(bits) bytes per (page, layer, K/V, kv-head) with
// the 16 tokens of the page:
//   angles  [16][16 * bits]   bytes 0 ..            (token t at t * 16 * bits)
//   signs   [16][8]           QJL sign bits (K only; bit j = residual . jl_j > 0)
//   radius  [16]              fp16 final polar radius
//   norms   [16]              fp16 residual norm (K only)
// V slices use the angles and radius fields only (same offsets).
//
// Angle record of one token: four quarters of 4 * bits bytes.  Quarter g holds
// the 31 angles of the subtree over dims 32 g .. 32 g + 31 plus one spare slot
// that carries a top-level angle, so that a decode lane owning those dims
// reads one aligned 4 * bits-byte word.  For bits <= 3 a node's angle is
// followed by its two children's, so that the index of a two-level product
// table (node bin + NB * child-0 bin + NB^2 * child-1 bin, NB = 2^bits) is one
// contiguous 3 * bits-bit field:
//   slots 3 j, 3 j + 1, 3 j + 2       (j = 0 .. 7) level 1 angle 8 g + j,
//                                     then level 0 angles 16 g + 2 j, 16 g + 2 j + 1
//   slots 24 + 3 j .. 26 + 3 j        (j = 0, 1) level 3 angle 2 g + j, then
//                                     level 2 angles 4 g + 2 j, 4 g + 2 j + 1
//   slot 30                           level 4 angle g
// For bits == 4 the levels are in order (the decode reads siblings in pairs):
//   slot 0 level 4 angle g; slots 1, 2 level 3 angles 2 g, 2 g + 1; slots
//   3 .. 6 level 2 angles 4 g ..; slots 7 .. 14 level 1 angles 8 g ..; slots
//   15 .. 30 level 0 angles 16 g ..
// For every bits:
//   slot 31   quarter 0: level 6 angle; quarter 1: level 5 angle 0;
//             quarter 2: level 5 angle 1; quarter 3: 0
// Slot s occupies bits [s * bits, (s + 1) * bits) of its quarter, bit i of a
// quarter being bit i % 8 of its byte i / 8 (little-endian).  The record has
// exactly the 127 * bits bits of the reference's packed angles (plus bits
// padding bits).  Angle levels and indices are those of the reference's
// level-major bins (core/kv_quantizer.py:262-287): level l holds 64 >> l
// angles and angle i of level l pairs elements 2 i, 2 i + 1 of level l - 1.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace vrm {
namespace tq {

constexpr int kPD = 128;      // padded head dimension
constexpr int kLevels = 7;    // log2(kPD)
constexpr int kAngles = 127;  // kPD - 1
constexpr int kQjl = 64;      // QJL projection rows
constexpr int kTokens = 16;   // tokens per page

__host__ __device__ constexpr int angle_bytes(int bits) { return 16 * bits; }        // per token
__host__ __device__ constexpr int signs_offset(int bits) { return kTokens * angle_bytes(bits); }
__host__ __device__ constexpr int radius_offset(int bits) { return signs_offset(bits) + kTokens * 8; }
__host__ __device__ constexpr int norms_offset(int bits) { return radius_offset(bits) + kTokens * 2; }
__host__ __device__ constexpr int slice_bytes(int bits) { return norms_offset(bits) + kTokens * 2; }

// Offset of level l in the reference's level-major bin array: sum_{i<l} 64 >> i.
__host__ __device__ constexpr int level_offset(int l) { return kPD - (kPD >> l); }

// (quarter, slot) of angle i of level l.
__host__ __device__ inline void slot_of(int l, int i, int bits, int& quarter, int& slot) {
  if (l <= 4) {
    const int per = 1 << (4 - l);  // angles of level l per quarter
    quarter = i / per;
    const int a = i % per;  // angle within the quarter
    if (bits == 4) {
      slot = (per - 1) + a;
      return;
    }
    switch (l) {
      case 0: slot = 3 * (a >> 1) + 1 + (a & 1); break;
      case 1: slot = 3 * a; break;
      case 2: slot = 24 + 3 * (a >> 1) + 1 + (a & 1); break;
      case 3: slot = 24 + 3 * a; break;
      default: slot = 30; break;
    }
  } else if (l == 5) {
    quarter = 1 + i;
    slot = 31;
  } else {
    quarter = 0;
    slot = 31;
  }
}

// Level-major bin index (reference order) of slot s of quarter g, or -1 for
// the unused spare of quarter 3.
__host__ __device__ inline int bin_index_of(int g, int s, int bits) {
  if (s == 31) return g == 0 ? level_offset(6) : (g <= 2 ? level_offset(5) + (g - 1) : -1);
  if (bits == 4) {  // slots 2^m - 1 .. 2^(m+1) - 2 hold the 2^m angles of level 4 - m
    const int m = 31 - __builtin_clz(s + 1);
    return level_offset(4 - m) + g * (1 << m) + (s + 1 - (1 << m));
  }
  if (s == 30) return level_offset(4) + g;
  if (s >= 24) {
    const int k = (s - 24) / 3, r = (s - 24) % 3;
    return r == 0 ? level_offset(3) + 2 * g + k : level_offset(2) + 4 * g + 2 * k + (r - 1);
  }
  const int j = s / 3, r = s % 3;
  return r == 0 ? level_offset(1) + 8 * g + j : level_offset(0) + 16 * g + 2 * j + (r - 1);
}

// ---------------------------------------------------------------------------
// Generic page layout: every other setting of the compressor (head_dim 33 ..
// 256, i.e. padded_dim 64 / 128 / 256, 1 to 8 bits per angle, qjl_dim 1 ..
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
  int pd;        // padded dim (64, 128, 256)
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

// Padded dim of a head_dim: the next power of two (the reference's
// 2^ceil(log2 head_dim), core/kv_quantizer.py:225), or 0 outside 33 .. 256.
__host__ __device__ inline int padded_dim_of(int head_dim) {
  if (head_dim < 33 || head_dim > 256) return 0;
  int pd = 64;
  while (pd < head_dim) pd <<= 1;
  return pd;
}

__host__ __device__ inline GenLayout gen_layout(int head_dim, int bits, int qjl, int ps) {
  GenLayout g{};
  g.pd = padded_dim_of(head_dim);
  g.levels = g.pd == 64 ? 6 : g.pd == 128 ? 7 : 8;
  g.bits = bits;
  g.qjl = qjl;
  g.ps = ps;
  g.angle_dw = ((g.pd - 1) * bits + 31) / 32;
  g.sign_dw = (qjl + 31) / 32;
  return g;
}

// True for the settings the tuned layout above (and its decode kernel) serves:
// padded dim 128 (head_dim 65 .. 128, zero-padded before the rotation as the
// compressor pads), 64 QJL rows, 16-token pages, 2 to 4 bits.
__host__ __device__ inline bool tuned_layout(int head_dim, int bits, int qjl, int ps) {
  return head_dim > kPD / 2 && head_dim <= kPD && qjl == kQjl && ps == kTokens && bits >= 2 && bits <= 4;
}

// True for settings the generic layout serves.
__host__ __device__ inline bool generic_ok(int head_dim, int bits, int qjl, int ps) {
  return padded_dim_of(head_dim) != 0 && bits >= 1 && bits <= 8 && qjl >= 1 && qjl <= 256 && ps >= 1;
}

}  // namespace tq
}  // namespace vrm
