// Types shared by the decode kernels of libvrm_paged.so.
#pragma once
#include "vrm_common.h"

namespace vrm {
namespace dec {

constexpr int kPS = 16;               // tokens per page (the reference's default)
constexpr int kMaxPagesPerSplit = 64;  // one page id per lane of a wavefront
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
  float* part_acc;            // [B][H][nsplit][D]
  float* part_ml;             // [B][H][nsplit][2]
  int H, KH, L, P, max_pp, layer;
  float qscale;               // scale * log2(e): scores live in the log2 domain
  int pages_per_split, nsplit;
};

// Matrix-core (MFMA) split pass for the quantized pools; KIND is K_I8 or
// K_FP8, D the head dimension, G the query heads per wavefront (<= 16).
hipError_t launch_quant_mfma(const DecodeArgs& a, int kind, int B, int D, int G, hipStream_t st);

// Largest divisor of the GQA group size that is <= max_tile.
inline int pick_group_tile(int group, int max_tile) {
  for (int g = max_tile; g >= 1; --g)
    if (group % g == 0) return g;
  return 1;
}

}  // namespace dec
}  // namespace vrm
