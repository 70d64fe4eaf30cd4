// Bit packing of TurboQuant codes for storage and transfer: the packed format
// of KVCacheCompressor (core/kv_quantizer.py:46-105, 337-371).  Each row of M
// values contributes the low `bits` bits of every value, most significant bit
// first, value after value; the bit stream is cut into bytes, the first bit in
// bit 7 of byte 0, and the last byte is zero-padded.  QJL signs are the case
// bits = 1, angle bins the case bits = bits_per_angle over the level-major
// concatenation of a row's bins.
#include "vrm_common.h"

namespace vrm {
namespace {

constexpr int kThreads = 256;

// Row and column of flat element x of a [rows][width] array; 32-bit division
// when the whole array indexes in 31 bits (the caller's uniform choice).
__device__ __forceinline__ void split_index(long long x, int width, bool narrow, long long& row, int& col) {
  if (narrow) {
    const uint32_t r = (uint32_t)x / (uint32_t)width;
    row = r;
    col = (int)((uint32_t)x - r * (uint32_t)width);
  } else {
    row = x / width;
    col = (int)(x - row * width);
  }
}

// One thread per packed byte; global byte x = row * nbytes + j.  The byte's
// 8 bits walk the stream from bit 8 j: one division finds the first value,
// then the position inside the value advances bit by bit.
__global__ void __launch_bounds__(kThreads) pack_kernel(const uint8_t* vals, long long rows, int M, int bits,
                                                        int nbytes, uint8_t* out) {
  const long long x = (long long)blockIdx.x * kThreads + threadIdx.x;
  const long long n = rows * nbytes;
  if (x >= n) return;
  long long row;
  int j;
  split_index(x, nbytes, n <= 0x7fffffffLL, row, j);
  const uint8_t* v = vals + row * M;
  const int total = M * bits;
  int pos = 8 * j;  // bit position in the row's stream
  int i = pos / bits;
  int from_msb = pos - i * bits;
  uint32_t byte = 0;
  for (int k = 0; k < 8; ++k, ++pos) {
    const uint32_t bit = pos < total ? (v[i] >> (bits - 1 - from_msb)) & 1u : 0u;
    byte |= bit << (7 - k);
    if (++from_msb == bits) {
      from_msb = 0;
      ++i;
    }
  }
  out[x] = (uint8_t)byte;
}

// One thread per value; global value x = row * M + i.
__global__ void __launch_bounds__(kThreads) unpack_kernel(const uint8_t* packed, long long rows, int M, int bits,
                                                          int nbytes, uint8_t* vals) {
  const long long x = (long long)blockIdx.x * kThreads + threadIdx.x;
  const long long n = rows * M;
  if (x >= n) return;
  long long row;
  int i;
  split_index(x, M, n <= 0x7fffffffLL, row, i);
  const uint8_t* p = packed + row * nbytes;
  uint32_t v = 0;
  for (int b = 0; b < bits; ++b) {
    const int pos = i * bits + b;
    v = (v << 1) | ((p[pos >> 3] >> (7 - (pos & 7))) & 1u);
  }
  vals[x] = (uint8_t)v;
}

int check_pack(long long rows, int M, int bits, const void* a, const void* b, const char* who) {
  if (rows < 0 || M < 0 || bits < 1 || bits > 8) {
    set_error("%s: bad sizes (rows=%lld M=%d bits=%d)", who, rows, M, bits);
    return VRM_ERR_ARG;
  }
  const long long nbytes = ((long long)M * bits + 7) / 8;
  if (rows * (nbytes > M ? nbytes : M) > 0x7fffffffLL * kThreads) {
    set_error("%s: too many elements", who);
    return VRM_ERR_UNSUPPORTED;
  }
  if (rows > 0 && M > 0 && (!a || !b)) {
    set_error("%s: null pointer argument", who);
    return VRM_ERR_ARG;
  }
  return VRM_OK;
}

}  // namespace
}  // namespace vrm

using namespace vrm;

extern "C" int vrm_pack_bits(const uint8_t* vals, long long rows, int M, int bits, uint8_t* packed,
                             vrm_stream_t stream) {
  const char* who = "vrm_pack_bits";
  int rc = check_pack(rows, M, bits, vals, packed, who);
  if (rc) return rc;
  const int nbytes = (int)(((long long)M * bits + 7) / 8);
  const long long n = rows * nbytes;
  if (n == 0) {
    clear_error();
    return VRM_OK;
  }
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), vals, rows, M, bits, nbytes, packed);
  return launch_status(who);
}

extern "C" int vrm_unpack_bits(const uint8_t* packed, long long rows, int M, int bits, uint8_t* vals,
                               vrm_stream_t stream) {
  const char* who = "vrm_unpack_bits";
  int rc = check_pack(rows, M, bits, packed, vals, who);
  if (rc) return rc;
  const int nbytes = (int)(((long long)M * bits + 7) / 8);
  const long long n = rows * M;
  if (n == 0) {
    clear_error();
    return VRM_OK;
  }
  hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), packed, rows, M, bits, nbytes, vals);
  return launch_status(who);
}
