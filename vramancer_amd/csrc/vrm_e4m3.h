// float32 -> OCP e4m3fn encoding with round-to-nearest-even, matching the
// cast `tensor.to(torch.float8_e4m3fn)`: magnitudes >= 480 (the first value
// past the largest finite 448) and NaN give the NaN code 0x7f (with the sign),
// magnitudes below 2^-6 are rounded into the subnormal range by one float add
// against 2^14 so that the hardware's round-to-nearest-even does the rounding.
// Plain C++ so the host unit test and the gfx950 kernels share it.
#pragma once
#include <stdint.h>
#include <string.h>

#ifdef __HIPCC__
#define VRM_E4M3_HD __host__ __device__ __forceinline__
#else
#define VRM_E4M3_HD static inline
#endif

namespace vrm_e4m3 {

VRM_E4M3_HD uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
VRM_E4M3_HD float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

VRM_E4M3_HD uint8_t encode(float f) {
#pragma clang fp contract(off)
  const uint32_t kFirstOverflow = 0x43f00000u;  // 480.0f
  const uint32_t kDenormMagic = 141u << 23;     // 2^14: aligns 2^-9 with the float ulp
  uint32_t bits = f2u(f);
  const uint32_t sign = bits & 0x80000000u;
  bits ^= sign;
  uint32_t code;
  if (bits >= kFirstOverflow) {  // includes NaN and infinities
    code = 0x7fu;
  } else if (bits < (121u << 23)) {  // below 2^-6: subnormal or zero
    code = f2u(u2f(bits) + u2f(kDenormMagic)) - kDenormMagic;
  } else {
    const uint32_t odd = (bits >> 20) & 1u;            // lsb of the kept mantissa
    bits += ((uint32_t)(7 - 127) << 23) + 0x7ffffu + odd;  // rebias + round half to even
    code = bits >> 20;
  }
  return (uint8_t)(code | (sign >> 24));
}

// e4m3fn byte -> float32 (exact).
VRM_E4M3_HD float decode(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 24;
  const uint32_t e = (b >> 3) & 0xfu;
  const uint32_t m = b & 0x7u;
  float mag;
  if (e == 0) {
    mag = (float)m * 0.001953125f;
  } else if (e == 0xfu && m == 0x7u) {
    mag = u2f(0x7fc00000u);
  } else {
    mag = u2f(((e + 120u) << 23) | (m << 20));
  }
  return u2f(f2u(mag) | sign);
}

}  // namespace vrm_e4m3
