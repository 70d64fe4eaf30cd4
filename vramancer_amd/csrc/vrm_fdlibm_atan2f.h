// Single-precision atan2 following the fdlibm algorithm (Sun Microsystems,
// 1993; float conversion by Ian Lance Taylor, Cygnus Support), which is the
// implementation behind glibc 2.35's scalar atan2f on x86_64.
//
//   Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//   Developed at SunPro, a Sun Microsystems, Inc. business.
//   Permission to use, copy, modify, and distribute this software is freely
//   granted, provided that this notice is preserved.
//
// Why this exists: the PolarQuant encoder bins atan2(b, a) into 2^bits
// uniform sectors, and the reference computes that angle with PyTorch's CPU
// kernel on strided views, i.e. with the C library's scalar atan2f
// (core/kv_quantizer.py:272).  That routine is not correctly rounded (about
// 16% of random inputs differ from the correctly rounded value by one ulp),
// so reproducing its exact float steps is the only way to get bit-identical
// angle bins near sector edges.  Every operation below is a single IEEE
// binary32 operation; callers must compile it without FP contraction.
//
// The header is plain C++ so that the same code is unit-tested against the
// host libm with g++ and compiled into the gfx950 kernels with hipcc.
#pragma once
#include <stdint.h>
#include <string.h>

#ifdef __HIPCC__
#define VRM_HD __host__ __device__ __forceinline__
#else
#define VRM_HD static inline
#endif

namespace vrm_fdlibm {

VRM_HD uint32_t fbits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
VRM_HD float bitsf(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

// atan(x) for float x: reduce |x| to one of five ranges around the nodes
// 0, 1/2, 1, 3/2, inf and evaluate an 11-term odd polynomial split into
// even/odd halves in z = x^2.
VRM_HD float atanf(float x) {
#pragma clang fp contract(off)
  const float atanhi0 = 4.6364760399e-01f, atanhi1 = 7.8539812565e-01f,
              atanhi2 = 9.8279368877e-01f, atanhi3 = 1.5707962513e+00f;
  const float atanlo0 = 5.0121582440e-09f, atanlo1 = 3.7748947079e-08f,
              atanlo2 = 3.4473217170e-08f, atanlo3 = 7.5497894159e-08f;
  const float aT0 = 3.3333334327e-01f, aT1 = -2.0000000298e-01f,
              aT2 = 1.4285714924e-01f, aT3 = -1.1111110449e-01f,
              aT4 = 9.0908870101e-02f, aT5 = -7.6918758452e-02f,
              aT6 = 6.6610731184e-02f, aT7 = -5.8335702866e-02f,
              aT8 = 4.9768779427e-02f, aT9 = -3.6531571299e-02f,
              aT10 = 1.6285819933e-02f;
  const float one = 1.0f;
  uint32_t hx = fbits(x);
  uint32_t ix = hx & 0x7fffffffu;
  int id;
  if (ix >= 0x4c000000u) {              // |x| >= 2^25
    if (ix > 0x7f800000u) return x + x;  // NaN
    return (hx >> 31) ? -atanhi3 - atanlo3 : atanhi3 + atanlo3;
  }
  if (ix < 0x3ee00000u) {               // |x| < 0.4375
    if (ix < 0x31000000u) return x;      // |x| < 2^-29
    id = -1;
  } else {
    x = bitsf(ix);                       // fabsf
    if (ix < 0x3f980000u) {              // |x| < 1.1875
      if (ix < 0x3f300000u) {            // 7/16 <= |x| < 11/16
        id = 0; x = (2.0f * x - one) / (2.0f + x);
      } else {                           // 11/16 <= |x| < 19/16
        id = 1; x = (x - one) / (x + one);
      }
    } else {
      if (ix < 0x401c0000u) {            // |x| < 2.4375
        id = 2; x = (x - 1.5f) / (one + 1.5f * x);
      } else {                           // 2.4375 <= |x| < 2^25
        id = 3; x = -1.0f / x;
      }
    }
  }
  float z = x * x;
  float w = z * z;
  float s1 = z * (aT0 + w * (aT2 + w * (aT4 + w * (aT6 + w * (aT8 + w * aT10)))));
  float s2 = w * (aT1 + w * (aT3 + w * (aT5 + w * (aT7 + w * aT9))));
  if (id < 0) return x - x * (s1 + s2);
  float hi = id == 0 ? atanhi0 : id == 1 ? atanhi1 : id == 2 ? atanhi2 : atanhi3;
  float lo = id == 0 ? atanlo0 : id == 1 ? atanlo1 : id == 2 ? atanlo2 : atanlo3;
  z = hi - ((x * (s1 + s2) - lo) - x);
  return (hx >> 31) ? -z : z;
}

// atan2(y, x) with the fdlibm quadrant logic.
VRM_HD float atan2f(float y, float x) {
#pragma clang fp contract(off)
  const float tiny = 1.0e-30f, pi_o_4 = 7.8539818525e-01f,
              pi_o_2 = 1.5707963705e+00f, pi = 3.1415927410e+00f,
              pi_lo = -8.7422776573e-08f;
  uint32_t hx = fbits(x), hy = fbits(y);
  uint32_t ix = hx & 0x7fffffffu, iy = hy & 0x7fffffffu;
  if (ix > 0x7f800000u || iy > 0x7f800000u) return x + y;  // NaN
  if (hx == 0x3f800000u) return atanf(y);                    // x == 1
  int m = (int)((hy >> 31) & 1u) | (int)((hx >> 30) & 2u);   // 2*sign(x)+sign(y)
  if (iy == 0) {
    switch (m) {
      case 0: case 1: return y;
      case 2: return pi + tiny;
      default: return -pi - tiny;
    }
  }
  if (ix == 0) return (hy >> 31) ? -pi_o_2 - tiny : pi_o_2 + tiny;
  if (ix == 0x7f800000u) {
    if (iy == 0x7f800000u) {
      switch (m) {
        case 0: return pi_o_4 + tiny;
        case 1: return -pi_o_4 - tiny;
        case 2: return 3.0f * pi_o_4 + tiny;
        default: return -3.0f * pi_o_4 - tiny;
      }
    }
    switch (m) {
      case 0: return 0.0f;
      case 1: return -0.0f;
      case 2: return pi + tiny;
      default: return -pi - tiny;
    }
  }
  if (iy == 0x7f800000u) return (hy >> 31) ? -pi_o_2 - tiny : pi_o_2 + tiny;
  int k = ((int)iy - (int)ix) >> 23;
  float z;
  if (k > 60) z = pi_o_2 + 0.5f * pi_lo;
  else if ((hx >> 31) && k < -60) z = 0.0f;
  else z = atanf(bitsf(fbits(y / x) & 0x7fffffffu));
  switch (m) {
    case 0: return z;
    case 1: return -z;
    case 2: return pi - (z - pi_lo);
    default: return (z - pi_lo) - pi;
  }
}

}  // namespace vrm_fdlibm
