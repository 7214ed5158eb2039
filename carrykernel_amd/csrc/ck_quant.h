// Scalar quantizer steps shared by both state layouts. The two arithmetic modes
// are defined bit-for-bit here and replayed by the CPU oracle.
#pragma once

#include "ck_device.h"

namespace ck {

enum QuantMode : int { kFast = 0, kExact = 1 };

// Rounds t / s to the nearest integer (ties to even) and returns it as a float;
// the low byte / nibble of `ybits` is the two's-complement code.
//  FAST : rne(t * inv) of the exact product, one fma (inv = RN(1/s)).
//  EXACT: rne(RN(t / s)). RN(t / s) comes from Markstein's correction of the
//         reciprocal product (P. Markstein, "Computation of elementary
//         functions on the IBM RISC System/6000 processor", IBM J. Res. Dev.
//         34(1), 1990): q0 = RN(t*inv), r = t - q0*s (exact in an fma),
//         q = RN(q0 + r*inv), which is the correctly rounded quotient when
//         inv = RN(1/s); then rne(q) by adding 1.5*2^23.
template <int MODE>
__device__ __forceinline__ float quantize(float t, float s, float inv, uint32_t& ybits) {
  float y;
  if constexpr (MODE == kFast) {
    y = fmaf(t, inv, kMagic);
  } else {
    const float q0 = t * inv;
    const float r = fmaf(-q0, s, t);
    const float q = fmaf(r, inv, q0);
    y = q + kMagic;
  }
  ybits = __float_as_uint(y);
  return y - kMagic;
}

// Error-feedback residual t - code * s.
//  FAST : one rounding (fma).  EXACT: RN(t - RN(code * s)).
template <int MODE>
__device__ __forceinline__ float residual(float t, float code, float s) {
  if constexpr (MODE == kFast) {
    return fmaf(-code, s, t);
  } else {
    return t - code * s;
  }
}

// a + x * y:  FAST: fma.  EXACT: RN(a + RN(x * y)).
template <int MODE>
__device__ __forceinline__ float madd(float x, float y, float a) {
  if constexpr (MODE == kFast) {
    return fmaf(x, y, a);
  } else {
    return a + x * y;
  }
}

}  // namespace ck
