// Deterministic fp32 exp / log / gate functions for the GDN decode kernels.
//
// The kernels derive the decay alpha = exp(-exp(A_log) * softplus(a + dt_bias))
// and the write strength beta = sigmoid(b) in-kernel, as
// vllm_integration/quantized_packed_decode.py:174-182 does. Library
// transcendentals (OCML on the GPU, glibc on the host) are accurate but not
// bit-identical to each other, and a one-ulp difference in alpha moves every
// downstream fp32 value of the step. These functions are written only with
// IEEE-754 fp32 add/mul/fma/div and round-to-nearest-even rint, so the same
// source evaluates to the same bits on the GPU and in a host build compiled
// with -ffp-contract=off.
//
// Method (published, not a vendor library):
//  * exp: Cody & Waite argument reduction (W. J. Cody, W. Waite, "Software
//    Manual for the Elementary Functions", 1980): x = n*ln2 + r, |r| <= ln2/2,
//    with ln2 split into a 16-bit head (so n*head is exact for |n| < 2^8) and
//    a tail; e^r by its Taylor series to degree 8 (coefficients 1/k!) in
//    Horner form; scaling by 2^n in two exact power-of-two steps.
//  * log: y = m * 2^e with m in [sqrt(1/2), sqrt(2)); log m = 2*atanh(s),
//    s = (m-1)/(m+1), by the odd series 2*(s + s^3/3 + ... + s^13/13).
// Accuracy is a few ulp; the unit tests bound it against float64.
#pragma once

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define CK_GM_FN __device__ __forceinline__
#else
#include <math.h>
#include <stdint.h>
#include <string.h>
#define CK_GM_FN static inline
#endif

CK_GM_FN float ck_gm_bits_to_float(uint32_t u) {
#if defined(__HIPCC__)
  return __uint_as_float(u);
#else
  float f;
  memcpy(&f, &u, 4);
  return f;
#endif
}

CK_GM_FN uint32_t ck_gm_float_to_bits(float f) {
#if defined(__HIPCC__)
  return __float_as_uint(f);
#else
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
#endif
}

// 2^n for an integer n in [-126, 127], exactly.
CK_GM_FN float ck_gm_pow2i(int n) { return ck_gm_bits_to_float((uint32_t)(n + 127) << 23); }

CK_GM_FN float ck_expf(float x) {
  if (x != x) return x;                              // NaN passes through
  if (x > 88.72283172607421875f) return ck_gm_bits_to_float(0x7f800000u);  // +inf
  if (x < -103.97208404541015625f) return 0.0f;       // below half the least subnormal
  const float kLog2e = 1.44269502162933349609375f;    // RN(log2(e))
  const float kLn2Hi = 0.693145751953125f;            // ln2 truncated to 16 bits
  const float kLn2Lo = 1.42860676533018704503775e-06f;  // RN(ln2 - kLn2Hi)
  const float n = rintf(x * kLog2e);
  float r = fmaf(-n, kLn2Hi, x);                     // exact: n*kLn2Hi has <= 24 bits
  r = fmaf(-n, kLn2Lo, r);
  // Taylor series of e^r, degree 8, Horner form.
  float p = 2.48015873015873015873e-05f;             // 1/8!
  p = fmaf(p, r, 1.98412698412698412698e-04f);       // 1/7!
  p = fmaf(p, r, 1.38888888888888888889e-03f);       // 1/6!
  p = fmaf(p, r, 8.33333333333333333333e-03f);       // 1/5!
  p = fmaf(p, r, 4.16666666666666666667e-02f);       // 1/4!
  p = fmaf(p, r, 1.66666666666666666667e-01f);       // 1/3!
  p = fmaf(p, r, 0.5f);                              // 1/2!
  p = fmaf(p, r, 1.0f);                              // 1/1!
  p = fmaf(p, r, 1.0f);                              // 1/0!
  const int ni = (int)n;                             // in [-150, 128]
  const int n1 = ni / 2;
  const int n2 = ni - n1;
  return (p * ck_gm_pow2i(n1)) * ck_gm_pow2i(n2);
}

// Natural log for y > 0 (normal or subnormal); log(0) = -inf, log(inf) = inf,
// log(negative or NaN) = NaN.
CK_GM_FN float ck_logf(float y) {
  if (y != y || y < 0.0f) return ck_gm_bits_to_float(0x7fc00000u);
  if (y == 0.0f) return ck_gm_bits_to_float(0xff800000u);
  if (y > 3.40282346638528859812e+38f) return y;     // +inf
  int e = 0;
  if (y < 1.17549435082228750797e-38f) {             // subnormal: rescale by 2^24
    y = y * 16777216.0f;
    e = -24;
  }
  const uint32_t u = ck_gm_float_to_bits(y);
  e += (int)((u >> 23) & 0xffu) - 127;
  float m = ck_gm_bits_to_float((u & 0x007fffffu) | 0x3f800000u);  // [1, 2)
  if (m > 1.41421353816986083984f) {                 // RN(sqrt(2))
    m = m * 0.5f;
    e += 1;
  }
  const float s = (m - 1.0f) / (m + 1.0f);           // m-1 is exact (Sterbenz)
  const float s2 = s * s;
  float p = 7.69230769230769230769e-02f;             // 1/13
  p = fmaf(p, s2, 9.09090909090909090909e-02f);      // 1/11
  p = fmaf(p, s2, 1.11111111111111111111e-01f);      // 1/9
  p = fmaf(p, s2, 1.42857142857142857143e-01f);      // 1/7
  p = fmaf(p, s2, 2.0e-01f);                         // 1/5
  p = fmaf(p, s2, 3.33333333333333333333e-01f);      // 1/3
  // log m = 2s + 2 s^3 * p
  const float logm = fmaf(2.0f * s, s2 * p, 2.0f * s);
  const float fe = (float)e;
  const float kLn2Hi = 0.693145751953125f;
  const float kLn2Lo = 1.42860676533018704503775e-06f;
  return fmaf(fe, kLn2Hi, fmaf(fe, kLn2Lo, logm));
}

// Gates of one (request, value-head), following
// vllm_integration/quantized_packed_decode.py:179-182:
//   x = a + dt_bias; softplus = x <= 20 ? log(1 + exp(x)) : x
//   g = -exp(A_log) * softplus; alpha = exp(g); beta = sigmoid(b)
CK_GM_FN void ck_gates(float a, float b, float A_log, float dt_bias, float* alpha, float* beta) {
  const float x = a + dt_bias;
  const float sp = (x <= 20.0f) ? ck_logf(1.0f + ck_expf(x)) : x;
  const float g = -ck_expf(A_log) * sp;
  *alpha = ck_expf(g);
  *beta = 1.0f / (1.0f + ck_expf(-b));
}
