// Device-side helpers shared by the CarryKernel GDN decode kernels (gfx950).
//
// All kernels are compiled with -ffp-contract=off: every fused multiply-add in
// them is an explicit fmaf(), so the fp32 operation sequence is exactly the one
// the CPU oracle replays.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ck_gate_math.h"

namespace ck {

// 1.5 * 2^23. For |x| < 2^22, fmaf(t, inv, kMagic) rounds t*inv (exact product)
// to the nearest integer, ties to even, and leaves that integer in the low
// mantissa bits in two's complement: the low byte is the int8 code and the low
// nibble the int4 code. Subtracting kMagic recovers the code as a float exactly.
constexpr float kMagic = 12582912.0f;
constexpr float kEps = 1e-12f;

enum DType : int { kF32 = 0, kBF16 = 1, kF16 = 2 };

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float load_act(const void* p, int64_t i, int dtype) {
  if (dtype == kF32) return static_cast<const float*>(p)[i];
  if (dtype == kBF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  return (float)static_cast<const _Float16*>(p)[i];
}

__device__ __forceinline__ void store_act(void* p, int64_t i, int dtype, float v) {
  if (dtype == kF32) {
    static_cast<float*>(p)[i] = v;
  } else if (dtype == kBF16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_rne(v);
  } else {
    static_cast<_Float16*>(p)[i] = (_Float16)v;  // round to nearest even
  }
}

// Load 16 consecutive activations starting at element i (i a multiple of 16 for
// fp32 alignment of the vector path; falls back to scalar loads otherwise).
__device__ __forceinline__ void load_act16(const void* p, int64_t i, int dtype, float (&x)[16]) {
  if (dtype == kF32 && ((reinterpret_cast<uintptr_t>(static_cast<const float*>(p) + i) & 15u) == 0)) {
    const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float4 v = q[j];
      x[4 * j + 0] = v.x;
      x[4 * j + 1] = v.y;
      x[4 * j + 2] = v.z;
      x[4 * j + 3] = v.w;
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) x[j] = load_act(p, i + j, dtype);
}

// ---------------------------------------------------------------------------
// Cross-lane reductions over aligned groups of N lanes (N = 1, 2, 4, 8, 16),
// built from DPP moves. Each step adds the value of a partner lane; because
// fp32 addition is commutative both partners obtain the same bits, so the
// result is the balanced tree ((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+p7)) ... in
// every lane of the group, independent of which lane is "self".
// ---------------------------------------------------------------------------
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141; // lane i <-> 7-i within 8
constexpr int kDppRowMirror = 0x140;     // lane i <-> 15-i within 16

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

template <int N>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group size");
  if constexpr (N >= 2) x = x + dpp_f<kDppQuadXor1>(x);
  if constexpr (N >= 4) x = x + dpp_f<kDppQuadXor2>(x);
  if constexpr (N >= 8) x = x + dpp_f<kDppRowHalfMirror>(x);
  if constexpr (N >= 16) x = x + dpp_f<kDppRowMirror>(x);
  return x;
}

template <int N>
__device__ __forceinline__ float group_max(float x) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group size");
  if constexpr (N >= 2) x = fmaxf(x, dpp_f<kDppQuadXor1>(x));
  if constexpr (N >= 4) x = fmaxf(x, dpp_f<kDppQuadXor2>(x));
  if constexpr (N >= 8) x = fmaxf(x, dpp_f<kDppRowHalfMirror>(x));
  if constexpr (N >= 16) x = fmaxf(x, dpp_f<kDppRowMirror>(x));
  return x;
}

// Max over a whole wavefront (64 lanes), result valid in every lane.
__device__ __forceinline__ float wave_max(float x) {
  x = group_max<16>(x);
  // combine the four rows of 16 lanes through lane reads (uniform results)
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// ---------------------------------------------------------------------------
// Byte / nibble packing of magic-rounded codes.
// ---------------------------------------------------------------------------

// Low bytes of four dwords -> one dword (byte j from w[j]).
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
  // v_perm_b32(S0, S1, sel): selector bytes 0-3 pick S1 bytes, 4-7 pick S0
  // bytes, 0x0c yields 0x00.
  const uint32_t lo = __builtin_amdgcn_perm(w1, w0, 0x0c0c0400u);  // [w0.b0, w1.b0, 0, 0]
  const uint32_t hi = __builtin_amdgcn_perm(w3, w2, 0x04000c0cu);  // [0, 0, w2.b0, w3.b0]
  return lo | hi;
}

// Eight codes (low nibbles of w[0..7], element j at bits 4j..4j+3) -> dword.
// Even elements take the low nibble of each byte, odd elements the high one,
// matching vllm_integration/quantized_packed_decode.py:221-237.
__device__ __forceinline__ uint32_t pack_nibbles8(const uint32_t (&w)[8]) {
  const uint32_t ev = pack_low_bytes(w[0], w[2], w[4], w[6]);
  const uint32_t od = pack_low_bytes(w[1], w[3], w[5], w[7]);
  return (ev & 0x0f0f0f0fu) | ((od << 4) & 0xf0f0f0f0u);
}

// Sign-extended int8 code b (0..3) of dword d, as float.
__device__ __forceinline__ float code_i8(uint32_t d, int b) {
  return (float)(int)(signed char)(d >> (8 * b));
}

// Sign-extended int4 code n (0..7) of dword d, as float.
__device__ __forceinline__ float code_i4(uint32_t d, int n) {
  return (float)(int)__builtin_amdgcn_sbfe((int)d, 4 * n, 4);
}

}  // namespace ck
