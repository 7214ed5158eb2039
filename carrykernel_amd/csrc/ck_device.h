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

// Element i of a tensor of runtime dtype as one 4-byte load (for a 16-bit
// element: the aligned dword that holds it, which lies inside any
// allocation, 4-byte aligned and 4-byte granular), decoded after the load.
// No conversion sits next to a load, so the compiler need not wait for a
// load (and every load issued before it) until the value is decoded, and
// several such loads can be in flight before the first is needed.
struct ActBits {
  uint32_t word;
  uint32_t hi;  // 16-bit element in the high half of the word
};

__device__ __forceinline__ ActBits load_act_bits(const void* p, int64_t i, int dtype) {
  ActBits r;
  if (dtype == kF32) {
    r.word = static_cast<const uint32_t*>(p)[i];
    r.hi = 0;
  } else {
    const char* e = static_cast<const char*>(p) + 2 * i;
    const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(e) & 3u;  // 0 or 2
    r.word = *reinterpret_cast<const uint32_t*>(e - mis);  // pointer arithmetic keeps the global address space
    r.hi = mis >> 1;
  }
  return r;
}

// load_act_bits without a branch on the dtype: the element's byte offset is
// selected, so a uniform index gives one scalar load whatever the dtype (a
// load in each arm of a dtype branch would be joined by a copy that waits for
// it). An fp32 element is 4-byte aligned (as every float is), so hi is 0 for it.
__device__ __forceinline__ ActBits load_act_bits_sel(const void* p, int64_t i, int dtype) {
  const char* e = static_cast<const char*>(p) + (dtype == kF32 ? 4 * i : 2 * i);
  const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(e) & 3u;  // 0 or 2
  ActBits r;
  r.word = *reinterpret_cast<const uint32_t*>(e - mis);
  r.hi = mis >> 1;
  return r;
}

__device__ __forceinline__ float decode_act_bits(ActBits b, int dtype) {
  if (dtype == kF32) return __uint_as_float(b.word);
  const uint32_t h16 = b.hi ? (b.word >> 16) : (b.word & 0xffffu);
  if (dtype == kBF16) return __uint_as_float(h16 << 16);
  _Float16 h;
  const uint16_t r16 = (uint16_t)h16;
  __builtin_memcpy(&h, &r16, 2);
  return (float)h;
}

// Raw bits of one activation of ESZ bytes (4: fp32, 2: bf16 / fp16) at a
// uniform base plus a 32-bit byte offset. Conversion is deferred to
// act_decode so that issuing the load never waits for its data.
template <int ESZ>
__device__ __forceinline__ uint32_t load_act_raw(const char* base, uint32_t off) {
  if constexpr (ESZ == 4) {
    return *reinterpret_cast<const uint32_t*>(base + off);
  } else {
    return (uint32_t)*reinterpret_cast<const uint16_t*>(base + off);
  }
}

// Bytes of one activation of dtype ACT, and its decode from raw bits with the
// dtype fixed at compile time.
template <int ACT>
constexpr int act_bytes = ACT == kF32 ? 4 : 2;

template <int ACT>
__device__ __forceinline__ float act_decode(uint32_t raw) {
  if constexpr (ACT == kF32) {
    return __uint_as_float(raw);
  } else if constexpr (ACT == kBF16) {
    return __uint_as_float(raw << 16);
  } else {
    _Float16 h;
    const uint16_t r16 = (uint16_t)raw;
    __builtin_memcpy(&h, &r16, 2);
    return (float)h;
  }
}

// Access at a uniform base plus a 32-bit byte offset (lets the compiler use
// the scalar-base + 32-bit vector-offset addressing form).
template <typename T>
__device__ __forceinline__ T ld_at(const void* base, uint32_t byte_off) {
  return *reinterpret_cast<const T*>(static_cast<const char*>(base) + byte_off);
}
template <typename T>
__device__ __forceinline__ void st_at(void* base, uint32_t byte_off, T v) {
  *reinterpret_cast<T*>(static_cast<char*>(base) + byte_off) = v;
}

// Store one activation at a uniform base plus a 32-bit element offset.
__device__ __forceinline__ void store_act_at(void* base, uint32_t i, int dtype, float v) {
  if (dtype == kF32) {
    st_at<float>(base, i * 4u, v);
  } else if (dtype == kBF16) {
    st_at<uint16_t>(base, i * 2u, f32_to_bf16_rne(v));
  } else {
    st_at<_Float16>(base, i * 2u, (_Float16)v);  // round to nearest even
  }
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
// Cross-lane reductions over aligned groups of N lanes (N = 1, 2, 4, 8, 16,
// 32, 64), built from DPP moves within a row of 16 lanes and ds_swizzle /
// ds_bpermute lane exchanges (__shfl_xor) across rows. Each step adds the
// value of a partner lane; because
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
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16 || N == 32 || N == 64, "group size");
  if constexpr (N >= 2) x = x + dpp_f<kDppQuadXor1>(x);
  if constexpr (N >= 4) x = x + dpp_f<kDppQuadXor2>(x);
  if constexpr (N >= 8) x = x + dpp_f<kDppRowHalfMirror>(x);
  if constexpr (N >= 16) x = x + dpp_f<kDppRowMirror>(x);
  if constexpr (N >= 32) x = x + __shfl_xor(x, 16);
  if constexpr (N >= 64) x = x + __shfl_xor(x, 32);
  return x;
}

// Max over a group of N lanes of non-negative floats (absolute values). For
// x >= 0 (and +inf) the IEEE order equals the unsigned order of the bit
// patterns, so the cross-lane steps are v_max_u32 with a fused DPP source,
// which avoids the NaN-quieting extra op of an IEEE fmaxf on a DPP result.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}

template <int N>
__device__ __forceinline__ float group_max(float x) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16 || N == 32 || N == 64, "group size");
  uint32_t u = __float_as_uint(x);
  if constexpr (N >= 2) u = max(u, dpp_u<kDppQuadXor1>(u));
  if constexpr (N >= 4) u = max(u, dpp_u<kDppQuadXor2>(u));
  if constexpr (N >= 8) u = max(u, dpp_u<kDppRowHalfMirror>(u));
  if constexpr (N >= 16) u = max(u, dpp_u<kDppRowMirror>(u));
  if constexpr (N >= 32) u = max(u, (uint32_t)__shfl_xor((int)u, 16));
  if constexpr (N >= 64) u = max(u, (uint32_t)__shfl_xor((int)u, 32));
  return __uint_as_float(u);
}

// Max over a whole wavefront (64 lanes) of non-negative floats, result valid
// in every lane.
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

// v_cvt_off_f32_i4 on byte B of d: sext(low nibble of that byte) / 16, exactly.
// One VALU op per code. (Checked on gfx950 for all 256 byte values and all
// four byte selects.)
template <int B>
__device__ __forceinline__ float cvt_off_i4(uint32_t d) {
  float r;
  if constexpr (B == 0) {
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(d));
  } else if constexpr (B == 1) {
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(d));
  } else if constexpr (B == 2) {
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(d));
  } else {
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(d));
  }
  return r;
}

// Eight int4 codes of dword d (element j at bits 4j..4j+3), each divided by 16.
__device__ __forceinline__ void decode_i4x8_div16(uint32_t d, float* out) {
  const uint32_t hi = d >> 4;  // odd elements' nibbles moved to the low half of each byte
  out[0] = cvt_off_i4<0>(d);
  out[1] = cvt_off_i4<0>(hi);
  out[2] = cvt_off_i4<1>(d);
  out[3] = cvt_off_i4<1>(hi);
  out[4] = cvt_off_i4<2>(d);
  out[5] = cvt_off_i4<2>(hi);
  out[6] = cvt_off_i4<3>(d);
  out[7] = cvt_off_i4<3>(hi);
}

// ---------------------------------------------------------------------------
// Correctly rounded scalar divisions without the generic IEEE division
// sequence.
// ---------------------------------------------------------------------------

// RN(a / q) for an integer q in 1..127, given rq = RN(1 / q): Markstein's
// correction of the reciprocal product. Checked exhaustively (all 2^23
// mantissas of a at five exponents, every q in 1..127) to equal the IEEE
// quotient.
__device__ __forceinline__ float div_small_int(float a, float q, float rq) {
  const float q0 = a * rq;
  const float r = fmaf(-q0, q, a);
  return fmaf(r, rq, q0);
}

// RN(1 / s) for a normal s whose reciprocal is normal: v_rcp_f32 followed by
// one Newton step in fma form. Checked on gfx950 against the IEEE quotient for
// all 2^23 mantissas at exponents spanning the fp32 range.
__device__ __forceinline__ float recip_rn(float s) {
  const float y = __builtin_amdgcn_rcpf(s);
  const float e = fmaf(-s, y, 1.0f);
  return fmaf(e, y, y);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Streaming (non-temporal) 16- and 8-byte accesses: the state and residual are
// touched once per step, so they should not displace reusable lines.
__device__ __forceinline__ u32x4 ld_stream16(const int8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x2 ld_stream8(const int8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}
__device__ __forceinline__ void st_stream16(int8_t* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}
__device__ __forceinline__ void st_stream8(int8_t* p, u32x2 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x2*>(p));
}

}  // namespace ck
