// Fused GDN decode step in the statequant layout: state [B, HV, K, V] int8
// (V contiguous) with one scale per V-column (amax over K), error-feedback
// residual stored as fp32, fp16, fp8 e5m2 or int8 with a per-column scale.
// Out of place (in place also works: a workgroup reads its whole tile before
// writing it). Counterpart of statequant/kernel.py:260-341 (_gdn_quant_kernel),
// cuda/gdn_state_kernel.cu:141-246 and the launcher at :310-348; plus the fp32
// baseline step (statequant/kernel.py:211-248, cuda/gdn_state_kernel.cu:251-297).
//
// Work mapping. A workgroup covers one (request, head) and a tile of 32 column
// groups of CPT consecutive V-columns; thread t owns column group t % 32 and
// one of S K-slices: S = 8 slices of K/8 rows for K <= 128 (256 threads),
// S = 16 slices of 16 rows at K = 256 (512 threads), so a thread's rows always
// fit its registers. Column sums over K are a sequential fma chain over the
// thread's rows, then the S slice partials are combined through LDS by a
// balanced pairwise tree (S = 8: ((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7))). Four
// such exchanges per step (h.k, h.q, amax, and the int8 residual's amax), one
// barrier each.
//
// Any K in 1..256: the reference's CUDA launcher loops over its K rows
// (cuda/gdn_state_kernel.cu:141-246) and the Triton kernel masks its BK =
// next_pow2(K) rows (statequant/kernel.py:277-279). Here the rows are padded
// with zeros to KP = max(16, next_pow2(K)) and the KP kernel runs on them (MK:
// rows at or past K load nothing, contribute zero products and zero to every
// amax, and store nothing), so the sums keep the KP slice order.
//
// Columns per thread. CPT = 4 when V % 4 == 0 and every tensor is 16-byte
// aligned: a thread's columns are one vector access per row (a dword of
// codes), so each half-wave reads 128 contiguous bytes of a row. Otherwise
// (any V, as the reference's masked offs_v < V; offset views) CPT = 1: one
// element per thread and row, 32 contiguous elements per half-wave, and the
// threads past V load nothing and store nothing. One column per thread keeps
// that path at 24-106 VGPRs, two or more waves per SIMD, which its narrow
// loads need (four columns 32 apart per thread, 128-column tiles, ran 1.5-2x
// slower at one wave per SIMD).
#include <hip/hip_runtime.h>

#include "ck_capi_common.h"
#include "ck_device.h"
#include "ck_quant.h"

namespace ck {
namespace qs {

constexpr int kResFp32 = CK_RES_FP32;
constexpr int kResFp16 = CK_RES_FP16;
constexpr int kResFp8 = CK_RES_FP8;
constexpr int kResInt8 = CK_RES_INT8;

constexpr int kGroups = 32;  // column groups per workgroup (one half-wave)

// K-slices per workgroup, one half-wave each.
template <int K>
constexpr int kSlicesFor = K <= 128 ? 8 : K / 16;
template <int K>
constexpr int kThreadsFor = kGroups * kSlicesFor<K>;

// fp8 e5m2 (OCP: sign | 5-bit exponent, bias 15 | 2-bit mantissa, with
// infinities and NaNs) through gfx950's conversion instructions: encoding
// rounds to nearest even, keeps subnormals (m * 2^-16) and sends values at or
// past the midpoint above the largest finite 57344 to infinity, the format's
// own definition (the reference's torch.float8_e5m2 casts). Two values per
// v_cvt_pk_bf8_f32 into one 16-bit half of the result; decoding picks a byte.
template <int CPT>
__device__ __forceinline__ uint32_t f32_to_e5m2(const float (&x)[CPT]) {
  if constexpr (CPT == 4) {
    const int lo = __builtin_amdgcn_cvt_pk_bf8_f32(x[0], x[1], 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(x[2], x[3], lo, true);
  } else {
    return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(x[0], 0.0f, 0, false) & 0xffu;
  }
}

// Byte j (0..3, unrolled to a constant) of d as an e5m2 value.
__device__ __forceinline__ float e5m2_byte(uint32_t d, int j) {
  switch (j) {
    case 0: return __builtin_amdgcn_cvt_f32_bf8((int)d, 0);
    case 1: return __builtin_amdgcn_cvt_f32_bf8((int)d, 1);
    case 2: return __builtin_amdgcn_cvt_f32_bf8((int)d, 2);
    default: return __builtin_amdgcn_cvt_f32_bf8((int)d, 3);
  }
}

__device__ __forceinline__ float half_bits_to_f32(uint32_t h) {
  _Float16 x;
  const uint16_t b = (uint16_t)h;
  __builtin_memcpy(&x, &b, 2);
  return (float)x;
}

__device__ __forceinline__ uint32_t f32_to_half_bits(float f) {
  const _Float16 x = (_Float16)f;  // round to nearest even, subnormals kept
  uint16_t b;
  __builtin_memcpy(&b, &x, 2);
  return b;
}

// Balanced pairwise tree over the S slice partials of LDS column `col`.
template <int S, int NC>
__device__ __forceinline__ float slice_tree_sum(const float (*red)[NC], int col) {
  float c[S];
#pragma unroll
  for (int s = 0; s < S; ++s) c[s] = red[s][col];
#pragma unroll
  for (int w = 1; w < S; w *= 2)
#pragma unroll
    for (int i = 0; i + w < S; i += 2 * w) c[i] = c[i] + c[i + w];
  return c[0];
}

template <int S, int NC>
__device__ __forceinline__ float slice_max(const float (*red)[NC], int col) {
  float m = red[0][col];
#pragma unroll
  for (int s = 1; s < S; ++s) m = fmaxf(m, red[s][col]);
  return m;
}

// CPT consecutive columns of one row at p: CPT = 4 is one naturally aligned
// vector access, CPT = 1 one element. 8-bit values travel packed in a dword
// (column j in byte j), 16-bit values two to a dword.
template <int CPT>
__device__ __forceinline__ void ld_f32(const float* p, float (&x)[CPT]) {
  if constexpr (CPT == 4) {
    const float4 f = *reinterpret_cast<const float4*>(p);
    x[0] = f.x, x[1] = f.y, x[2] = f.z, x[3] = f.w;
  } else {
    x[0] = *p;
  }
}

template <int CPT>
__device__ __forceinline__ uint32_t ld_b8(const void* p) {
  if constexpr (CPT == 4) return *reinterpret_cast<const uint32_t*>(p);
  else return *static_cast<const uint8_t*>(p);
}

template <int CPT>
__device__ __forceinline__ void ld_b16(const uint16_t* p, uint32_t (&w)[(CPT + 1) / 2]) {
  if constexpr (CPT == 4) {
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    w[0] = x.x, w[1] = x.y;
  } else {
    w[0] = *p;
  }
}

template <int CPT>
__device__ __forceinline__ void st_f32(float* p, const float (&x)[CPT]) {
  if constexpr (CPT == 4) *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
  else *p = x[0];
}

template <int CPT>
__device__ __forceinline__ void st_b8(void* p, uint32_t x) {
  if constexpr (CPT == 4) *reinterpret_cast<uint32_t*>(p) = x;
  else *static_cast<uint8_t*>(p) = (uint8_t)x;
}

template <int CPT>
__device__ __forceinline__ void st_b16(uint16_t* p, const uint32_t (&w)[(CPT + 1) / 2]) {
  if constexpr (CPT == 4) *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
  else *p = (uint16_t)w[0];
}

// Low bytes of the CPT codes, column j in byte j.
template <int CPT>
__device__ __forceinline__ uint32_t pack_codes(const uint32_t (&yb)[CPT]) {
  if constexpr (CPT == 4) return pack_low_bytes(yb[0], yb[1], yb[2], yb[3]);
  else return yb[0] & 0xffu;
}

struct StepParams {
  const int8_t* h_in;
  const float* scale_in;
  const void* e_in;
  const float* e_scale_in;
  const float* q;
  const float* k;
  const float* v;
  const float* alpha;
  const float* beta;
  float* o;
  int8_t* h_out;
  float* scale_out;
  void* e_out;
  float* e_scale_out;
  int HV, V, nvt;
  int K;  // rows that exist (the kernel's K template argument is the padded count)
  float qmax, rqmax;
};

template <int K, int RES, int MODE, int CPT, bool MK>
__global__ __launch_bounds__(kThreadsFor<K>) void quant_step_kernel(const StepParams p) {
  constexpr int S = kSlicesFor<K>;
  constexpr int RPS = K / S;            // rows per slice
  constexpr int NC = kGroups * CPT;     // columns per workgroup
  __shared__ float red[4][S][NC];

  const int t = threadIdx.x;
  const int cg = t % kGroups;
  const int ks = t / kGroups;
  const int vt = blockIdx.x % p.nvt;
  const int w = blockIdx.x / p.nvt;  // (request, head)
  const int lc = cg * CPT;           // local column
  const int c0 = vt * NC + lc;
  const bool colok = c0 < p.V;       // CPT = 4 only with V % 4 == 0: all 4 columns or none
  const int r0 = ks * RPS;
  const int KA = MK ? p.K : K;       // rows that exist
  const int64_t mb = (int64_t)w * KA * p.V;
  const int64_t vb = (int64_t)w * p.V;
  const float alpha = p.alpha[w];
  const float beta = p.beta[w];

  uint32_t cw[RPS];
  // the residual stays in its stored form until t = h + e (one dword per row
  // and 4 columns for 8-bit formats, two for fp16, four for fp32)
  constexpr int EWD = RES == kResFp32 ? CPT : RES == kResFp16 ? (CPT + 1) / 2 : 1;
  uint32_t ew[RPS][EWD];
  float sc[CPT], esc[CPT], vv[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) sc[j] = esc[j] = vv[j] = 0.f;
  float kk[RPS], qq[RPS];
#pragma unroll
  for (int r = 0; r < RPS; ++r) {
    kk[r] = qq[r] = 0.f;
    if (!MK || r0 + r < KA) {
      kk[r] = p.k[(int64_t)w * KA + r0 + r];
      qq[r] = p.q[(int64_t)w * KA + r0 + r];
    }
  }
  if (colok) {
    ld_f32<CPT>(p.scale_in + vb + c0, sc);
    ld_f32<CPT>(p.v + vb + c0, vv);
    if constexpr (RES == kResInt8) ld_f32<CPT>(p.e_scale_in + vb + c0, esc);
#pragma unroll
    for (int r = 0; r < RPS; ++r) {
      if (MK && r0 + r >= KA) {  // padding row: zero codes and residual (decodes to +0 in every format)
        cw[r] = 0;
#pragma unroll
        for (int j = 0; j < EWD; ++j) ew[r][j] = 0u;
        continue;
      }
      const int64_t i = mb + (int64_t)(r0 + r) * p.V + c0;
      cw[r] = ld_b8<CPT>(p.h_in + i);
      if constexpr (RES == kResFp32) {
        float e[CPT];
        ld_f32<CPT>(static_cast<const float*>(p.e_in) + i, e);
#pragma unroll
        for (int j = 0; j < CPT; ++j) ew[r][j] = __float_as_uint(e[j]);
      } else if constexpr (RES == kResFp16) {
        ld_b16<CPT>(static_cast<const uint16_t*>(p.e_in) + i, ew[r]);
      } else {
        ew[r][0] = ld_b8<CPT>(static_cast<const uint8_t*>(p.e_in) + i);
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < RPS; ++r) {
      cw[r] = 0;
#pragma unroll
      for (int j = 0; j < EWD; ++j) ew[r][j] = 0u;   // decodes to +0 in every format
    }
  }

  // dequantize + decay
  float h[RPS][CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const float sa = sc[j] * alpha;
#pragma unroll
    for (int r = 0; r < RPS; ++r) {
      const float code = code_i8(cw[r], j);
      h[r][j] = (MODE == kFast) ? code * sa : (code * sc[j]) * alpha;
    }
  }
  // rd = h^T k
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    float acc = h[0][j] * kk[0];
#pragma unroll
    for (int r = 1; r < RPS; ++r) acc = fmaf(h[r][j], kk[r], acc);
    red[0][ks][lc + j] = acc;
  }
  __syncthreads();
  float dv[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) dv[j] = beta * (vv[j] - slice_tree_sum<S, NC>(red[0], lc + j));
  // h += k dv; o = h^T q
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
#pragma unroll
    for (int r = 0; r < RPS; ++r) h[r][j] = madd<MODE>(kk[r], dv[j], h[r][j]);
    float acc = h[0][j] * qq[0];
#pragma unroll
    for (int r = 1; r < RPS; ++r) acc = fmaf(h[r][j], qq[r], acc);
    red[1][ks][lc + j] = acc;
  }
  // t = h + e (the residual decoded here)
#pragma unroll
  for (int r = 0; r < RPS; ++r) {
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      float ev;
      if constexpr (RES == kResFp32) {
        ev = __uint_as_float(ew[r][j]);
      } else if constexpr (RES == kResFp16) {
        ev = half_bits_to_f32(j % 2 ? ew[r][j / 2] >> 16 : ew[r][j / 2] & 0xffffu);
      } else if constexpr (RES == kResFp8) {
        ev = e5m2_byte(ew[r][0], j);
      } else {
        ev = code_i8(ew[r][0], j);
      }
      if constexpr (RES == kResInt8) {
        h[r][j] = madd<MODE>(ev, esc[j], h[r][j]);
      } else {
        h[r][j] = h[r][j] + ev;
      }
    }
  }
  // amax over K per column
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    float m = fabsf(h[0][j]);
#pragma unroll
    for (int r = 1; r < RPS; ++r) m = fmaxf(m, fabsf(h[r][j]));
    red[2][ks][lc + j] = m;
  }
  __syncthreads();
  if (ks == 0 && colok) {
    float o4[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) o4[j] = slice_tree_sum<S, NC>(red[1], lc + j);
    st_f32<CPT>(p.o + vb + c0, o4);
  }
  float s[CPT], inv[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    s[j] = fmaxf(div_small_int(slice_max<S, NC>(red[2], lc + j), p.qmax, p.rqmax), kEps);
    inv[j] = recip_rn(s[j]);
  }
  // requantize, store codes, form the residual
  float ea[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) ea[j] = 0.f;
#pragma unroll
  for (int r = 0; r < RPS; ++r) {
    uint32_t yb[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const float code = quantize<MODE>(h[r][j], s[j], inv[j], yb[j]);
      h[r][j] = residual<MODE>(h[r][j], code, s[j]);
      ea[j] = fmaxf(ea[j], fabsf(h[r][j]));
    }
    if (colok && (!MK || r0 + r < KA)) st_b8<CPT>(p.h_out + mb + (int64_t)(r0 + r) * p.V + c0, pack_codes<CPT>(yb));
  }
  if (ks == 0 && colok) st_f32<CPT>(p.scale_out + vb + c0, s);

  if constexpr (RES == kResInt8) {
#pragma unroll
    for (int j = 0; j < CPT; ++j) red[3][ks][lc + j] = ea[j];
    __syncthreads();
    float es[CPT], inv_e[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      es[j] = fmaxf(div_small_int(slice_max<S, NC>(red[3], lc + j), p.qmax, p.rqmax), kEps);
      inv_e[j] = recip_rn(es[j]);
    }
    if (colok) {
#pragma unroll
      for (int r = 0; r < RPS; ++r) {
        if (MK && r0 + r >= KA) continue;
        uint32_t eb[CPT];
#pragma unroll
        for (int j = 0; j < CPT; ++j) (void)quantize<MODE>(h[r][j], es[j], inv_e[j], eb[j]);
        st_b8<CPT>(static_cast<int8_t*>(p.e_out) + mb + (int64_t)(r0 + r) * p.V + c0, pack_codes<CPT>(eb));
      }
      if (ks == 0) st_f32<CPT>(p.e_scale_out + vb + c0, es);
    }
  } else if (colok) {
#pragma unroll
    for (int r = 0; r < RPS; ++r) {
      if (MK && r0 + r >= KA) continue;
      const int64_t i = mb + (int64_t)(r0 + r) * p.V + c0;
      if constexpr (RES == kResFp32) {
        st_f32<CPT>(static_cast<float*>(p.e_out) + i, h[r]);
      } else if constexpr (RES == kResFp16) {
        uint32_t hw[(CPT + 1) / 2];
#pragma unroll
        for (int j = 0; j < CPT; j += 2)
          hw[j / 2] = f32_to_half_bits(h[r][j]) | (j + 1 < CPT ? f32_to_half_bits(h[r][j + 1]) << 16 : 0u);
        st_b16<CPT>(static_cast<uint16_t*>(p.e_out) + i, hw);
      } else {
        st_b8<CPT>(static_cast<uint8_t*>(p.e_out) + i, f32_to_e5m2<CPT>(h[r]));
      }
    }
  }
}

struct Fp32Params {
  const float* h_in;
  const float* q;
  const float* k;
  const float* v;
  const float* alpha;
  const float* beta;
  float* o;
  float* h_out;
  int V, nvt;
  int K;  // rows that exist (the kernel's K template argument is the padded count)
};

template <int K, int CPT, bool MK>
__global__ __launch_bounds__(kThreadsFor<K>) void fp32_step_kernel(const Fp32Params p) {
  constexpr int S = kSlicesFor<K>;
  constexpr int RPS = K / S;
  constexpr int NC = kGroups * CPT;
  __shared__ float red[2][S][NC];
  const int t = threadIdx.x;
  const int cg = t % kGroups;
  const int ks = t / kGroups;
  const int vt = blockIdx.x % p.nvt;
  const int w = blockIdx.x / p.nvt;
  const int lc = cg * CPT;
  const int c0 = vt * NC + lc;
  const bool colok = c0 < p.V;
  const int r0 = ks * RPS;
  const int KA = MK ? p.K : K;  // rows that exist
  const int64_t mb = (int64_t)w * KA * p.V;
  const int64_t vb = (int64_t)w * p.V;
  const float alpha = p.alpha[w];
  const float beta = p.beta[w];
  float h[RPS][CPT], kk[RPS], qq[RPS], vv[CPT];
#pragma unroll
  for (int r = 0; r < RPS; ++r) {
    const bool rin = !MK || r0 + r < KA;
    kk[r] = qq[r] = 0.f;
    if (rin) {
      kk[r] = p.k[(int64_t)w * KA + r0 + r];
      qq[r] = p.q[(int64_t)w * KA + r0 + r];
    }
    float x[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) x[j] = 0.f;
    if (colok && rin) ld_f32<CPT>(p.h_in + mb + (int64_t)(r0 + r) * p.V + c0, x);
#pragma unroll
    for (int j = 0; j < CPT; ++j) h[r][j] = x[j] * alpha;
  }
#pragma unroll
  for (int j = 0; j < CPT; ++j) vv[j] = 0.f;
  if (colok) ld_f32<CPT>(p.v + vb + c0, vv);
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    float acc = h[0][j] * kk[0];
#pragma unroll
    for (int r = 1; r < RPS; ++r) acc = fmaf(h[r][j], kk[r], acc);
    red[0][ks][lc + j] = acc;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const float dv = beta * (vv[j] - slice_tree_sum<S, NC>(red[0], lc + j));
#pragma unroll
    for (int r = 0; r < RPS; ++r) h[r][j] = fmaf(kk[r], dv, h[r][j]);
    float acc = h[0][j] * qq[0];
#pragma unroll
    for (int r = 1; r < RPS; ++r) acc = fmaf(h[r][j], qq[r], acc);
    red[1][ks][lc + j] = acc;
  }
  if (colok) {
#pragma unroll
    for (int r = 0; r < RPS; ++r)
      if (!MK || r0 + r < KA) st_f32<CPT>(p.h_out + mb + (int64_t)(r0 + r) * p.V + c0, h[r]);
  }
  __syncthreads();
  if (ks == 0 && colok) {
    float o4[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) o4[j] = slice_tree_sum<S, NC>(red[1], lc + j);
    st_f32<CPT>(p.o + vb + c0, o4);
  }
}

template <int K, int MODE, int CPT, bool MK>
int launch_quant(const StepParams& p, int64_t grid, int res_fmt, hipStream_t s) {
  const dim3 g((unsigned)grid), b(kThreadsFor<K>);
  switch (res_fmt) {
    case kResFp32: hipLaunchKernelGGL((quant_step_kernel<K, kResFp32, MODE, CPT, MK>), g, b, 0, s, p); break;
    case kResFp16: hipLaunchKernelGGL((quant_step_kernel<K, kResFp16, MODE, CPT, MK>), g, b, 0, s, p); break;
    case kResFp8: hipLaunchKernelGGL((quant_step_kernel<K, kResFp8, MODE, CPT, MK>), g, b, 0, s, p); break;
    default: hipLaunchKernelGGL((quant_step_kernel<K, kResInt8, MODE, CPT, MK>), g, b, 0, s, p); break;
  }
  return check_launch("ck_gdn_quant_step");
}

// K padded to KP = max(16, next_pow2(K)) (K <= 256)
inline int padded_k(int K) {
  int kp = 16;
  while (kp < K) kp *= 2;
  return kp;
}

template <int MODE, int CPT, bool MK>
int launch_quant_kp(const StepParams& p, int64_t grid, int KP, int res_fmt, hipStream_t s) {
  switch (KP) {
    case 16: return launch_quant<16, MODE, CPT, MK>(p, grid, res_fmt, s);
    case 32: return launch_quant<32, MODE, CPT, MK>(p, grid, res_fmt, s);
    case 64: return launch_quant<64, MODE, CPT, MK>(p, grid, res_fmt, s);
    case 128: return launch_quant<128, MODE, CPT, MK>(p, grid, res_fmt, s);
    default: return launch_quant<256, MODE, CPT, MK>(p, grid, res_fmt, s);
  }
}

template <int MODE, int CPT>
int launch_quant_k(const StepParams& p, int64_t grid, int K, int res_fmt, hipStream_t s) {
  const int KP = padded_k(K);
  return KP == K ? launch_quant_kp<MODE, CPT, false>(p, grid, KP, res_fmt, s)
                 : launch_quant_kp<MODE, CPT, true>(p, grid, KP, res_fmt, s);
}

template <int CPT, bool MK>
int launch_fp32_kp(const Fp32Params& p, int64_t grid, int KP, hipStream_t s) {
  const dim3 g((unsigned)grid);
  switch (KP) {
    case 16: hipLaunchKernelGGL((fp32_step_kernel<16, CPT, MK>), g, dim3(kThreadsFor<16>), 0, s, p); break;
    case 32: hipLaunchKernelGGL((fp32_step_kernel<32, CPT, MK>), g, dim3(kThreadsFor<32>), 0, s, p); break;
    case 64: hipLaunchKernelGGL((fp32_step_kernel<64, CPT, MK>), g, dim3(kThreadsFor<64>), 0, s, p); break;
    case 128: hipLaunchKernelGGL((fp32_step_kernel<128, CPT, MK>), g, dim3(kThreadsFor<128>), 0, s, p); break;
    default: hipLaunchKernelGGL((fp32_step_kernel<256, CPT, MK>), g, dim3(kThreadsFor<256>), 0, s, p); break;
  }
  return check_launch("ck_gdn_fp32_step");
}

template <int CPT>
int launch_fp32(const Fp32Params& p, int64_t grid, int K, hipStream_t s) {
  const int KP = padded_k(K);
  return KP == K ? launch_fp32_kp<CPT, false>(p, grid, KP, s) : launch_fp32_kp<CPT, true>(p, grid, KP, s);
}

inline bool valid_k(int K) { return K >= 1 && K <= 256; }

// Bitwise OR of the addresses: its low bits are zero only if every pointer is
// aligned that far.
template <typename... P>
inline uintptr_t addr_bits(const P*... ptrs) {
  return (reinterpret_cast<uintptr_t>(ptrs) | ... | (uintptr_t)0);
}

// Column tiles per (request, head) for CPT columns per thread.
inline int col_tiles(int V, int cpt) { return (V + kGroups * cpt - 1) / (kGroups * cpt); }

}  // namespace qs
}  // namespace ck

extern "C" int ck_gdn_quant_step(const int8_t* h_in, const float* scale_in, const void* e_in,
                                 const float* e_scale_in,
                                 const float* q, const float* k, const float* v,
                                 const float* alpha, const float* beta,
                                 float* o, int8_t* h_out, float* scale_out, void* e_out, float* e_scale_out,
                                 int B, int HV, int K, int V, float qmax, int res_fmt, int quant_mode,
                                 void* stream) {
  using namespace ck;
  using namespace ck::qs;
  if (B < 0 || HV <= 0 || K <= 0 || V <= 0) return fail(CK_EINVAL, "bad sizes B=%d HV=%d K=%d V=%d", B, HV, K, V);
  if (!valid_k(K)) return fail(CK_EUNSUPPORTED, "K must be in 1..256, got %d", K);
  if (res_fmt < CK_RES_FP32 || res_fmt > CK_RES_INT8) return fail(CK_EINVAL, "unknown residual format %d", res_fmt);
  if (quant_mode != CK_QUANT_FAST && quant_mode != CK_QUANT_EXACT)
    return fail(CK_EINVAL, "quant_mode must be CK_QUANT_FAST or CK_QUANT_EXACT, got %d", quant_mode);
  const int iq = (int)qmax;
  if ((float)iq != qmax || iq < 1 || iq > 127) return fail(CK_EINVAL, "qmax must be an integer in 1..127");
  if (B == 0) return ok();
  if (!h_in || !scale_in || !e_in || !q || !k || !v || !alpha || !beta || !o || !h_out || !scale_out || !e_out)
    return fail(CK_EINVAL, "null pointer argument");
  if (res_fmt == CK_RES_INT8 && (!e_scale_in || !e_scale_out)) return fail(CK_EINVAL, "int8 residual needs e_scale");
  const bool int8_res = res_fmt == CK_RES_INT8;
  const uintptr_t fbits = addr_bits(scale_in, q, k, v, alpha, beta, o, scale_out) |
                          (int8_res ? addr_bits(e_scale_in, e_scale_out) : 0);
  const int esz = res_fmt == CK_RES_FP32 ? 4 : res_fmt == CK_RES_FP16 ? 2 : 1;
  const uintptr_t ebits = addr_bits(e_in, e_out);
  if ((fbits & 3) || (ebits & (esz - 1)))
    return fail(CK_EINVAL, "fp32 tensors must be 4-byte aligned and the residual %d-byte aligned", esz);
  // four columns per thread when every 4-column group of every row is one aligned access
  const bool vec = V % 4 == 0 && ((fbits | ebits | addr_bits(h_in, h_out)) & 15) == 0;
  StepParams p{};
  p.h_in = h_in;
  p.scale_in = scale_in;
  p.e_in = e_in;
  p.e_scale_in = e_scale_in;
  p.q = q;
  p.k = k;
  p.v = v;
  p.alpha = alpha;
  p.beta = beta;
  p.o = o;
  p.h_out = h_out;
  p.scale_out = scale_out;
  p.e_out = e_out;
  p.e_scale_out = e_scale_out;
  p.HV = HV;
  p.V = V;
  p.nvt = col_tiles(V, vec ? 4 : 1);
  p.K = K;
  volatile float one = 1.0f;
  p.qmax = qmax;
  p.rqmax = one / qmax;
  const int64_t grid = (int64_t)B * HV * p.nvt;
  if (grid > 0x7fffffff) return fail(CK_EUNSUPPORTED, "grid too large");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (quant_mode == CK_QUANT_EXACT)
    return vec ? launch_quant_k<kExact, 4>(p, grid, K, res_fmt, s) : launch_quant_k<kExact, 1>(p, grid, K, res_fmt, s);
  return vec ? launch_quant_k<kFast, 4>(p, grid, K, res_fmt, s) : launch_quant_k<kFast, 1>(p, grid, K, res_fmt, s);
}

extern "C" int ck_gdn_fp32_step(const float* h_in, const float* q, const float* k, const float* v,
                                const float* alpha, const float* beta, float* o, float* h_out,
                                int B, int HV, int K, int V, void* stream) {
  using namespace ck;
  using namespace ck::qs;
  if (B < 0 || HV <= 0 || K <= 0 || V <= 0) return fail(CK_EINVAL, "bad sizes B=%d HV=%d K=%d V=%d", B, HV, K, V);
  if (!valid_k(K)) return fail(CK_EUNSUPPORTED, "K must be in 1..256, got %d", K);
  if (B == 0) return ok();
  if (!h_in || !q || !k || !v || !alpha || !beta || !o || !h_out) return fail(CK_EINVAL, "null pointer argument");
  const uintptr_t bits = addr_bits(h_in, q, k, v, alpha, beta, o, h_out);
  if (bits & 3) return fail(CK_EINVAL, "fp32 tensors must be 4-byte aligned");
  const bool vec = V % 4 == 0 && (bits & 15) == 0;
  Fp32Params p{h_in, q, k, v, alpha, beta, o, h_out, V, col_tiles(V, vec ? 4 : 1), K};
  const int64_t grid = (int64_t)B * HV * p.nvt;
  if (grid > 0x7fffffff) return fail(CK_EUNSUPPORTED, "grid too large");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return vec ? launch_fp32<4>(p, grid, K, s) : launch_fp32<1>(p, grid, K, s);
}
