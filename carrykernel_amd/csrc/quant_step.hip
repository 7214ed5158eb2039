// Fused GDN decode step in the statequant layout: state [B, HV, K, V] int8
// (V contiguous) with one scale per V-column (amax over K), error-feedback
// residual stored as fp32, fp16, fp8 e5m2 or int8 with a per-column scale.
// Out of place (in place also works: a workgroup reads its whole tile before
// writing it). Counterpart of statequant/kernel.py:260-341 (_gdn_quant_kernel),
// cuda/gdn_state_kernel.cu:141-246 and the launcher at :310-348; plus the fp32
// baseline step (statequant/kernel.py:211-248, cuda/gdn_state_kernel.cu:251-297).
//
// Work mapping. A workgroup of 256 threads covers one (request, head) and a
// tile of 128 V-columns. Thread t owns 4 consecutive columns (one dword of
// codes per K-row, so each half-wave reads 128 contiguous bytes of a row) and
// one of 8 K-slices of K/8 rows. Column sums over K are a sequential fma chain
// over the thread's rows, then the 8 slice partials are combined through LDS
// as ((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7)). Four such exchanges per step (h.k,
// h.q, amax, and the int8 residual's amax), one barrier each.
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

constexpr int kCols = 128;   // V-columns per workgroup
constexpr int kSlices = 8;   // K-slices per workgroup
constexpr int kThreads = 256;

// fp8 e5m2 (OCP: sign | 5-bit exponent, bias 15 | 2-bit mantissa, with
// infinities and NaNs) through gfx950's conversion instructions: encoding
// rounds to nearest even, keeps subnormals (m * 2^-16) and sends values at or
// past the midpoint above the largest finite 57344 to infinity, the format's
// own definition (the reference's torch.float8_e5m2 casts). Two values per
// v_cvt_pk_bf8_f32 into one 16-bit half of the result; decoding picks a byte.
__device__ __forceinline__ uint32_t f32x4_to_e5m2x4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(c, d, lo, true);
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

// Balanced tree over the 8 slice partials of LDS column `col`.
__device__ __forceinline__ float slice_tree_sum(const float (*red)[kCols], int col) {
  const float s01 = red[0][col] + red[1][col];
  const float s23 = red[2][col] + red[3][col];
  const float s45 = red[4][col] + red[5][col];
  const float s67 = red[6][col] + red[7][col];
  return (s01 + s23) + (s45 + s67);
}

__device__ __forceinline__ float slice_max(const float (*red)[kCols], int col) {
  float m = red[0][col];
#pragma unroll
  for (int s = 1; s < kSlices; ++s) m = fmaxf(m, red[s][col]);
  return m;
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
  float qmax, rqmax;
};

template <int K, int RES, int MODE>
__global__ __launch_bounds__(kThreads) void quant_step_kernel(const StepParams p) {
  constexpr int RPS = K / kSlices;  // rows per slice
  __shared__ float red[4][kSlices][kCols];

  const int t = threadIdx.x;
  const int cg = t % 32;
  const int ks = t / 32;
  const int vt = blockIdx.x % p.nvt;
  const int w = blockIdx.x / p.nvt;  // (request, head)
  const int lc = cg * 4;             // local column
  const int c0 = vt * kCols + lc;
  const bool colok = c0 < p.V;  // V % 4 == 0, so all 4 columns or none
  const int r0 = ks * RPS;
  const int64_t mb = (int64_t)w * K * p.V;
  const int64_t vb = (int64_t)w * p.V;
  const float alpha = p.alpha[w];
  const float beta = p.beta[w];

  uint32_t cw[RPS];
  // the residual stays in its stored form until t = h + e (16, 32 or 64
  // registers for 8-bit, fp16 and fp32 residuals instead of 64 floats)
  constexpr int EWD = RES == kResFp32 ? 4 : RES == kResFp16 ? 2 : 1;
  uint32_t ew[RPS][EWD];
  float4 sc = make_float4(0.f, 0.f, 0.f, 0.f), esc = make_float4(0.f, 0.f, 0.f, 0.f),
         vv = make_float4(0.f, 0.f, 0.f, 0.f);
  float kk[RPS], qq[RPS];
#pragma unroll
  for (int r = 0; r < RPS; ++r) {
    kk[r] = p.k[(int64_t)w * K + r0 + r];
    qq[r] = p.q[(int64_t)w * K + r0 + r];
  }
  if (colok) {
    sc = *reinterpret_cast<const float4*>(p.scale_in + vb + c0);
    vv = *reinterpret_cast<const float4*>(p.v + vb + c0);
    if constexpr (RES == kResInt8) esc = *reinterpret_cast<const float4*>(p.e_scale_in + vb + c0);
#pragma unroll
    for (int r = 0; r < RPS; ++r) {
      const int64_t i = mb + (int64_t)(r0 + r) * p.V + c0;
      cw[r] = *reinterpret_cast<const uint32_t*>(p.h_in + i);
      if constexpr (RES == kResFp32) {
        const uint4 e4 = *reinterpret_cast<const uint4*>(static_cast<const float*>(p.e_in) + i);
        ew[r][0] = e4.x, ew[r][1] = e4.y, ew[r][2] = e4.z, ew[r][3] = e4.w;
      } else if constexpr (RES == kResFp16) {
        const uint2 e2 = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p.e_in) + i);
        ew[r][0] = e2.x, ew[r][1] = e2.y;
      } else if constexpr (RES == kResFp8) {
        ew[r][0] = *reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(p.e_in) + i);
      } else {
        ew[r][0] = *reinterpret_cast<const uint32_t*>(static_cast<const int8_t*>(p.e_in) + i);
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
  const float scv[4] = {sc.x, sc.y, sc.z, sc.w};
  const float escv[4] = {esc.x, esc.y, esc.z, esc.w};
  const float vvv[4] = {vv.x, vv.y, vv.z, vv.w};

  // dequantize + decay
  float h[RPS][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float sa = scv[j] * alpha;
#pragma unroll
    for (int r = 0; r < RPS; ++r) {
      const float code = code_i8(cw[r], j);
      h[r][j] = (MODE == kFast) ? code * sa : (code * scv[j]) * alpha;
    }
  }
  // rd = h^T k
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float acc = h[0][j] * kk[0];
#pragma unroll
    for (int r = 1; r < RPS; ++r) acc = fmaf(h[r][j], kk[r], acc);
    red[0][ks][lc + j] = acc;
  }
  __syncthreads();
  float dv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) dv[j] = beta * (vvv[j] - slice_tree_sum(red[0], lc + j));
  // h += k dv; o = h^T q
#pragma unroll
  for (int j = 0; j < 4; ++j) {
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
    float ev[4];
    if constexpr (RES == kResFp32) {
#pragma unroll
      for (int j = 0; j < 4; ++j) ev[j] = __uint_as_float(ew[r][j]);
    } else if constexpr (RES == kResFp16) {
      ev[0] = half_bits_to_f32(ew[r][0] & 0xffffu), ev[1] = half_bits_to_f32(ew[r][0] >> 16);
      ev[2] = half_bits_to_f32(ew[r][1] & 0xffffu), ev[3] = half_bits_to_f32(ew[r][1] >> 16);
    } else if constexpr (RES == kResFp8) {
      ev[0] = __builtin_amdgcn_cvt_f32_bf8((int)ew[r][0], 0);
      ev[1] = __builtin_amdgcn_cvt_f32_bf8((int)ew[r][0], 1);
      ev[2] = __builtin_amdgcn_cvt_f32_bf8((int)ew[r][0], 2);
      ev[3] = __builtin_amdgcn_cvt_f32_bf8((int)ew[r][0], 3);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) ev[j] = code_i8(ew[r][0], j);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (RES == kResInt8) {
        h[r][j] = madd<MODE>(ev[j], escv[j], h[r][j]);
      } else {
        h[r][j] = h[r][j] + ev[j];
      }
    }
  }
  // amax over K per column
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float m = fabsf(h[0][j]);
#pragma unroll
    for (int r = 1; r < RPS; ++r) m = fmaxf(m, fabsf(h[r][j]));
    red[2][ks][lc + j] = m;
  }
  __syncthreads();
  if (ks == 0 && colok) {
    float o4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o4[j] = slice_tree_sum(red[1], lc + j);
    *reinterpret_cast<float4*>(p.o + vb + c0) = make_float4(o4[0], o4[1], o4[2], o4[3]);
  }
  float s[4], inv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    s[j] = fmaxf(div_small_int(slice_max(red[2], lc + j), p.qmax, p.rqmax), kEps);
    inv[j] = recip_rn(s[j]);
  }
  // requantize, store codes, form the residual
  float ea[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < RPS; ++r) {
    uint32_t yb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float code = quantize<MODE>(h[r][j], s[j], inv[j], yb[j]);
      h[r][j] = residual<MODE>(h[r][j], code, s[j]);
      ea[j] = fmaxf(ea[j], fabsf(h[r][j]));
    }
    if (colok)
      *reinterpret_cast<uint32_t*>(p.h_out + mb + (int64_t)(r0 + r) * p.V + c0) =
          pack_low_bytes(yb[0], yb[1], yb[2], yb[3]);
  }
  if (ks == 0 && colok) *reinterpret_cast<float4*>(p.scale_out + vb + c0) = make_float4(s[0], s[1], s[2], s[3]);

  if constexpr (RES == kResInt8) {
#pragma unroll
    for (int j = 0; j < 4; ++j) red[3][ks][lc + j] = ea[j];
    __syncthreads();
    float es[4], inv_e[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      es[j] = fmaxf(div_small_int(slice_max(red[3], lc + j), p.qmax, p.rqmax), kEps);
      inv_e[j] = recip_rn(es[j]);
    }
    if (colok) {
#pragma unroll
      for (int r = 0; r < RPS; ++r) {
        uint32_t eb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) (void)quantize<MODE>(h[r][j], es[j], inv_e[j], eb[j]);
        *reinterpret_cast<uint32_t*>(static_cast<int8_t*>(p.e_out) + mb + (int64_t)(r0 + r) * p.V + c0) =
            pack_low_bytes(eb[0], eb[1], eb[2], eb[3]);
      }
      if (ks == 0) *reinterpret_cast<float4*>(p.e_scale_out + vb + c0) = make_float4(es[0], es[1], es[2], es[3]);
    }
  } else if (colok) {
#pragma unroll
    for (int r = 0; r < RPS; ++r) {
      const int64_t i = mb + (int64_t)(r0 + r) * p.V + c0;
      if constexpr (RES == kResFp32) {
        *reinterpret_cast<float4*>(static_cast<float*>(p.e_out) + i) = make_float4(h[r][0], h[r][1], h[r][2], h[r][3]);
      } else if constexpr (RES == kResFp16) {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.e_out) + i) =
            make_uint2(f32_to_half_bits(h[r][0]) | (f32_to_half_bits(h[r][1]) << 16),
                       f32_to_half_bits(h[r][2]) | (f32_to_half_bits(h[r][3]) << 16));
      } else {
        *reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(p.e_out) + i) =
            f32x4_to_e5m2x4(h[r][0], h[r][1], h[r][2], h[r][3]);
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
};

template <int K>
__global__ __launch_bounds__(kThreads) void fp32_step_kernel(const Fp32Params p) {
  constexpr int RPS = K / kSlices;
  __shared__ float red[2][kSlices][kCols];
  const int t = threadIdx.x;
  const int cg = t % 32;
  const int ks = t / 32;
  const int vt = blockIdx.x % p.nvt;
  const int w = blockIdx.x / p.nvt;
  const int lc = cg * 4;
  const int c0 = vt * kCols + lc;
  const bool colok = c0 < p.V;
  const int r0 = ks * RPS;
  const int64_t mb = (int64_t)w * K * p.V;
  const int64_t vb = (int64_t)w * p.V;
  const float alpha = p.alpha[w];
  const float beta = p.beta[w];
  float h[RPS][4], kk[RPS], qq[RPS];
  float4 vv = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int r = 0; r < RPS; ++r) {
    kk[r] = p.k[(int64_t)w * K + r0 + r];
    qq[r] = p.q[(int64_t)w * K + r0 + r];
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (colok) x = *reinterpret_cast<const float4*>(p.h_in + mb + (int64_t)(r0 + r) * p.V + c0);
    h[r][0] = x.x * alpha, h[r][1] = x.y * alpha, h[r][2] = x.z * alpha, h[r][3] = x.w * alpha;
  }
  if (colok) vv = *reinterpret_cast<const float4*>(p.v + vb + c0);
  const float vvv[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float acc = h[0][j] * kk[0];
#pragma unroll
    for (int r = 1; r < RPS; ++r) acc = fmaf(h[r][j], kk[r], acc);
    red[0][ks][lc + j] = acc;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float dv = beta * (vvv[j] - slice_tree_sum(red[0], lc + j));
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
      *reinterpret_cast<float4*>(p.h_out + mb + (int64_t)(r0 + r) * p.V + c0) =
          make_float4(h[r][0], h[r][1], h[r][2], h[r][3]);
  }
  __syncthreads();
  if (ks == 0 && colok) {
    float o4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o4[j] = slice_tree_sum(red[1], lc + j);
    *reinterpret_cast<float4*>(p.o + vb + c0) = make_float4(o4[0], o4[1], o4[2], o4[3]);
  }
}

template <int K, int MODE>
int launch_quant(const StepParams& p, int64_t grid, int res_fmt, hipStream_t s) {
  switch (res_fmt) {
    case kResFp32: hipLaunchKernelGGL((quant_step_kernel<K, kResFp32, MODE>), dim3(grid), dim3(kThreads), 0, s, p); break;
    case kResFp16: hipLaunchKernelGGL((quant_step_kernel<K, kResFp16, MODE>), dim3(grid), dim3(kThreads), 0, s, p); break;
    case kResFp8: hipLaunchKernelGGL((quant_step_kernel<K, kResFp8, MODE>), dim3(grid), dim3(kThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((quant_step_kernel<K, kResInt8, MODE>), dim3(grid), dim3(kThreads), 0, s, p); break;
  }
  return check_launch("ck_gdn_quant_step");
}

template <int MODE>
int launch_quant_k(const StepParams& p, int64_t grid, int K, int res_fmt, hipStream_t s) {
  switch (K) {
    case 16: return launch_quant<16, MODE>(p, grid, res_fmt, s);
    case 32: return launch_quant<32, MODE>(p, grid, res_fmt, s);
    case 64: return launch_quant<64, MODE>(p, grid, res_fmt, s);
    default: return launch_quant<128, MODE>(p, grid, res_fmt, s);
  }
}

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
  if (K != 16 && K != 32 && K != 64 && K != 128)
    return fail(CK_EUNSUPPORTED, "K must be one of 16, 32, 64, 128, got %d", K);
  if (V % 4 != 0) return fail(CK_EUNSUPPORTED, "V must be a multiple of 4, got %d", V);
  if (res_fmt < CK_RES_FP32 || res_fmt > CK_RES_INT8) return fail(CK_EINVAL, "unknown residual format %d", res_fmt);
  if (quant_mode != CK_QUANT_FAST && quant_mode != CK_QUANT_EXACT)
    return fail(CK_EINVAL, "quant_mode must be CK_QUANT_FAST or CK_QUANT_EXACT, got %d", quant_mode);
  const int iq = (int)qmax;
  if ((float)iq != qmax || iq < 1 || iq > 127) return fail(CK_EINVAL, "qmax must be an integer in 1..127");
  if (B == 0) return ok();
  if (!h_in || !scale_in || !e_in || !q || !k || !v || !alpha || !beta || !o || !h_out || !scale_out || !e_out)
    return fail(CK_EINVAL, "null pointer argument");
  if (res_fmt == CK_RES_INT8 && (!e_scale_in || !e_scale_out)) return fail(CK_EINVAL, "int8 residual needs e_scale");
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
  p.nvt = (V + kCols - 1) / kCols;
  volatile float one = 1.0f;
  p.qmax = qmax;
  p.rqmax = one / qmax;
  const int64_t grid = (int64_t)B * HV * p.nvt;
  if (grid > 0x7fffffff) return fail(CK_EUNSUPPORTED, "grid too large");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return quant_mode == CK_QUANT_EXACT ? launch_quant_k<kExact>(p, grid, K, res_fmt, s)
                                      : launch_quant_k<kFast>(p, grid, K, res_fmt, s);
}

extern "C" int ck_gdn_fp32_step(const float* h_in, const float* q, const float* k, const float* v,
                                const float* alpha, const float* beta, float* o, float* h_out,
                                int B, int HV, int K, int V, void* stream) {
  using namespace ck;
  using namespace ck::qs;
  if (B < 0 || HV <= 0 || K <= 0 || V <= 0) return fail(CK_EINVAL, "bad sizes B=%d HV=%d K=%d V=%d", B, HV, K, V);
  if (K != 16 && K != 32 && K != 64 && K != 128)
    return fail(CK_EUNSUPPORTED, "K must be one of 16, 32, 64, 128, got %d", K);
  if (V % 4 != 0) return fail(CK_EUNSUPPORTED, "V must be a multiple of 4, got %d", V);
  if (B == 0) return ok();
  if (!h_in || !q || !k || !v || !alpha || !beta || !o || !h_out) return fail(CK_EINVAL, "null pointer argument");
  Fp32Params p{h_in, q, k, v, alpha, beta, o, h_out, V, (V + kCols - 1) / kCols};
  const int64_t grid = (int64_t)B * HV * p.nvt;
  if (grid > 0x7fffffff) return fail(CK_EUNSUPPORTED, "grid too large");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (K) {
    case 16: hipLaunchKernelGGL(fp32_step_kernel<16>, dim3(grid), dim3(kThreads), 0, s, p); break;
    case 32: hipLaunchKernelGGL(fp32_step_kernel<32>, dim3(grid), dim3(kThreads), 0, s, p); break;
    case 64: hipLaunchKernelGGL(fp32_step_kernel<64>, dim3(grid), dim3(kThreads), 0, s, p); break;
    default: hipLaunchKernelGGL(fp32_step_kernel<128>, dim3(grid), dim3(kThreads), 0, s, p); break;
  }
  return check_launch("ck_gdn_fp32_step");
}
