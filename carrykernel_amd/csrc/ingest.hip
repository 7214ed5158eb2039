// State ingest: quantize a float state into the int8 pool.
//   ck_quantize_rows: rows of K (vLLM [.., V, K] layout), one scale per row,
//     init_quantized_state semantics (vllm_integration/quantized_packed_decode.py:347-351):
//     scale = max(amax, 1e-12) / qmax, code = clamp(rne(x / scale), +-qmax),
//     evaluated in the precision of x as torch evaluates that expression on a
//     tensor of x's dtype: fp32 and float64 arithmetic as such; for bf16 and
//     fp16 every operation is computed in fp32 and rounded (to nearest even)
//     to x's dtype, so the scale is the 16-bit value RN16(RN(max(amax, RN16(
//     1e-12)) / qmax)) and the quotient RN16(RN(x / scale)) is rounded to an
//     integer from there (it can reach qmax + 1 in bf16, where the clamp then
//     binds). A float64 scale is stored rounded to fp32.
//   ck_quantize_cols: [K, V] matrices, one scale per V-column (amax over K),
//     per_v_channel_quantize semantics (statequant/kernel.py:99-113).
// Both divide correctly rounded (IEEE division, or the reciprocal with
// Markstein's correction), so the codes equal torch.round(x / scale).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "ck_capi_common.h"
#include "ck_device.h"
#include "ck_quant.h"

namespace ck {
namespace {

// x rounded to nearest even to the 16-bit dtype DT and back to fp32 (fp32:
// unchanged); subnormal fp16 results are kept (the conversion honours fp16
// denormals), values past the largest finite fp16 become inf.
template <int DT>
__device__ __forceinline__ float round16(float x) {
  if constexpr (DT == kBF16) {
    return bf16_to_f32(f32_to_bf16_rne(x));
  } else if constexpr (DT == kF16) {
    return (float)(_Float16)x;
  } else {
    return x;
  }
}

__device__ __forceinline__ float round16_rt(int dt, float x) {
  return dt == kBF16 ? round16<kBF16>(x) : dt == kF16 ? round16<kF16>(x) : x;
}

// RN(t / s) from inv = RN(1 / s) by Markstein's correction (the EXACT quotient
// of ck_quant.h, before its rounding to an integer).
__device__ __forceinline__ float quantize_quotient(float t, float s, float inv) {
  const float q0 = t * inv;
  const float r = fmaf(-q0, s, t);
  return fmaf(r, inv, q0);
}

// Rows of K = 16 * LPR (K <= 256), 16-byte aligned: a lane owns 16 consecutive
// elements of a row (vector loads, one 16-byte store of codes), the LPR lanes
// of a row take the row amax by DPP, and each element is divided by the row
// scale through RN(1/s) with Markstein's correction (ck_quant.h, EXACT mode),
// which is the correctly rounded quotient. |x / s| <= qmax (1 + 2^-23) < qmax
// + 1/2 since s >= RN(amax / qmax), so no code exceeds qmax and the clamp of
// the reference never binds. Waves stride over row groups. A lane's 64 (fp32)
// or 32 (16-bit) bytes are read in 16-byte loads, so one load instruction
// covers part of every line the wave touches: the loads are cached (the next
// instruction's bytes are then L2 hits), which measured 1.3x faster than
// non-temporal loads here.
template <int LPR, int DT>
__global__ __launch_bounds__(256) void quantize_rows16_kernel(const char* __restrict__ x, int64_t stride_row_bytes,
                                                              int64_t rows, float qmax, int8_t* __restrict__ codes,
                                                              float* __restrict__ scale) {
  constexpr int RPW = 64 / LPR;  // rows per wave
  constexpr int K = 16 * LPR;
  const int lane = threadIdx.x & 63;
  const int c = lane % LPR;
  const int g = lane / LPR;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  for (int64_t r0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW; r0 < rows; r0 += nwaves * RPW) {
    const int64_t row = r0 + g;
    const bool valid = row < rows;
    const char* p = x + (valid ? row : rows - 1) * stride_row_bytes + c * 16 * (DT == kF32 ? 4 : 2);
    float v[16];
    if constexpr (DT == kF32) {
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const u32x4 w = reinterpret_cast<const u32x4*>(p)[h];
        v[4 * h] = __uint_as_float(w.x), v[4 * h + 1] = __uint_as_float(w.y);
        v[4 * h + 2] = __uint_as_float(w.z), v[4 * h + 3] = __uint_as_float(w.w);
      }
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const u32x4 w = reinterpret_cast<const u32x4*>(p)[h];
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[8 * h + 2 * i] = act_decode<DT>(ws[i] & 0xffffu);
          v[8 * h + 2 * i + 1] = act_decode<DT>(ws[i] >> 16);
        }
      }
    }
    float am = fabsf(v[0]);
#pragma unroll
    for (int j = 1; j < 16; ++j) am = fmaxf(am, fabsf(v[j]));
    am = group_max<LPR>(am);
    uint32_t yb[16];
    float s;
    if constexpr (DT == kF32) {
      s = fmaxf(am, kEps) / qmax;
      const float inv = recip_rn(s);
#pragma unroll
      for (int j = 0; j < 16; ++j) (void)quantize<kExact>(v[j], s, inv, yb[j]);
    } else {
      // in x's precision: RN16 after every fp32 operation (see the header)
      s = round16<DT>(fmaxf(am, round16<DT>(kEps)) / qmax);
      if (s > 0.0f) {
        const float inv = recip_rn(s);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float q = round16<DT>(quantize_quotient(v[j], s, inv));
          yb[j] = __float_as_uint(fminf(fmaxf(rintf(q), -qmax), qmax) + kMagic);
        }
      } else {
        // fp16 only (RN16(1e-12) = 0): the row's scale rounded to 0, so x / 0
        // is +-inf (clamped to +-qmax) for x != 0 and NaN for x = 0, which
        // the reference's int8 conversion turns into 0
#pragma unroll
        for (int j = 0; j < 16; ++j)
          yb[j] = __float_as_uint((v[j] > 0.0f ? qmax : v[j] < 0.0f ? -qmax : 0.0f) + kMagic);
      }
    }
    if (valid) {
      __builtin_nontemporal_store(u32x4{pack_low_bytes(yb[0], yb[1], yb[2], yb[3]),
                                        pack_low_bytes(yb[4], yb[5], yb[6], yb[7]),
                                        pack_low_bytes(yb[8], yb[9], yb[10], yb[11]),
                                        pack_low_bytes(yb[12], yb[13], yb[14], yb[15])},
                                  reinterpret_cast<u32x4*>(codes + row * K + c * 16));
      if (c == 0) scale[row] = s;
    }
  }
}

template <int LPR>
void launch_rows16(const void* x, int dtype, int64_t stride_row, int64_t rows, float qmax, int8_t* codes,
                   float* scale, hipStream_t stream) {
  constexpr int RPW = 64 / LPR;
  const int64_t waves = (rows + RPW - 1) / RPW;
  const int64_t grid = std::min<int64_t>((waves + 3) / 4, 256 * 32);
  const int esz = dtype == kF32 ? 4 : 2;
  const char* xb = static_cast<const char*>(x);
  if (dtype == kF32)
    hipLaunchKernelGGL((quantize_rows16_kernel<LPR, kF32>), dim3((unsigned)grid), dim3(256), 0, stream, xb,
                       stride_row * esz, rows, qmax, codes, scale);
  else if (dtype == kBF16)
    hipLaunchKernelGGL((quantize_rows16_kernel<LPR, kBF16>), dim3((unsigned)grid), dim3(256), 0, stream, xb,
                       stride_row * esz, rows, qmax, codes, scale);
  else
    hipLaunchKernelGGL((quantize_rows16_kernel<LPR, kF16>), dim3((unsigned)grid), dim3(256), 0, stream, xb,
                       stride_row * esz, rows, qmax, codes, scale);
}

// Any K, any alignment: one wavefront per row; lanes stride over K. 16-bit
// dtypes in their own precision (RN16 after each fp32 operation).
__global__ __launch_bounds__(256) void quantize_rows_kernel(const void* __restrict__ x, int dtype, int64_t stride_row,
                                                            int64_t rows, int K, float qmax,
                                                            int8_t* __restrict__ codes, float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wavefront exits together
  const int64_t base = row * stride_row;
  float am = 0.0f;
  for (int j = lane; j < K; j += 64) am = fmaxf(am, fabsf(load_act(x, base + j, dtype)));
  am = wave_max(am);
  const float s = round16_rt(dtype, fmaxf(am, round16_rt(dtype, kEps)) / qmax);
  for (int j = lane; j < K; j += 64) {
    // IEEE division: an fp16 scale that rounded to 0 gives +-inf (clamped to
    // +-qmax) for x != 0 and NaN for x = 0, which the int8 conversion of the
    // reference turns into 0
    const float q = round16_rt(dtype, load_act(x, base + j, dtype) / s);
    const float c = q != q ? 0.0f : fminf(fmaxf(rintf(q), -qmax), qmax);
    codes[row * K + j] = (int8_t)(int)c;
  }
  if (lane == 0) scale[row] = s;
}

// float64 rows (any K, alignment of a double): one wavefront per row, the
// arithmetic in float64 as torch does for a float64 h0; the scale is stored
// rounded to fp32 (the pool's scale dtype), the codes use the float64 scale.
__global__ __launch_bounds__(256) void quantize_rows_f64_kernel(const double* __restrict__ x, int64_t stride_row,
                                                                int64_t rows, int K, double qmax,
                                                                int8_t* __restrict__ codes, float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wavefront exits together
  const double* xr = x + row * stride_row;
  double am = 0.0;
  for (int j = lane; j < K; j += 64) am = fmax(am, fabs(xr[j]));
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) am = fmax(am, __shfl_xor(am, m, 64));
  const double s = fmax(am, 1e-12) / qmax;
  for (int j = lane; j < K; j += 64) codes[row * K + j] = (int8_t)(int)fmin(fmax(rint(xr[j] / s), -qmax), qmax);
  if (lane == 0) scale[row] = (float)s;
}

// [M, K, V] matrices with K in {16, 32, 64, 128, 256}, V % 4 == 0, 16-byte aligned:
// a lane owns 4 consecutive columns over K/8 rows (its whole slice stays in
// registers, no second read), lane = column group * 8 + K-slice, so one load
// instruction reads 8 rows of 128 contiguous bytes; the column amax combines
// the 8 K-slice lanes by DPP, the division is the exact reciprocal form of
// quantize_rows16_kernel, and each row's 4 codes go out as one dword. A
// workgroup of 4 waves covers 128 columns of one matrix.
template <int K>
__global__ __launch_bounds__(256) void quantize_cols4_kernel(const float* __restrict__ x, int V, float qmax,
                                                             int8_t* __restrict__ codes, float* __restrict__ scale) {
  constexpr int R = K / 8;  // rows per lane
  const int lane = threadIdx.x & 63;
  const int kc = lane & 7;
  const int col0 = (int)blockIdx.x * 128 + (int)(threadIdx.x >> 6) * 32 + (lane >> 3) * 4;
  const int64_t m = blockIdx.y;
  const bool valid = col0 < V;
  const int col = valid ? col0 : V - 4;  // re-read the last group (no store)
  const float* xm = x + m * K * V + (int64_t)(kc * R) * V + col;
  float v[R][4];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const float4 f = *reinterpret_cast<const float4*>(xm + (int64_t)j * V);
    v[j][0] = f.x, v[j][1] = f.y, v[j][2] = f.z, v[j][3] = f.w;
  }
  float s[4], inv[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float am = fabsf(v[0][c]);
#pragma unroll
    for (int j = 1; j < R; ++j) am = fmaxf(am, fabsf(v[j][c]));
    am = group_max<8>(am);
    s[c] = fmaxf(am, kEps) / qmax;
    inv[c] = recip_rn(s[c]);
  }
  if (!valid) return;
  int8_t* cm = codes + m * K * V + (int64_t)(kc * R) * V + col;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    uint32_t yb[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) (void)quantize<kExact>(v[j][c], s[c], inv[c], yb[c]);
    *reinterpret_cast<uint32_t*>(cm + (int64_t)j * V) = pack_low_bytes(yb[0], yb[1], yb[2], yb[3]);
  }
  if (kc == 0) *reinterpret_cast<float4*>(scale + m * V + col) = make_float4(s[0], s[1], s[2], s[3]);
}

// Any shape: one thread per (matrix, V-column); consecutive threads take
// consecutive columns so every K-row access is coalesced.
__global__ __launch_bounds__(256) void quantize_cols_kernel(const float* __restrict__ x, int64_t M, int K, int V,
                                                            float qmax, int8_t* __restrict__ codes,
                                                            float* __restrict__ scale) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= M * V) return;
  const int64_t m = t / V;
  const int c = (int)(t % V);
  const float* xm = x + m * K * V + c;
  float am = 0.0f;
  for (int j = 0; j < K; ++j) am = fmaxf(am, fabsf(xm[(int64_t)j * V]));
  const float s = fmaxf(am, kEps) / qmax;
  int8_t* cm = codes + m * K * V + c;
  for (int j = 0; j < K; ++j) {
    const float q = fminf(fmaxf(rintf(xm[(int64_t)j * V] / s), -qmax), qmax);
    cm[(int64_t)j * V] = (int8_t)(int)q;
  }
  scale[m * V + c] = s;
}

}  // namespace
}  // namespace ck

extern "C" int ck_quantize_rows(const void* x, int x_dtype, int64_t stride_row, int64_t rows, int K, float qmax,
                                int8_t* codes, float* scale, void* stream) {
  using namespace ck;
  if (rows < 0 || K <= 0 || stride_row < K) return fail(CK_EINVAL, "bad sizes rows=%lld K=%d", (long long)rows, K);
  if (!valid_dtype(x_dtype) && x_dtype != CK_DTYPE_F64) return fail(CK_EINVAL, "unsupported dtype code %d", x_dtype);
  if (!(qmax >= 1.0f && qmax <= 127.0f)) return fail(CK_EINVAL, "qmax must be in [1, 127]");
  if (rows == 0) return ok();
  if (!x || !codes || !scale) return fail(CK_EINVAL, "null pointer argument");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (x_dtype == CK_DTYPE_F64) {
    if (reinterpret_cast<uintptr_t>(x) & 7) return fail(CK_EINVAL, "float64 rows must be 8-byte aligned");
    const int64_t grid = (rows + 3) / 4;
    if (grid > 0x7fffffff) return fail(CK_EUNSUPPORTED, "too many rows");
    hipLaunchKernelGGL(quantize_rows_f64_kernel, dim3((unsigned)grid), dim3(256), 0, s, static_cast<const double*>(x),
                       stride_row, rows, K, (double)qmax, codes, scale);
    return check_launch("ck_quantize_rows");
  }
  const int esz = x_dtype == kF32 ? 4 : 2;
  const bool aligned = ((reinterpret_cast<uintptr_t>(x) | (uintptr_t)(stride_row * esz) |
                         reinterpret_cast<uintptr_t>(codes)) & 15) == 0;
  if (aligned && (K == 16 || K == 32 || K == 64 || K == 128 || K == 256)) {
    switch (K) {
      case 16: launch_rows16<1>(x, x_dtype, stride_row, rows, qmax, codes, scale, s); break;
      case 32: launch_rows16<2>(x, x_dtype, stride_row, rows, qmax, codes, scale, s); break;
      case 64: launch_rows16<4>(x, x_dtype, stride_row, rows, qmax, codes, scale, s); break;
      case 128: launch_rows16<8>(x, x_dtype, stride_row, rows, qmax, codes, scale, s); break;
      default: launch_rows16<16>(x, x_dtype, stride_row, rows, qmax, codes, scale, s); break;
    }
    return check_launch("ck_quantize_rows");
  }
  const int64_t grid = (rows + 3) / 4;
  if (grid > 0x7fffffff) return fail(CK_EUNSUPPORTED, "too many rows");
  hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)grid), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     x, x_dtype, stride_row, rows, K, qmax, codes, scale);
  return check_launch("ck_quantize_rows");
}

extern "C" int ck_quantize_cols(const float* x, int64_t M, int K, int V, float qmax, int8_t* codes, float* scale,
                                void* stream) {
  using namespace ck;
  if (M < 0 || K <= 0 || V <= 0) return fail(CK_EINVAL, "bad sizes M=%lld K=%d V=%d", (long long)M, K, V);
  if (!(qmax >= 1.0f && qmax <= 127.0f)) return fail(CK_EINVAL, "qmax must be in [1, 127]");
  if (M == 0) return ok();
  if (!x || !codes || !scale) return fail(CK_EINVAL, "null pointer argument");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool aligned = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(codes) |
                         reinterpret_cast<uintptr_t>(scale)) & 15) == 0;
  if (aligned && V % 4 == 0 && M <= 65535 && (K == 16 || K == 32 || K == 64 || K == 128 || K == 256)) {
    const dim3 grid((unsigned)((V + 127) / 128), (unsigned)M);
    switch (K) {
      case 16: hipLaunchKernelGGL(quantize_cols4_kernel<16>, grid, dim3(256), 0, s, x, V, qmax, codes, scale); break;
      case 32: hipLaunchKernelGGL(quantize_cols4_kernel<32>, grid, dim3(256), 0, s, x, V, qmax, codes, scale); break;
      case 64: hipLaunchKernelGGL(quantize_cols4_kernel<64>, grid, dim3(256), 0, s, x, V, qmax, codes, scale); break;
      case 128: hipLaunchKernelGGL(quantize_cols4_kernel<128>, grid, dim3(256), 0, s, x, V, qmax, codes, scale); break;
      default: hipLaunchKernelGGL(quantize_cols4_kernel<256>, grid, dim3(256), 0, s, x, V, qmax, codes, scale); break;
    }
    return check_launch("ck_quantize_cols");
  }
  const int64_t grid = (M * V + 255) / 256;
  if (grid > 0x7fffffff) return fail(CK_EUNSUPPORTED, "too many columns");
  hipLaunchKernelGGL(quantize_cols_kernel, dim3((unsigned)grid), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     x, M, K, V, qmax, codes, scale);
  return check_launch("ck_quantize_cols");
}
