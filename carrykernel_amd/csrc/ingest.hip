// State ingest: quantize a float state into the int8 pool.
//   ck_quantize_rows: rows of K (vLLM [.., V, K] layout), one scale per row,
//     init_quantized_state semantics (vllm_integration/quantized_packed_decode.py:347-351):
//     scale = max(amax, 1e-12) / qmax, code = clamp(rne(x / scale), +-qmax).
//   ck_quantize_cols: [K, V] matrices, one scale per V-column (amax over K),
//     per_v_channel_quantize semantics (statequant/kernel.py:99-113).
// Both use IEEE divisions, so the codes equal torch.round(x / scale).
#include <hip/hip_runtime.h>

#include "ck_capi_common.h"
#include "ck_device.h"

namespace ck {
namespace {

// One wavefront per row; lanes stride over K.
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
  const float s = fmaxf(am, kEps) / qmax;
  for (int j = lane; j < K; j += 64) {
    const float c = fminf(fmaxf(rintf(load_act(x, base + j, dtype) / s), -qmax), qmax);
    codes[row * K + j] = (int8_t)(int)c;
  }
  if (lane == 0) scale[row] = s;
}

// One thread per (matrix, V-column); consecutive threads take consecutive
// columns so every K-row access is coalesced.
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
  if (!valid_dtype(x_dtype)) return fail(CK_EINVAL, "unsupported dtype code %d", x_dtype);
  if (!(qmax >= 1.0f && qmax <= 127.0f)) return fail(CK_EINVAL, "qmax must be in [1, 127]");
  if (rows == 0) return ok();
  if (!x || !codes || !scale) return fail(CK_EINVAL, "null pointer argument");
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
  const int64_t grid = (M * V + 255) / 256;
  if (grid > 0x7fffffff) return fail(CK_EUNSUPPORTED, "too many columns");
  hipLaunchKernelGGL(quantize_cols_kernel, dim3((unsigned)grid), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     x, M, K, V, qmax, codes, scale);
  return check_launch("ck_quantize_cols");
}
