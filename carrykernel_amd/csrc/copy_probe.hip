// Streaming device copy used as the measured HBM ceiling next to the decode's
// spec-sheet roofline. The reference measures its peak with a device-to-device
// copy (experiments/cuda_bench.py:39-60); this kernel is the best copy found
// on gfx950 for the byte counts of the decode steps: one 16-byte
// non-temporal load and store per lane per iteration, grid-stride, 512
// threads per workgroup.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "ck_capi_common.h"

namespace ck {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(512) void hbm_copy_kernel(const u32x4_t* __restrict__ src, u32x4_t* __restrict__ dst,
                                                       int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

}  // namespace
}  // namespace ck

extern "C" int ck_hbm_copy(const void* src, void* dst, int64_t bytes, int grid, void* stream) {
  using namespace ck;
  if (bytes < 0 || (bytes & 15)) return fail(CK_EINVAL, "bytes must be a non-negative multiple of 16, got %lld",
                                             (long long)bytes);
  if (grid < 0 || grid > (1 << 20)) return fail(CK_EINVAL, "grid must be in [0, 2^20], got %d", grid);
  if (bytes == 0) return ok();
  if (!src || !dst) return fail(CK_EINVAL, "null pointer argument");
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15)
    return fail(CK_EINVAL, "src and dst must be 16-byte aligned");
  const int64_t n = bytes / 16;
  const int64_t need = (n + 511) / 512;
  const int g = (int)(grid == 0 ? (need < 4096 ? need : 4096) : (need < grid ? need : grid));
  hipLaunchKernelGGL(hbm_copy_kernel, dim3((unsigned)g), dim3(512), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const u32x4_t*>(src), static_cast<u32x4_t*>(dst), n);
  return check_launch("ck_hbm_copy");
}
