// Slot-level operations on the quantized state pool, for the engine's cache
// management around the decode step: the error-feedback residual is
// per-request state that has to move with the codes and scales when a
// request's state is forked (prefix-cache reuse), checkpointed (speculative
// decoding), swapped out and back (preemption) or released.
//
//   ck_pool_copy_slots:  for each pair i, copy slot src_ids[i] of one pool to
//                        slot dst_ids[i] of another (or the same) pool: state
//                        codes, state scales, residual codes, residual scales.
//   ck_pool_reset_slots: zero those four regions of the listed slots (a fresh
//                        request starts from a zero state and residual).
//
// A slot id outside [1, num_slots) of its pool skips the pair (slot 0 is the
// NULL block). The per-slot regions are contiguous (the host checks it), so a
// pair is four flat byte ranges; each is moved in 16-byte units when its size
// and both bases allow, else in 4-byte units (every region is a multiple of 4
// bytes). HBM-bound: 2 bytes moved per byte of slot copied, 1 per byte reset.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ck_capi_common.h"

namespace ck {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kRegions = 4;  // state codes, state scales, residual codes, residual scales
constexpr int kThreads = 256;
constexpr int kUnitsPerThread = 4;

struct PoolView {
  char* base[kRegions];       // region bases (slot 0)
  int64_t stride[kRegions];   // slot stride in bytes
  int64_t num_slots;
};

struct RegionPlan {
  int64_t bytes[kRegions];    // bytes of one slot in each region
  int vec16[kRegions];        // 1: move 16-byte units
};

// grid: x = chunks of kThreads * kUnitsPerThread units, y = pair, z = region.
__global__ __launch_bounds__(kThreads) void pool_slots_kernel(PoolView src, PoolView dst, RegionPlan plan,
                                                              const int32_t* __restrict__ src_ids,
                                                              const int32_t* __restrict__ dst_ids, int reset) {
  const int pair = (int)blockIdx.y;
  const int reg = (int)blockIdx.z;
  const int64_t d = dst_ids[pair];
  if (d <= 0 || d >= dst.num_slots) return;  // whole workgroup
  int64_t s = 0;
  if (!reset) {
    s = src_ids[pair];
    if (s <= 0 || s >= src.num_slots) return;
  }
  const int64_t bytes = plan.bytes[reg];
  char* out = dst.base[reg] + d * dst.stride[reg];
  const char* in = reset ? nullptr : src.base[reg] + s * src.stride[reg];
  const int64_t first = ((int64_t)blockIdx.x * kUnitsPerThread) * kThreads + threadIdx.x;
  // every load of the thread is issued before its first store: the source and
  // destination may be the same pool, so the compiler could not hoist a load
  // above an earlier store, and one unit at a time would be in flight
  if (plan.vec16[reg]) {
    const int64_t n = bytes >> 4;
    u32x4_t v[kUnitsPerThread];
#pragma unroll
    for (int u = 0; u < kUnitsPerThread; ++u) {
      const int64_t i = first + (int64_t)u * kThreads;
      v[u] = (reset || i >= n) ? u32x4_t{0u, 0u, 0u, 0u}
                               : __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(in) + i);
    }
#pragma unroll
    for (int u = 0; u < kUnitsPerThread; ++u) {
      const int64_t i = first + (int64_t)u * kThreads;
      if (i < n) __builtin_nontemporal_store(v[u], reinterpret_cast<u32x4_t*>(out) + i);
    }
  } else {
    const int64_t n = bytes >> 2;
    uint32_t v[kUnitsPerThread];
#pragma unroll
    for (int u = 0; u < kUnitsPerThread; ++u) {
      const int64_t i = first + (int64_t)u * kThreads;
      v[u] = (reset || i >= n) ? 0u : reinterpret_cast<const uint32_t*>(in)[i];
    }
#pragma unroll
    for (int u = 0; u < kUnitsPerThread; ++u) {
      const int64_t i = first + (int64_t)u * kThreads;
      if (i < n) reinterpret_cast<uint32_t*>(out)[i] = v[u];
    }
  }
}

// Every region in 16-byte units (the usual layout): each region of a slot is
// split into runs of kThreads * kFlatUnits consecutive units (16 KB), and a
// pair's runs are numbered region by region along blockIdx.x, so a workgroup
// lies in one region (its base, stride and length are uniform) and only a
// region's last run is partly empty. Each thread issues all its loads before
// its stores (the source and destination may be the same pool, so the
// compiler could not hoist a load above an earlier store). Loads are
// non-temporal; a copy's stores are ordinary (write-back) stores, a reset's
// non-temporal. Measured on MI355X, 256 random int4 per-head slots of a
// 1025-slot pool (HV=32, K=V=128): copy 83.5 us with non-temporal stores
// against 67.6 us with ordinary ones (6.1 TB/s), reset 42.1 against 43.4 us;
// the earlier layout (32 KB runs over the pair's four regions as one range,
// every unit tested against every region) took 86.2 / 43.0 us.
constexpr int kFlatUnits = 4;
constexpr int64_t kRunUnits = (int64_t)kThreads * kFlatUnits;

struct FlatPlan {
  int64_t units[kRegions];     // 16-byte units of one slot in each region
  int32_t run0[kRegions + 1];  // first run of each region; run0[kRegions] = runs per pair
};

template <bool RESET>
__global__ __launch_bounds__(kThreads) void pool_slots_flat_kernel(PoolView src, PoolView dst, FlatPlan f,
                                                                   const int32_t* __restrict__ src_ids,
                                                                   const int32_t* __restrict__ dst_ids) {
  const int pair = (int)blockIdx.y;
  const int64_t d = dst_ids[pair];
  if (d <= 0 || d >= dst.num_slots) return;  // whole workgroup
  int64_t s = 0;
  if (!RESET) {
    s = src_ids[pair];
    if (s <= 0 || s >= src.num_slots) return;
  }
  const int bx = (int)blockIdx.x;
  const int r = (bx >= f.run0[1]) + (bx >= f.run0[2]) + (bx >= f.run0[3]);
  // uniform selection (a dynamic index into the argument arrays would go
  // through memory)
  const char* ib = r == 0 ? src.base[0] : r == 1 ? src.base[1] : r == 2 ? src.base[2] : src.base[3];
  const int64_t is = r == 0 ? src.stride[0] : r == 1 ? src.stride[1] : r == 2 ? src.stride[2] : src.stride[3];
  char* ob = r == 0 ? dst.base[0] : r == 1 ? dst.base[1] : r == 2 ? dst.base[2] : dst.base[3];
  const int64_t os = r == 0 ? dst.stride[0] : r == 1 ? dst.stride[1] : r == 2 ? dst.stride[2] : dst.stride[3];
  const int64_t n = r == 0 ? f.units[0] : r == 1 ? f.units[1] : r == 2 ? f.units[2] : f.units[3];
  const int run = bx - (r == 0 ? f.run0[0] : r == 1 ? f.run0[1] : r == 2 ? f.run0[2] : f.run0[3]);
  const u32x4_t* in = reinterpret_cast<const u32x4_t*>(ib + s * is);
  u32x4_t* out = reinterpret_cast<u32x4_t*>(ob + d * os);
  const int64_t first = (int64_t)run * kRunUnits + threadIdx.x;
  u32x4_t v[kFlatUnits];
#pragma unroll
  for (int u = 0; u < kFlatUnits; ++u) {
    const int64_t i = first + (int64_t)u * kThreads;
    v[u] = (RESET || i >= n) ? u32x4_t{0u, 0u, 0u, 0u} : __builtin_nontemporal_load(in + i);
  }
#pragma unroll
  for (int u = 0; u < kFlatUnits; ++u) {
    const int64_t i = first + (int64_t)u * kThreads;
    if (i < n) {
      if (RESET) {
        __builtin_nontemporal_store(v[u], out + i);
      } else {
        out[i] = v[u];
      }
    }
  }
}

// Validates one pool and fills its view; element strides are per slot.
int make_view(const char* name, int8_t* state, int64_t stride_state, float* sscale, int64_t stride_sscale,
              int8_t* resid, int64_t stride_resid, float* rscale, int64_t stride_rscale, int64_t num_slots,
              const RegionPlan& plan, PoolView* v) {
  if (!state || !sscale || !resid || !rscale) return fail(CK_EINVAL, "%s: null pointer argument", name);
  if (num_slots <= 0) return fail(CK_EINVAL, "%s: num_slots must be positive", name);
  const int64_t strides[kRegions] = {stride_state, stride_sscale * 4, stride_resid, stride_rscale * 4};
  char* bases[kRegions] = {reinterpret_cast<char*>(state), reinterpret_cast<char*>(sscale),
                           reinterpret_cast<char*>(resid), reinterpret_cast<char*>(rscale)};
  for (int r = 0; r < kRegions; ++r) {
    if (strides[r] < plan.bytes[r])
      return fail(CK_EINVAL, "%s: slot stride of region %d (%lld B) is smaller than a slot (%lld B)", name, r,
                  (long long)strides[r], (long long)plan.bytes[r]);
    if ((reinterpret_cast<uintptr_t>(bases[r]) | (uintptr_t)strides[r]) & 3)
      return fail(CK_EINVAL, "%s: region %d is not 4-byte aligned", name, r);
    v->base[r] = bases[r];
    v->stride[r] = strides[r];
  }
  v->num_slots = num_slots;
  return CK_OK;
}

int launch(const PoolView& src, const PoolView& dst, RegionPlan plan, const int32_t* src_ids, const int32_t* dst_ids,
           int n, int reset, void* stream, const char* what) {
  int64_t max_units = 0;
  for (int r = 0; r < kRegions; ++r) {
    const uintptr_t align = (uintptr_t)dst.base[r] | (uintptr_t)dst.stride[r] | (uintptr_t)plan.bytes[r] |
                            (reset ? 0 : ((uintptr_t)src.base[r] | (uintptr_t)src.stride[r]));
    plan.vec16[r] = (align & 15) == 0;
    const int64_t units = plan.bytes[r] >> (plan.vec16[r] ? 4 : 2);
    max_units = units > max_units ? units : max_units;
  }
  if (n == 0 || max_units == 0) return ok();
  if (plan.vec16[0] && plan.vec16[1] && plan.vec16[2] && plan.vec16[3]) {
    FlatPlan f;
    int64_t runs = 0;
    for (int r = 0; r < kRegions; ++r) {
      f.units[r] = plan.bytes[r] >> 4;
      f.run0[r] = (int32_t)(runs < 0x7fffffff ? runs : 0x7fffffff);
      runs += (f.units[r] + kRunUnits - 1) / kRunUnits;
    }
    if (runs > 0x7fffffff || n > 65535) return fail(CK_EUNSUPPORTED, "%s: too many slots or too large a slot", what);
    f.run0[kRegions] = (int32_t)runs;
    const dim3 grid((unsigned)runs, (unsigned)n);
    if (reset) {
      hipLaunchKernelGGL(pool_slots_flat_kernel<true>, grid, dim3(kThreads), 0, reinterpret_cast<hipStream_t>(stream),
                         src, dst, f, src_ids, dst_ids);
    } else {
      hipLaunchKernelGGL(pool_slots_flat_kernel<false>, grid, dim3(kThreads), 0,
                         reinterpret_cast<hipStream_t>(stream), src, dst, f, src_ids, dst_ids);
    }
    return check_launch(what);
  }
  const int64_t chunks = (max_units + (int64_t)kThreads * kUnitsPerThread - 1) / ((int64_t)kThreads * kUnitsPerThread);
  if (chunks > 0x7fffffff || n > 65535) return fail(CK_EUNSUPPORTED, "%s: too many slots or too large a slot", what);
  hipLaunchKernelGGL(pool_slots_kernel, dim3((unsigned)chunks, (unsigned)n, kRegions), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), src, dst, plan, src_ids, dst_ids, reset);
  return check_launch(what);
}

int plan_regions(int HV, int V, int K, int resid_fmt, int rscale_mode, RegionPlan* plan) {
  if (HV <= 0 || V <= 0 || K <= 0) return fail(CK_EINVAL, "bad sizes HV=%d V=%d K=%d", HV, V, K);
  if (resid_fmt != CK_RESID_INT8 && resid_fmt != CK_RESID_INT4)
    return fail(CK_EINVAL, "resid_fmt must be CK_RESID_INT8 or CK_RESID_INT4, got %d", resid_fmt);
  if (rscale_mode != CK_RSCALE_PER_ROW && rscale_mode != CK_RSCALE_PER_HEAD)
    return fail(CK_EINVAL, "rscale_mode must be CK_RSCALE_PER_ROW or CK_RSCALE_PER_HEAD, got %d", rscale_mode);
  if (K % 8 != 0) return fail(CK_EINVAL, "K must be a multiple of 8, got %d", K);
  const int64_t rows = (int64_t)HV * V;
  plan->bytes[0] = rows * K;
  plan->bytes[1] = rows * 4;
  plan->bytes[2] = resid_fmt == CK_RESID_INT4 ? rows * (K / 2) : rows * K;
  plan->bytes[3] = rscale_mode == CK_RSCALE_PER_HEAD ? (int64_t)HV * 4 : rows * 4;
  return CK_OK;
}

}  // namespace
}  // namespace ck

extern "C" int ck_pool_copy_slots(const int8_t* src_state, int64_t src_stride_state, const float* src_sscale,
                                  int64_t src_stride_sscale, const int8_t* src_resid, int64_t src_stride_resid,
                                  const float* src_rscale, int64_t src_stride_rscale, int64_t src_num_slots,
                                  int8_t* dst_state, int64_t dst_stride_state, float* dst_sscale,
                                  int64_t dst_stride_sscale, int8_t* dst_resid, int64_t dst_stride_resid,
                                  float* dst_rscale, int64_t dst_stride_rscale, int64_t dst_num_slots,
                                  const int32_t* src_ids, const int32_t* dst_ids, int n,
                                  int HV, int V, int K, int resid_fmt, int rscale_mode, void* stream) {
  using namespace ck;
  RegionPlan plan{};
  int st = plan_regions(HV, V, K, resid_fmt, rscale_mode, &plan);
  if (st != CK_OK) return st;
  if (n < 0) return fail(CK_EINVAL, "n must be non-negative, got %d", n);
  if (n > 0 && (!src_ids || !dst_ids)) return fail(CK_EINVAL, "null slot id array");
  PoolView src{}, dst{};
  st = make_view("source pool", const_cast<int8_t*>(src_state), src_stride_state, const_cast<float*>(src_sscale),
                 src_stride_sscale, const_cast<int8_t*>(src_resid), src_stride_resid,
                 const_cast<float*>(src_rscale), src_stride_rscale, src_num_slots, plan, &src);
  if (st != CK_OK) return st;
  st = make_view("destination pool", dst_state, dst_stride_state, dst_sscale, dst_stride_sscale, dst_resid,
                 dst_stride_resid, dst_rscale, dst_stride_rscale, dst_num_slots, plan, &dst);
  if (st != CK_OK) return st;
  return launch(src, dst, plan, src_ids, dst_ids, n, 0, stream, "ck_pool_copy_slots");
}

extern "C" int ck_pool_reset_slots(int8_t* state, int64_t stride_state, float* sscale, int64_t stride_sscale,
                                   int8_t* resid, int64_t stride_resid, float* rscale, int64_t stride_rscale,
                                   int64_t num_slots, const int32_t* ids, int n,
                                   int HV, int V, int K, int resid_fmt, int rscale_mode, void* stream) {
  using namespace ck;
  RegionPlan plan{};
  int st = plan_regions(HV, V, K, resid_fmt, rscale_mode, &plan);
  if (st != CK_OK) return st;
  if (n < 0) return fail(CK_EINVAL, "n must be non-negative, got %d", n);
  if (n > 0 && !ids) return fail(CK_EINVAL, "null slot id array");
  PoolView dst{};
  st = make_view("pool", state, stride_state, sscale, stride_sscale, resid, stride_resid, rscale, stride_rscale,
                 num_slots, plan, &dst);
  if (st != CK_OK) return st;
  return launch(dst, dst, plan, ids, ids, n, 1, stream, "ck_pool_reset_slots");
}
