// C ABI entry point of the vLLM-layout fused decode: argument validation and
// dispatch to the per-K instantiations (packed_decode_k*.hip). The kernels and
// their design are in packed_decode_impl.h.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdlib>
#include <mutex>

#include "packed_decode_masked.h"

namespace ck {
namespace pd {

int launch_masked(const PackedParams& p, int B, int resid_fmt, int per_head, int mode, int access,
                  hipStream_t stream) {
  if (p.K <= 16) return launch_masked_k<16>(p, B, resid_fmt, per_head, mode, access, stream);
  if (p.K <= 32) return launch_masked_k<32>(p, B, resid_fmt, per_head, mode, access, stream);
  if (p.K <= 64) return launch_masked_k<64>(p, B, resid_fmt, per_head, mode, access, stream);
  if (p.K <= 128) return launch_masked_k<128>(p, B, resid_fmt, per_head, mode, access, stream);
  if (p.K <= 256) return launch_masked_k<256>(p, B, resid_fmt, per_head, mode, access, stream);
  if (p.K <= 512) return launch_masked_k<512>(p, B, resid_fmt, per_head, mode, access, stream);
  return launch_masked_k<1024>(p, B, resid_fmt, per_head, mode, access, stream);
}

namespace {
std::atomic<int64_t> g_max_items{0};
std::once_flag g_max_items_env;

// CARRYKERNEL_MAX_ITEMS_PER_LAUNCH, read on the first launch (not at every
// call: getenv can race a setenv of another thread)
void read_max_items_env() {
  std::call_once(g_max_items_env, [] {
    if (const char* e = getenv("CARRYKERNEL_MAX_ITEMS_PER_LAUNCH")) {
      const long long v = atoll(e);
      if (v > 0) g_max_items.store(v, std::memory_order_relaxed);
    }
  });
}
}  // namespace

int64_t max_items_override() {
  read_max_items_env();
  return g_max_items.load(std::memory_order_relaxed);
}

namespace {
std::atomic<int> g_decode_kernel{kDecodeKernelAuto};
std::once_flag g_decode_kernel_env;

// CARRYKERNEL_DECODE_KERNEL (1: persistent, 2: one-item), read on the first
// launch like CARRYKERNEL_MAX_ITEMS_PER_LAUNCH
void read_decode_kernel_env() {
  std::call_once(g_decode_kernel_env, [] {
    if (const char* e = getenv("CARRYKERNEL_DECODE_KERNEL")) {
      const int v = atoi(e);
      if (v == kDecodeKernelPersistent || v == kDecodeKernelOneItem) g_decode_kernel.store(v, std::memory_order_relaxed);
    }
  });
}
}  // namespace

int decode_kernel_override() {
  read_decode_kernel_env();
  return g_decode_kernel.load(std::memory_order_relaxed);
}

int resident_workgroups(const void* fn, int block, int* per_cu_out) {
  static std::mutex mu;
  struct Entry {
    const void* fn;
    int device;
    int block;
    int n;
    int per_cu;
  };
  static Entry cache[512];
  static int ncache = 0;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return -1;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < ncache; ++i)
    if (cache[i].fn == fn && cache[i].device == device && cache[i].block == block) {
      if (per_cu_out) *per_cu_out = cache[i].per_cu;
      return cache[i].n;
    }
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, block, 0) != hipSuccess || per_cu <= 0) return -1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0) return -1;
  const int n = per_cu * cus;
  if (ncache < 512) cache[ncache++] = {fn, device, block, n, per_cu};
  if (per_cu_out) *per_cu_out = per_cu;
  return n;
}

}  // namespace pd
}  // namespace ck

#if CK_TIMELINE
static void* g_timeline = nullptr;
#endif

// Shared body of ck_gdn_packed_decode (dst_indices == NULL: in place) and
// ck_gdn_packed_decode_to.
static int packed_decode_impl(const void* mixed_qkv, int qkv_dtype, int64_t stride_qkv_tok,
                              const void* a, int a_dtype, int64_t stride_a_tok,
                              const void* b, int b_dtype, int64_t stride_b_tok,
                              const void* A_log, int A_log_dtype,
                              const void* dt_bias, int dt_bias_dtype,
                              float scale,
                              int8_t* state_codes, int64_t stride_state_slot,
                              float* state_scale, int64_t stride_sscale_slot,
                              int8_t* resid_codes, int64_t stride_resid_slot,
                              float* resid_scale, int64_t stride_rscale_slot,
                              void* out, int out_dtype,
                              const int32_t* ssm_state_indices, int64_t stride_indices,
                              const int32_t* dst_indices, int64_t stride_dst_indices,
                              int64_t num_slots,
                              int B, int H, int HV, int K, int V,
                              int use_qk_l2norm, int resid_fmt, int rscale_mode,
                              int state_bits, int quant_mode,
                              void* stream) {
  using namespace ck;
  using namespace ck::pd;
  if (B < 0 || H <= 0 || HV <= 0 || K <= 0 || V <= 0)
    return fail(CK_EINVAL, "bad sizes B=%d H=%d HV=%d K=%d V=%d", B, H, HV, K, V);
  if (HV % H != 0) return fail(CK_EINVAL, "HV (%d) must be a multiple of H (%d)", HV, H);
  if (!valid_dtype(qkv_dtype) || !valid_dtype(a_dtype) || !valid_dtype(b_dtype) || !valid_dtype(A_log_dtype) ||
      !valid_dtype(dt_bias_dtype) || !valid_dtype(out_dtype))
    return fail(CK_EINVAL, "unsupported dtype code");
  if (resid_fmt != CK_RESID_INT8 && resid_fmt != CK_RESID_INT4)
    return fail(CK_EINVAL, "resid_fmt must be CK_RESID_INT8 or CK_RESID_INT4, got %d", resid_fmt);
  if (rscale_mode != CK_RSCALE_PER_ROW && rscale_mode != CK_RSCALE_PER_HEAD)
    return fail(CK_EINVAL, "rscale_mode must be CK_RSCALE_PER_ROW or CK_RSCALE_PER_HEAD, got %d", rscale_mode);
  if (quant_mode != CK_QUANT_FAST && quant_mode != CK_QUANT_EXACT)
    return fail(CK_EINVAL, "quant_mode must be CK_QUANT_FAST or CK_QUANT_EXACT, got %d", quant_mode);
  if (state_bits < 2 || state_bits > 8) return fail(CK_EINVAL, "state_bits must be in 2..8, got %d", state_bits);
  if (num_slots <= 0) return fail(CK_EINVAL, "num_slots must be positive");
  if (K > 1024) return fail(CK_EUNSUPPORTED, "K must be at most 1024, got %d", K);
  if (resid_fmt == CK_RESID_INT4 && K % 2 != 0)
    return fail(CK_EINVAL, "int4 residual packing needs an even K, got %d", K);
  if (B == 0) return ok();
  if (!mixed_qkv || !a || !b || !A_log || !dt_bias || !state_codes || !state_scale || !resid_codes || !resid_scale ||
      !out || !ssm_state_indices)
    return fail(CK_EINVAL, "null pointer argument");
  // The bandwidth kernels take power-of-two K from 16 and rows their lanes
  // load whole (16 state bytes and 8 (int4) or 16 (int8) residual bytes per
  // lane); any other K or row alignment runs the masked kernel.
  const int ealign = (resid_fmt == CK_RESID_INT4) ? 8 : 16;
  const bool pow2_k = K == 16 || K == 32 || K == 64 || K == 128 || K == 256;
  const bool rows_aligned = !(reinterpret_cast<uintptr_t>(state_codes) & 15) && stride_state_slot % 16 == 0 &&
                            !(reinterpret_cast<uintptr_t>(resid_codes) & (ealign - 1)) &&
                            stride_resid_slot % ealign == 0;
  // per-lane offsets inside one (slot, head) and one row of mixed_qkv are 32-bit
  if ((int64_t)V * K >= ((int64_t)1 << 31) || (2 * (int64_t)H * K + (int64_t)HV * V) * 4 >= ((int64_t)1 << 31))
    return fail(CK_EUNSUPPORTED, "head or activation row too large");

  const int64_t strides[] = {stride_qkv_tok, stride_a_tok, stride_b_tok, stride_state_slot, stride_sscale_slot,
                             stride_resid_slot, stride_rscale_slot, stride_indices, stride_dst_indices};
  for (int64_t st : strides)
    if (st < 0 || st > INT32_MAX) return fail(CK_EUNSUPPORTED, "strides must be in [0, 2^31) elements");
  if (num_slots > INT32_MAX) return fail(CK_EUNSUPPORTED, "num_slots must be < 2^31");

  PackedParams p{};
  p.mixed = mixed_qkv;
  p.a = a;
  p.b = b;
  p.A_log = A_log;
  p.dt_bias = dt_bias;
  p.state = state_codes;
  p.sscale = state_scale;
  p.resid = resid_codes;
  p.rscale = resid_scale;
  p.out = out;
  p.idx = ssm_state_indices;
  p.dst_idx = dst_indices;
  p.stride_mixed = (int32_t)stride_qkv_tok;
  p.stride_a = (int32_t)stride_a_tok;
  p.stride_b = (int32_t)stride_b_tok;
  p.stride_state = (int32_t)stride_state_slot;
  p.stride_sscale = (int32_t)stride_sscale_slot;
  p.stride_resid = (int32_t)stride_resid_slot;
  p.stride_rscale = (int32_t)stride_rscale_slot;
  p.stride_idx = (int32_t)stride_indices;
  p.stride_dst_idx = (int32_t)stride_dst_indices;
  p.num_slots = (int32_t)num_slots;
  p.scale = scale;
  const int qmax = (1 << (state_bits - 1)) - 1;
  volatile float one = 1.0f;  // RN(1/q) computed in fp32 on the host
  p.qmax = (float)qmax;
  p.rqmax = one / (float)qmax;
  p.dtypes = qkv_dtype | (a_dtype << 4) | (b_dtype << 8) | (A_log_dtype << 12) | (dt_bias_dtype << 16) |
             (out_dtype << 20);
  p.H = H;
  p.HV = HV;
  p.div_grp = make_fastdiv((uint32_t)(HV / H));
  p.V = V;
  p.K = K;
  p.l2norm = use_qk_l2norm ? 1 : 0;
#if CK_TIMELINE
  p.timeline = static_cast<uint64_t*>(g_timeline);
#endif
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int per_head = rscale_mode == CK_RSCALE_PER_HEAD;
  const int mode = quant_mode == CK_QUANT_EXACT ? kExact : kFast;
  if (!pow2_k || !rows_aligned) {
    // 4-byte state rows (and int8 residual rows; int4 residual rows of K / 2
    // bytes are then 2-byte aligned) take word accesses
    const int walign = resid_fmt == CK_RESID_INT4 ? 2 : 4;
    const bool words = K % 4 == 0 && !(reinterpret_cast<uintptr_t>(state_codes) & 3) && stride_state_slot % 4 == 0 &&
                       !(reinterpret_cast<uintptr_t>(resid_codes) & (walign - 1)) && stride_resid_slot % walign == 0;
    const int access = rows_aligned && K % 16 == 0 ? kMaskLanes : words ? kMaskWords : kMaskBytes;
    return launch_masked(p, B, resid_fmt, per_head, mode, access, s);
  }
  switch (K) {
    case 16: return launch_for_k<16>(p, B, resid_fmt, per_head, mode, qkv_dtype, s);
    case 32: return launch_for_k<32>(p, B, resid_fmt, per_head, mode, qkv_dtype, s);
    case 64: return launch_for_k<64>(p, B, resid_fmt, per_head, mode, qkv_dtype, s);
    case 128: return launch_for_k<128>(p, B, resid_fmt, per_head, mode, qkv_dtype, s);
    default: return launch_for_k<256>(p, B, resid_fmt, per_head, mode, qkv_dtype, s);
  }
}

extern "C" int ck_gdn_packed_decode(const void* mixed_qkv, int qkv_dtype, int64_t stride_qkv_tok,
                                    const void* a, int a_dtype, int64_t stride_a_tok,
                                    const void* b, int b_dtype, int64_t stride_b_tok,
                                    const void* A_log, int A_log_dtype,
                                    const void* dt_bias, int dt_bias_dtype,
                                    float scale,
                                    int8_t* state_codes, int64_t stride_state_slot,
                                    float* state_scale, int64_t stride_sscale_slot,
                                    int8_t* resid_codes, int64_t stride_resid_slot,
                                    float* resid_scale, int64_t stride_rscale_slot,
                                    void* out, int out_dtype,
                                    const int32_t* ssm_state_indices, int64_t stride_indices,
                                    int64_t num_slots,
                                    int B, int H, int HV, int K, int V,
                                    int use_qk_l2norm, int resid_fmt, int rscale_mode,
                                    int state_bits, int quant_mode,
                                    void* stream) {
  return packed_decode_impl(mixed_qkv, qkv_dtype, stride_qkv_tok, a, a_dtype, stride_a_tok, b, b_dtype, stride_b_tok,
                            A_log, A_log_dtype, dt_bias, dt_bias_dtype, scale, state_codes, stride_state_slot,
                            state_scale, stride_sscale_slot, resid_codes, stride_resid_slot, resid_scale,
                            stride_rscale_slot, out, out_dtype, ssm_state_indices, stride_indices, nullptr, 0,
                            num_slots, B, H, HV, K, V, use_qk_l2norm, resid_fmt, rscale_mode, state_bits, quant_mode,
                            stream);
}

extern "C" int ck_gdn_packed_decode_to(const void* mixed_qkv, int qkv_dtype, int64_t stride_qkv_tok,
                                       const void* a, int a_dtype, int64_t stride_a_tok,
                                       const void* b, int b_dtype, int64_t stride_b_tok,
                                       const void* A_log, int A_log_dtype,
                                       const void* dt_bias, int dt_bias_dtype,
                                       float scale,
                                       int8_t* state_codes, int64_t stride_state_slot,
                                       float* state_scale, int64_t stride_sscale_slot,
                                       int8_t* resid_codes, int64_t stride_resid_slot,
                                       float* resid_scale, int64_t stride_rscale_slot,
                                       void* out, int out_dtype,
                                       const int32_t* ssm_state_indices, int64_t stride_indices,
                                       const int32_t* dst_state_indices, int64_t stride_dst_indices,
                                       int64_t num_slots,
                                       int B, int H, int HV, int K, int V,
                                       int use_qk_l2norm, int resid_fmt, int rscale_mode,
                                       int state_bits, int quant_mode,
                                       void* stream) {
  // an empty batch (B = 0) may pass NULL id arrays, as an empty tensor's data pointer is
  if (!dst_state_indices && B != 0)
    return ck::fail(CK_EINVAL, "dst_state_indices is NULL (use ck_gdn_packed_decode)");
  return packed_decode_impl(mixed_qkv, qkv_dtype, stride_qkv_tok, a, a_dtype, stride_a_tok, b, b_dtype, stride_b_tok,
                            A_log, A_log_dtype, dt_bias, dt_bias_dtype, scale, state_codes, stride_state_slot,
                            state_scale, stride_sscale_slot, resid_codes, stride_resid_slot, resid_scale,
                            stride_rscale_slot, out, out_dtype, ssm_state_indices, stride_indices, dst_state_indices,
                            stride_dst_indices, num_slots, B, H, HV, K, V, use_qk_l2norm, resid_fmt, rscale_mode,
                            state_bits, quant_mode, stream);
}

extern "C" const char* ck_last_error(void) { return ck::last_error().c_str(); }

extern "C" int ck_abi_version(void) { return 2; }

extern "C" int ck_set_max_items_per_launch(int64_t cap) {
  if (cap < 0) return ck::fail(CK_EINVAL, "the item limit must be >= 0, got %lld", (long long)cap);
  ck::pd::read_max_items_env();  // so that a later first launch does not overwrite it
  ck::pd::g_max_items.store(cap, std::memory_order_relaxed);
  return ck::ok();
}

extern "C" int ck_set_decode_kernel(int which) {
  if (which != ck::pd::kDecodeKernelAuto && which != ck::pd::kDecodeKernelPersistent &&
      which != ck::pd::kDecodeKernelOneItem)
    return ck::fail(CK_EINVAL, "the decode kernel must be 0 (automatic), 1 (persistent) or 2 (one-item), got %d", which);
  ck::pd::read_decode_kernel_env();  // so that a later first launch does not overwrite it
  ck::pd::g_decode_kernel.store(which, std::memory_order_relaxed);
  return ck::ok();
}

#if CK_TIMELINE
// Timeline build only: device buffer of kTlMaxWorkgroups x kTlSlots uint64
// that the following ck_gdn_packed_decode launches write their timestamps to
// (NULL: none). Not thread-safe; for measurement runs.
extern "C" int ck_timeline_set(void* device_buffer) {
  g_timeline = device_buffer;
  return CK_OK;
}
#endif
