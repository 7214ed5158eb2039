// Argument checks and launch of the quantized packed decode for the Python
// front end, carrykernel_amd/vllm_integration/quantized_packed_decode.py, in
// C++ over torch's tensor metadata (host code only: built with g++ into a
// CPython extension that calls the C ABI's ck_gdn_packed_decode[_to]).
//
// The front end's checks in Python read about 60 tensor attributes and cost
// ~6 us per eager call, more than the device time of a small batch. Here the
// same checks read the metadata straight from the TensorImpl. This module
// only ever ACCEPTS: a call whose arguments pass every check of the Python
// front end (the reference's, quantized_packed_decode.py:268-309, and the
// ones it adds) is launched here with the arguments the Python front end
// would pass; any other call returns kDeclined and the Python front end runs
// its own checks, which raise the reference's errors. The set accepted here
// is a subset of the Python front end's (degenerate sizes, zero batches and
// anything unusual stay on the Python side).
//
// The C entry points are called through the addresses the front end binds
// (bind()), taken from the library its ctypes loader opened, so both paths
// reach the same loaded library and its process-wide settings.

#include <torch/extension.h>
#include <pybind11/stl.h>

#include <climits>
#include <cstdint>
#include <optional>

#include "carrykernel_gdn.h"

namespace {

constexpr int64_t kDeclined = -1;   // ck_status values are >= 0
constexpr int64_t kMaxK = 1024;     // MAX_K of the Python front end
constexpr int64_t kResidInt8 = 0, kResidInt4 = 1;
constexpr int64_t kQuantFast = 0;

decltype(&ck_gdn_packed_decode) g_decode = nullptr;
decltype(&ck_gdn_packed_decode_to) g_decode_to = nullptr;

// enum ck_dtype of a float tensor, -1 for any other dtype
int dtype_code(const at::Tensor& t) {
  switch (t.scalar_type()) {
    case at::kFloat: return 0;
    case at::kBFloat16: return 1;
    case at::kHalf: return 2;
    default: return -1;
  }
}

// every dim after the slot dim is row-major dense (size-1 dims: any stride)
bool dense_after_slot(const at::Tensor& t) {
  const auto sh = t.sizes();
  const auto st = t.strides();
  int64_t expect = 1;
  for (int64_t i = (int64_t)sh.size() - 1; i > 0; --i) {
    if (sh[i] != 1 && st[i] != expect) return false;
    expect *= sh[i];
  }
  return true;
}

bool fits_int(int64_t v) { return v > 0 && v <= INT_MAX; }

// The arguments of ck_gdn_packed_decode[_to] (stream aside).
struct DecodeArgs {
  const void *qkv, *a, *b, *A_log, *dt_bias;
  int qkv_dt, a_dt, b_dt, A_log_dt, dt_bias_dt, out_dt;
  int64_t qkv_st, a_st, b_st;
  float scale;
  int8_t* sc;
  float* ss;
  int8_t* rc;
  float* rs;
  int64_t sc_st, ss_st, rc_st, rs_st;
  void* out;
  const int32_t* idx;
  int64_t idx_st;
  const int32_t* dst;
  int64_t dst_st;
  int64_t num_slots;
  int B, H, HV, K, V, l2norm, resid_fmt, rscale_mode, state_bits, quant_mode;
};

// Fills `r` and returns true when the Python front end would accept the call
// with these arguments (`require_cuda`: every tensor on one GPU).
bool accept(const at::Tensor& qkv, const at::Tensor& a, const at::Tensor& b, const at::Tensor& A_log,
            const at::Tensor& dt_bias, double scale, const at::Tensor& sc, const at::Tensor& ss,
            const at::Tensor& rc, const at::Tensor& rs, const at::Tensor& out, const at::Tensor& idx,
            const std::optional<at::Tensor>& dst, bool l2norm, int64_t resid_fmt, int64_t state_bits,
            int64_t quant_mode, bool require_cuda, DecodeArgs& r) {
  if (qkv.dim() != 2 || qkv.stride(1) != 1) return false;
  if (sc.dim() != 4 || sc.stride(3) != 1 || rc.dim() != 4) return false;
  if (sc.scalar_type() != at::kChar || rc.scalar_type() != at::kChar) return false;
  const int64_t S = sc.size(0), HV = sc.size(1), V = sc.size(2), K = sc.size(3), B = qkv.size(0);
  if (!fits_int(B) || !fits_int(HV) || !fits_int(V) || !fits_int(K) || S <= 0) return false;
  if (resid_fmt == kResidInt4) {
    if (rc.size(3) * 2 != K) return false;          // also rejects an odd K
  } else if (resid_fmt == kResidInt8) {
    if (rc.size(3) != K) return false;
  } else {
    return false;
  }
  if (rc.size(0) != S || rc.size(1) != HV || rc.size(2) != V) return false;
  if (idx.dim() != 1 || idx.scalar_type() != at::kInt || idx.size(0) < B) return false;
  if (out.dim() != 4 || out.size(0) != B || out.size(1) != 1 || out.size(2) != HV || out.size(3) != V ||
      !out.is_contiguous())
    return false;
  // H from the packed width, as the Python front end infers it
  const int64_t qk_dim = qkv.size(1) - HV * V;
  if (qk_dim <= 0 || qk_dim % 2 != 0) return false;
  const int64_t H = (qk_dim / 2) / K;
  if (H <= 0 || 2 * H * K != qk_dim || HV % H != 0) return false;
  if (K > kMaxK) return false;
  if (ss.scalar_type() != at::kFloat || ss.dim() != 3 || ss.size(0) != S || ss.size(1) != HV ||
      ss.size(2) != V)
    return false;
  if (rs.scalar_type() != at::kFloat) return false;
  int rscale_mode;
  if (rs.dim() == 3 && rs.size(0) == S && rs.size(1) == HV && rs.size(2) == V) {
    rscale_mode = 0;   // per V-row
  } else if (rs.dim() == 2 && rs.size(0) == S && rs.size(1) == HV) {
    rscale_mode = 1;   // per head
  } else {
    return false;
  }
  if (!dense_after_slot(sc) || !dense_after_slot(ss) || !dense_after_slot(rc) || !dense_after_slot(rs))
    return false;
  for (const at::Tensor* t : {&a, &b}) {
    if (t->dim() != 2 || t->size(0) != B || t->size(1) != HV || t->stride(1) != 1) return false;
  }
  for (const at::Tensor* t : {&A_log, &dt_bias}) {
    if (t->dim() != 1 || t->size(0) != HV || t->stride(0) != 1) return false;
  }
  if (state_bits < 2 || state_bits > 8) return false;
  if (dst) {
    if (dst->dim() != 1 || dst->scalar_type() != at::kInt || quant_mode != kQuantFast || dst->size(0) < B)
      return false;
  }
  r.qkv_dt = dtype_code(qkv);
  r.a_dt = dtype_code(a);
  r.b_dt = dtype_code(b);
  r.A_log_dt = dtype_code(A_log);
  r.dt_bias_dt = dtype_code(dt_bias);
  r.out_dt = dtype_code(out);
  if ((r.qkv_dt | r.a_dt | r.b_dt | r.A_log_dt | r.dt_bias_dt | r.out_dt) < 0) return false;
  if (require_cuda) {
    if (!sc.is_cuda()) return false;
    const at::Device dev = sc.device();
    for (const at::Tensor* t : {&qkv, &a, &b, &A_log, &dt_bias, &ss, &rc, &rs, &out, &idx}) {
      if (t->device() != dev) return false;
    }
    if (dst && dst->device() != dev) return false;
  }
  r.qkv = qkv.data_ptr();
  r.qkv_st = qkv.stride(0);
  r.a = a.data_ptr();
  r.a_st = a.stride(0);
  r.b = b.data_ptr();
  r.b_st = b.stride(0);
  r.A_log = A_log.data_ptr();
  r.dt_bias = dt_bias.data_ptr();
  r.scale = (float)scale;
  r.sc = static_cast<int8_t*>(sc.data_ptr());
  r.sc_st = sc.stride(0);
  r.ss = static_cast<float*>(ss.data_ptr());
  r.ss_st = ss.stride(0);
  r.rc = static_cast<int8_t*>(rc.data_ptr());
  r.rc_st = rc.stride(0);
  r.rs = static_cast<float*>(rs.data_ptr());
  r.rs_st = rs.stride(0);
  r.out = out.data_ptr();
  r.idx = static_cast<const int32_t*>(idx.data_ptr());
  r.idx_st = idx.stride(0);
  r.dst = dst ? static_cast<const int32_t*>(dst->data_ptr()) : nullptr;
  r.dst_st = dst ? dst->stride(0) : 0;
  r.num_slots = S;
  r.B = (int)B;
  r.H = (int)H;
  r.HV = (int)HV;
  r.K = (int)K;
  r.V = (int)V;
  r.l2norm = l2norm ? 1 : 0;
  r.resid_fmt = (int)resid_fmt;
  r.rscale_mode = rscale_mode;
  r.state_bits = (int)state_bits;
  r.quant_mode = (int)quant_mode;
  return true;
}

void bind(uintptr_t decode, uintptr_t decode_to) {
  g_decode = reinterpret_cast<decltype(g_decode)>(decode);
  g_decode_to = reinterpret_cast<decltype(g_decode_to)>(decode_to);
}

// The ck_status of the launch, or kDeclined (nothing launched).
int64_t packed_decode(const at::Tensor& qkv, const at::Tensor& a, const at::Tensor& b, const at::Tensor& A_log,
                      const at::Tensor& dt_bias, double scale, const at::Tensor& sc, const at::Tensor& ss,
                      const at::Tensor& rc, const at::Tensor& rs, const at::Tensor& out, const at::Tensor& idx,
                      const std::optional<at::Tensor>& dst, bool l2norm, int64_t resid_fmt, int64_t state_bits,
                      int64_t quant_mode, uintptr_t stream) {
  if (g_decode == nullptr || g_decode_to == nullptr) return kDeclined;
  DecodeArgs r;
  if (!accept(qkv, a, b, A_log, dt_bias, scale, sc, ss, rc, rs, out, idx, dst, l2norm, resid_fmt, state_bits,
              quant_mode, true, r))
    return kDeclined;
  void* s = reinterpret_cast<void*>(stream);
  pybind11::gil_scoped_release nogil;   // as a ctypes call does
  if (r.dst == nullptr) {
    return g_decode(r.qkv, r.qkv_dt, r.qkv_st, r.a, r.a_dt, r.a_st, r.b, r.b_dt, r.b_st, r.A_log, r.A_log_dt,
                    r.dt_bias, r.dt_bias_dt, r.scale, r.sc, r.sc_st, r.ss, r.ss_st, r.rc, r.rc_st, r.rs, r.rs_st,
                    r.out, r.out_dt, r.idx, r.idx_st, r.num_slots, r.B, r.H, r.HV, r.K, r.V, r.l2norm,
                    r.resid_fmt, r.rscale_mode, r.state_bits, r.quant_mode, s);
  }
  return g_decode_to(r.qkv, r.qkv_dt, r.qkv_st, r.a, r.a_dt, r.a_st, r.b, r.b_dt, r.b_st, r.A_log, r.A_log_dt,
                     r.dt_bias, r.dt_bias_dt, r.scale, r.sc, r.sc_st, r.ss, r.ss_st, r.rc, r.rc_st, r.rs, r.rs_st,
                     r.out, r.out_dt, r.idx, r.idx_st, r.dst, r.dst_st, r.num_slots, r.B, r.H, r.HV, r.K, r.V,
                     r.l2norm, r.resid_fmt, r.rscale_mode, r.state_bits, r.quant_mode, s);
}

// For tests: the C-ABI arguments (stream aside) in ck_gdn_packed_decode_to's
// order, pointers as integers, or None where packed_decode would decline.
// require_cuda=false leaves out the device checks (CPU tensors).
pybind11::object launch_args(const at::Tensor& qkv, const at::Tensor& a, const at::Tensor& b,
                             const at::Tensor& A_log, const at::Tensor& dt_bias, double scale,
                             const at::Tensor& sc, const at::Tensor& ss, const at::Tensor& rc,
                             const at::Tensor& rs, const at::Tensor& out, const at::Tensor& idx,
                             const std::optional<at::Tensor>& dst, bool l2norm, int64_t resid_fmt,
                             int64_t state_bits, int64_t quant_mode, bool require_cuda) {
  DecodeArgs r;
  if (!accept(qkv, a, b, A_log, dt_bias, scale, sc, ss, rc, rs, out, idx, dst, l2norm, resid_fmt, state_bits,
              quant_mode, require_cuda, r))
    return pybind11::none();
  auto p = [](const void* x) { return (uintptr_t)x; };
  return pybind11::make_tuple(
      p(r.qkv), r.qkv_dt, r.qkv_st, p(r.a), r.a_dt, r.a_st, p(r.b), r.b_dt, r.b_st, p(r.A_log), r.A_log_dt,
      p(r.dt_bias), r.dt_bias_dt, r.scale, p(r.sc), r.sc_st, p(r.ss), r.ss_st, p(r.rc), r.rc_st, p(r.rs), r.rs_st,
      p(r.out), r.out_dt, p(r.idx), r.idx_st, p(r.dst), r.dst_st, r.num_slots, r.B, r.H, r.HV, r.K, r.V,
      r.l2norm, r.resid_fmt, r.rscale_mode, r.state_bits, r.quant_mode);
}

}  // namespace

PYBIND11_MODULE(_ck_front, m) {
  m.doc() = "argument checks and launch of the quantized packed decode (host C++ over the C ABI)";
  m.attr("DECLINED") = kDeclined;
  m.attr("MAX_K") = kMaxK;
  m.attr("RESID_INT8") = kResidInt8;
  m.attr("RESID_INT4") = kResidInt4;
  m.attr("QUANT_FAST") = kQuantFast;
  m.def("bind", &bind, "set the addresses of ck_gdn_packed_decode and ck_gdn_packed_decode_to");
  m.def("packed_decode", &packed_decode);
  m.def("launch_args", &launch_args);
}
