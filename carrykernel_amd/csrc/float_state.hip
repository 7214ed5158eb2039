// GDN decode step on an unquantized state pool (fp32 or bf16), vLLM's paged
// [slots, HV, V, K] layout, updated in place. This is the comparison arm for
// the quantized step: the semantics of the upstream packed decode that
// vllm_integration/quantized_packed_decode.py:1-7 replaces (same gates, GQA,
// optional L2 norm, NULL-slot padding), with vLLM's default bf16 state.
//
// Same work mapping as packed_decode.hip: a lane owns 16 consecutive K of a
// V-row (64 bytes of fp32 or 32 bytes of bf16), K/16 lanes per row, DPP row
// reductions, 4 rows per lane, one wave per workgroup.
#include <hip/hip_runtime.h>

#include "ck_capi_common.h"
#include "ck_device.h"

namespace ck {
namespace {

struct FloatStateParams {
  const void* mixed;
  int64_t stride_mixed;
  const void* a;
  int64_t stride_a;
  const void* b;
  int64_t stride_b;
  const void* A_log;
  const void* dt_bias;
  void* state;
  int64_t stride_state;
  void* out;
  const int32_t* idx;
  int64_t stride_idx;
  int64_t num_slots;
  float scale;
  int mixed_dtype, a_dtype, b_dtype, A_log_dtype, dt_bias_dtype, out_dtype;
  int B, H, HV, V;
  int nvt;
  int l2norm;
};

template <int K, int RPL, bool BF16>
__global__ __launch_bounds__(64) void float_state_kernel(const FloatStateParams p) {
  constexpr int LPR = K / 16;
  constexpr int RPI = 64 / LPR;
  constexpr int ROWS_WG = RPI * RPL;

  const int lane = threadIdx.x;
  const int c = lane % LPR;
  const int g = lane / LPR;
  int bid = blockIdx.x;
  const int vt = bid % p.nvt;
  bid /= p.nvt;
  const int hv = bid % p.HV;
  const int n = bid / p.HV;
  const int row0 = vt * ROWS_WG + g;
  const int64_t obase = ((int64_t)n * p.HV + hv) * p.V;

  const int64_t slot = (int64_t)p.idx[(int64_t)n * p.stride_idx];
  if (slot <= 0 || slot >= p.num_slots) {
    const float fill = (slot <= 0) ? 0.0f : __uint_as_float(0x7fc00000u);
    if (c == 0) {
#pragma unroll
      for (int i = 0; i < RPL; ++i) {
        const int r = row0 + i * RPI;
        if (r < p.V) store_act(p.out, obase + r, p.out_dtype, fill);
      }
    }
    return;
  }

  const int64_t sbase = slot * p.stride_state + ((int64_t)hv * p.V) * K + c * 16;
  const int64_t mrow = (int64_t)n * p.stride_mixed;
  const int hq = hv / (p.HV / p.H);

  float h[RPL][16];
  float vv[RPL];
#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const int r = row0 + i * RPI;
    if (r < p.V) {
      if constexpr (BF16) {
        const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.state) + sbase + (int64_t)r * K);
#pragma unroll
        for (int q4 = 0; q4 < 2; ++q4) {
          const uint4 w = src[q4];
          const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            h[i][q4 * 8 + 2 * j] = __uint_as_float(ws[j] << 16);
            h[i][q4 * 8 + 2 * j + 1] = __uint_as_float(ws[j] & 0xffff0000u);
          }
        }
      } else {
        const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(p.state) + sbase + (int64_t)r * K);
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const float4 w = src[q4];
          h[i][4 * q4 + 0] = w.x;
          h[i][4 * q4 + 1] = w.y;
          h[i][4 * q4 + 2] = w.z;
          h[i][4 * q4 + 3] = w.w;
        }
      }
      vv[i] = load_act(p.mixed, mrow + 2 * (int64_t)p.H * K + (int64_t)hv * p.V + r, p.mixed_dtype);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) h[i][j] = 0.0f;
      vv[i] = 0.0f;
    }
  }

  float qq[16], kk[16];
  load_act16(p.mixed, mrow + (int64_t)hq * K + c * 16, p.mixed_dtype, qq);
  load_act16(p.mixed, mrow + (int64_t)p.H * K + (int64_t)hq * K + c * 16, p.mixed_dtype, kk);
  if (p.l2norm) {
    float sq = qq[0] * qq[0];
    float sk = kk[0] * kk[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) {
      sq = fmaf(qq[j], qq[j], sq);
      sk = fmaf(kk[j], kk[j], sk);
    }
    sq = group_sum<LPR>(sq);
    sk = group_sum<LPR>(sk);
    const float dq = sqrtf(sq + 1e-6f);
    const float dk = sqrtf(sk + 1e-6f);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      qq[j] = qq[j] / dq;
      kk[j] = kk[j] / dk;
    }
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) qq[j] = qq[j] * p.scale;

  float alpha, beta;
  ck_gates(load_act(p.a, (int64_t)n * p.stride_a + hv, p.a_dtype),
           load_act(p.b, (int64_t)n * p.stride_b + hv, p.b_dtype),
           load_act(p.A_log, hv, p.A_log_dtype), load_act(p.dt_bias, hv, p.dt_bias_dtype), &alpha, &beta);

#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const int r = row0 + i * RPI;
#pragma unroll
    for (int j = 0; j < 16; ++j) h[i][j] = h[i][j] * alpha;
    float rd = h[i][0] * kk[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) rd = fmaf(h[i][j], kk[j], rd);
    rd = group_sum<LPR>(rd);
    const float dv = beta * (vv[i] - rd);
#pragma unroll
    for (int j = 0; j < 16; ++j) h[i][j] = fmaf(kk[j], dv, h[i][j]);
    float o = h[i][0] * qq[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) o = fmaf(h[i][j], qq[j], o);
    o = group_sum<LPR>(o);
    if (r < p.V) {
      if (c == 0) store_act(p.out, obase + r, p.out_dtype, o);
      if constexpr (BF16) {
        uint4* dst = reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.state) + sbase + (int64_t)r * K);
#pragma unroll
        for (int q4 = 0; q4 < 2; ++q4) {
          uint32_t ws[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            ws[j] = (uint32_t)f32_to_bf16_rne(h[i][q4 * 8 + 2 * j]) |
                    ((uint32_t)f32_to_bf16_rne(h[i][q4 * 8 + 2 * j + 1]) << 16);
          dst[q4] = make_uint4(ws[0], ws[1], ws[2], ws[3]);
        }
      } else {
        float4* dst = reinterpret_cast<float4*>(static_cast<float*>(p.state) + sbase + (int64_t)r * K);
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          dst[q4] = make_float4(h[i][4 * q4], h[i][4 * q4 + 1], h[i][4 * q4 + 2], h[i][4 * q4 + 3]);
      }
    }
  }
}

template <int K, bool BF16>
int launch_fs(FloatStateParams p, hipStream_t stream) {
  constexpr int RPL = 4;
  constexpr int ROWS_WG = (64 / (K / 16)) * RPL;
  p.nvt = (p.V + ROWS_WG - 1) / ROWS_WG;
  const int64_t grid = (int64_t)p.B * p.HV * p.nvt;
  if (grid > 0x7fffffff) return fail(CK_EUNSUPPORTED, "grid too large");
  if (grid == 0) return ok();
  hipLaunchKernelGGL((float_state_kernel<K, RPL, BF16>), dim3((unsigned)grid), dim3(64), 0, stream, p);
  return check_launch("ck_gdn_packed_decode_float_state");
}

template <bool BF16>
int launch_fs_k(const FloatStateParams& p, int K, hipStream_t s) {
  switch (K) {
    case 16: return launch_fs<16, BF16>(p, s);
    case 32: return launch_fs<32, BF16>(p, s);
    case 64: return launch_fs<64, BF16>(p, s);
    case 128: return launch_fs<128, BF16>(p, s);
    case 256: return launch_fs<256, BF16>(p, s);
    default: return fail(CK_EUNSUPPORTED, "K must be one of 16, 32, 64, 128, 256, got %d", K);
  }
}

}  // namespace
}  // namespace ck

extern "C" int ck_gdn_packed_decode_float_state(const void* mixed_qkv, int qkv_dtype, int64_t stride_qkv_tok,
                                                const void* a, int a_dtype, int64_t stride_a_tok,
                                                const void* b, int b_dtype, int64_t stride_b_tok,
                                                const void* A_log, int A_log_dtype,
                                                const void* dt_bias, int dt_bias_dtype,
                                                float scale,
                                                void* state, int state_dtype, int64_t stride_state_slot,
                                                void* out, int out_dtype,
                                                const int32_t* ssm_state_indices, int64_t stride_indices,
                                                int64_t num_slots,
                                                int B, int H, int HV, int K, int V,
                                                int use_qk_l2norm, void* stream) {
  using namespace ck;
  if (B < 0 || H <= 0 || HV <= 0 || K <= 0 || V <= 0)
    return fail(CK_EINVAL, "bad sizes B=%d H=%d HV=%d K=%d V=%d", B, H, HV, K, V);
  if (HV % H != 0) return fail(CK_EINVAL, "HV (%d) must be a multiple of H (%d)", HV, H);
  if (!valid_dtype(qkv_dtype) || !valid_dtype(a_dtype) || !valid_dtype(b_dtype) || !valid_dtype(A_log_dtype) ||
      !valid_dtype(dt_bias_dtype) || !valid_dtype(out_dtype))
    return fail(CK_EINVAL, "unsupported dtype code");
  if (state_dtype != CK_DTYPE_F32 && state_dtype != CK_DTYPE_BF16)
    return fail(CK_EINVAL, "state dtype must be float32 or bfloat16");
  if (num_slots <= 0) return fail(CK_EINVAL, "num_slots must be positive");
  if (B == 0) return ok();
  if (!mixed_qkv || !a || !b || !A_log || !dt_bias || !state || !out || !ssm_state_indices)
    return fail(CK_EINVAL, "null pointer argument");
  const int esz = state_dtype == CK_DTYPE_F32 ? 4 : 2;
  if ((reinterpret_cast<uintptr_t>(state) & 15) || ((stride_state_slot * esz) % 16))
    return fail(CK_EINVAL, "state rows must be 16-byte aligned");
  FloatStateParams p{};
  p.mixed = mixed_qkv;
  p.stride_mixed = stride_qkv_tok;
  p.a = a;
  p.stride_a = stride_a_tok;
  p.b = b;
  p.stride_b = stride_b_tok;
  p.A_log = A_log;
  p.dt_bias = dt_bias;
  p.state = state;
  p.stride_state = stride_state_slot;
  p.out = out;
  p.idx = ssm_state_indices;
  p.stride_idx = stride_indices;
  p.num_slots = num_slots;
  p.scale = scale;
  p.mixed_dtype = qkv_dtype;
  p.a_dtype = a_dtype;
  p.b_dtype = b_dtype;
  p.A_log_dtype = A_log_dtype;
  p.dt_bias_dtype = dt_bias_dtype;
  p.out_dtype = out_dtype;
  p.B = B;
  p.H = H;
  p.HV = HV;
  p.V = V;
  p.l2norm = use_qk_l2norm ? 1 : 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return state_dtype == CK_DTYPE_BF16 ? launch_fs_k<true>(p, K, s) : launch_fs_k<false>(p, K, s);
}
