// Fused GDN decode step with INT8 per-V-row state and INT8 / packed-INT4
// error-feedback residual, in vLLM's paged [slots, HV, V, K] layout (K
// contiguous), updated in place. Counterpart of
// vllm_integration/quantized_packed_decode.py:101-239 (device) and :242-327
// (host launcher), written for gfx950.
//
// Work mapping. A lane owns 16 consecutive K of one V-row: one 16-byte load of
// state codes and one 8-byte (int4) or 16-byte (int8) load of residual codes.
// LPR = K/16 lanes cover a row, so one wave instruction covers 64/LPR
// consecutive rows = one contiguous 1 KB span at K=128. Each lane keeps RPL
// rows; a workgroup of WAVES waves covers RPL*WAVES*64/LPR rows of one
// (request, value-head). Row reductions over K (h.k, h.q, amax) are a
// partial sum over the lane's 16 elements followed by a DPP butterfly over the
// LPR lanes of the row. The whole tile is in VGPRs from load to store, so the
// state is read once and written once.
//
// Arithmetic per row (FAST mode; EXACT differs where ck_quant.h says):
//   sa = s_in * alpha;  h_j = code_j * sa
//   rd = sum_j h_j k_j;  dv = beta * (v - rd);  h_j = fma(k_j, dv, h_j)
//   o  = sum_j h_j q_j
//   t_j = fma(e_code_j, e_scale_in, h_j)
//   s = max(amax_j |t_j| / qmax, 1e-12);  code_j = rne(t_j / s)
//   e_j = t_j - code_j * s
//   es = max(amax |e| / qmax_e, 1e-12);  e_code_j = rne(e_j / es)
// The clamps of the reference (quantized_packed_decode.py:208,215) are
// omitted: |t_j| <= amax and s >= RN(amax/qmax) bound |t_j / s| by
// qmax * (1 + 2^-23) < qmax + 1/2, so the rounded code never exceeds qmax.
#include <hip/hip_runtime.h>

#include "ck_capi_common.h"
#include "ck_device.h"
#include "ck_quant.h"

namespace ck {
namespace {

struct PackedParams {
  const void* mixed;
  int64_t stride_mixed;
  const void* a;
  int64_t stride_a;
  const void* b;
  int64_t stride_b;
  const void* A_log;
  const void* dt_bias;
  int8_t* state;
  int64_t stride_state;
  float* sscale;
  int64_t stride_sscale;
  int8_t* resid;
  int64_t stride_resid;
  float* rscale;
  int64_t stride_rscale;
  void* out;
  const int32_t* idx;
  int64_t stride_idx;
  int64_t num_slots;
  float scale;
  float qmax;
  float qmax_e;
  int mixed_dtype, a_dtype, b_dtype, A_log_dtype, dt_bias_dtype, out_dtype;
  int B, H, HV, V;
  int nvt;     // V-tiles per (request, head)
  int l2norm;
};

constexpr int kResidInt8 = CK_RESID_INT8;
constexpr int kResidInt4 = CK_RESID_INT4;

template <int K, int RPL, int WAVES, int RESID, bool PER_HEAD, int MODE>
__global__ __launch_bounds__(WAVES * 64) void packed_decode_kernel(const PackedParams p) {
  constexpr int LPR = K / 16;          // lanes per V-row
  constexpr int RPI = 64 / LPR;        // rows per wave instruction
  constexpr int ROWS_WAVE = RPI * RPL;
  constexpr int ROWS_WG = ROWS_WAVE * WAVES;
  constexpr int RK = (RESID == kResidInt4) ? K / 2 : K;  // residual bytes per row

  __shared__ float red[WAVES];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane % LPR;
  const int g = lane / LPR;

  int bid = blockIdx.x;
  const int vt = bid % p.nvt;
  bid /= p.nvt;
  const int hv = bid % p.HV;
  const int n = bid / p.HV;
  const int row0 = vt * ROWS_WG + wave * ROWS_WAVE + g;
  const int64_t obase = ((int64_t)n * p.HV + hv) * p.V;

  const int64_t slot = (int64_t)p.idx[(int64_t)n * p.stride_idx];
  if (slot <= 0 || slot >= p.num_slots) {
    // NULL block (slot <= 0): emit zeros, touch no state
    // (quantized_packed_decode.py:132-136). Out-of-range ids emit NaN.
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

  // ---- state / residual / scale loads first, so they are all in flight ----
  const int64_t sbase = slot * p.stride_state + (int64_t)hv * p.V * K + c * 16;
  const int64_t ebase = slot * p.stride_resid + (int64_t)hv * p.V * RK + c * (RK / LPR);
  const int64_t scbase = slot * p.stride_sscale + (int64_t)hv * p.V;
  const int64_t rsbase = PER_HEAD ? slot * p.stride_rscale + hv : slot * p.stride_rscale + (int64_t)hv * p.V;

  uint4 cw[RPL];
  uint32_t ew[RPL][RESID == kResidInt4 ? 2 : 4];
  float s_in[RPL], e_in_scale[RPL], vv[RPL];

  const int hq = hv / (p.HV / p.H);
  const int64_t mrow = (int64_t)n * p.stride_mixed;

#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const int r = row0 + i * RPI;
    if (r < p.V) {
      cw[i] = *reinterpret_cast<const uint4*>(p.state + sbase + (int64_t)r * K);
      if constexpr (RESID == kResidInt4) {
        const uint2 t = *reinterpret_cast<const uint2*>(p.resid + ebase + (int64_t)r * RK);
        ew[i][0] = t.x;
        ew[i][1] = t.y;
      } else {
        const uint4 t = *reinterpret_cast<const uint4*>(p.resid + ebase + (int64_t)r * RK);
        ew[i][0] = t.x;
        ew[i][1] = t.y;
        ew[i][2] = t.z;
        ew[i][3] = t.w;
      }
      s_in[i] = p.sscale[scbase + r];
      if constexpr (!PER_HEAD) e_in_scale[i] = p.rscale[rsbase + r];
      vv[i] = load_act(p.mixed, mrow + 2 * (int64_t)p.H * K + (int64_t)hv * p.V + r, p.mixed_dtype);
    } else {
      cw[i] = make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < (RESID == kResidInt4 ? 2 : 4); ++j) ew[i][j] = 0;
      s_in[i] = 0.0f;
      e_in_scale[i] = 0.0f;
      vv[i] = 0.0f;
    }
  }
  float e_head_scale = 0.0f;
  if constexpr (PER_HEAD) e_head_scale = p.rscale[rsbase];

  // ---- q, k (this lane's 16 K positions), optional L2 norm, q scale ----
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

  // ---- gates (quantized_packed_decode.py:175-182) ----
  float alpha, beta;
  ck_gates(load_act(p.a, (int64_t)n * p.stride_a + hv, p.a_dtype),
           load_act(p.b, (int64_t)n * p.stride_b + hv, p.b_dtype),
           load_act(p.A_log, hv, p.A_log_dtype), load_act(p.dt_bias, hv, p.dt_bias_dtype), &alpha, &beta);

  float ekeep[PER_HEAD ? RPL : 1][16];
  float eamax_local = 0.0f;

#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const int r = row0 + i * RPI;
    const bool valid = r < p.V;
    const uint32_t cws[4] = {cw[i].x, cw[i].y, cw[i].z, cw[i].w};

    // dequantize + decay
    float h[16];
    if constexpr (MODE == kFast) {
      const float sa = s_in[i] * alpha;
#pragma unroll
      for (int j = 0; j < 16; ++j) h[j] = code_i8(cws[j >> 2], j & 3) * sa;
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) h[j] = (code_i8(cws[j >> 2], j & 3) * s_in[i]) * alpha;
    }

    // delta rule: rd = h^T k, dv = beta (v - rd), h += k dv, o = h^T q
    float rd = h[0] * kk[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) rd = fmaf(h[j], kk[j], rd);
    rd = group_sum<LPR>(rd);
    const float dv = beta * (vv[i] - rd);
#pragma unroll
    for (int j = 0; j < 16; ++j) h[j] = madd<MODE>(kk[j], dv, h[j]);
    float o = h[0] * qq[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) o = fmaf(h[j], qq[j], o);
    o = group_sum<LPR>(o);
    if (c == 0 && valid) store_act(p.out, obase + r, p.out_dtype, o);

    // add the carried residual
    const float es_in = PER_HEAD ? e_head_scale : e_in_scale[i];
    float t[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float ec;
      if constexpr (RESID == kResidInt4) {
        ec = code_i4(ew[i][j >> 3], j & 7);
      } else {
        ec = code_i8(ew[i][j >> 2], j & 3);
      }
      t[j] = madd<MODE>(ec, es_in, h[j]);
    }

    // requantize the state
    float am = fabsf(t[0]);
#pragma unroll
    for (int j = 1; j < 16; ++j) am = fmaxf(am, fabsf(t[j]));
    am = group_max<LPR>(am);
    const float s_new = fmaxf(am / p.qmax, kEps);
    const float inv = 1.0f / s_new;
    uint32_t yb[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float code = quantize<MODE>(t[j], s_new, inv, yb[j]);
      t[j] = residual<MODE>(t[j], code, s_new);
    }
    if (valid) {
      uint4 st;
      st.x = pack_low_bytes(yb[0], yb[1], yb[2], yb[3]);
      st.y = pack_low_bytes(yb[4], yb[5], yb[6], yb[7]);
      st.z = pack_low_bytes(yb[8], yb[9], yb[10], yb[11]);
      st.w = pack_low_bytes(yb[12], yb[13], yb[14], yb[15]);
      *reinterpret_cast<uint4*>(p.state + sbase + (int64_t)r * K) = st;
      if (c == 0) p.sscale[scbase + r] = s_new;
    }

    float ea = fabsf(t[0]);
#pragma unroll
    for (int j = 1; j < 16; ++j) ea = fmaxf(ea, fabsf(t[j]));

    if constexpr (PER_HEAD) {
#pragma unroll
      for (int j = 0; j < 16; ++j) ekeep[i][j] = t[j];
      eamax_local = fmaxf(eamax_local, ea);
    } else {
      // per-row residual scale: finish this row now
      ea = group_max<LPR>(ea);
      const float es = fmaxf(ea / p.qmax_e, kEps);
      const float inv_e = 1.0f / es;
      uint32_t eb[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) (void)quantize<MODE>(t[j], es, inv_e, eb[j]);
      if (valid) {
        if constexpr (RESID == kResidInt4) {
          const uint32_t w0[8] = {eb[0], eb[1], eb[2], eb[3], eb[4], eb[5], eb[6], eb[7]};
          const uint32_t w1[8] = {eb[8], eb[9], eb[10], eb[11], eb[12], eb[13], eb[14], eb[15]};
          *reinterpret_cast<uint2*>(p.resid + ebase + (int64_t)r * RK) = make_uint2(pack_nibbles8(w0), pack_nibbles8(w1));
        } else {
          uint4 st;
          st.x = pack_low_bytes(eb[0], eb[1], eb[2], eb[3]);
          st.y = pack_low_bytes(eb[4], eb[5], eb[6], eb[7]);
          st.z = pack_low_bytes(eb[8], eb[9], eb[10], eb[11]);
          st.w = pack_low_bytes(eb[12], eb[13], eb[14], eb[15]);
          *reinterpret_cast<uint4*>(p.resid + ebase + (int64_t)r * RK) = st;
        }
        if (c == 0) p.rscale[rsbase + r] = es;
      }
    }
  }

  if constexpr (PER_HEAD) {
    // one residual scale for the whole (slot, head): amax over every row of
    // every wave (rows past V hold zeros and do not move the max)
    const float wm = wave_max(eamax_local);
    if (lane == 0) red[wave] = wm;
    __syncthreads();
    float ea = red[0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) ea = fmaxf(ea, red[w]);
    const float es = fmaxf(ea / p.qmax_e, kEps);
    const float inv_e = 1.0f / es;
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
      const int r = row0 + i * RPI;
      uint32_t eb[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) (void)quantize<MODE>(ekeep[i][j], es, inv_e, eb[j]);
      if (r < p.V) {
        if constexpr (RESID == kResidInt4) {
          const uint32_t w0[8] = {eb[0], eb[1], eb[2], eb[3], eb[4], eb[5], eb[6], eb[7]};
          const uint32_t w1[8] = {eb[8], eb[9], eb[10], eb[11], eb[12], eb[13], eb[14], eb[15]};
          *reinterpret_cast<uint2*>(p.resid + ebase + (int64_t)r * RK) = make_uint2(pack_nibbles8(w0), pack_nibbles8(w1));
        } else {
          uint4 st;
          st.x = pack_low_bytes(eb[0], eb[1], eb[2], eb[3]);
          st.y = pack_low_bytes(eb[4], eb[5], eb[6], eb[7]);
          st.z = pack_low_bytes(eb[8], eb[9], eb[10], eb[11]);
          st.w = pack_low_bytes(eb[12], eb[13], eb[14], eb[15]);
          *reinterpret_cast<uint4*>(p.resid + ebase + (int64_t)r * RK) = st;
        }
      }
    }
    if (threadIdx.x == 0) p.rscale[rsbase] = es;
  }
}

// ---------------------------------------------------------------------------
// Launch configuration
// ---------------------------------------------------------------------------

template <int K, int RPL, int WAVES, int RESID, bool PER_HEAD, int MODE>
int launch_cfg(PackedParams p, hipStream_t stream) {
  constexpr int ROWS_WG = (64 / (K / 16)) * RPL * WAVES;
  p.nvt = PER_HEAD ? 1 : (p.V + ROWS_WG - 1) / ROWS_WG;
  const int64_t grid = (int64_t)p.B * p.HV * p.nvt;
  if (grid > 0x7fffffff) return fail(CK_EUNSUPPORTED, "grid of %lld workgroups is too large", (long long)grid);
  if (grid == 0) return ok();
  hipLaunchKernelGGL((packed_decode_kernel<K, RPL, WAVES, RESID, PER_HEAD, MODE>), dim3((unsigned)grid),
                     dim3(WAVES * 64), 0, stream, p);
  return check_launch("ck_gdn_packed_decode");
}

// Rows per lane and waves per workgroup. Per-row residual scales split a head
// into V-tiles of 32 rows at K=128 (one wave, 4 rows per lane). A per-head
// residual scale needs the whole head in one workgroup: 4 rows per lane and
// enough waves to cover V.
template <int K, int RESID, bool PER_HEAD, int MODE>
int launch_k(const PackedParams& p, hipStream_t stream) {
  constexpr int RPI = 64 / (K / 16);
  if constexpr (!PER_HEAD) {
    return launch_cfg<K, 4, 1, RESID, false, MODE>(p, stream);
  } else {
    const int need = p.V;
    if (need <= RPI * 4 * 1) return launch_cfg<K, 4, 1, RESID, true, MODE>(p, stream);
    if (need <= RPI * 4 * 2) return launch_cfg<K, 4, 2, RESID, true, MODE>(p, stream);
    if (need <= RPI * 4 * 4) return launch_cfg<K, 4, 4, RESID, true, MODE>(p, stream);
    if (need <= RPI * 4 * 8) return launch_cfg<K, 4, 8, RESID, true, MODE>(p, stream);
    return fail(CK_EUNSUPPORTED, "per-head residual scale supports V <= %d at K=%d, got V=%d", RPI * 32, K, p.V);
  }
}

template <int RESID, bool PER_HEAD, int MODE>
int launch_resid(const PackedParams& p, int K, hipStream_t stream) {
  switch (K) {
    case 16: return launch_k<16, RESID, PER_HEAD, MODE>(p, stream);
    case 32: return launch_k<32, RESID, PER_HEAD, MODE>(p, stream);
    case 64: return launch_k<64, RESID, PER_HEAD, MODE>(p, stream);
    case 128: return launch_k<128, RESID, PER_HEAD, MODE>(p, stream);
    case 256: return launch_k<256, RESID, PER_HEAD, MODE>(p, stream);
    default: return fail(CK_EUNSUPPORTED, "K must be one of 16, 32, 64, 128, 256, got %d", K);
  }
}

template <int MODE>
int launch_mode(const PackedParams& p, int K, int resid_fmt, int per_head, hipStream_t stream) {
  if (resid_fmt == CK_RESID_INT4) {
    return per_head ? launch_resid<kResidInt4, true, MODE>(p, K, stream)
                    : launch_resid<kResidInt4, false, MODE>(p, K, stream);
  }
  return per_head ? launch_resid<kResidInt8, true, MODE>(p, K, stream)
                  : launch_resid<kResidInt8, false, MODE>(p, K, stream);
}

}  // namespace
}  // namespace ck

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
  using namespace ck;
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
  if (B == 0) return ok();
  if (!mixed_qkv || !a || !b || !A_log || !dt_bias || !state_codes || !state_scale || !resid_codes || !resid_scale ||
      !out || !ssm_state_indices)
    return fail(CK_EINVAL, "null pointer argument");
  // lanes load 16 state bytes and 8 (int4) or 16 (int8) residual bytes
  const int ealign = (resid_fmt == CK_RESID_INT4) ? 8 : 16;
  if ((reinterpret_cast<uintptr_t>(state_codes) & 15) || (stride_state_slot % 16))
    return fail(CK_EINVAL, "state_codes rows must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(resid_codes) & (ealign - 1)) || (stride_resid_slot % ealign))
    return fail(CK_EINVAL, "resid_codes rows must be %d-byte aligned", ealign);

  PackedParams p{};
  p.mixed = mixed_qkv;
  p.stride_mixed = stride_qkv_tok;
  p.a = a;
  p.stride_a = stride_a_tok;
  p.b = b;
  p.stride_b = stride_b_tok;
  p.A_log = A_log;
  p.dt_bias = dt_bias;
  p.state = state_codes;
  p.stride_state = stride_state_slot;
  p.sscale = state_scale;
  p.stride_sscale = stride_sscale_slot;
  p.resid = resid_codes;
  p.stride_resid = stride_resid_slot;
  p.rscale = resid_scale;
  p.stride_rscale = stride_rscale_slot;
  p.out = out;
  p.idx = ssm_state_indices;
  p.stride_idx = stride_indices;
  p.num_slots = num_slots;
  p.scale = scale;
  p.qmax = (float)((1 << (state_bits - 1)) - 1);
  p.qmax_e = (resid_fmt == CK_RESID_INT4) ? 7.0f : 127.0f;
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
  const int per_head = rscale_mode == CK_RSCALE_PER_HEAD;
  if (quant_mode == CK_QUANT_EXACT) return launch_mode<kExact>(p, K, resid_fmt, per_head, s);
  return launch_mode<kFast>(p, K, resid_fmt, per_head, s);
}

extern "C" const char* ck_last_error(void) { return ck::last_error().c_str(); }

extern "C" int ck_abi_version(void) { return 1; }
