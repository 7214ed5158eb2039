// Fused decode for any pool row length K in 1 .. 1024 and any row alignment:
// the reference masks its K lanes with o_k < K and loads zeros past K
// (vllm_integration/quantized_packed_decode.py:123-127, :158, :165-166,
// :196-202; BK = next_pow2(K) at :303), so a row of
// K codes computes as the same row padded with zeros to KP, the power of two
// >= max(K, 16) that the reference's BK also rounds to. This kernel runs the
// arithmetic of packed_decode_impl.h (process_item) on that padded row: the
// lane map of KP, every value past K zero in registers, stores of the K
// existing bytes only. Loads and stores are byte-granular (kMaskBytes: a row
// of K bytes has any alignment) or, for K a multiple of 16 with aligned rows,
// whole 16-byte lanes (kMaskLanes: a lane's 16 codes are all in the row or all
// past it). An item is loaded before it is computed, one item per workgroup,
// with no cross-item pipelining: the bandwidth-tuned kernel covers the
// power-of-two K of real models, this one every other shape.
#pragma once

#include "packed_decode_impl.h"

namespace ck {
namespace pd {

// Every load of one live item, zero past p.K, activations converted to fp32
// bits (the kernel computes with ACT = fp32 whatever the activation dtype).
template <int KP, int RPL, int WAVES, int RESID, bool PER_HEAD, int MASK>
__device__ __forceinline__ void load_item_masked(const PackedParams& p, const ItemCoord& ic, int row0, int c,
                                                 ItemRegs<RPL, Layout<KP, RPL, WAVES, RESID, PER_HEAD>::EW,
                                                          Layout<KP, RPL, WAVES, RESID, PER_HEAD>::QKT>& R) {
  using L = Layout<KP, RPL, WAVES, RESID, PER_HEAD>;
  constexpr int RKL = L::RK / L::LPR;  // residual bytes per lane: 8 (int4) or 16 (int8)
  const int K = p.K;
  const int RKA = RESID == kResidInt4 ? K / 2 : K;
  const int8_t* sbase = p.state + ic.slot * p.stride_state + (int64_t)ic.hv * p.V * K;
  const int8_t* ebase = p.resid + ic.slot * p.stride_resid + (int64_t)ic.hv * p.V * RKA;
  const float* scb = p.sscale + ic.slot * p.stride_sscale + (int64_t)ic.hv * p.V;
  const float* rsb = p.rscale + ic.slot * p.stride_rscale + (int64_t)ic.hv * p.V;
  const int adt = p.mixed_dtype();
  const int64_t mrow = (int64_t)ic.n * p.stride_mixed;  // the token's activation row, in elements
#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const int r = min(row0 + i * L::RPI, p.V - 1);  // rows past V re-read row V-1 (never stored)
    const int8_t* srow = sbase + (int64_t)r * K;
    const int8_t* erow = ebase + (int64_t)r * RKA;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    uint32_t e[4] = {0u, 0u, 0u, 0u};
    if constexpr (MASK == kMaskLanes) {
      if (c * 16 < K) {
        const u32x4 w4 = ld_stream16(srow + c * 16);
        w[0] = w4.x, w[1] = w4.y, w[2] = w4.z, w[3] = w4.w;
        if constexpr (RESID == kResidInt4) {
          const u32x2 e2 = ld_stream8(erow + c * RKL);
          e[0] = e2.x, e[1] = e2.y;
        } else {
          const u32x4 e4 = ld_stream16(erow + c * RKL);
          e[0] = e4.x, e[1] = e4.y, e[2] = e4.z, e[3] = e4.w;
        }
      }
    } else if constexpr (MASK == kMaskWords) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c * 16 + 4 * j < K) w[j] = *reinterpret_cast<const uint32_t*>(srow + c * 16 + 4 * j);
      if constexpr (RESID == kResidInt4) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (c * RKL + 2 * j < RKA)
            e[j >> 1] |= (uint32_t)*reinterpret_cast<const uint16_t*>(erow + c * RKL + 2 * j) << (16 * (j & 1));
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (c * RKL + 4 * j < RKA) e[j] = *reinterpret_cast<const uint32_t*>(erow + c * RKL + 4 * j);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int k = c * 16 + j;
        if (k < K) w[j >> 2] |= (uint32_t)(uint8_t)srow[k] << (8 * (j & 3));
      }
#pragma unroll
      for (int j = 0; j < RKL; ++j) {
        const int bidx = c * RKL + j;
        if (bidx < RKA) e[j >> 2] |= (uint32_t)(uint8_t)erow[bidx] << (8 * (j & 3));
      }
    }
    R.cw[i] = u32x4{w[0], w[1], w[2], w[3]};
#pragma unroll
    for (int j = 0; j < L::EW; ++j) R.ew[i][j] = e[j];
    R.s_in[i] = scb[r];
    if constexpr (!PER_HEAD) R.es_in[i] = rsb[r];
    const int64_t vi = mrow + 2 * (int64_t)p.H * K + (int64_t)ic.hv * p.V + r;
    R.vv[i] = __float_as_uint(decode_act_bits(load_act_bits(p.mixed, vi, adt), adt));
  }
  if constexpr (PER_HEAD) R.es_in[0] = p.rscale[ic.slot * p.stride_rscale + ic.hv];
  const int64_t head = fdiv((uint32_t)ic.hv, p.div_grp);
#pragma unroll
  for (int j = 0; j < L::QKT; ++j) {
    const int e = min((int)threadIdx.x + j * L::NT, 2 * KP - 1);  // [q | k], each padded to KP
    const int isk = e >= KP;
    const int kk = e - isk * KP;
    float x = 0.0f;
    if (kk < K) {
      const int64_t qi = mrow + isk * (int64_t)p.H * K + head * K + kk;
      x = decode_act_bits(load_act_bits(p.mixed, qi, adt), adt);
    }
    R.qk[j] = __float_as_uint(x);
  }
}

template <int KP, int RPL, int WAVES, int RESID, bool PER_HEAD, int MODE, bool DST, int MASK>
__global__ __launch_bounds__(WAVES * 64) void packed_decode_masked_kernel(const PackedParams p,
                                                                          const int32_t* __restrict__ idx,
                                                                          const int32_t* __restrict__ dst_idx) {
  using L = Layout<KP, RPL, WAVES, RESID, PER_HEAD>;
  __shared__ __attribute__((aligned(16))) float s_qk[4][2 * KP];  // [parity] staged, [2 + parity] raw
  __shared__ float s_red[2][WAVES];
  __shared__ float4 s_ek[kResidInLds<RPL, RESID, PER_HEAD> ? WAVES * RPL * 4 * 64 : 1];
  __shared__ float2 s_gate[1];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane % L::LPR;
  const int g = lane / L::LPR;
  const Geom gm = geom_of(p);
  const ItemCoord ic = xcd_item_coord<DST>(p, gm, idx, dst_idx, (int)blockIdx.x, gm.share_n);  // share_n: xcd_base
  const int row0 = ic.vt * L::ROWS_WG + wave * L::ROWS_WAVE + g;
  const GateBits gbits = load_item_gate_bits(p, ic);  // before the item's loads (see stage_item_gates)
  ItemRegs<RPL, L::EW, L::QKT> R{};
  if (ic.live) load_item_masked<KP, RPL, WAVES, RESID, PER_HEAD, MASK>(p, ic, row0, c, R);
  stage_item_gates(p, gbits, wave, lane, s_gate);  // wave 0 evaluates this item's gates into LDS
  __syncthreads();
  const float2 gab = s_gate[0];
  process_item<KP, RPL, WAVES, RESID, PER_HEAD, MODE, kF32, DST, MASK>(p, ic, row0, c, lane, wave, 0, gab.x, gab.y, R,
                                                                        s_qk, s_red, s_ek);
}

template <int KP, int RPL, int WAVES, int RESID, bool PER_HEAD, int MODE, bool DST, int MASK>
int launch_masked_cfg(PackedParams p, int B, hipStream_t stream) {
  using L = Layout<KP, RPL, WAVES, RESID, PER_HEAD>;
  const int nvt = PER_HEAD ? 1 : (p.V + L::ROWS_WG - 1) / L::ROWS_WG;
  const int64_t items = (int64_t)B * p.HV * nvt;
  if (items > 0x7fffffff) return fail(CK_EUNSUPPORTED, "%lld work items is too many", (long long)items);
  if (items == 0) return ok();
  p.items = (int)items;
  p.div_nvt = make_fastdiv((uint32_t)nvt);
  p.div_hv = make_fastdiv((uint32_t)p.HV);
  p.cu_share_n = xcd_base(B, p.HV * nvt);  // the base of xcd_item_coord
  p.cu_shares = 0;
  hipLaunchKernelGGL((packed_decode_masked_kernel<KP, RPL, WAVES, RESID, PER_HEAD, MODE, DST, MASK>), dim3((unsigned)items),
                     dim3(WAVES * 64), 0, stream, p, p.idx, p.dst_idx);
  return check_launch("ck_gdn_packed_decode");
}

// Shapes: per-row residual scales take tiles of RPI * 4 rows, as 4 waves of
// one row per lane with byte or word accesses (more loads in flight) or with
// fewer than 2048 tiles (a small batch's rows over more SIMDs), else one wave
// of 4 rows per lane (per-workgroup set-up spread over more rows): K=100
// bytes, B=1 / 8 / 64 at HV=32: 18.5 / 23.4 / 112 -> 8.2 / 17.0 / 105 us;
// K=100 words, B=64: 32.7 us (37.1 with 4 rows per lane); K=96 lanes: B=1 / 8
// 6.8 / 7.7 -> 4.5 / 6.7 us, B=64 24.3 us kept (31.6 with one row per lane).
// A per-head scale needs the whole head in one workgroup: at KP=128 a head of
// 65 to 128 rows takes 8 waves of 2 rows per lane (two workgroups per CU, as
// the bandwidth kernel's shape; B=64, HV=32, V=128: K=100 int4 words 40.9 ->
// 34.3 us, K=128 one byte off alignment 121.0 -> 105.7 us against 4 waves of 4
// rows), at KP=256 a head of 65 to 128 rows 16 waves of 2 rows per lane (K=200
// int4 100.7 -> 87.2 us, K=256 misaligned 232.5 -> 209.2 us against 8 waves of
// 4 rows), otherwise the fewest waves of 4 rows per lane that cover V.
template <int KP, int RESID, bool PER_HEAD, int MODE, bool DST, int MASK>
int launch_masked_shape(const PackedParams& p, int B, hipStream_t s) {
  constexpr int RPI = 64 / (KP / 16);
  if constexpr (!PER_HEAD) {
    if constexpr (MASK == kMaskBytes || MASK == kMaskWords) {
      return launch_masked_cfg<KP, 1, 4, RESID, false, MODE, DST, MASK>(p, B, s);
    } else {
      const int64_t tiles = (int64_t)B * p.HV * ((p.V + RPI * 4 - 1) / (RPI * 4));
      if (tiles < 2048) return launch_masked_cfg<KP, 1, 4, RESID, false, MODE, DST, MASK>(p, B, s);
      return launch_masked_cfg<KP, 4, 1, RESID, false, MODE, DST, MASK>(p, B, s);
    }
  } else {
    if constexpr (KP == 128) {
      if (p.V > RPI * 4 * 2 && p.V <= RPI * 2 * 8) return launch_masked_cfg<KP, 2, 8, RESID, true, MODE, DST, MASK>(p, B, s);
    }
    if constexpr (KP == 256) {
      if (p.V > RPI * 4 * 4 && p.V <= RPI * 2 * 16)
        return launch_masked_cfg<KP, 2, 16, RESID, true, MODE, DST, MASK>(p, B, s);
    }
    if (p.V <= RPI * 4 * 1) return launch_masked_cfg<KP, 4, 1, RESID, true, MODE, DST, MASK>(p, B, s);
    if (p.V <= RPI * 4 * 2) return launch_masked_cfg<KP, 4, 2, RESID, true, MODE, DST, MASK>(p, B, s);
    if (p.V <= RPI * 4 * 4) return launch_masked_cfg<KP, 4, 4, RESID, true, MODE, DST, MASK>(p, B, s);
    if (p.V <= RPI * 4 * 8) return launch_masked_cfg<KP, 4, 8, RESID, true, MODE, DST, MASK>(p, B, s);
    // rows of 512 or 1024 codes: 2 or 1 rows per wave instruction, so a head
    // of V = 128 or 64 rows takes 16 waves of 4 rows per lane
    constexpr int kMaxWaves = KP >= 512 ? 16 : 8;
    if constexpr (KP >= 512) {
      if (p.V <= RPI * 4 * 16) return launch_masked_cfg<KP, 4, 16, RESID, true, MODE, DST, MASK>(p, B, s);
    }
    return fail(CK_EUNSUPPORTED, "per-head residual scale supports V <= %d at K=%d, got V=%d", RPI * 4 * kMaxWaves,
                p.K, p.V);
  }
}

// Dispatch over residual format, scale granularity, mode and destination for
// one padded K and access mode.
template <int KP, int MASK>
int launch_masked_mode(const PackedParams& p, int B, int resid_fmt, int per_head, int mode, hipStream_t s) {
  const bool i4 = resid_fmt == CK_RESID_INT4;
  if (p.dst_idx) {  // out-of-place step: instantiated for the FAST arithmetic only
    if (mode != kFast) return fail(CK_EUNSUPPORTED, "dst_state_indices needs quant_mode FAST");
    return i4 ? (per_head ? launch_masked_shape<KP, kResidInt4, true, kFast, true, MASK>(p, B, s)
                          : launch_masked_shape<KP, kResidInt4, false, kFast, true, MASK>(p, B, s))
              : (per_head ? launch_masked_shape<KP, kResidInt8, true, kFast, true, MASK>(p, B, s)
                          : launch_masked_shape<KP, kResidInt8, false, kFast, true, MASK>(p, B, s));
  }
  if (mode == kFast)
    return i4 ? (per_head ? launch_masked_shape<KP, kResidInt4, true, kFast, false, MASK>(p, B, s)
                          : launch_masked_shape<KP, kResidInt4, false, kFast, false, MASK>(p, B, s))
              : (per_head ? launch_masked_shape<KP, kResidInt8, true, kFast, false, MASK>(p, B, s)
                          : launch_masked_shape<KP, kResidInt8, false, kFast, false, MASK>(p, B, s));
  return i4 ? (per_head ? launch_masked_shape<KP, kResidInt4, true, kExact, false, MASK>(p, B, s)
                        : launch_masked_shape<KP, kResidInt4, false, kExact, false, MASK>(p, B, s))
            : (per_head ? launch_masked_shape<KP, kResidInt8, true, kExact, false, MASK>(p, B, s)
                        : launch_masked_shape<KP, kResidInt8, false, kExact, false, MASK>(p, B, s));
}

// access: kMaskLanes when p.K is a multiple of 16 and the rows are aligned for
// whole-lane accesses (only below a power-of-two KP >= 64: K = 16 and 32 are
// powers of two, which the bandwidth kernel takes when aligned), kMaskWords
// when p.K is a multiple of 4 with 4-byte-aligned rows, else kMaskBytes.
template <int KP>
int launch_masked_k(const PackedParams& p, int B, int resid_fmt, int per_head, int mode, int access, hipStream_t s);

#define CK_PD_DEFINE_MASKED_FOR_K(KP)                                                                        \
  template <>                                                                                                \
  int launch_masked_k<KP>(const PackedParams& p, int B, int resid_fmt, int per_head, int mode, int access,   \
                          hipStream_t s) {                                                                   \
    if constexpr (KP >= 64) {                                                                                \
      if (access == kMaskLanes) return launch_masked_mode<KP, kMaskLanes>(p, B, resid_fmt, per_head, mode, s); \
    }                                                                                                        \
    if (access == kMaskWords || access == kMaskLanes)                                                        \
      return launch_masked_mode<KP, kMaskWords>(p, B, resid_fmt, per_head, mode, s);                         \
    return launch_masked_mode<KP, kMaskBytes>(p, B, resid_fmt, per_head, mode, s);                           \
  }

}  // namespace pd
}  // namespace ck
