// Fused GDN decode step with INT8 per-V-row state and INT8 / packed-INT4
// error-feedback residual, in vLLM's paged [slots, HV, V, K] layout (K
// contiguous), updated in place. Counterpart of
// vllm_integration/quantized_packed_decode.py:101-239 (device) and :242-327
// (host launcher), written for gfx950. The templates are instantiated per K in
// packed_decode_k*.hip; ck_gdn_packed_decode (packed_decode.hip) dispatches.
//
// Work items. An item is one (request, value-head, V-tile); with a per-head
// residual scale the tile is the whole head. A workgroup of WAVES waves covers
// a tile: a lane owns 16 consecutive K of a V-row (one 16-byte load of state
// codes, one 8-byte (int4) or 16-byte (int8) load of residual codes), LPR =
// K/16 lanes cover a row, one wave instruction covers 64/LPR consecutive rows
// (a contiguous 1 KB span at K=128), and each lane keeps RPL rows. The tile
// stays in VGPRs from load to store: state and residual are read once and
// written once.
//
// Two kernels compute items with the same code (process_item), so their bits
// are the same; launch_cfg picks one per launch.
//  * One-item kernel (packed_decode_single_kernel): one workgroup per item;
//    the hardware dispatcher starts the next workgroup on whichever CU frees
//    a slot, and the workgroups that share a CU overlap one's loads with
//    another's arithmetic. It runs every launch except a per-head K=256 batch
//    above one item per resident workgroup.
//  * Persistent kernel (packed_decode_kernel): the grid holds as many
//    workgroups as fit on the GPU at once; each loops over its items. While
//    an item is computed, the next item's codes, residual, scales, v and q/k
//    load into a second register set. The gates of all of a workgroup's items
//    are evaluated before its item loop, one item per lane, into an LDS table
//    (stage_gates).
// Loads carry raw bits (activation conversion happens at use), so issuing them
// never waits. q and k are staged once per item through LDS (one barrier per
// item).
//
// Arithmetic per row (FAST mode; EXACT differs where ck_quant.h says):
//   sa = s_in * alpha;  h_j = code_j * sa
//   rd = sum_j h_j k_j;  dv = beta * (v - rd);  h_j = fma(k_j, dv, h_j)
//   o  = sum_j h_j q_j
//   t_j = fma(e_code_j, e_scale_in, h_j)
//   s = max(amax_j |t_j| / qmax, 1e-12);  code_j = rne(t_j * RN(1/s))
//   e_j = fma(-code_j, s, t_j)
//   es = max(amax |e| / qmax_e, 1e-12);  e_code_j = rne(e_j * RN(1/es))
// K-sums are 16-element fma chains per lane combined by a DPP butterfly. The
// clamps of the reference (quantized_packed_decode.py:208,215) are omitted:
// |t_j| <= amax and s >= RN(amax/qmax) bound |t_j / s| by qmax * (1 + 2^-23)
// < qmax + 1/2, so no rounded code exceeds qmax.
#pragma once

#include <hip/hip_runtime.h>


#include "ck_capi_common.h"
#include "ck_device.h"
#include "ck_quant.h"

namespace ck {
namespace pd {

// Unsigned division by a runtime constant d as (x * m) >> (31 + l), exact for
// 0 <= x < 2^31 with l = ceil(log2 d), m = ceil(2^(31+l) / d) < 2^32
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, Theorem 4.2 with N = 31).
// For l >= 1, (x * m) >> (31 + l) = mulhi(x, m) >> (l - 1), a scalar
// s_mul_hi_u32 on uniform operands; d = 1 is passed through.
struct FastDiv {
  uint32_t d, m, sh;  // sh = l - 1 (unused when d == 1)
};

inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  const uint64_t m = ((1ull << (31 + l)) + d - 1) / d;
  return FastDiv{d, (uint32_t)m, l == 0 ? 0u : l - 1};
}

__device__ __forceinline__ uint32_t fdiv(uint32_t x, const FastDiv& f) {
  return f.d == 1 ? x : (__umulhi(x, f.m) >> f.sh);
}

// A FastDiv used for quotients only, in two words: m, and sh with bit 8 set
// when d == 1 (d itself is then not kept).
inline uint32_t quotient_word(const FastDiv& f) { return f.sh | (f.d == 1 ? 0x100u : 0u); }
__device__ __forceinline__ FastDiv quotient_fastdiv(uint32_t m, uint32_t w) {
  return FastDiv{(w & 0x100u) ? 1u : 0u, m, w & 0xffu};
}

struct PackedParams {
  const void* mixed;
  const void* a;
  const void* b;
  const void* A_log;
  const void* dt_bias;
  int8_t* state;
  float* sscale;
  int8_t* resid;
  float* rscale;
  void* out;
  // strides in elements; validated on the host to fit in 32 bits
  int32_t stride_mixed, stride_a, stride_b, stride_state, stride_sscale, stride_resid, stride_rscale;
  int32_t num_slots;
  float scale;
  float qmax, rqmax;      // state code range and RN(1/qmax)
  int32_t dtypes;         // mixed | a << 4 | b << 8 | A_log << 12 | dt_bias << 16 | out << 20
  int32_t H, HV, V;
  int32_t l2norm;
  FastDiv div_grp;        // HV / H: value heads per q/k head
  // Fields the one-item kernel does not read come after the ones it does: its
  // kernel-argument loads then hold no unused dwords, whose registers the
  // compiler would give to the slot id, so that load waited for them (B=1
  // 5.44 -> 5.34 us, B=64 -0.8 %, three A/B pairs).
  const int32_t* idx;
  const int32_t* dst_idx;  // slot ids the updated state is written to (NULL: in place, to idx's slots)
  int32_t stride_idx, stride_dst_idx;
  int32_t K;              // pool row length; the template K of the masked kernel is K rounded up to a power of two
  int32_t items;          // B * HV * nvt
  int32_t cu_share_n;     // workgroups per CU that share their items unevenly (<= 1: plain stride); see work_seq
  uint32_t cu_shares;     // byte a: share of the age-a workgroup, in 64ths
  uint64_t* timeline;     // timeline build only (CK_TIMELINE): per-workgroup timestamps, else unused
  FastDiv div_nvt, div_hv;  // nvt = V-tiles per (request, head)

  __device__ __forceinline__ int mixed_dtype() const { return dtypes & 15; }
  __device__ __forceinline__ int a_dtype() const { return (dtypes >> 4) & 15; }
  __device__ __forceinline__ int b_dtype() const { return (dtypes >> 8) & 15; }
  __device__ __forceinline__ int A_log_dtype() const { return (dtypes >> 12) & 15; }
  __device__ __forceinline__ int dt_bias_dtype() const { return (dtypes >> 16) & 15; }
  __device__ __forceinline__ int out_dtype() const { return (dtypes >> 20) & 15; }
};

constexpr int kResidInt8 = CK_RESID_INT8;
constexpr int kResidInt4 = CK_RESID_INT4;

// Residual code range qmax_e (7 for int4, 127 for int8) and RN(1 / qmax_e),
// fixed by the residual format.
template <int RESID>
struct ResidRange {
  static constexpr float q = RESID == kResidInt4 ? 7.0f : 127.0f;
  static constexpr uint32_t rq_bits = RESID == kResidInt4 ? 0x3e124925u : 0x3c010204u;  // RN(1/7), RN(1/127)
};

template <int K, int RPL, int WAVES, int RESID, bool PER_HEAD>
struct Layout {
  static constexpr int LPR = K / 16;    // lanes per V-row
  static constexpr int RPI = 64 / LPR;  // rows per wave instruction
  static constexpr int ROWS_WAVE = RPI * RPL;
  static constexpr int ROWS_WG = ROWS_WAVE * WAVES;
  static constexpr int NT = WAVES * 64;
  static constexpr int QKT = (2 * K + NT - 1) / NT;  // staged q/k values per thread
  static constexpr int EW = (RESID == kResidInt4) ? 2 : 4;
  static constexpr int RK = (RESID == kResidInt4) ? K / 2 : K;  // residual bytes per row
};

// Per-head residual mode keeps every row's unquantized residual until the
// head's amax is known. In the persistent kernel, with int8 residual rows at
// 2 rows per lane, the 32 values go to LDS (each lane reads back only its
// own) instead of VGPRs, so the 8-wave shape fits 128 VGPRs beside the second
// register set. The one-item kernel has no second set and keeps them in VGPRs
// (process_item's EK_REGS).
template <int RPL, int RESID, bool PER_HEAD>
constexpr bool kResidInLds = PER_HEAD && RESID == CK_RESID_INT8 && RPL == 2;

// Everything one lane needs from memory for one item.
template <int RPL, int EW, int QKT>
struct ItemRegs {
  u32x4 cw[RPL];         // state codes, 16 per row
  uint32_t ew[RPL][EW];  // residual codes
  float s_in[RPL];       // state scale per row
  float es_in[RPL];      // residual scale per row (per-row mode); [0] per head
  uint32_t vv[RPL];      // v per row (raw activation bits)
  uint32_t qk[QKT];      // this thread's share of [q | k] (raw activation bits)
};

struct ItemCoord {
  int n, hv, vt;
  int64_t slot;   // slot the state is read from
  int64_t dslot;  // slot the updated state is written to
  bool live;      // slot in [1, num_slots)
  bool dlive;     // dslot in [1, num_slots): the update is stored
};

// Launch geometry: item count, the divisors that split an item number into
// (request, head, V-tile), the slot-id stride and the item sharing. The
// bandwidth kernel takes these as its leading scalar arguments, which the
// compiler preloads into SGPRs (-amdgpu-kernarg-preload-count), so the first
// slot-id load depends on no kernel-argument load; other kernels read them
// from PackedParams (geom_of).
struct Geom {
  int items, stride_idx, share_n;
  uint32_t shares;
  FastDiv nvt, hv;
  int grid;  // workgroups in the launch (gridDim.x)
};

__device__ __forceinline__ Geom geom_of(const PackedParams& p) {
  return Geom{p.items, p.stride_idx, p.cu_share_n, p.cu_shares, p.div_nvt, p.div_hv, (int)gridDim.x};
}

template <bool DST>
__device__ __forceinline__ void slot_coord(const PackedParams& p, const Geom& gm, const int32_t* __restrict__ idx,
                                           const int32_t* __restrict__ dst_idx, ItemCoord& ic);

// Coordinates of an item. `item` is uniform; readfirstlane keeps the results
// in SGPRs so that the slot id is a scalar load (a vector load here would be
// ordered behind the prefetch in the vector memory counter).
// DST: the step writes to the slots in dst_idx (a second scalar load per
// item); otherwise the destination is the source slot.
template <bool ONE_TILE = false, bool DST = false>  // ONE_TILE: one V-tile per (request, head), vt = 0
__device__ __forceinline__ ItemCoord item_coord(const PackedParams& p, const Geom& gm, const int32_t* __restrict__ idx,
                                                const int32_t* __restrict__ dst_idx, int item) {
  ItemCoord ic;
  item = __builtin_amdgcn_readfirstlane(item);
  const uint32_t nh = ONE_TILE ? (uint32_t)item : fdiv((uint32_t)item, gm.nvt);
  ic.vt = ONE_TILE ? 0 : item - (int)(nh * gm.nvt.d);
  const uint32_t n = fdiv(nh, gm.hv);
  ic.hv = __builtin_amdgcn_readfirstlane((int)(nh - n * gm.hv.d));
  ic.n = __builtin_amdgcn_readfirstlane((int)n);
  ic.vt = __builtin_amdgcn_readfirstlane(ic.vt);
  slot_coord<DST>(p, gm, idx, dst_idx, ic);
  return ic;
}

// The slots of an item whose (n, hv, vt) are set.
template <bool DST>
__device__ __forceinline__ void slot_coord(const PackedParams& p, const Geom& gm, const int32_t* __restrict__ idx,
                                           const int32_t* __restrict__ dst_idx, ItemCoord& ic) {
  ic.slot = (int64_t)idx[(int64_t)ic.n * gm.stride_idx];
  ic.live = ic.slot > 0 && ic.slot < p.num_slots;
  if constexpr (DST) {
    ic.dslot = (int64_t)dst_idx[(int64_t)ic.n * p.stride_dst_idx];
    ic.dlive = ic.dslot > 0 && ic.dslot < p.num_slots;
  } else {
    (void)dst_idx;
    ic.dslot = ic.slot;
    ic.dlive = ic.live;
  }
}

// Issue every load of one item, branch-free: the number of loads is the same
// on every path, so the compiler's wait counts let this item's loads stay in
// flight while the previous item is computed. A prefetch that is not needed
// (dead item: NULL or out-of-range slot; past the last item) collapses every
// lane onto the first bytes of slot 0 / head 0, one cache line per load, and
// its values are never used. Rows past V re-read row V-1. Bases are uniform;
// per-lane offsets are 32-bit.
template <int K, int RPL, int WAVES, int RESID, bool PER_HEAD, int ACT>
__device__ __forceinline__ void load_item(const PackedParams& p, const ItemCoord& ic, bool needed, int row0, int c,
                                          ItemRegs<RPL, Layout<K, RPL, WAVES, RESID, PER_HEAD>::EW,
                                                   Layout<K, RPL, WAVES, RESID, PER_HEAD>::QKT>& R) {
  using L = Layout<K, RPL, WAVES, RESID, PER_HEAD>;
  constexpr int ESZ = act_bytes<ACT>;
  const bool real = needed && ic.live;
  const uint32_t keep = real ? 0xffffffffu : 0u;  // per-lane offset mask
  const int64_t slot = real ? ic.slot : 0;
  const int hv = real ? ic.hv : 0;
  const int8_t* sbase = p.state + slot * p.stride_state + (int64_t)hv * p.V * K;
  const int8_t* ebase = p.resid + slot * p.stride_resid + (int64_t)hv * p.V * L::RK;
  const float* scb = p.sscale + slot * p.stride_sscale + (int64_t)hv * p.V;
  const float* rsb = p.rscale + slot * p.stride_rscale + (int64_t)hv * p.V;  // per-row mode only
  const char* mrow = static_cast<const char*>(p.mixed) + (int64_t)ic.n * p.stride_mixed * ESZ;
  const char* vbase = mrow + (2 * (int64_t)p.H * K + (int64_t)hv * p.V) * ESZ;
#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const uint32_t r = (uint32_t)min(row0 + i * L::RPI, p.V - 1) & keep;
    const uint32_t cc = (uint32_t)c & keep;
    R.cw[i] = ld_stream16(sbase + (r * K + cc * 16));
    if constexpr (RESID == kResidInt4) {
      const u32x2 t = ld_stream8(ebase + (r * L::RK + cc * 8));
      R.ew[i][0] = t.x;
      R.ew[i][1] = t.y;
    } else {
      const u32x4 t = ld_stream16(ebase + (r * L::RK + cc * 16));
      R.ew[i][0] = t.x;
      R.ew[i][1] = t.y;
      R.ew[i][2] = t.z;
      R.ew[i][3] = t.w;
    }
    R.s_in[i] = ld_at<float>(scb, r * 4u);
    if constexpr (!PER_HEAD) R.es_in[i] = ld_at<float>(rsb, r * 4u);
    R.vv[i] = load_act_raw<ESZ>(vbase, r * ESZ);
  }
  if constexpr (PER_HEAD) {
    // one scale per (slot, head) at a uniform address: a scalar load in the
    // one-item kernel, a vector load in the persistent kernel's item loop
    const float* rsh = p.rscale + slot * p.stride_rscale + hv;
    R.es_in[0] = ld_at<float>(rsh, 0u * (uint32_t)c);
  }
  // the q/k head by a scalar multiply-shift (two integer divisions in VALU before)
  const char* qbase = mrow + (int64_t)fdiv((uint32_t)hv, p.div_grp) * K * ESZ;
  const uint32_t koff = (uint32_t)((p.H - 1) * K);  // k of this head sits H*K after q
#pragma unroll
  for (int j = 0; j < L::QKT; ++j) {
    const uint32_t e = min((uint32_t)threadIdx.x + j * L::NT, (uint32_t)(2 * K - 1));  // q then k
    R.qk[j] = load_act_raw<ESZ>(qbase, ((e < K ? e : e + koff) * ESZ) & keep);
  }
}

template <int RESID>
__device__ __forceinline__ void store_resid(int8_t* dst, const uint32_t (&eb)[16]) {
  if constexpr (RESID == kResidInt4) {
    const uint32_t w0[8] = {eb[0], eb[1], eb[2], eb[3], eb[4], eb[5], eb[6], eb[7]};
    const uint32_t w1[8] = {eb[8], eb[9], eb[10], eb[11], eb[12], eb[13], eb[14], eb[15]};
    st_stream8(dst, u32x2{pack_nibbles8(w0), pack_nibbles8(w1)});
  } else {
    st_stream16(dst, u32x4{pack_low_bytes(eb[0], eb[1], eb[2], eb[3]), pack_low_bytes(eb[4], eb[5], eb[6], eb[7]),
                           pack_low_bytes(eb[8], eb[9], eb[10], eb[11]),
                           pack_low_bytes(eb[12], eb[13], eb[14], eb[15])});
  }
}

// Stage one item's q and k in LDS buffer `parity`: q * scale and k, both
// L2-normalised first when the flag is set (one division per staged value).
// qk holds this thread's share of the raw activation bits, element
// threadIdx.x + j * NT of [q | k]. A thread computes the norm of the vector
// its element belongs to: the lanes of a row group (LPR lanes) each sum the
// squares of one 16-element slice in order, then group_sum adds the slices,
// so every thread of q (or of k) gets the same sum. Threads with no element
// (a wave past 2K) skip the norm. Ends with a barrier after which every thread
// may read the staged values.
template <int K, int QKT, int NT, int ACT>
__device__ __forceinline__ void stage_qk(const PackedParams& p, const uint32_t (&qk)[QKT], int c, int parity,
                                         float (*s_qk)[2 * K]) {
  constexpr int LPR = K / 16;
  float* buf = s_qk[parity];
  if (p.l2norm) {
    float* raw = s_qk[2 + parity];
#pragma unroll
    for (int j = 0; j < QKT; ++j) {
      const int e = (int)threadIdx.x + j * NT;
      if (e < 2 * K) raw[e] = act_decode<ACT>(qk[j]);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < QKT; ++j) {
      const int e = (int)threadIdx.x + j * NT;
      // uniform over a wave for all but its last partial group of elements
      if ((int)(threadIdx.x & ~63u) + j * NT < 2 * K) {
        const bool isq = e < K;
        const float4* x4 = reinterpret_cast<const float4*>(raw + (isq ? 0 : K) + c * 16);
        float xv[16];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float4 a4 = x4[t];
          xv[4 * t] = a4.x, xv[4 * t + 1] = a4.y, xv[4 * t + 2] = a4.z, xv[4 * t + 3] = a4.w;
        }
        float ss = xv[0] * xv[0];
#pragma unroll
        for (int t = 1; t < 16; ++t) ss = fmaf(xv[t], xv[t], ss);
        ss = group_sum<LPR>(ss);
        const float d = sqrtf(ss + 1e-6f);
        if (e < 2 * K) buf[e] = isq ? (raw[e] / d) * p.scale : raw[e] / d;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < QKT; ++j) {
      const int e = (int)threadIdx.x + j * NT;
      if (e < 2 * K) {
        const float x = act_decode<ACT>(qk[j]);
        buf[e] = (e < K) ? x * p.scale : x;
      }
    }
  }
  __syncthreads();
}

// The first n bytes (n clamped to 0 .. 4 NW) of w, byte j from dword j / 4,
// one byte store each: the masked kernel's rows have any length and alignment.
template <int NW>
__device__ __forceinline__ void st_bytes_masked(int8_t* dst, const uint32_t (&w)[NW], int n) {
#pragma unroll
  for (int j = 0; j < 4 * NW; ++j)
    if (j < n) dst[j] = (int8_t)(w[j >> 2] >> (8 * (j & 3)));
}

template <int RESID>
__device__ __forceinline__ void store_resid_masked(int8_t* dst, const uint32_t (&eb)[16], int n) {
  if constexpr (RESID == kResidInt4) {
    const uint32_t w0[8] = {eb[0], eb[1], eb[2], eb[3], eb[4], eb[5], eb[6], eb[7]};
    const uint32_t w1[8] = {eb[8], eb[9], eb[10], eb[11], eb[12], eb[13], eb[14], eb[15]};
    const uint32_t w[2] = {pack_nibbles8(w0), pack_nibbles8(w1)};
    st_bytes_masked<2>(dst, w, n);
  } else {
    const uint32_t w[4] = {pack_low_bytes(eb[0], eb[1], eb[2], eb[3]), pack_low_bytes(eb[4], eb[5], eb[6], eb[7]),
                           pack_low_bytes(eb[8], eb[9], eb[10], eb[11]), pack_low_bytes(eb[12], eb[13], eb[14], eb[15])};
    st_bytes_masked<4>(dst, w, n);
  }
}

// How the masked kernel's rows are accessed: rows are p.K codes long (K is
// p.K rounded up to a power of two, at least 16; the loader zero-fills every
// value past p.K). kMaskBytes: any p.K and alignment, byte by byte.
// kMaskLanes: p.K a multiple of 16 with aligned rows, so a lane's 16 codes
// (and 8 or 16 residual bytes) are all there or all past p.K, and it loads and
// stores them whole. kMaskWords: p.K a multiple of 4 with 4-byte-aligned state
// rows (and int8 residual rows; an int4 residual row of p.K / 2 bytes is then
// 2-byte aligned): 4-byte state and int8-residual accesses, 2-byte int4
// residual ones, each all there or all past p.K.
constexpr int kMaskNone = 0;
constexpr int kMaskBytes = 1;
constexpr int kMaskLanes = 2;
constexpr int kMaskWords = 3;

// The first n bytes (n a multiple of 4, clamped to 0 .. 4 NW) of w, one
// 4-byte store per word.
template <int NW>
__device__ __forceinline__ void st_words_masked(int8_t* dst, const uint32_t (&w)[NW], int n) {
#pragma unroll
  for (int j = 0; j < NW; ++j)
    if (4 * j < n) *reinterpret_cast<uint32_t*>(dst + 4 * j) = w[j];
}

// A lane's residual bytes under kMaskWords: int8 in 4-byte words, int4 (n
// even) in 2-byte halves.
template <int RESID>
__device__ __forceinline__ void store_resid_words(int8_t* dst, const uint32_t (&eb)[16], int n) {
  if constexpr (RESID == kResidInt4) {
    const uint32_t w0[8] = {eb[0], eb[1], eb[2], eb[3], eb[4], eb[5], eb[6], eb[7]};
    const uint32_t w1[8] = {eb[8], eb[9], eb[10], eb[11], eb[12], eb[13], eb[14], eb[15]};
    const uint32_t w[2] = {pack_nibbles8(w0), pack_nibbles8(w1)};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (2 * j < n) *reinterpret_cast<uint16_t*>(dst + 2 * j) = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
  } else {
    const uint32_t w[4] = {pack_low_bytes(eb[0], eb[1], eb[2], eb[3]), pack_low_bytes(eb[4], eb[5], eb[6], eb[7]),
                           pack_low_bytes(eb[8], eb[9], eb[10], eb[11]), pack_low_bytes(eb[12], eb[13], eb[14], eb[15])};
    st_words_masked<4>(dst, w, n);
  }
}

// Compute and store one item whose registers are loaded (MASK: see above).
// EK_REGS: the per-head residual waits in VGPRs even where kResidInLds would
// put it in LDS (the one-item kernel).
template <int K, int RPL, int WAVES, int RESID, bool PER_HEAD, int MODE, int ACT, bool DST, int MASK = kMaskNone,
          bool EK_REGS = false>
__device__ __forceinline__ void process_item(const PackedParams& p, const ItemCoord& ic, int row0, int c, int lane,
                                             int wave, int parity, float alpha, float beta,
                                             const ItemRegs<RPL, Layout<K, RPL, WAVES, RESID, PER_HEAD>::EW,
                                                            Layout<K, RPL, WAVES, RESID, PER_HEAD>::QKT>& R,
                                             float (*s_qk)[2 * K], float (*s_red)[WAVES], float4* s_ek) {
  using L = Layout<K, RPL, WAVES, RESID, PER_HEAD>;
  constexpr bool EK_LDS = kResidInLds<RPL, RESID, PER_HEAD> && !EK_REGS;
  constexpr int LPR = L::LPR;
  const int odt = p.out_dtype();
  char* obase = static_cast<char*>(p.out) + ((int64_t)ic.n * p.HV + ic.hv) * p.V * (odt == kF32 ? 4 : 2);

  if (!ic.live) {
    // NULL block (slot <= 0): zeros, no state access
    // (quantized_packed_decode.py:132-136); out-of-range ids: NaN.
    const float fill = (ic.slot <= 0) ? 0.0f : __uint_as_float(0x7fc00000u);
    if (c == 0) {
#pragma unroll
      for (int i = 0; i < RPL; ++i) {
        const int r = row0 + i * L::RPI;
        if (r < p.V) store_act_at(obase, (uint32_t)r, odt, fill);
      }
    }
    return;
  }

  stage_qk<K, L::QKT, L::NT, ACT>(p, R.qk, c, parity, s_qk);
  const float* buf = s_qk[parity];
  // k and q are read from LDS for every row (not held in registers across
  // rows): 32 fewer VGPRs, so more waves per SIMD hide latency.
  const float4* q4 = reinterpret_cast<const float4*>(buf + c * 16);
  const float4* k4 = reinterpret_cast<const float4*>(buf + K + c * 16);

  // the updated state goes to the destination slot (the source slot when the
  // step is in place); a destination outside [1, num_slots) stores nothing
  const bool dst_ok = DST ? ic.dlive : true;
  const int64_t dslot = DST ? (ic.dlive ? ic.dslot : 0) : ic.slot;
  constexpr bool MASKED = MASK != kMaskNone;
  const int KA = MASKED ? p.K : K;  // state bytes per row
  const int RKA = MASKED ? (RESID == kResidInt4 ? p.K / 2 : p.K) : L::RK;  // residual bytes per row
  const bool lane_in = MASK != kMaskLanes || c * 16 < KA;  // kMaskLanes: the lane's bytes exist
  constexpr int RKL = L::RK / LPR;  // residual bytes per lane
  int8_t* sbase = p.state + dslot * p.stride_state + (int64_t)ic.hv * p.V * KA;
  int8_t* ebase = p.resid + dslot * p.stride_resid + (int64_t)ic.hv * p.V * RKA;
  float* scb = p.sscale + dslot * p.stride_sscale + (int64_t)ic.hv * p.V;
  float* rsb = PER_HEAD ? p.rscale + dslot * p.stride_rscale + ic.hv
                        : p.rscale + dslot * p.stride_rscale + (int64_t)ic.hv * p.V;
  const float es_head = R.es_in[0];

  float ekeep[PER_HEAD && !EK_LDS ? RPL : 1][16];
  // Per-row residual scales: lane c of a row group stores row c's output and
  // both scales after the row loop (every lane of the group holds the reduced
  // values), so one store instruction covers the group's RPL rows instead of
  // one 32-byte piece per row (per-row int4, us: B=1 4.76 -> 4.68, B=128
  // 47.3 -> 46.4; the per-head shape measured level and keeps its stores).
  constexpr bool MERGED = !PER_HEAD && LPR >= RPL;
  float o_keep[RPL], s_keep[RPL], es_keep[RPL];
  float4* ek = s_ek + (wave * RPL * 4) * 64 + lane;  // this lane's slots (EK_LDS)
  float eamax_local = 0.0f;

#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const int r = row0 + i * L::RPI;
    const bool valid = r < p.V;
    const uint32_t cws[4] = {R.cw[i].x, R.cw[i].y, R.cw[i].z, R.cw[i].w};
    asm volatile("" ::: "memory");  // re-read k, q from LDS for this row
    float kk[16], qq[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 b4 = k4[j];
      kk[4 * j] = b4.x, kk[4 * j + 1] = b4.y, kk[4 * j + 2] = b4.z, kk[4 * j + 3] = b4.w;
    }

    // dequantize + decay
    float h[16];
    if constexpr (MODE == kFast) {
      const float sa = R.s_in[i] * alpha;
#pragma unroll
      for (int j = 0; j < 16; ++j) h[j] = code_i8(cws[j >> 2], j & 3) * sa;
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) h[j] = (code_i8(cws[j >> 2], j & 3) * R.s_in[i]) * alpha;
    }

    // delta rule: rd = h^T k, dv = beta (v - rd), h += k dv, o = h^T q
    float rd = h[0] * kk[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) rd = fmaf(h[j], kk[j], rd);
    rd = group_sum<LPR>(rd);
    const float dv = beta * (act_decode<ACT>(R.vv[i]) - rd);
#pragma unroll
    for (int j = 0; j < 16; ++j) h[j] = madd<MODE>(kk[j], dv, h[j]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 a4 = q4[j];
      qq[4 * j] = a4.x, qq[4 * j + 1] = a4.y, qq[4 * j + 2] = a4.z, qq[4 * j + 3] = a4.w;
    }
    float o = h[0] * qq[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) o = fmaf(h[j], qq[j], o);
    o = group_sum<LPR>(o);
    asm volatile("" : "+v"(o));  // finish the sum here, where its DPP steps fuse into adds
    if constexpr (MERGED) {
      o_keep[i] = o;
    } else {
      if (c == 0 && valid) store_act_at(obase, (uint32_t)r, odt, o);
    }

    // add the carried residual: t = h + e_code * e_scale
    const float es_in = PER_HEAD ? es_head : R.es_in[i];
    float t[16];
    if constexpr (RESID == kResidInt4) {
      // codes arrive as code/16 (exact), so scale by 16*es (exact)
      float ec[16];
      decode_i4x8_div16(R.ew[i][0], ec);
      decode_i4x8_div16(R.ew[i][1], ec + 8);
      const float es16 = es_in * 16.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j) t[j] = madd<MODE>(ec[j], es16, h[j]);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) t[j] = madd<MODE>(code_i8(R.ew[i][j >> 2], j & 3), es_in, h[j]);
    }

    // requantize the state
    float am = fabsf(t[0]);
#pragma unroll
    for (int j = 1; j < 16; ++j) am = fmaxf(am, fabsf(t[j]));
    am = group_max<LPR>(am);
    const float s_new = fmaxf(div_small_int(am, p.qmax, p.rqmax), kEps);
    const float inv = recip_rn(s_new);
    uint32_t yb[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float code = quantize<MODE>(t[j], s_new, inv, yb[j]);
      t[j] = residual<MODE>(t[j], code, s_new);
    }
    const bool store = valid && dst_ok;
    if (store) {
      const uint32_t w[4] = {pack_low_bytes(yb[0], yb[1], yb[2], yb[3]), pack_low_bytes(yb[4], yb[5], yb[6], yb[7]),
                             pack_low_bytes(yb[8], yb[9], yb[10], yb[11]), pack_low_bytes(yb[12], yb[13], yb[14], yb[15])};
      if constexpr (MASK == kMaskBytes) {
        st_bytes_masked<4>(sbase + (uint32_t)(r * KA + c * 16), w, KA - c * 16);
      } else if constexpr (MASK == kMaskWords) {
        st_words_masked<4>(sbase + (uint32_t)(r * KA + c * 16), w, KA - c * 16);
      } else if constexpr (MASK == kMaskLanes) {
        if (lane_in) st_stream16(sbase + (uint32_t)(r * KA + c * 16), u32x4{w[0], w[1], w[2], w[3]});
      } else {
        st_stream16(sbase + (uint32_t)(r * K + c * 16), u32x4{w[0], w[1], w[2], w[3]});
      }
      if constexpr (!MERGED) {
        if (c == 0) st_at<float>(scb, (uint32_t)r * 4u, s_new);
      }
    }
    if constexpr (MERGED) s_keep[i] = s_new;

    float ea = fabsf(t[0]);
#pragma unroll
    for (int j = 1; j < 16; ++j) ea = fmaxf(ea, fabsf(t[j]));

    if constexpr (PER_HEAD) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if constexpr (EK_LDS) {
          if ((j & 3) == 3) ek[(i * 4 + (j >> 2)) * 64] = make_float4(t[j - 3], t[j - 2], t[j - 1], t[j]);
        } else {
          ekeep[i][j] = t[j];
        }
      }
      eamax_local = fmaxf(eamax_local, valid ? ea : 0.0f);  // rows past V hold re-read data
    } else {
      ea = group_max<LPR>(ea);
      const float es = fmaxf(div_small_int(ea, ResidRange<RESID>::q, __uint_as_float(ResidRange<RESID>::rq_bits)), kEps);
      const float inv_e = recip_rn(es);
      uint32_t eb[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) (void)quantize<MODE>(t[j], es, inv_e, eb[j]);
      if (store) {
        if constexpr (MASK == kMaskBytes) {
          store_resid_masked<RESID>(ebase + (uint32_t)(r * RKA + c * RKL), eb, RKA - c * RKL);
        } else if constexpr (MASK == kMaskWords) {
          store_resid_words<RESID>(ebase + (uint32_t)(r * RKA + c * RKL), eb, RKA - c * RKL);
        } else if (lane_in) {
          store_resid<RESID>(ebase + (uint32_t)(r * RKA + c * RKL), eb);
        }
        if constexpr (!MERGED) {
          if (c == 0) st_at<float>(rsb, (uint32_t)r * 4u, es);
        }
      }
      if constexpr (MERGED) es_keep[i] = es;
    }
  }
  if constexpr (MERGED) {
    if (c < RPL) {
      float ov = o_keep[0], sv = s_keep[0], ev = es_keep[0];
#pragma unroll
      for (int j = 1; j < RPL; ++j) {
        ov = c == j ? o_keep[j] : ov;
        sv = c == j ? s_keep[j] : sv;
        ev = c == j ? es_keep[j] : ev;
      }
      const int r = row0 + c * L::RPI;
      if (r < p.V) {
        store_act_at(obase, (uint32_t)r, odt, ov);
        if (dst_ok) {
          st_at<float>(scb, (uint32_t)r * 4u, sv);
          st_at<float>(rsb, (uint32_t)r * 4u, ev);
        }
      }
    }
  }

  if constexpr (PER_HEAD) {
    // one residual scale for the whole (slot, head)
    const float wm = wave_max(eamax_local);
    if (lane == 0) s_red[parity][wave] = wm;
    __syncthreads();
    float ea = s_red[parity][0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) ea = fmaxf(ea, s_red[parity][w]);
    const float es = fmaxf(div_small_int(ea, ResidRange<RESID>::q, __uint_as_float(ResidRange<RESID>::rq_bits)), kEps);
    const float inv_e = recip_rn(es);
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
      const int r = row0 + i * L::RPI;
      uint32_t eb[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float ev;
        if constexpr (EK_LDS) {
          const float4 e4 = ek[(i * 4 + (j >> 2)) * 64];
          ev = (j & 3) == 0 ? e4.x : (j & 3) == 1 ? e4.y : (j & 3) == 2 ? e4.z : e4.w;
        } else {
          ev = ekeep[i][j];
        }
        (void)quantize<MODE>(ev, es, inv_e, eb[j]);
      }
      if (r < p.V && dst_ok) {
        if constexpr (MASK == kMaskBytes) {
          store_resid_masked<RESID>(ebase + (uint32_t)(r * RKA + c * RKL), eb, RKA - c * RKL);
        } else if constexpr (MASK == kMaskWords) {
          store_resid_words<RESID>(ebase + (uint32_t)(r * RKA + c * RKL), eb, RKA - c * RKL);
        } else if (lane_in) {
          store_resid<RESID>(ebase + (uint32_t)(r * RKA + c * RKL), eb);
        }
      }
    }
    if (threadIdx.x == 0 && dst_ok) *rsb = es;
  }
}

// Timeline build (compiled with CK_TIMELINE=1 into a separate library; the
// product library has none of this): lane 0 of each workgroup writes
// s_memrealtime (a 100 MHz counter) into p.timeline[blockIdx.x * kTlSlots + s]:
// s = 0 at its start; for item k (k >= 9 reuses k = 9's slots) s = 1 + 3k when
// the item's processing begins, 2 + 3k once all of its loads have landed,
// 3 + 3k when its stores are issued; s = 31 holds the HW_ID register (low
// word) and the XCC id (high word) of the CU it ran on; s = 32 once the
// first item's slot id is known, 33 once its loads are issued, 34 once the
// first gates are computed.
constexpr int kTlSlots = 40;
constexpr int kTlMaxWorkgroups = 8192;

__device__ __forceinline__ void tl_mark(const PackedParams& p, int slot) {
#if CK_TIMELINE
  const uint64_t t = __builtin_amdgcn_s_memrealtime();
  if (p.timeline && threadIdx.x == 0 && blockIdx.x < kTlMaxWorkgroups) p.timeline[blockIdx.x * kTlSlots + slot] = t;
#else
  (void)p;
  (void)slot;
#endif
}

__device__ __forceinline__ void tl_start(const PackedParams& p) {
#if CK_TIMELINE
  tl_mark(p, 0);
  if (p.timeline && threadIdx.x == 0 && blockIdx.x < kTlMaxWorkgroups) {
    const uint32_t hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);    // HW_REG_HW_ID
    const uint32_t xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);  // HW_REG_XCC_ID
    p.timeline[blockIdx.x * kTlSlots + 31] = ((uint64_t)xcc << 32) | hw;
  }
#else
  (void)p;
#endif
}

__device__ __forceinline__ int tl_item_slot(int k, int phase) { return 1 + 3 * (k < 9 ? k : 9) + phase; }

// Timeline build: wait until every load of the item in R has landed (the
// vector memory counter retires in order, so waiting for the last-issued
// values waits for all of them), then mark.
template <typename Regs>
__device__ __forceinline__ void tl_data_ready(const PackedParams& p, int k, const Regs& R) {
#if CK_TIMELINE
  constexpr int rpl = sizeof(R.s_in) / sizeof(R.s_in[0]);
  constexpr int qkt = sizeof(R.qk) / sizeof(R.qk[0]);
  asm volatile("" ::"v"(R.cw[rpl - 1].w), "v"(R.ew[rpl - 1][0]), "v"(R.qk[qkt - 1]), "v"(R.es_in[0]),
               "v"(R.vv[rpl - 1]), "v"(R.s_in[rpl - 1]));
  tl_mark(p, tl_item_slot(k, 1));
#else
  (void)p;
  (void)k;
  (void)R;
#endif
}

// The items of one workgroup: first, first + step, ... (count of them).
struct WorkSeq {
  int first, step, count;
};

// Item sequence of this workgroup. Plain: blockIdx.x + j * gridDim.x.
//
// Shared (P = cu_share_n > 1 resident workgroups per CU, a grid of P x CUs,
// at least two items per workgroup): the dispatcher places one workgroup on
// every CU before it fills the next slot, so with m = G / P the workgroups
// q, q + m, ..., q + (P-1) m share a CU, in order of age a = b / m, and the
// instruction arbiter issues from the oldest waves first. Measured on MI355X
// (per-workgroup timestamps of one launch) an older workgroup computes an
// item in a fraction of a younger one's time; with an even split the older
// ones finish first and the last ones run alone at a fraction of the CU's
// wave count. So the group's items q + j m (j = 0 .. n-1) are shared
// unevenly: age a takes the j from ceil(n * c_a / 64) up to the next age's
// start, where c_a is the sum of the shares (bytes of cu_shares) of the
// older ages. Any shares are correct (each item is taken exactly once); they
// only change when the workgroups of a CU finish.
__device__ __forceinline__ WorkSeq work_seq(int items, int share_n, uint32_t shares, int G) {
  const int b = (int)blockIdx.x;
  WorkSeq w;
  if (share_n > 1 && G % share_n == 0 && items >= 2 * G) {
    const int m = G / share_n;
    const int age = b / m;
    const int q = b - age * m;
    const int n = (items - q + m - 1) / m;
    int c_lo = 0;
    for (int a = 0; a < age; ++a) c_lo += (int)((shares >> (8 * a)) & 0xffu);
    const int c_hi = c_lo + (int)((shares >> (8 * age)) & 0xffu);
    const int j0 = (n * c_lo + 63) / 64;
    const int j1 = age == share_n - 1 ? n : (n * c_hi + 63) / 64;
    w.first = q + j0 * m;
    w.step = m;
    w.count = max(j1 - j0, 0);
  } else {
    w.first = b;
    w.step = G;
    w.count = b < items ? (items - b + G - 1) / G : 0;
  }
  w.first = __builtin_amdgcn_readfirstlane(w.first);
  w.step = __builtin_amdgcn_readfirstlane(w.step);
  w.count = __builtin_amdgcn_readfirstlane(w.count);
  return w;
}

// Shares (64ths, byte a = age a) for two and for four resident workgroups
// per CU, from the per-age item times measured on the int4 steps: two 8-wave
// workgroups (per-head residual scale) about 5:3; four 4-wave workgroups
// (per-row residual scale) about 19:17:15:13.
#ifndef CK_CU_SHARES2
#define CK_CU_SHARES2 (40u | (24u << 8))
#endif
#ifndef CK_CU_SHARES4
#define CK_CU_SHARES4 (19u | (17u << 8) | (15u << 16) | (13u << 24))
#endif

// Sets the item sharing of a persistent launch of `grid` workgroups, given
// the kernel's occupancy per CU and the resident grid.
inline void set_cu_shares(PackedParams& p, int grid, int resident, int per_cu) {
  p.cu_share_n = 0;
  p.cu_shares = 0;
  if (grid != resident) return;
  if (per_cu == 2) {
    p.cu_share_n = 2;
    p.cu_shares = CK_CU_SHARES2;
  } else if (per_cu == 4) {
    p.cu_share_n = 4;
    p.cu_shares = CK_CU_SHARES4;
  }
}

// Gates of this workgroup's items number kbase .. kbase+63 (one per lane).
__device__ __forceinline__ void gates_for_items(const PackedParams& p, const Geom& gm, const WorkSeq& w, int kbase,
                                                int lane, float& alpha_v, float& beta_v) {
  // Branch-free over lanes (lanes past the last item recompute the last
  // item's gates, which are never read): a divergent region here would move
  // the uniform dtype/stride values into VGPRs that stay live over the loop.
  const int item = min(w.first + (kbase + lane) * w.step, gm.items - 1);
  const uint32_t nh = fdiv((uint32_t)item, gm.nvt);
  const uint32_t n = fdiv(nh, gm.hv);
  const int hv = (int)(nh - n * gm.hv.d);
  // all four loads are issued before any value is decoded: a conversion next
  // to its load would wait for every load in flight (including the items')
  const ActBits ra = load_act_bits(p.a, (int64_t)n * p.stride_a + hv, p.a_dtype());
  const ActBits rb = load_act_bits(p.b, (int64_t)n * p.stride_b + hv, p.b_dtype());
  const ActBits rA = load_act_bits(p.A_log, hv, p.A_log_dtype());
  const ActBits rd = load_act_bits(p.dt_bias, hv, p.dt_bias_dtype());
  ck_gates(decode_act_bits(ra, p.a_dtype()), decode_act_bits(rb, p.b_dtype()), decode_act_bits(rA, p.A_log_dtype()),
           decode_act_bits(rd, p.dt_bias_dtype()), &alpha_v, &beta_v);
}

// Gates (alpha, beta) of every item of a workgroup, computed before its item
// loop into LDS: chunk v of 64 items goes to wave v (ROTATE: wave v - b mod
// WAVES in workgroup b), the next to wave v + WAVES, so a workgroup of up to
// 64 items evaluates them in one wave. Nothing in the item loop refers to the
// gate inputs, so their pointers, strides and dtype tests are dead there (a
// refresh of a per-wave gate table inside the loop kept them live and spilled
// 36 SGPRs to VGPR lanes in the K=128 8-wave kernel). The item loop reads
// them after a barrier ahead of its first item; the host keeps a launch's
// items per workgroup at or below kGateCap (launch_item_cap).
//
// A wave with no chunk waits here for its first item's loads, as a gate wave
// does for the gate inputs issued after them (the vector memory counter
// retires in order), so no wave issues its second item's loads while its
// first item's are still arriving: at start-up every workgroup of the grid
// loads at once, and the first items' data then lands earlier (per-head int4,
// us: B=1 6.3 -> 5.9, B=64 27.0 -> 26.7, B=256 84.8 -> 84.4). Which wave
// evaluates the gates was measured per shape: the first-dispatched wave for
// the 8-wave per-head workgroups (rotated: B=1 6.3), rotated for the four
// 4-wave per-row workgroups of a CU (wave 0 in every one: B=128 47.3 us
// against 45.5).
constexpr int kGateCap = 256;
constexpr int kWaitVmcnt0 = 0x0f70;  // s_waitcnt simm16: vmcnt 0, expcnt 7, lgkmcnt 15 (vector memory only)

// One item's gates into s_gate[0], for the kernels with one item per
// workgroup: every wave issues the item's four gate-input loads (uniform
// addresses: scalar loads, which retire independently of the vector loads)
// next to the item's own loads; wave 0 evaluates the gates once those arrive,
// while the item's bytes are still in flight (graph-replayed, int4 per head,
// HV=32, us: B=1 5.35 -> 5.09, B=8 6.33 -> 5.82, B=64 25.06 -> 24.58, three
// A/B pairs), against loading them after the item and evaluating them lane-
// parallel as stage_gates does. The caller issues its item's vector loads
// before stage_item_gates (the one-item kernel issues them before
// load_item_gate_bits too) and passes a barrier before reading s_gate[0].
struct GateBits {
  ActBits a, b, A_log, dt_bias;
};

__device__ __forceinline__ GateBits load_item_gate_bits(const PackedParams& p, const ItemCoord& ic) {
  return GateBits{load_act_bits_sel(p.a, (int64_t)ic.n * p.stride_a + ic.hv, p.a_dtype()),
                  load_act_bits_sel(p.b, (int64_t)ic.n * p.stride_b + ic.hv, p.b_dtype()),
                  load_act_bits_sel(p.A_log, ic.hv, p.A_log_dtype()),
                  load_act_bits_sel(p.dt_bias, ic.hv, p.dt_bias_dtype())};
}

__device__ __forceinline__ void stage_item_gates(const PackedParams& p, const GateBits& g, int wave, int lane,
                                                 float2* s_gate) {
  // All four words are required here at once, so their scalar loads are issued
  // together and waited for with one counter wait. Left alone, the compiler
  // sinks each load next to its decode, behind the previous input's dtype
  // branch: four load latencies in a row (B=64 24.61 -> 24.15 us, B=128 per
  // head 43.5 -> 43.0 us).
  asm volatile("" ::"s"(g.a.word), "s"(g.b.word), "s"(g.A_log.word), "s"(g.dt_bias.word));
  if (wave == 0) {
    float alpha, beta;
    ck_gates(decode_act_bits(g.a, p.a_dtype()), decode_act_bits(g.b, p.b_dtype()),
             decode_act_bits(g.A_log, p.A_log_dtype()), decode_act_bits(g.dt_bias, p.dt_bias_dtype()), &alpha, &beta);
    if (lane == 0) s_gate[0] = make_float2(alpha, beta);
  }
}

template <int WAVES, bool ROTATE>
__device__ __forceinline__ void stage_gates(const PackedParams& p, const Geom& gm, const WorkSeq& w, int wave,
                                            int lane, float2* s_gate) {
  const int n = min(w.count, kGateCap);
  const int v = ROTATE ? (wave + (int)blockIdx.x) % WAVES : wave;
  for (int kb = v * 64; kb < n; kb += WAVES * 64) {
    float a, b;
    gates_for_items(p, gm, w, kb, lane, a, b);
    if (kb + lane < n) s_gate[kb + lane] = make_float2(a, b);
  }
  if (v * 64 >= n) __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
}

// Item of workgroup b in the kernels with one item per workgroup. The
// dispatcher hands workgroups to the 8 XCDs in turn (b % 8), each XCD with its
// own L2. This bijection of [0, items) keeps each request's items (its heads
// and their row tiles) on one XCD, against a request's heads spread over all
// eight in blockIdx order (graph-replayed, int4 per head, HV=32, three A/B
// pairs, us: B=1 5.00 -> 4.87, B=8 5.83 -> 5.47, B=64 24.02 -> 23.53, B=128
// 43.1 -> 42.2, B=256 80.4 -> 78.2). It deals the first 8 * (B / 8) requests
// to the XCDs in turn, XCD x taking x, x + 8, x + 16, ..., in that order on
// even XCDs and in reverse on odd ones; the items of the last B % 8 requests
// are cut into 8 contiguous ranges, one per XCD. Against 8 contiguous ranges
// of the whole launch (B / 8 requests per XCD), dealing keeps a batch padded
// at its end with NULL slot ids (a captured batch size) spread over all
// XCDs, and the reversal keeps the requests running at one time apart in
// memory (two A/B pairs, us: 24 layers x B=64 with 48 live requests 492 ->
// 433 per token, all live 548 -> 531; B=64 on consecutive slots 24.6 ->
// 23.8; random slots B=40 17.06 -> 17.01, B=64 24.36 -> 24.33, B=256 79.07
// -> 78.85; dealing without the reversal: 440, 539, 24.3, 17.20, 24.52,
// 79.06). `base` = (B / 8) * items per request, each XCD's workgroups before
// that tail (0: the whole launch in contiguous ranges). Any other dispatch
// order leaves it a permutation of the items.
template <bool DST>
__device__ __forceinline__ ItemCoord xcd_item_coord(const PackedParams& p, const Geom& gm,
                                                    const int32_t* __restrict__ idx,
                                                    const int32_t* __restrict__ dst_idx, int b, int base) {
  const int x = b & 7, j = b >> 3;
  const bool dealt = j < base;  // XCD x's i-th dealt request is request x + 8 i
  const int tail = gm.items - 8 * base;
  const int q = tail >> 3, r = tail & 7;  // XCDs below r take q + 1 tail items, the others q
  // the item's number within the XCD's dealt requests (odd XCDs: from the
  // last), or within the launch
  const uint32_t u = dealt ? (uint32_t)((x & 1) ? base - 1 - j : j)
                           : (uint32_t)(8 * base + x * q + min(x, r) + (j - base));
  const uint32_t nh = fdiv(u, gm.nvt);
  const uint32_t i = fdiv(nh, gm.hv);
  ItemCoord ic;
  ic.vt = __builtin_amdgcn_readfirstlane((int)(u - nh * gm.nvt.d));
  ic.hv = __builtin_amdgcn_readfirstlane((int)(nh - i * gm.hv.d));
  ic.n = __builtin_amdgcn_readfirstlane(dealt ? x + 8 * (int)i : (int)i);
  slot_coord<DST>(p, gm, idx, dst_idx, ic);
  return ic;
}

// (B / 8) * items per request: the `base` of xcd_item_coord.
inline int xcd_base(int B, int per_request) { return (B >> 3) * per_request; }

// The decode kernel chosen for the process (tests): automatic, or one of the
// two for every launch (CARRYKERNEL_DECODE_KERNEL, read once, or
// ck_set_decode_kernel in packed_decode.hip).
constexpr int kDecodeKernelAuto = 0;
constexpr int kDecodeKernelPersistent = 1;
constexpr int kDecodeKernelOneItem = 2;
int decode_kernel_override();

// A lower limit on the items of one launch set for the process (0: none):
// CARRYKERNEL_MAX_ITEMS_PER_LAUNCH, read once, or ck_set_max_items_per_launch
// (packed_decode.hip). Used by the tests of the split.
int64_t max_items_override();

// Items one launch may hold so that no workgroup gets more than kGateCap:
// a workgroup's items come from one CU group of ceil(items / m) items, m =
// resident / per_cu (work_seq; the plain stride gives fewer), or fewer if the
// process sets a lower limit (max_items_override).
inline int64_t launch_item_cap(int resident, int per_cu) {
  int64_t cap = (int64_t)kGateCap * (resident / (per_cu > 1 ? per_cu : 1));
  const int64_t v = max_items_override();
  if (v > 0 && v < cap) cap = v;
  return cap;
}

// The same step for requests n0 .. of p: per-request inputs, outputs and ids
// advanced by n0 requests (the pool and the per-head inputs are shared).
inline PackedParams requests_from(const PackedParams& p, int n0) {
  auto esz = [](int dt) { return dt == kF32 ? 4 : 2; };
  PackedParams q = p;
  q.mixed = static_cast<const char*>(p.mixed) + (int64_t)n0 * p.stride_mixed * esz(p.dtypes & 15);
  q.a = static_cast<const char*>(p.a) + (int64_t)n0 * p.stride_a * esz((p.dtypes >> 4) & 15);
  q.b = static_cast<const char*>(p.b) + (int64_t)n0 * p.stride_b * esz((p.dtypes >> 8) & 15);
  q.out = static_cast<char*>(p.out) + (int64_t)n0 * p.HV * p.V * esz((p.dtypes >> 20) & 15);
  q.idx = p.idx + (int64_t)n0 * p.stride_idx;
  if (p.dst_idx) q.dst_idx = p.dst_idx + (int64_t)n0 * p.stride_dst_idx;
  return q;
}

// Waves per SIMD the register allocation must allow: two 8-wave or four
// 4-wave workgroups per CU need 4 (<= 128 VGPRs); other shapes take what they
// need.
template <int RPL, int WAVES>
constexpr int kMinWavesPerEU = (RPL == 2 && (WAVES == 8 || WAVES == 4)) ? 4 : 1;

// The one-item kernel's register budget: the per-head 8-wave shape at 80
// VGPRs (six waves per SIMD: three workgroups per CU), others as above.
template <int RPL, int WAVES, bool PER_HEAD>
constexpr int kSingleWavesPerEU = (PER_HEAD && RPL == 2 && WAVES == 8) ? 6 : kMinWavesPerEU<RPL, WAVES>;

template <int K, int RPL, int WAVES, int RESID, bool PER_HEAD, int MODE, int ACT, bool DST>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(kMinWavesPerEU<RPL, WAVES>)))
void packed_decode_kernel(const int32_t* __restrict__ idx, int items, int stride_idx, uint32_t nvt_d, uint32_t nvt_m,
                          uint32_t nvt_sh, uint32_t hv_d, uint32_t hv_m, uint32_t hv_sh, int share_n, uint32_t shares,
                          int grid, const PackedParams p, const int32_t* __restrict__ dst_idx) {
  using L = Layout<K, RPL, WAVES, RESID, PER_HEAD>;
  const Geom gm{items, stride_idx, share_n, shares, FastDiv{nvt_d, nvt_m, nvt_sh}, FastDiv{hv_d, hv_m, hv_sh}, grid};
  __shared__ __attribute__((aligned(16))) float s_qk[4][2 * K];  // [parity] staged, [2 + parity] raw
  __shared__ float s_red[2][WAVES];
  __shared__ float4 s_ek[kResidInLds<RPL, RESID, PER_HEAD> ? WAVES * RPL * 4 * 64 : 1];
  __shared__ float2 s_gate[kGateCap];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane % L::LPR;
  const int g = lane / L::LPR;
  tl_start(p);

  const WorkSeq w = work_seq(gm.items, gm.share_n, gm.shares, gm.grid);
  if (w.count <= 0) return;  // whole workgroup
  int item = w.first;
  const int last = gm.items - 1;
  const int item_end = w.first + w.count * w.step;  // one past this workgroup's last item

  // LDS buffers alternate between consecutive live items (a NULL item skips
  // the barriers, so the parity follows a count of live items): two uses of
  // one buffer are always separated by the barrier of the live item between.
  ItemRegs<RPL, L::EW, L::QKT> A, B;
  ItemCoord ca = item_coord<false, DST>(p, gm, idx, dst_idx, item), cb;
#if CK_TIMELINE
  asm volatile("" ::"s"((int)ca.slot));
  tl_mark(p, 32);
#endif
  load_item<K, RPL, WAVES, RESID, PER_HEAD, ACT>(p, ca, true, ca.vt * L::ROWS_WG + wave * L::ROWS_WAVE + g, c, A);
  tl_mark(p, 33);
  stage_gates<WAVES, !PER_HEAD>(p, gm, w, wave, lane, s_gate);  // its loads overlap the first item's
  tl_mark(p, 34);
  int k = 0;     // item number within this workgroup
  int live = 0;  // live items processed so far
  for (;;) {
    // ---- item k in A; prefetch item k+1 into B (past the end: re-read the last item) ----
    int next = item + w.step;
    cb = item_coord<false, DST>(p, gm, idx, dst_idx, min(next, last));
    load_item<K, RPL, WAVES, RESID, PER_HEAD, ACT>(p, cb, next < item_end, cb.vt * L::ROWS_WG + wave * L::ROWS_WAVE + g, c, B);
    {
      if (k == 0) __syncthreads();  // the staged gates are visible from here on
      const float2 gab = s_gate[min(k, kGateCap - 1)];
      tl_mark(p, tl_item_slot(k, 0));
      tl_data_ready(p, k, A);
      process_item<K, RPL, WAVES, RESID, PER_HEAD, MODE, ACT, DST>(p, ca, ca.vt * L::ROWS_WG + wave * L::ROWS_WAVE + g, c,
                                                          lane, wave, live & 1, gab.x, gab.y, A, s_qk, s_red, s_ek);
      live += ca.live ? 1 : 0;
      tl_mark(p, tl_item_slot(k, 2));
    }
    if (next >= item_end) break;
    ++k;
    item = next;

    // ---- item k in B; prefetch item k+1 into A ----
    next = item + w.step;
    ca = item_coord<false, DST>(p, gm, idx, dst_idx, min(next, last));
    load_item<K, RPL, WAVES, RESID, PER_HEAD, ACT>(p, ca, next < item_end, ca.vt * L::ROWS_WG + wave * L::ROWS_WAVE + g, c, A);
    {
      const float2 gab = s_gate[min(k, kGateCap - 1)];
      tl_mark(p, tl_item_slot(k, 0));
      tl_data_ready(p, k, B);
      process_item<K, RPL, WAVES, RESID, PER_HEAD, MODE, ACT, DST>(p, cb, cb.vt * L::ROWS_WG + wave * L::ROWS_WAVE + g, c,
                                                          lane, wave, live & 1, gab.x, gab.y, B, s_qk, s_red, s_ek);
      live += cb.live ? 1 : 0;
      tl_mark(p, tl_item_slot(k, 2));
    }
    if (next >= item_end) break;
    ++k;
    item = next;
  }
}

// One item per workgroup: its loads, the gates, the item, with no prefetch of
// a next item; the grid is one workgroup per item and the hardware dispatcher
// starts the next one on whichever CU frees a slot. Used (launch_cfg) when a
// launch has no more items than resident workgroups, and for larger launches
// when this kernel holds more workgroups per CU than the persistent one does
// with its second register set, or as many and at least two (a CU then
// overlaps one workgroup's loads with another's arithmetic without a
// prefetch).
//  * Small launches: the persistent loop would issue a past-the-end prefetch
//    before the item and, at the joins of its conditional stores, wait for
//    some of those loads; this kernel has no younger loads to wait for
//    (graph-replayed, int4, HV=32, us: per head B=1 5.70 -> 5.13, B=8 6.89 ->
//    6.36; per row B=1 4.53 -> 4.01).
//  * Larger launches: at K=128 per head it takes 80 VGPRs, three 8-wave
//    workgroups per CU against the persistent kernel's two (128 VGPRs), and
//    per row 56-62 VGPRs, eight 4-wave workgroups against four; the
//    dispatcher then also balances the end of the launch across CUs (two A/B
//    pairs on one box, us: per head B=64 28.57 -> 28.15, B=128 48.80 -> 47.24,
//    B=256 86.49 -> 85.08; per row B=64 28.07 -> 26.81, B=128 47.74 -> 46.49;
//    per row K=64 B=64 16.03 -> 15.27). With the int8 residual per head it
//    keeps the head's unquantized residual in VGPRs (80, three workgroups per
//    CU) where the persistent kernel needs a 64 KB LDS table (two): int8 per
//    head B=64 30.95 -> 28.61, B=256 107.7 -> 101.8 (three A/B pairs). At
//    equal occupancy it is faster too, once its start-up chain was shortened
//    (one box, us: per head K=64 B=256 45.3 -> 42.6, K=32 29.4 -> 26.5, K=16
//    18.9 -> 16.3; per row K=32 B=256 28.7 -> 25.9, K=16 18.9 -> 16.5).
// process_item computes the item in both kernels, so the results are the same
// bits.
template <int K, int RPL, int WAVES, int RESID, bool PER_HEAD, int MODE, int ACT, bool DST>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(kSingleWavesPerEU<RPL, WAVES, PER_HEAD>)))
void packed_decode_single_kernel(const int32_t* __restrict__ idx, int items, int stride_idx, uint32_t nvt_d,
                                 uint32_t nvt_m, uint32_t nvt_sh, uint32_t hv_d, uint32_t hv_m, uint32_t hv_sh,
                                 int xcd_base, uint32_t grp_m, uint32_t grp_w, const PackedParams p_arg,
                                 const int32_t* __restrict__ dst_idx) {
  using L = Layout<K, RPL, WAVES, RESID, PER_HEAD>;
  const Geom gm{items, stride_idx, 0, 0u, FastDiv{nvt_d, nvt_m, nvt_sh}, FastDiv{hv_d, hv_m, hv_sh}, items};
  // div_grp from two preloaded arguments: the kernel then reads no kernel-
  // argument dword past l2norm, and no load of the struct's tail (div_grp
  // and its padding dword, whose register the compiler could reuse for the
  // item coordinates, making them wait for that load) precedes the slot id
  PackedParams p = p_arg;
  p.div_grp = quotient_fastdiv(grp_m, grp_w);
  __shared__ __attribute__((aligned(16))) float s_qk[4][2 * K];  // [0] staged, [2] raw
  __shared__ float s_red[2][WAVES];
  __shared__ float4 s_ek[1];  // unused: the per-head residual waits in VGPRs (EK_REGS)
  __shared__ float2 s_gate[1];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane % L::LPR;
  const int g = lane / L::LPR;
  tl_start(p);
  const ItemCoord ca = xcd_item_coord<DST>(p, gm, idx, dst_idx, (int)blockIdx.x, xcd_base);
#if CK_TIMELINE
  asm volatile("" ::"s"((int)ca.slot));
  tl_mark(p, 32);
#endif
  const int row0 = ca.vt * L::ROWS_WG + wave * L::ROWS_WAVE + g;
  ItemRegs<RPL, L::EW, L::QKT> A;
  load_item<K, RPL, WAVES, RESID, PER_HEAD, ACT>(p, ca, true, row0, c, A);
  // the item's vector loads are issued first; the gate inputs' address
  // arithmetic and scalar loads follow (scheduled ahead, they delayed the
  // first vector load)
  __builtin_amdgcn_sched_barrier(0);
  const GateBits gbits = load_item_gate_bits(p, ca);
  tl_mark(p, 33);
  stage_item_gates(p, gbits, wave, lane, s_gate);
  tl_mark(p, 34);
  __syncthreads();
  const float2 gab = s_gate[0];
  tl_mark(p, tl_item_slot(0, 0));
  tl_data_ready(p, 0, A);
  process_item<K, RPL, WAVES, RESID, PER_HEAD, MODE, ACT, DST, kMaskNone, true>(p, ca, row0, c, lane, wave, 0, gab.x,
                                                                               gab.y, A, s_qk, s_red, s_ek);
  tl_mark(p, tl_item_slot(0, 2));
}

// Resident workgroups per GPU for a kernel (occupancy x CUs), cached per
// device; *per_cu (if given) receives the occupancy per CU.
int resident_workgroups(const void* fn, int block, int* per_cu = nullptr);

template <int K, int RPL, int WAVES, int RESID, bool PER_HEAD, int MODE, int ACT, bool DST>
int launch_cfg(PackedParams p, int B, hipStream_t stream) {
  using L = Layout<K, RPL, WAVES, RESID, PER_HEAD>;
  const int nvt = PER_HEAD ? 1 : (p.V + L::ROWS_WG - 1) / L::ROWS_WG;
  const int64_t items = (int64_t)B * p.HV * nvt;
  if (items > 0x7fffffff) return fail(CK_EUNSUPPORTED, "%lld work items is too many", (long long)items);
  if (items == 0) return ok();
  p.items = (int)items;
  p.div_nvt = make_fastdiv((uint32_t)nvt);
  p.div_hv = make_fastdiv((uint32_t)p.HV);
  auto fn = packed_decode_kernel<K, RPL, WAVES, RESID, PER_HEAD, MODE, ACT, DST>;
  int per_cu = 0;
  const int resident = resident_workgroups(reinterpret_cast<const void*>(fn), WAVES * 64, &per_cu);
  if (resident <= 0) return fail(CK_ELAUNCH, "cannot query the device occupancy");
  // the one-item kernel (packed_decode_single_kernel): for a launch with no
  // more items than resident workgroups, and for a larger one when it fits
  // more workgroups per CU, or as many and at least two. With one workgroup
  // per CU the persistent kernel's prefetch is the only overlap of loads and
  // arithmetic (per head K=256, 16 waves, B=256: 208 against 240 us).
  bool single = items <= resident;
  if (!single) {
    int single_per_cu = 0;
    const void* sfn = reinterpret_cast<const void*>(packed_decode_single_kernel<K, RPL, WAVES, RESID, PER_HEAD, MODE,
                                                                               ACT, DST>);
    single = resident_workgroups(sfn, WAVES * 64, &single_per_cu) > 0 &&
             (single_per_cu > per_cu || (single_per_cu == per_cu && per_cu >= 2));
  }
  const int forced = decode_kernel_override();
  if (forced != kDecodeKernelAuto) single = forced == kDecodeKernelOneItem;
  // the persistent kernel's gate table bounds its items per launch; the
  // one-item kernel has no table, so only a process-wide limit splits it
  const int64_t override_cap = max_items_override();
  const int64_t cap = single ? (override_cap > 0 ? override_cap : items) : launch_item_cap(resident, per_cu);
  if (items > cap) {  // consecutive launches over slices of the requests
    const int64_t per_request = (int64_t)p.HV * nvt;
    if (per_request > cap) return fail(CK_EUNSUPPORTED, "%lld work items per request is too many", (long long)per_request);
    const int chunk = (int)(cap / per_request);
    for (int n0 = 0; n0 < B; n0 += chunk) {
      const int rc = launch_cfg<K, RPL, WAVES, RESID, PER_HEAD, MODE, ACT, DST>(requests_from(p, n0), min(chunk, B - n0),
                                                                              stream);
      if (rc != CK_OK) return rc;
    }
    return ok();
  }
  if (single) {
    hipLaunchKernelGGL((packed_decode_single_kernel<K, RPL, WAVES, RESID, PER_HEAD, MODE, ACT, DST>),
                       dim3((unsigned)p.items), dim3(WAVES * 64), 0, stream, p.idx, p.items, p.stride_idx,
                       p.div_nvt.d, p.div_nvt.m, p.div_nvt.sh, p.div_hv.d, p.div_hv.m, p.div_hv.sh,
                       xcd_base(B, p.HV * nvt), p.div_grp.m, quotient_word(p.div_grp), p, p.dst_idx);
    return check_launch("ck_gdn_packed_decode");
  }
  // fewest items per workgroup, then the fewest workgroups achieving it
  const int per_wg = (p.items + resident - 1) / resident;
  const int grid = (p.items + per_wg - 1) / per_wg;
  set_cu_shares(p, grid, resident, per_cu);
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(WAVES * 64), 0, stream, p.idx, p.items, p.stride_idx, p.div_nvt.d,
                     p.div_nvt.m, p.div_nvt.sh, p.div_hv.d, p.div_hv.m, p.div_hv.sh, p.cu_share_n, p.cu_shares, grid,
                     p, p.dst_idx);
  return check_launch("ck_gdn_packed_decode");
}

// Workgroup shape (numbers for K=128, where a lane row is 16 K and a wave
// instruction covers 8 rows). With per-row residual scales a workgroup is 4
// waves of 2 rows per lane (64-row tiles, four workgroups per CU) when that
// gives 512 tiles or more, else 4 waves of 1 row per lane (32-row tiles): a
// small batch's rows then spread over four times as many SIMDs, each wave
// computing a quarter of what one wave of 4 rows per lane would (B=1 to 4 at
// HV=32: 6.5 / 6.6 / 7.3 us -> 4.7 / 4.7 / 5.7 us; from B=8 the 64-row tiles
// are faster). A
// per-head residual scale needs the whole head in one workgroup; at K=128 that
// is 8 waves of 2 rows per lane: three workgroups per CU in the one-item
// kernel (80 VGPRs), two in the persistent one (128 VGPRs; the int8
// residual's unquantized values wait for the head amax in LDS there); K=64,
// 32 and 16 spread a 128-row head over more waves (below); other shapes keep
// 4 rows per lane.
template <int K, int RESID, bool PER_HEAD, int MODE, int ACT, bool DST>
int launch_k(const PackedParams& p, int B, hipStream_t stream) {
  constexpr int RPI = 64 / (K / 16);
  if constexpr (!PER_HEAD) {
    // at K=16 and 32 a wave instruction covers 64 / 32 rows, so the shapes
    // below would leave most lanes of a V=128 head idle; 128-row tiles instead
    // (per-row int4, HV=32, B=64: K=16 12.1 -> 8.5 us, K=32 13.4 -> 11.3 us)
    if constexpr (K == 16) {
      return launch_cfg<K, 1, 2, RESID, false, MODE, ACT, DST>(p, B, stream);
    } else if constexpr (K == 32) {
      return launch_cfg<K, 1, 4, RESID, false, MODE, ACT, DST>(p, B, stream);
    } else {
      if ((int64_t)B * p.HV * ((p.V + RPI * 8 - 1) / (RPI * 8)) >= 512)
        return launch_cfg<K, 2, 4, RESID, false, MODE, ACT, DST>(p, B, stream);
      return launch_cfg<K, 1, 4, RESID, false, MODE, ACT, DST>(p, B, stream);
    }
  } else {
    const int need = p.V;
    if constexpr (K == 128) {
      if (need > RPI * 4 * 2 && need <= RPI * 2 * 8) return launch_cfg<K, 2, 8, RESID, true, MODE, ACT, DST>(p, B, stream);
    }
    // K=256: 8 waves of 4 rows per lane take 230 VGPRs, one 8-wave workgroup
    // per CU; from one head per CU on, 16 waves of 2 rows (128 VGPRs, four
    // waves per SIMD) hide more latency (int4 per head, H=HV=32, graph-
    // replayed, us: B=8 10.3 -> 9.8, B=16 16.8 -> 16.0, B=64 51.1 -> 49.5);
    // fewer heads stay on the 8-wave shape (B=1 9.1 against 9.7)
    if constexpr (K == 256) {
      if (need > RPI * 4 * 4 && need <= RPI * 2 * 16 && (int64_t)B * p.HV >= 256)
        return launch_cfg<K, 2, 16, RESID, true, MODE, ACT, DST>(p, B, stream);
    }
    // fewer rows per lane over more waves for a V=128 head at small K (per-head,
    // int4, HV=32, us at B=1 / 64): K=64 2 rows x 4 waves 6.9 / 16.1 -> 5.7 /
    // 14.8; K=16 1 row x 2 waves 6.2 / 9.2 -> 4.9 / 8.7; K=32 1 row x 4 waves
    // 6.5 -> 5.0 at B=1 but 10.3 -> 11.9 at B=64, so only up to one item per CU
    if constexpr (K == 64) {
      if (need > RPI * 4 * 1 && need <= RPI * 2 * 4) return launch_cfg<K, 2, 4, RESID, true, MODE, ACT, DST>(p, B, stream);
    }
    if constexpr (K == 32) {
      if (need > RPI * 2 && need <= RPI * 4 && (int64_t)B * p.HV <= 256)
        return launch_cfg<K, 1, 4, RESID, true, MODE, ACT, DST>(p, B, stream);
    }
    if constexpr (K == 16) {
      if (need > RPI && need <= RPI * 2) return launch_cfg<K, 1, 2, RESID, true, MODE, ACT, DST>(p, B, stream);
    }
    if (need <= RPI * 4 * 1) return launch_cfg<K, 4, 1, RESID, true, MODE, ACT, DST>(p, B, stream);
    if (need <= RPI * 4 * 2) return launch_cfg<K, 4, 2, RESID, true, MODE, ACT, DST>(p, B, stream);
    if (need <= RPI * 4 * 4) return launch_cfg<K, 4, 4, RESID, true, MODE, ACT, DST>(p, B, stream);
    if (need <= RPI * 4 * 8) return launch_cfg<K, 4, 8, RESID, true, MODE, ACT, DST>(p, B, stream);
    return fail(CK_EUNSUPPORTED, "per-head residual scale supports V <= %d at K=%d, got V=%d", RPI * 32, K, p.V);
  }
}

// Dispatch over residual format, scale granularity, mode and activation dtype
// for one K (launch_for_k is defined in packed_decode_k<K>.hip).
template <int K, int ACT>
int launch_for_act(const PackedParams& p, int B, int resid_fmt, int per_head, int mode, hipStream_t s) {
  const bool i4 = resid_fmt == CK_RESID_INT4;
  if (p.dst_idx) {  // out-of-place step: instantiated for the FAST arithmetic only
    if (mode != kFast) return fail(CK_EUNSUPPORTED, "dst_state_indices needs quant_mode FAST");
    return i4 ? (per_head ? launch_k<K, kResidInt4, true, kFast, ACT, true>(p, B, s)
                          : launch_k<K, kResidInt4, false, kFast, ACT, true>(p, B, s))
              : (per_head ? launch_k<K, kResidInt8, true, kFast, ACT, true>(p, B, s)
                          : launch_k<K, kResidInt8, false, kFast, ACT, true>(p, B, s));
  }
  if (mode == kFast)
    return i4 ? (per_head ? launch_k<K, kResidInt4, true, kFast, ACT, false>(p, B, s)
                          : launch_k<K, kResidInt4, false, kFast, ACT, false>(p, B, s))
              : (per_head ? launch_k<K, kResidInt8, true, kFast, ACT, false>(p, B, s)
                          : launch_k<K, kResidInt8, false, kFast, ACT, false>(p, B, s));
  return i4 ? (per_head ? launch_k<K, kResidInt4, true, kExact, ACT, false>(p, B, s)
                        : launch_k<K, kResidInt4, false, kExact, ACT, false>(p, B, s))
            : (per_head ? launch_k<K, kResidInt8, true, kExact, ACT, false>(p, B, s)
                        : launch_k<K, kResidInt8, false, kExact, ACT, false>(p, B, s));
}

template <int K>
int launch_for_k(const PackedParams& p, int B, int resid_fmt, int per_head, int mode, int act, hipStream_t stream);

// Any K in 1 .. 256 and any row alignment (packed_decode_masked.h): the lane
// map of K rounded up to a power of two (at least 16), values past p.K zero,
// one item per workgroup; access: kMaskLanes (p.K a multiple of 16, aligned
// rows), kMaskWords (p.K a multiple of 4, 4-byte-aligned rows) or kMaskBytes.
int launch_masked(const PackedParams& p, int B, int resid_fmt, int per_head, int mode, int access,
                  hipStream_t stream);

#define CK_PD_DEFINE_LAUNCH_FOR_K(KV)                                                                     \
  template <>                                                                                             \
  int launch_for_k<KV>(const PackedParams& p, int B, int resid_fmt, int per_head, int mode, int act,      \
                       hipStream_t s) {                                                                   \
    if (act == kF32) return launch_for_act<KV, kF32>(p, B, resid_fmt, per_head, mode, s);                 \
    if (act == kBF16) return launch_for_act<KV, kBF16>(p, B, resid_fmt, per_head, mode, s);               \
    return launch_for_act<KV, kF16>(p, B, resid_fmt, per_head, mode, s);                                  \
  }

}  // namespace pd
}  // namespace ck
