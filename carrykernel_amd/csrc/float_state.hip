// GDN decode step on an unquantized state pool (fp32 or bf16), vLLM's paged
// [slots, HV, V, K] layout, updated in place. This is the comparison arm for
// the quantized step: the semantics of the upstream packed decode that
// vllm_integration/quantized_packed_decode.py:1-7 replaces (same gates, GQA,
// optional L2 norm, NULL-slot padding), with vLLM's default bf16 state.
//
// It runs on the quantized decode's machinery (packed_decode_impl.h): the same
// lane map (a lane owns 16 consecutive K of a V-row: 64 bytes of fp32 or 32 of
// bf16), persistent workgroups of 4 waves x 2 rows per lane (64-row tiles)
// looping over items with the next item's state rows, v and q/k prefetched
// into a second register set, q/k staged once per item in LDS, the gates of
// all of a workgroup's items evaluated lane-parallel into LDS before the item
// loop, DPP row reductions. Per row:
//   h_j = h_j * alpha;  rd = sum_j h_j k_j;  dv = beta * (v - rd)
//   h_j = fma(k_j, dv, h_j);  o = sum_j h_j q_j;  state <- h (bf16: RNE)
#include <hip/hip_runtime.h>

#include "ck_capi_common.h"
#include "ck_device.h"
#include "packed_decode_impl.h"

namespace ck {
namespace fs {

using pd::ItemCoord;
using pd::PackedParams;

// state dwords per lane per row: 16 fp32 or 16 bf16
template <bool BF16>
constexpr int kStateWords = BF16 ? 8 : 16;

template <int RPL, int QKT, bool BF16>
struct FloatItemRegs {
  u32x4 sw[RPL][kStateWords<BF16> / 4];  // state row chunk, raw
  uint32_t vv[RPL];                      // v per row (raw activation bits)
  uint32_t qk[QKT];                      // this thread's share of [q | k]
};

template <int K, int RPL, int WAVES>
using FLayout = pd::Layout<K, RPL, WAVES, pd::kResidInt8, false>;

// All loads of one item, branch-free (see pd::load_item): an unneeded item
// collapses onto the first bytes of slot 0; rows past V re-read row V-1.
template <int K, int RPL, int WAVES, bool BF16, int ACT>
__device__ __forceinline__ void load_fitem(const PackedParams& p, const ItemCoord& ic, bool needed, int row0, int c,
                                           FloatItemRegs<RPL, FLayout<K, RPL, WAVES>::QKT, BF16>& R) {
  using L = FLayout<K, RPL, WAVES>;
  constexpr uint32_t SB = BF16 ? 2u : 4u;  // state bytes per element
  constexpr int ESZ = act_bytes<ACT>;
  const bool real = needed && ic.live;
  const uint32_t keep = real ? 0xffffffffu : 0u;
  const int64_t slot = real ? ic.slot : 0;
  const int hv = real ? ic.hv : 0;
  const int8_t* sbase = p.state + (slot * p.stride_state + (int64_t)hv * p.V * K) * SB;
  const char* mrow = static_cast<const char*>(p.mixed) + (int64_t)ic.n * p.stride_mixed * ESZ;
  const char* vbase = mrow + (2 * (int64_t)p.H * K + (int64_t)hv * p.V) * ESZ;
#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const uint32_t r = (uint32_t)min(row0 + i * L::RPI, p.V - 1) & keep;
    const uint32_t off = ((r * K + ((uint32_t)c & keep) * 16) * SB);
    // fp32 rows: a lane's 64 bytes sit 64 bytes apart from its neighbour's, so
    // one instruction touches a quarter of each line; the ordinary (cached)
    // forms let the lines merge, where the streaming ones lose a third of the
    // bandwidth. bf16 rows (32 bytes per lane) stream.
#pragma unroll
    for (int w = 0; w < kStateWords<BF16> / 4; ++w)
      R.sw[i][w] = BF16 ? ld_stream16(sbase + off + 16u * w) : ld_at<u32x4>(sbase, off + 16u * w);
    R.vv[i] = load_act_raw<ESZ>(vbase, r * ESZ);
  }
  const char* qbase = mrow + (int64_t)pd::fdiv((uint32_t)hv, p.div_grp) * K * ESZ;
  const uint32_t koff = (uint32_t)((p.H - 1) * K);
#pragma unroll
  for (int j = 0; j < L::QKT; ++j) {
    const uint32_t e = min((uint32_t)threadIdx.x + j * L::NT, (uint32_t)(2 * K - 1));
    R.qk[j] = load_act_raw<ESZ>(qbase, ((e < K ? e : e + koff) * ESZ) & keep);
  }
}

template <int K, int RPL, int WAVES, bool BF16, int ACT>
__device__ __forceinline__ void process_fitem(const PackedParams& p, const ItemCoord& ic, int row0, int c,
                                              int parity, float alpha, float beta,
                                              const FloatItemRegs<RPL, FLayout<K, RPL, WAVES>::QKT, BF16>& R,
                                              float (*s_qk)[2 * K]) {
  using L = FLayout<K, RPL, WAVES>;
  constexpr int LPR = L::LPR;
  constexpr uint32_t SB = BF16 ? 2u : 4u;
  const int odt = p.out_dtype();
  char* obase = static_cast<char*>(p.out) + ((int64_t)ic.n * p.HV + ic.hv) * p.V * (odt == kF32 ? 4 : 2);
  if (!ic.live) {
    // NULL block (slot <= 0): zeros, no state access; out-of-range ids: NaN
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
  pd::stage_qk<K, L::QKT, L::NT, ACT>(p, R.qk, c, parity, s_qk);
  const float* buf = s_qk[parity];
  const float4* q4 = reinterpret_cast<const float4*>(buf + c * 16);
  const float4* k4 = reinterpret_cast<const float4*>(buf + K + c * 16);
  int8_t* sbase = p.state + (ic.slot * p.stride_state + (int64_t)ic.hv * p.V * K) * SB;
#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const int r = row0 + i * L::RPI;
    asm volatile("" ::: "memory");  // re-read k, q from LDS for this row
    float kk[16], qq[16], h[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 b4 = k4[j];
      kk[4 * j] = b4.x, kk[4 * j + 1] = b4.y, kk[4 * j + 2] = b4.z, kk[4 * j + 3] = b4.w;
    }
#pragma unroll
    for (int w = 0; w < kStateWords<BF16> / 4; ++w) {
      const uint32_t ws[4] = {R.sw[i][w].x, R.sw[i][w].y, R.sw[i][w].z, R.sw[i][w].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (BF16) {
          h[8 * w + 2 * j] = __uint_as_float(ws[j] << 16) * alpha;
          h[8 * w + 2 * j + 1] = __uint_as_float(ws[j] & 0xffff0000u) * alpha;
        } else {
          h[4 * w + j] = __uint_as_float(ws[j]) * alpha;
        }
      }
    }
    float rd = h[0] * kk[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) rd = fmaf(h[j], kk[j], rd);
    rd = group_sum<LPR>(rd);
    const float dv = beta * (act_decode<ACT>(R.vv[i]) - rd);
#pragma unroll
    for (int j = 0; j < 16; ++j) h[j] = fmaf(kk[j], dv, h[j]);
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
    if (r < p.V) {
      if (c == 0) store_act_at(obase, (uint32_t)r, odt, o);
      const uint32_t off = ((uint32_t)r * K + (uint32_t)c * 16) * SB;
      if constexpr (BF16) {
        typedef float f2 __attribute__((ext_vector_type(2)));
        typedef __bf16 b2 __attribute__((ext_vector_type(2)));
        uint32_t ws[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const b2 bb = __builtin_convertvector((f2){h[2 * j], h[2 * j + 1]}, b2);  // round to nearest even
          __builtin_memcpy(&ws[j], &bb, 4);
        }
        st_stream16(sbase + off, u32x4{ws[0], ws[1], ws[2], ws[3]});
        st_stream16(sbase + off + 16u, u32x4{ws[4], ws[5], ws[6], ws[7]});
      } else {
#pragma unroll
        for (int w = 0; w < 4; ++w)
          st_at<u32x4>(sbase, off + 16u * w, u32x4{__float_as_uint(h[4 * w]), __float_as_uint(h[4 * w + 1]),
                                                   __float_as_uint(h[4 * w + 2]), __float_as_uint(h[4 * w + 3])});
      }
    }
  }
}

template <int K, int RPL, int WAVES, bool BF16, int ACT>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(4)))
void float_decode_kernel(const PackedParams p, const int32_t* __restrict__ idx) {
  using L = FLayout<K, RPL, WAVES>;
  __shared__ __attribute__((aligned(16))) float s_qk[4][2 * K];  // [parity] staged, [2 + parity] raw
  __shared__ float2 s_gate[pd::kGateCap];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane % L::LPR;
  const int g = lane / L::LPR;
  const pd::Geom gm = pd::geom_of(p);
  const pd::WorkSeq w = pd::work_seq(gm.items, gm.share_n, gm.shares, gm.grid);
  if (w.count <= 0) return;  // whole workgroup
  int item = w.first;
  const int last = p.items - 1;
  const int item_end = w.first + w.count * w.step;  // one past this workgroup's last item
  // q/k staging buffers alternate between consecutive live items (see
  // packed_decode_kernel)
  FloatItemRegs<RPL, L::QKT, BF16> A, B;
  ItemCoord ca = pd::item_coord(p, gm, idx, nullptr, item), cb;
  load_fitem<K, RPL, WAVES, BF16, ACT>(p, ca, true, ca.vt * L::ROWS_WG + wave * L::ROWS_WAVE + g, c, A);
  pd::stage_gates<WAVES, true>(p, gm, w, wave, lane, s_gate);
  int k = 0, live = 0;
  for (;;) {
    int next = item + w.step;
    cb = pd::item_coord(p, gm, idx, nullptr, min(next, last));
    load_fitem<K, RPL, WAVES, BF16, ACT>(p, cb, next < item_end, cb.vt * L::ROWS_WG + wave * L::ROWS_WAVE + g, c, B);
    if (k == 0) __syncthreads();  // the staged gates are visible from here on
    float2 gab = s_gate[min(k, pd::kGateCap - 1)];
    process_fitem<K, RPL, WAVES, BF16, ACT>(p, ca, ca.vt * L::ROWS_WG + wave * L::ROWS_WAVE + g, c, live & 1, gab.x,
                                            gab.y, A, s_qk);
    live += ca.live ? 1 : 0;
    if (next >= item_end) break;
    ++k;
    item = next;

    next = item + w.step;
    ca = pd::item_coord(p, gm, idx, nullptr, min(next, last));
    load_fitem<K, RPL, WAVES, BF16, ACT>(p, ca, next < item_end, ca.vt * L::ROWS_WG + wave * L::ROWS_WAVE + g, c, A);
    gab = s_gate[min(k, pd::kGateCap - 1)];
    process_fitem<K, RPL, WAVES, BF16, ACT>(p, cb, cb.vt * L::ROWS_WG + wave * L::ROWS_WAVE + g, c, live & 1, gab.x,
                                            gab.y, B, s_qk);
    live += cb.live ? 1 : 0;
    if (next >= item_end) break;
    ++k;
    item = next;
  }
}

template <int K, bool BF16, int ACT>
int launch_fs(PackedParams p, int B, hipStream_t stream) {
  constexpr int RPL = 2, WAVES = 4;
  using L = FLayout<K, RPL, WAVES>;
  const int nvt = (p.V + L::ROWS_WG - 1) / L::ROWS_WG;
  const int64_t items = (int64_t)B * p.HV * nvt;
  if (items > 0x7fffffff) return fail(CK_EUNSUPPORTED, "%lld work items is too many", (long long)items);
  if (items == 0) return ok();
  p.items = (int)items;
  p.div_nvt = pd::make_fastdiv((uint32_t)nvt);
  p.div_hv = pd::make_fastdiv((uint32_t)p.HV);
  auto fn = float_decode_kernel<K, RPL, WAVES, BF16, ACT>;
  int per_cu = 0;
  const int resident = pd::resident_workgroups(reinterpret_cast<const void*>(fn), WAVES * 64, &per_cu);
  if (resident <= 0) return fail(CK_ELAUNCH, "cannot query the device occupancy");
  const int64_t cap = pd::launch_item_cap(resident, per_cu);
  if (items > cap) {  // consecutive launches over slices of the requests
    const int64_t per_request = (int64_t)p.HV * nvt;
    if (per_request > cap) return fail(CK_EUNSUPPORTED, "%lld work items per request is too many", (long long)per_request);
    const int chunk = (int)(cap / per_request);
    for (int n0 = 0; n0 < B; n0 += chunk) {
      const int rc = launch_fs<K, BF16, ACT>(pd::requests_from(p, n0), min(chunk, B - n0), stream);
      if (rc != CK_OK) return rc;
    }
    return ok();
  }
  const int per_wg = (p.items + resident - 1) / resident;
  const int grid = (p.items + per_wg - 1) / per_wg;
  pd::set_cu_shares(p, grid, resident, per_cu);
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(WAVES * 64), 0, stream, p, p.idx);
  return check_launch("ck_gdn_packed_decode_float_state");
}

template <bool BF16, int ACT>
int launch_fs_k(const PackedParams& p, int B, int K, hipStream_t s) {
  switch (K) {
    case 16: return launch_fs<16, BF16, ACT>(p, B, s);
    case 32: return launch_fs<32, BF16, ACT>(p, B, s);
    case 64: return launch_fs<64, BF16, ACT>(p, B, s);
    case 128: return launch_fs<128, BF16, ACT>(p, B, s);
    case 256: return launch_fs<256, BF16, ACT>(p, B, s);
    default: return fail(CK_EUNSUPPORTED, "K must be one of 16, 32, 64, 128, 256, got %d", K);
  }
}

}  // namespace fs
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
  if (K != 16 && K != 32 && K != 64 && K != 128 && K != 256)
    return fail(CK_EUNSUPPORTED, "K must be one of 16, 32, 64, 128, 256, got %d", K);
  if (B == 0) return ok();
  if (!mixed_qkv || !a || !b || !A_log || !dt_bias || !state || !out || !ssm_state_indices)
    return fail(CK_EINVAL, "null pointer argument");
  const int sesz = state_dtype == CK_DTYPE_F32 ? 4 : 2;
  if ((reinterpret_cast<uintptr_t>(state) & 15) || ((stride_state_slot * sesz) % 16))
    return fail(CK_EINVAL, "state rows must be 16-byte aligned");
  // per-lane byte offsets inside one (slot, head) and one row of mixed_qkv are 32-bit
  if ((int64_t)V * K * sesz >= ((int64_t)1 << 31) || (2 * (int64_t)H * K + (int64_t)HV * V) * 4 >= ((int64_t)1 << 31))
    return fail(CK_EUNSUPPORTED, "head or activation row too large");
  const int64_t strides[] = {stride_qkv_tok, stride_a_tok, stride_b_tok, stride_state_slot, stride_indices};
  for (int64_t st : strides)
    if (st < 0 || st > INT32_MAX) return fail(CK_EUNSUPPORTED, "strides must be in [0, 2^31) elements");
  if (num_slots > INT32_MAX) return fail(CK_EUNSUPPORTED, "num_slots must be < 2^31");

  pd::PackedParams p{};
  p.mixed = mixed_qkv;
  p.a = a;
  p.b = b;
  p.A_log = A_log;
  p.dt_bias = dt_bias;
  p.state = static_cast<int8_t*>(state);  // fp32 / bf16 elements, addressed in bytes
  p.out = out;
  p.idx = ssm_state_indices;
  p.stride_mixed = (int32_t)stride_qkv_tok;
  p.stride_a = (int32_t)stride_a_tok;
  p.stride_b = (int32_t)stride_b_tok;
  p.stride_state = (int32_t)stride_state_slot;
  p.stride_idx = (int32_t)stride_indices;
  p.num_slots = (int32_t)num_slots;
  p.scale = scale;
  p.dtypes = qkv_dtype | (a_dtype << 4) | (b_dtype << 8) | (A_log_dtype << 12) | (dt_bias_dtype << 16) |
             (out_dtype << 20);
  p.H = H;
  p.HV = HV;
  p.div_grp = pd::make_fastdiv((uint32_t)(HV / H));
  p.V = V;
  p.l2norm = use_qk_l2norm ? 1 : 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool bf16 = state_dtype == CK_DTYPE_BF16;
  if (qkv_dtype == CK_DTYPE_F32)
    return bf16 ? fs::launch_fs_k<true, kF32>(p, B, K, s) : fs::launch_fs_k<false, kF32>(p, B, K, s);
  if (qkv_dtype == CK_DTYPE_BF16)
    return bf16 ? fs::launch_fs_k<true, kBF16>(p, B, K, s) : fs::launch_fs_k<false, kBF16>(p, B, K, s);
  return bf16 ? fs::launch_fs_k<true, kF16>(p, B, K, s) : fs::launch_fs_k<false, kF16>(p, B, K, s);
}
