/*
 * carrykernel_gdn.h - C ABI of the MI355X (gfx950) fused Gated DeltaNet decode
 * step with error-feedback (EF) state quantization.
 *
 * Every entry point takes raw device pointers, element strides and sizes, and a
 * hipStream_t passed as void*. None allocates, none synchronises: kernels are
 * enqueued on `stream` and the call returns. The return value is a ck_status;
 * on failure ck_last_error() returns a message (thread-local).
 *
 * Reference interfaces replaced (paths relative to the tomalmog/carrykernel
 * repository root):
 *   ck_gdn_packed_decode      <- vllm_integration/quantized_packed_decode.py:242-327
 *                                (host) and _quant_int8_kernel :101-239 (device)
 *   ck_gdn_packed_decode_float_state
 *                             <- the upstream bf16/fp32-state packed decode that
 *                                quantized_packed_decode.py:1-7 replaces
 *                                (invoked at modal_vllm_headtohead.py:122-125)
 *   ck_gdn_quant_step         <- cuda/gdn_state_kernel.cu:310-348 (gdn_quant_step,
 *                                pybind at :373-377) and statequant/kernel.py:379-408
 *   ck_gdn_fp32_step          <- cuda/gdn_state_kernel.cu:350-371 (gdn_fp32_step)
 *                                and statequant/kernel.py:411-433
 *   ck_quantize_rows          <- vllm_integration/quantized_packed_decode.py:347-351
 *                                (init_quantized_state seeding from h0)
 *   ck_quantize_cols          <- statequant/kernel.py:99-113 (per_v_channel_quantize)
 *   ck_hbm_copy               <- measurement only: the device-to-device copy that
 *                                experiments/cuda_bench.py:39-60 times as the
 *                                measured bandwidth peak
 *   ck_gdn_packed_decode_to   <- the same step as ck_gdn_packed_decode with the
 *   ck_pool_copy_slots           updated state written to other slots, and slot
 *   ck_pool_reset_slots          copy / reset of the pool: the engine-side cache
 *                                operations the reference leaves open (its "Stage B":
 *                                the EF residual must move with the state through
 *                                paging, preemption, prefix-cache reuse and
 *                                speculative-decode rollback, CLAUDE.md:235-239,
 *                                266-273); no reference code implements them
 */
#ifndef CARRYKERNEL_GDN_H_
#define CARRYKERNEL_GDN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
enum ck_status {
  CK_OK = 0,
  CK_EINVAL = 1,       /* bad argument (null pointer, bad size/stride/dtype)   */
  CK_EUNSUPPORTED = 2, /* valid but not implemented here (e.g. K above 1024) */
  CK_ELAUNCH = 3       /* the HIP runtime rejected the kernel launch            */
};

/* Element types of activations / outputs / float state. CK_DTYPE_F64 is
 * accepted by ck_quantize_rows only (a float64 prefill state). */
enum ck_dtype { CK_DTYPE_F32 = 0, CK_DTYPE_BF16 = 1, CK_DTYPE_F16 = 2, CK_DTYPE_F64 = 3 };

/* Residual formats of the vLLM-layout path (quantized_packed_decode.py:82-83). */
enum ck_resid_fmt { CK_RESID_INT8 = 0, CK_RESID_INT4 = 1 };

/* Residual formats of the statequant-layout path (statequant/kernel.py:60-63). */
enum ck_res_fmt { CK_RES_FP32 = 0, CK_RES_FP16 = 1, CK_RES_FP8 = 2, CK_RES_INT8 = 3 };

/* Granularity of the residual scale in the vLLM-layout path. PER_ROW is the
 * reference's one scale per V-row (quantized_packed_decode.py:212-215);
 * PER_HEAD is one scale per (slot, value-head), amax over the whole [V, K]
 * tile, as configs 2/3 of the benchmark specify. */
enum ck_rscale_mode { CK_RSCALE_PER_ROW = 0, CK_RSCALE_PER_HEAD = 1 };

/* Arithmetic mode of the quantizer. FAST rounds rne(t * RN(1/s)) with one fma
 * and forms the residual with an fma; EXACT rounds rne(RN(t / s)) (the
 * correctly rounded quotient, as torch.round(target / scale) does) and forms
 * the residual as RN(t - RN(code * s)). */
enum ck_quant_mode { CK_QUANT_FAST = 0, CK_QUANT_EXACT = 1 };

/* Message of the last failed call on this thread ("" after a success). */
const char* ck_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int ck_abi_version(void);

/*
 * Lower, for the whole process, the number of work items one decode launch
 * holds (0: no lower limit, the default): a larger step then runs as
 * consecutive launches over slices of its requests, as steps past the
 * built-in limit do. It has no counterpart in the reference: it exists to
 * test the split. The environment variable CARRYKERNEL_MAX_ITEMS_PER_LAUNCH,
 * read once at the first launch, sets the same value. Thread-safe; affects
 * launches issued after it returns.
 */
int ck_set_max_items_per_launch(int64_t cap);

/*
 * Choose, for the whole process, which kernel runs the quantized decode
 * steps issued after it returns: 0 automatic (the default), 1 the persistent
 * kernel, 2 the one-item kernel, whatever the batch. It applies to K in
 * {16, 32, 64, 128, 256} with aligned pools; other K and unaligned pools run
 * the masked kernel, which has one form only. Both compute every item
 * with the same code, so the results are the same bits; the automatic choice
 * is the faster one. It has no counterpart in the reference: it exists so
 * that the tests run each kernel on shapes the automatic choice gives to the
 * other. The environment variable CARRYKERNEL_DECODE_KERNEL (1 or 2), read
 * once at the first launch, sets the same value. Thread-safe. Returns
 * CK_EINVAL for any other value.
 */
int ck_set_decode_kernel(int which);

/*
 * One decode step of the vLLM-layout quantized GDN, updated in place.
 *
 * mixed_qkv [B, 2*H*K + HV*V] (row stride stride_qkv_tok elements, last dim
 *   contiguous): q at i_h*K, k at H*K + i_h*K, v at 2*H*K + hv*V, with
 *   i_h = hv / (HV / H) (grouped-query mapping).
 * a, b [B, HV] (row strides given); A_log, dt_bias [HV].
 * State pool, per slot contiguous [HV, V, K] int8 codes; state_scale per slot
 *   [HV, V] fp32; resid_codes per slot [HV, V, K] int8 (CK_RESID_INT8) or
 *   [HV, V, K/2] packed nibbles (CK_RESID_INT4: even K in the low nibble);
 *   resid_scale per slot [HV, V] (CK_RSCALE_PER_ROW) or [HV] (CK_RSCALE_PER_HEAD).
 *   Slot strides are in elements of each tensor.
 * out [B, 1, HV, V] contiguous, dtype out_dtype.
 * ssm_state_indices [B] int32 (stride in elements): slot <= 0 is the NULL
 *   block (out gets zeros, state untouched); slot >= num_slots is out of range
 *   (out gets NaN, state untouched).
 * state_bits: the state code range is +-(2^(state_bits-1) - 1), bits in 2..8.
 * Requirements: K in 1..1024 (even for CK_RESID_INT4); HV % H == 0; with
 *   CK_RSCALE_PER_HEAD above K = 256, V <= 128 (K <= 512) or V <= 64. Rows of
 *   K = 16, 32, 64, 128 or 256 codes, 16-byte aligned (8-byte for int4
 *   residual rows), run the bandwidth kernel; any other K or alignment runs
 *   the masked kernel, which computes as if every row, q and k were
 *   zero-padded to max(16, next_pow2(K)), as the reference's masked lanes do
 *   (quantized_packed_decode.py:123-127,158,165-166,303), with whole 16-byte
 *   lane accesses when K is a multiple of 16 and rows are aligned, 4- and
 *   2-byte accesses when K is a multiple of 4 and rows are 4-byte aligned
 *   (2-byte for int4 residual rows), byte accesses otherwise.
 * B == 0 checks the sizes and codes, launches nothing and returns CK_OK; the
 *   pointer arguments may then be NULL (an empty tensor's data pointer).
 */
int ck_gdn_packed_decode(const void* mixed_qkv, int qkv_dtype, int64_t stride_qkv_tok,
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
                         void* stream);

/*
 * ck_gdn_packed_decode with the updated state written to the slots in
 * dst_state_indices [B] (int32, stride in elements) instead of back to the
 * slots it was read from: request n reads slot ssm_state_indices[n] and
 * writes slot dst_state_indices[n] of the same pool (the two may be equal).
 * A destination id outside [1, num_slots) discards the update (out is still
 * written). Reading a slot that another request of the same call writes is a
 * race. Chains of calls (token t reads the slot token t-1 wrote) keep every
 * intermediate state, which is what speculative decoding needs to roll back;
 * a shared prefix slot can be decoded into a request's own slot without a
 * copy. dst_state_indices must not be NULL unless B == 0 (as for
 * ck_gdn_packed_decode, nothing is then launched); quant_mode must be CK_QUANT_FAST
 * (other modes return CK_EUNSUPPORTED).
 */
int ck_gdn_packed_decode_to(const void* mixed_qkv, int qkv_dtype, int64_t stride_qkv_tok,
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
                            void* stream);

/*
 * Copy n slots between quantized pools of the same layout (HV, V, K,
 * resid_fmt, rscale_mode; the vLLM layout of ck_gdn_packed_decode): slot
 * src_ids[i] of the source pool -> slot dst_ids[i] of the destination pool,
 * all four regions (state codes and scales, residual codes and scales). The
 * pools may be the same tensors; a slot must not be both read and written by
 * one call. Pairs with an id outside [1, num_slots) of its pool are skipped.
 * Each slot's region must be contiguous; slot strides are in elements of the
 * region's type. n <= 65535. Device memory only.
 */
int ck_pool_copy_slots(const int8_t* src_state, int64_t src_stride_state, const float* src_sscale,
                       int64_t src_stride_sscale, const int8_t* src_resid, int64_t src_stride_resid,
                       const float* src_rscale, int64_t src_stride_rscale, int64_t src_num_slots,
                       int8_t* dst_state, int64_t dst_stride_state, float* dst_sscale,
                       int64_t dst_stride_sscale, int8_t* dst_resid, int64_t dst_stride_resid,
                       float* dst_rscale, int64_t dst_stride_rscale, int64_t dst_num_slots,
                       const int32_t* src_ids, const int32_t* dst_ids, int n,
                       int HV, int V, int K, int resid_fmt, int rscale_mode, void* stream);

/*
 * Zero the four regions of the n slots ids[i] (ids outside [1, num_slots) are
 * skipped): the state of a new request, as init_quantized_state without h0
 * gives (vllm_integration/quantized_packed_decode.py:341-345).
 */
int ck_pool_reset_slots(int8_t* state, int64_t stride_state, float* sscale, int64_t stride_sscale,
                        int8_t* resid, int64_t stride_resid, float* rscale, int64_t stride_rscale,
                        int64_t num_slots, const int32_t* ids, int n,
                        int HV, int V, int K, int resid_fmt, int rscale_mode, void* stream);

/*
 * Same step with an unquantized state pool (fp32 or bf16), the layout and
 * semantics of the upstream packed decode that the quantized op replaces:
 * state per slot contiguous [HV, V, K] of state_dtype, updated in place
 * (bf16 stores round to nearest even).
 */
int ck_gdn_packed_decode_float_state(const void* mixed_qkv, int qkv_dtype, int64_t stride_qkv_tok,
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
                                     int use_qk_l2norm, void* stream);

/*
 * One out-of-place step in the statequant layout: state [B, HV, K, V] int8
 * (V contiguous) with one scale per V-column (amax over K), residual e of
 * res_fmt (fp32 / fp16 / fp8 e5m2 / int8 with a per-V-column e_scale).
 * q, k [B, HV, K]; v [B, HV, V]; alpha, beta [B, HV]; all fp32, contiguous.
 * qmax = 2^(bits-1) - 1 is used for the state and, for CK_RES_INT8, for the
 * residual, as the reference's GPU kernels do (cuda/gdn_state_kernel.cu:210,233).
 * e_scale_in / e_scale_out are read / written only for CK_RES_INT8.
 * In-place use (h_out == h_in, e_out == e_in, ...) is allowed.
 * Requirements: K in 1..256 (rows past K zero-padded to max(16, next_pow2(K)),
 *   whose K-slices fix the reduction order); any V >= 1; fp32 tensors 4-byte
 * and the residual element-size aligned. V % 4 == 0 with 16-byte aligned
 * tensors takes one vector access per 4 columns, anything else one access
 * per column (statequant/kernel.py:277-279 masks offs_v < V the same way).
 */
int ck_gdn_quant_step(const int8_t* h_in, const float* scale_in, const void* e_in,
                      const float* e_scale_in,
                      const float* q, const float* k, const float* v,
                      const float* alpha, const float* beta,
                      float* o, int8_t* h_out, float* scale_out, void* e_out, float* e_scale_out,
                      int B, int HV, int K, int V, float qmax, int res_fmt, int quant_mode,
                      void* stream);

/* FP32 baseline step in the statequant layout (no quantization); the same K,
 * V and alignment rules as ck_gdn_quant_step. */
int ck_gdn_fp32_step(const float* h_in, const float* q, const float* k, const float* v,
                     const float* alpha, const float* beta, float* o, float* h_out,
                     int B, int HV, int K, int V, void* stream);

/*
 * Quantize rows of length K (contiguous, row stride `stride_row` elements) to
 * int8 codes with one scale per row: scale = max(amax, 1e-12) / qmax,
 * code = rne(x / scale) clamped to +-qmax (init_quantized_state semantics,
 * vllm_integration/quantized_packed_decode.py:347-351), evaluated in x's
 * precision as torch evaluates that expression on a tensor of x's dtype:
 * fp32 / float64 arithmetic for CK_DTYPE_F32 / CK_DTYPE_F64 (the float64
 * scale is stored rounded to fp32); for CK_DTYPE_BF16 / CK_DTYPE_F16 every
 * operation in fp32 rounded to nearest even to x's dtype (the scale is then
 * a bf16 / fp16 value, the quotient is rounded to x's dtype before rne, and
 * the clamp can bind). An fp16 row whose scale rounds to 0 (all zeros) gets
 * codes 0. codes are written contiguous [rows, K], scales [rows].
 */
int ck_quantize_rows(const void* x, int x_dtype, int64_t stride_row, int64_t rows, int K,
                     float qmax, int8_t* codes, float* scale, void* stream);

/*
 * Quantize M contiguous [K, V] matrices per V-column (amax over K), same
 * arithmetic as ck_quantize_rows: codes [M, K, V], scale [M, V].
 */
int ck_quantize_cols(const float* x, int64_t M, int K, int V, float qmax,
                     int8_t* codes, float* scale, void* stream);

/*
 * Measurement only (not on the decode path): copy `bytes` (a multiple of 16;
 * both pointers 16-byte aligned) from src to dst with a streaming kernel of
 * `grid` workgroups of 512 threads (0: min(4096, bytes / 8192)). Gives the
 * measured HBM copy ceiling the decode's bandwidth is compared with.
 */
int ck_hbm_copy(const void* src, void* dst, int64_t bytes, int grid, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CARRYKERNEL_GDN_H_ */
