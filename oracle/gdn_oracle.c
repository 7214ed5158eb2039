/*
 * CPU oracle for the fused GDN decode step with error-feedback state
 * quantization. TEST INFRASTRUCTURE ONLY: it is loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's CPU-baseline leg, as the checker;
 * the product never calls it.
 *
 * It restates the reference algorithm in plain C, one (request, value-head)
 * at a time:
 *   vllm_integration/quantized_packed_decode.py:116-239   (vLLM layout step)
 *   statequant/kernel.py:149-178 and :260-341             (statequant layout step)
 *   statequant/kernel.py:116-123, cuda/gdn_state_kernel.cu:251-297 (fp32 step)
 *   statequant/reference.py:20-34                         (GDN recurrence)
 *   statequant/quant.py:37-42, :65-80                     (per-axis quantizer, EF)
 *   vllm_integration/quantized_packed_decode.py:347-351   (init quantize)
 *
 * The reference leaves the fp32 evaluation order of its K-reductions to
 * torch.einsum / Triton and the quantizer's division to the backend. This
 * oracle fixes both, so that a GPU implementation following the same order is
 * checked bit for bit:
 *  - A K-reduction (dot product) is split into chunks of 16 consecutive K;
 *    each chunk is x0*y0 followed by fmaf(xj, yj, acc) for j = 1..15, and the
 *    K/16 chunk sums are combined as a balanced pairwise tree
 *    ((c0+c1)+(c2+c3))+((c4+c5)+(c6+c7)) ....
 *  - FAST quantizer mode: code = rne(t * RN(1/s)) of the exact product, the
 *    residual is fmaf(-code, s, t), dequantize-decay is code * RN(s*alpha),
 *    rank-1 update and residual add are fmaf.
 *  - EXACT quantizer mode: code = rne(RN(t / s)) with an IEEE division, the
 *    residual is RN(t - RN(code*s)), dequantize-decay is RN(RN(code*s)*alpha),
 *    rank-1 update and residual add are RN(a + RN(x*y)): the op-by-op rounding
 *    of statequant/kernel.py:165-177.
 * Clamping to +-qmax is applied (as the reference does); it never binds.
 * Build: see oracle/Makefile (-ffp-contract=off keeps every a*b+c unfused).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_EPS 1e-12f

/* ------------------------------------------------------------------------- */
/* Gate transcendentals: Cody-Waite exp with a degree-8 Taylor polynomial and  */
/* an atanh-series log, the method the kernels use (same fp32 operation        */
/* sequence, so the same bits). Accuracy is checked against float64 by tests. */
/* ------------------------------------------------------------------------- */
static float orc_bits_to_float(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t orc_float_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static float orc_pow2i(int n) { return orc_bits_to_float((uint32_t)(n + 127) << 23); }

float orc_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283172607421875f) return orc_bits_to_float(0x7f800000u);
  if (x < -103.97208404541015625f) return 0.0f;
  const float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.42860676533018704503775e-06f, r);
  float p = 2.48015873015873015873e-05f;
  p = fmaf(p, r, 1.98412698412698412698e-04f);
  p = fmaf(p, r, 1.38888888888888888889e-03f);
  p = fmaf(p, r, 8.33333333333333333333e-03f);
  p = fmaf(p, r, 4.16666666666666666667e-02f);
  p = fmaf(p, r, 1.66666666666666666667e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const int n1 = ni / 2;
  const int n2 = ni - n1;
  return (p * orc_pow2i(n1)) * orc_pow2i(n2);
}

float orc_logf(float y) {
  if (y != y || y < 0.0f) return orc_bits_to_float(0x7fc00000u);
  if (y == 0.0f) return orc_bits_to_float(0xff800000u);
  if (y > 3.40282346638528859812e+38f) return y;
  int e = 0;
  if (y < 1.17549435082228750797e-38f) {
    y = y * 16777216.0f;
    e = -24;
  }
  const uint32_t u = orc_float_to_bits(y);
  e += (int)((u >> 23) & 0xffu) - 127;
  float m = orc_bits_to_float((u & 0x007fffffu) | 0x3f800000u);
  if (m > 1.41421353816986083984f) {
    m = m * 0.5f;
    e += 1;
  }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float s2 = s * s;
  float p = 7.69230769230769230769e-02f;
  p = fmaf(p, s2, 9.09090909090909090909e-02f);
  p = fmaf(p, s2, 1.11111111111111111111e-01f);
  p = fmaf(p, s2, 1.42857142857142857143e-01f);
  p = fmaf(p, s2, 2.0e-01f);
  p = fmaf(p, s2, 3.33333333333333333333e-01f);
  const float logm = fmaf(2.0f * s, s2 * p, 2.0f * s);
  const float fe = (float)e;
  return fmaf(fe, 0.693145751953125f, fmaf(fe, 1.42860676533018704503775e-06f, logm));
}

/* quantized_packed_decode.py:179-182 */
void orc_gates(float a, float b, float A_log, float dt_bias, float* alpha, float* beta) {
  const float x = a + dt_bias;
  const float sp = (x <= 20.0f) ? orc_logf(1.0f + orc_expf(x)) : x;
  const float g = -orc_expf(A_log) * sp;
  *alpha = orc_expf(g);
  *beta = 1.0f / (1.0f + orc_expf(-b));
}

/* Vectorised entry points for tests (n values). */
void orc_expf_n(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_expf(x[i]);
}
void orc_logf_n(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_logf(x[i]);
}
void orc_gates_n(const float* a, const float* b, const float* A_log, const float* dt_bias, float* alpha,
                 float* beta, int64_t n) {
  for (int64_t i = 0; i < n; ++i) orc_gates(a[i], b[i], A_log[i], dt_bias[i], &alpha[i], &beta[i]);
}

/* ------------------------------------------------------------------------- */
/* Reductions in the fixed order described at the top.                       */
/* ------------------------------------------------------------------------- */
static float tree_sum(float* c, int n) {
  /* balanced pairwise tree over n (a power of two, at most 64) sums, in place */
  for (int w = 1; w < n; w *= 2)
    for (int i = 0; i + w < n; i += 2 * w) c[i] = c[i] + c[i + w];
  return c[0];
}

/* sum_k x[k*sx] * y[k*sy] over K (K a multiple of 16, K/16 a power of 2,
   K <= 1024). */
static float dot_k(const float* x, int64_t sx, const float* y, int64_t sy, int K) {
  float chunk[64];
  const int nc = K / 16;
  for (int cidx = 0; cidx < nc; ++cidx) {
    const float* xc = x + (int64_t)cidx * 16 * sx;
    const float* yc = y + (int64_t)cidx * 16 * sy;
    float acc = xc[0] * yc[0];
    for (int j = 1; j < 16; ++j) acc = fmaf(xc[(int64_t)j * sx], yc[(int64_t)j * sy], acc);
    chunk[cidx] = acc;
  }
  return tree_sum(chunk, nc);
}

/* ------------------------------------------------------------------------- */
/* Quantizer primitives.                                                       */
/* ------------------------------------------------------------------------- */
#define MODE_FAST 0
#define MODE_EXACT 1

static const float kMagic = 12582912.0f;

static float clampq(float c, float qmax) { return fminf(fmaxf(c, -qmax), qmax); }

/* rounded code (as float) of t at scale s, inv = RN(1/s) */
static float quant_code(float t, float s, float inv, float qmax, int mode) {
  float c;
  if (mode == MODE_FAST) {
    c = fmaf(t, inv, kMagic) - kMagic; /* rne of the exact product */
  } else {
    c = rintf(t / s); /* rne of the IEEE quotient */
  }
  return clampq(c, qmax);
}

static float resid_of(float t, float c, float s, int mode) {
  return mode == MODE_FAST ? fmaf(-c, s, t) : t - c * s;
}

static float madd(float x, float y, float a, int mode) { return mode == MODE_FAST ? fmaf(x, y, a) : a + x * y; }

/* two's-complement nibble of element j of a packed int4 row (qpd:196-199) */
static int unpack_i4(const int8_t* row, int j) {
  const int byte = row[j >> 1] & 0xff;
  int nib = (j & 1) ? (byte >> 4) & 0xf : byte & 0xf;
  return nib > 7 ? nib - 16 : nib;
}

/* qpd:226-230: byte = (c_even & 0xF) | (c_odd & 0xF) << 4 */
static void pack_i4_row(int8_t* row, const int* codes, int K) {
  for (int j = 0; j < K; j += 2) {
    const int byte = (codes[j] & 0xf) | ((codes[j + 1] & 0xf) << 4);
    row[j >> 1] = (int8_t)(uint8_t)byte;
  }
}

/* ------------------------------------------------------------------------- */
/* vLLM-layout fused decode step ([slots, HV, V, K], in place).                */
/* ------------------------------------------------------------------------- */
int orc_packed_decode(const float* mixed, int64_t stride_mixed,
                      const float* a, int64_t stride_a, const float* b, int64_t stride_b,
                      const float* A_log, const float* dt_bias, float scale,
                      int8_t* state, int64_t stride_state, float* sscale, int64_t stride_sscale,
                      int8_t* resid, int64_t stride_resid, float* rscale, int64_t stride_rscale,
                      float* out, const int32_t* idx, const int32_t* dst_idx, int64_t num_slots,
                      int B, int H, int HV, int K, int V,
                      int l2norm, int resid_fmt, int per_head, int state_bits, int mode, int nthreads) {
  /* dst_idx (may be NULL: in place): the updated state of request n goes to
     slot dst_idx[n]; one outside [1, num_slots) discards it (out is kept).
     Any K in 1..1024 (even for the int4 residual): the reference's lanes
     o_k < BK = next_pow2(K) load 0 past K (qpd:123-127, :158, :165-166,
     :196-202, :303), so the step runs on rows zero-padded to
     KP = max(16, next_pow2(K)) in the reduction order of KP and stores the
     K existing columns. */
  if (K < 1 || K > 1024 || HV % H != 0 || (resid_fmt == 1 && K % 2 != 0)) return 1;
  int KP = 16;
  while (KP < K) KP *= 2;
  const float qmax = (float)((1 << (state_bits - 1)) - 1);
  const float qmax_e = resid_fmt == 1 ? 7.0f : 127.0f;
  const int RK = resid_fmt == 1 ? K / 2 : K;
  const int64_t nwork = (int64_t)B * HV;
  (void)nthreads;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
  {
    float* q = (float*)malloc(sizeof(float) * KP);
    float* k = (float*)malloc(sizeof(float) * KP);
    float* h = (float*)malloc(sizeof(float) * KP);
    float* ebuf = (float*)malloc(sizeof(float) * (size_t)V * KP);
    int* codes = (int*)malloc(sizeof(int) * KP);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (int64_t w = 0; w < nwork; ++w) {
      const int n = (int)(w / HV);
      const int hv = (int)(w % HV);
      const int64_t slot = idx[n];
      float* o = out + ((int64_t)n * HV + hv) * V;
      if (slot <= 0 || slot >= num_slots) {
        const float fill = slot <= 0 ? 0.0f : NAN;
        for (int r = 0; r < V; ++r) o[r] = fill;
        continue;
      }
      const int hq = hv / (HV / H);
      const float* m = mixed + (int64_t)n * stride_mixed;
      for (int j = 0; j < KP; ++j) {
        q[j] = j < K ? m[(int64_t)hq * K + j] : 0.0f;
        k[j] = j < K ? m[(int64_t)H * K + (int64_t)hq * K + j] : 0.0f;
      }
      if (l2norm) { /* qpd:169-171 */
        const float dq = sqrtf(dot_k(q, 1, q, 1, KP) + 1e-6f);
        const float dk = sqrtf(dot_k(k, 1, k, 1, KP) + 1e-6f);
        for (int j = 0; j < KP; ++j) {
          q[j] = q[j] / dq;
          k[j] = k[j] / dk;
        }
      }
      for (int j = 0; j < KP; ++j) q[j] = q[j] * scale; /* qpd:172 */
      float alpha, beta;
      orc_gates(a[(int64_t)n * stride_a + hv], b[(int64_t)n * stride_b + hv], A_log[hv], dt_bias[hv], &alpha, &beta);

      const int64_t dslot = dst_idx ? (int64_t)dst_idx[n] : slot;
      const int store = dslot > 0 && dslot < num_slots;
      const int8_t* st = state + slot * stride_state + (int64_t)hv * V * K;
      const float* ss = sscale + slot * stride_sscale + (int64_t)hv * V;
      const int8_t* er = resid + slot * stride_resid + (int64_t)hv * V * RK;
      const float* rs = per_head ? rscale + slot * stride_rscale + hv : rscale + slot * stride_rscale + (int64_t)hv * V;
      const int64_t ws = store ? dslot : slot; /* write targets (used only when store) */
      int8_t* st_w = state + ws * stride_state + (int64_t)hv * V * K;
      float* ss_w = sscale + ws * stride_sscale + (int64_t)hv * V;
      int8_t* er_w = resid + ws * stride_resid + (int64_t)hv * V * RK;
      float* rs_w = per_head ? rscale + ws * stride_rscale + hv : rscale + ws * stride_rscale + (int64_t)hv * V;
      const float* vv = m + 2 * (int64_t)H * K + (int64_t)hv * V;
      const float rs_head = per_head ? rs[0] : 0.0f;
      float ea_head = 0.0f;

      for (int r = 0; r < V; ++r) {
        const int8_t* crow = st + (int64_t)r * K;
        const int8_t* erow = er + (int64_t)r * RK;
        int8_t* crow_w = st_w + (int64_t)r * K;
        int8_t* erow_w = er_w + (int64_t)r * RK;
        /* dequantize + decay (qpd:158, :185) */
        if (mode == MODE_FAST) {
          const float sa = ss[r] * alpha;
          for (int j = 0; j < KP; ++j) h[j] = (float)(j < K ? crow[j] : 0) * sa;
        } else {
          for (int j = 0; j < KP; ++j) h[j] = ((float)(j < K ? crow[j] : 0) * ss[r]) * alpha;
        }
        /* delta rule (qpd:186-190) */
        const float rd = dot_k(h, 1, k, 1, KP);
        const float dv = beta * (vv[r] - rd);
        for (int j = 0; j < KP; ++j) h[j] = madd(k[j], dv, h[j], mode);
        o[r] = dot_k(h, 1, q, 1, KP);
        /* residual add (qpd:195-203) */
        const float es_in = per_head ? rs_head : rs[r];
        for (int j = 0; j < KP; ++j) {
          const int ec = j >= K ? 0 : resid_fmt == 1 ? unpack_i4(erow, j) : (int)erow[j];
          h[j] = madd((float)ec, es_in, h[j], mode);
        }
        /* requantize (qpd:205-209) */
        float am = 0.0f;
        for (int j = 0; j < KP; ++j) am = fmaxf(am, fabsf(h[j]));
        const float s_new = fmaxf(am / qmax, ORC_EPS);
        const float inv = 1.0f / s_new;
        float* e = ebuf + (int64_t)r * KP;
        for (int j = 0; j < KP; ++j) {
          const float c = quant_code(h[j], s_new, inv, qmax, mode);
          if (store && j < K) crow_w[j] = (int8_t)c;
          e[j] = resid_of(h[j], c, s_new, mode);
        }
        if (store) ss_w[r] = s_new;
        if (per_head) {
          for (int j = 0; j < KP; ++j) ea_head = fmaxf(ea_head, fabsf(e[j]));
        } else { /* residual quantize, per V-row scale (qpd:211-215) */
          float ea = 0.0f;
          for (int j = 0; j < KP; ++j) ea = fmaxf(ea, fabsf(e[j]));
          const float es = fmaxf(ea / qmax_e, ORC_EPS);
          const float inv_e = 1.0f / es;
          for (int j = 0; j < K; ++j) codes[j] = (int)quant_code(e[j], es, inv_e, qmax_e, mode);
          if (store) {
            if (resid_fmt == 1) {
              pack_i4_row(erow_w, codes, K);
            } else {
              for (int j = 0; j < K; ++j) erow_w[j] = (int8_t)codes[j];
            }
            rs_w[r] = es;
          }
        }
      }
      if (per_head && store) { /* one residual scale per (slot, head) */
        const float es = fmaxf(ea_head / qmax_e, ORC_EPS);
        const float inv_e = 1.0f / es;
        for (int r = 0; r < V; ++r) {
          const float* e = ebuf + (int64_t)r * KP;
          int8_t* erow_w = er_w + (int64_t)r * RK;
          for (int j = 0; j < K; ++j) codes[j] = (int)quant_code(e[j], es, inv_e, qmax_e, mode);
          if (resid_fmt == 1) {
            pack_i4_row(erow_w, codes, K);
          } else {
            for (int j = 0; j < K; ++j) erow_w[j] = (int8_t)codes[j];
          }
        }
        rs_w[0] = es;
      }
    }
    free(q);
    free(k);
    free(h);
    free(ebuf);
    free(codes);
  }
  return 0;
}

/* ------------------------------------------------------------------------- */
/* init_quantized_state seeding (qpd:347-351): per row of K,                  */
/* scale = max(amax, eps) / qmax, code = clamp(rne(x / scale)).               */
/* ------------------------------------------------------------------------- */
void orc_quantize_rows(const float* x, int64_t rows, int K, float qmax, int8_t* codes, float* scale) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * K;
    float am = 0.0f;
    for (int j = 0; j < K; ++j) am = fmaxf(am, fabsf(xr[j]));
    const float s = fmaxf(am, ORC_EPS) / qmax;
    for (int j = 0; j < K; ++j) codes[r * K + j] = (int8_t)clampq(rintf(xr[j] / s), qmax);
    scale[r] = s;
  }
}

/* per_v_channel_quantize (statequant/kernel.py:99-113): [M, K, V], amax over K */
void orc_quantize_cols(const float* x, int64_t M, int K, int V, float qmax, int8_t* codes, float* scale) {
  for (int64_t mi = 0; mi < M; ++mi) {
    const float* xm = x + mi * K * V;
    for (int c = 0; c < V; ++c) {
      float am = 0.0f;
      for (int j = 0; j < K; ++j) am = fmaxf(am, fabsf(xm[(int64_t)j * V + c]));
      const float s = fmaxf(am, ORC_EPS) / qmax;
      for (int j = 0; j < K; ++j)
        codes[mi * K * V + (int64_t)j * V + c] = (int8_t)clampq(rintf(xm[(int64_t)j * V + c] / s), qmax);
      scale[mi * V + c] = s;
    }
  }
}

/* ------------------------------------------------------------------------- */
/* Residual storage codecs of the statequant layout (statequant/kernel.py:    */
/* 78-87): fp16 and fp8 e5m2 with round-to-nearest-even, written from the     */
/* format definitions (sign | exponent | mantissa, subnormals, overflow to    */
/* inf at and above the midpoint past the largest finite value).              */
/* ------------------------------------------------------------------------- */
uint16_t orc_f32_to_f16(float f) {
  const uint32_t u = orc_float_to_bits(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7e00u;       /* NaN */
  if (a >= 0x477ff000u) return sign | 0x7c00u;      /* >= 65520 rounds to inf */
  if (a < 0x38800000u) {                            /* below 2^-14: subnormal */
    const float scaled = orc_bits_to_float(a) * 16777216.0f; /* x 2^24, exact */
    return sign | (uint16_t)rintf(scaled);
  }
  const uint32_t lsb = (a >> 13) & 1u;
  uint32_t r = (a + 0xfffu + lsb) >> 13;
  r -= (127u - 15u) << 10;
  return sign | (uint16_t)r;
}

float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    const float v = (float)m * (1.0f / 16777216.0f); /* m x 2^-24, exact */
    return sign ? -v : v;
  }
  if (e == 31) return orc_bits_to_float(sign | 0x7f800000u | (m << 13));
  return orc_bits_to_float(sign | ((e - 15u + 127u) << 23) | (m << 13));
}

uint8_t orc_f32_to_e5m2(float f) {
  const uint32_t u = orc_float_to_bits(f);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;         /* NaN */
  if (a >= 0x47700000u) return sign | 0x7cu;        /* >= 61440 rounds to inf */
  if (a < 0x38800000u) {                            /* below 2^-14: subnormal */
    const float scaled = orc_bits_to_float(a) * 65536.0f; /* x 2^16, exact */
    return sign | (uint8_t)rintf(scaled);
  }
  const uint32_t lsb = (a >> 21) & 1u;
  uint32_t r = (a + 0xfffffu + lsb) >> 21;
  r -= (127u - 15u) << 2;
  return sign | (uint8_t)r;
}

float orc_e5m2_to_f32(uint8_t b) {
  const uint32_t sign = ((uint32_t)b & 0x80u) << 24;
  const uint32_t e = (b >> 2) & 0x1fu, m = b & 3u;
  if (e == 0) {
    const float v = (float)m * (1.0f / 65536.0f);   /* m x 2^-16, exact */
    return sign ? -v : v;
  }
  if (e == 31) return orc_bits_to_float(sign | 0x7f800000u | (m << 21));
  return orc_bits_to_float(sign | ((e - 15u + 127u) << 23) | (m << 21));
}

void orc_f32_to_f16_n(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_f16(x[i]);
}
void orc_f32_to_e5m2_n(const float* x, uint8_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_e5m2(x[i]);
}
void orc_e5m2_to_f32_n(const uint8_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_e5m2_to_f32(x[i]);
}

/* ------------------------------------------------------------------------- */
/* statequant layout: state [B, HV, K, V] (V contiguous), one scale per       */
/* V-column (amax over K). K-reductions: the K rows split into S slices of    */
/* consecutive rows, S = 8 for K <= 128 and K/16 (16 rows each) above; each   */
/* slice is x0*y0 then fmaf over its rows; the S slice sums combine by a      */
/* balanced pairwise tree (S = 8: ((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7))).       */
/* Any K in 1..1024: the rows are zero-padded to KP = max(16, next_pow2(K)),  */
/* as the reference's Triton kernel masks its BK = next_pow2(K) rows          */
/* (statequant/kernel.py:277-279), and the sums take KP's slices.             */
/* ------------------------------------------------------------------------- */
#define RES_FP32 0
#define RES_FP16 1
#define RES_FP8 2
#define RES_INT8 3

static int statequant_slices(int K) { return K <= 128 ? 8 : K / 16; }

static float dot_slices(const float* x, int64_t sx, const float* y, int K) {
  float part[64];
  const int ns = statequant_slices(K);
  const int rps = K / ns;
  for (int sl = 0; sl < ns; ++sl) {
    const int r0 = sl * rps;
    float acc = x[(int64_t)r0 * sx] * y[r0];
    for (int r = r0 + 1; r < r0 + rps; ++r) acc = fmaf(x[(int64_t)r * sx], y[r], acc);
    part[sl] = acc;
  }
  return tree_sum(part, ns);
}

static int statequant_k_ok(int K) { return K >= 1 && K <= 1024; }

/* KP = max(16, next_pow2(K)): the padded row count whose slices the sums take */
static int statequant_kp(int K) {
  int kp = 16;
  while (kp < K) kp *= 2;
  return kp;
}

/* statequant/kernel.py:149-178 (torch reference) and :260-341 (GPU kernel):
 * one out-of-place step. qmax applies to the state and to the int8 residual
 * (the GPU kernels' convention, cuda/gdn_state_kernel.cu:210,233). */
int orc_quant_step_kv(const int8_t* h_in, const float* scale_in, const void* e_in, const float* e_scale_in,
                      const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                      float* o, int8_t* h_out, float* scale_out, void* e_out, float* e_scale_out,
                      int B, int HV, int K, int V, float qmax, int res_fmt, int mode, int nthreads) {
  if (!statequant_k_ok(K) || V <= 0) return 1;
  (void)nthreads;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
  {
    const int KP = statequant_kp(K);
    /* rows K..KP-1 of h, kp and qp stay +0: zero codes, zero q and k */
    float* h = (float*)calloc((size_t)KP * V, sizeof(float));
    float* kp = (float*)calloc((size_t)KP, sizeof(float));
    float* qp = (float*)calloc((size_t)KP, sizeof(float));
    float* rd = (float*)malloc(sizeof(float) * V);
    float* col = (float*)malloc(sizeof(float) * K);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (int64_t w = 0; w < (int64_t)B * HV; ++w) {
      const int64_t mb = w * (int64_t)K * V, vb = w * V, kb = w * K;
      const float a = alpha[w], bt = beta[w];
      for (int r = 0; r < K; ++r) {
        kp[r] = k[kb + r];
        qp[r] = q[kb + r];
      }
      /* dequantize + decay (kernel.py:165-166) */
      for (int r = 0; r < K; ++r)
        for (int c = 0; c < V; ++c) {
          const float code = (float)h_in[mb + (int64_t)r * V + c];
          h[(int64_t)r * V + c] = mode == MODE_FAST ? code * (scale_in[vb + c] * a) : (code * scale_in[vb + c]) * a;
        }
      /* delta rule (kernel.py:167-170); a padding row stays +0 (its k is 0) */
      for (int c = 0; c < V; ++c) rd[c] = bt * (v[vb + c] - dot_slices(h + c, V, kp, KP));
      for (int r = 0; r < K; ++r)
        for (int c = 0; c < V; ++c) h[(int64_t)r * V + c] = madd(k[kb + r], rd[c], h[(int64_t)r * V + c], mode);
      for (int c = 0; c < V; ++c) o[vb + c] = dot_slices(h + c, V, qp, KP);
      /* residual add (kernel.py:172) */
      for (int r = 0; r < K; ++r)
        for (int c = 0; c < V; ++c) {
          const int64_t i = mb + (int64_t)r * V + c;
          float* t = &h[(int64_t)r * V + c];
          if (res_fmt == RES_INT8) {
            *t = madd((float)((const int8_t*)e_in)[i], e_scale_in[vb + c], *t, mode);
          } else if (res_fmt == RES_FP16) {
            *t = *t + orc_f16_to_f32(((const uint16_t*)e_in)[i]);
          } else if (res_fmt == RES_FP8) {
            *t = *t + orc_e5m2_to_f32(((const uint8_t*)e_in)[i]);
          } else {
            *t = *t + ((const float*)e_in)[i];
          }
        }
      /* requantize per V-column (kernel.py:173-177) */
      for (int c = 0; c < V; ++c) {
        float am = 0.0f;
        for (int r = 0; r < K; ++r) am = fmaxf(am, fabsf(h[(int64_t)r * V + c]));
        const float s = fmaxf(am / qmax, ORC_EPS);
        const float inv = 1.0f / s;
        float ea = 0.0f;
        for (int r = 0; r < K; ++r) {
          float* t = &h[(int64_t)r * V + c];
          const float code = quant_code(*t, s, inv, qmax, mode);
          h_out[mb + (int64_t)r * V + c] = (int8_t)code;
          *t = resid_of(*t, code, s, mode); /* now the residual e' */
          ea = fmaxf(ea, fabsf(*t));
          col[r] = *t;
        }
        scale_out[vb + c] = s;
        if (res_fmt == RES_INT8) {
          const float es = fmaxf(ea / qmax, ORC_EPS);
          const float inv_e = 1.0f / es;
          for (int r = 0; r < K; ++r)
            ((int8_t*)e_out)[mb + (int64_t)r * V + c] = (int8_t)quant_code(col[r], es, inv_e, qmax, mode);
          e_scale_out[vb + c] = es;
        } else {
          for (int r = 0; r < K; ++r) {
            const int64_t i = mb + (int64_t)r * V + c;
            if (res_fmt == RES_FP16) ((uint16_t*)e_out)[i] = orc_f32_to_f16(col[r]);
            else if (res_fmt == RES_FP8) ((uint8_t*)e_out)[i] = orc_f32_to_e5m2(col[r]);
            else ((float*)e_out)[i] = col[r];
          }
        }
      }
    }
    free(h);
    free(kp);
    free(qp);
    free(rd);
    free(col);
  }
  return 0;
}

/* FP32 GDN step in the statequant layout (statequant/kernel.py:116-123). */
int orc_fp32_step_kv(const float* h_in, const float* q, const float* k, const float* v, const float* alpha,
                     const float* beta, float* o, float* h_out, int B, int HV, int K, int V) {
  if (!statequant_k_ok(K) || V <= 0) return 1;
  const int KP = statequant_kp(K);
  float* rd = (float*)malloc(sizeof(float) * V);
  float* h = (float*)calloc((size_t)KP * V, sizeof(float)); /* rows K..KP-1 stay +0 */
  float* kp = (float*)calloc((size_t)KP, sizeof(float));
  float* qp = (float*)calloc((size_t)KP, sizeof(float));
  for (int64_t w = 0; w < (int64_t)B * HV; ++w) {
    const int64_t mb = w * (int64_t)K * V, vb = w * V, kb = w * K;
    for (int r = 0; r < K; ++r) {
      kp[r] = k[kb + r];
      qp[r] = q[kb + r];
    }
    for (int64_t i = 0; i < (int64_t)K * V; ++i) h[i] = h_in[mb + i] * alpha[w];
    for (int c = 0; c < V; ++c) rd[c] = beta[w] * (v[vb + c] - dot_slices(h + c, V, kp, KP));
    for (int r = 0; r < K; ++r)
      for (int c = 0; c < V; ++c) h[(int64_t)r * V + c] = fmaf(k[kb + r], rd[c], h[(int64_t)r * V + c]);
    for (int c = 0; c < V; ++c) o[vb + c] = dot_slices(h + c, V, qp, KP);
    for (int64_t i = 0; i < (int64_t)K * V; ++i) h_out[mb + i] = h[i];
  }
  free(rd);
  free(h);
  free(kp);
  free(qp);
  return 0;
}

/* vLLM-layout step with an unquantized fp32 or bf16 state pool (the
 * comparison arm): state [S, HV, V, K] as fp32 values; with bf16 != 0 the
 * stored state is rounded to bf16 (nearest even) and kept as fp32 values. */
static float bf16_round_f(float x) {
  uint32_t u = orc_float_to_bits(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return x;
  u += 0x7fffu + ((u >> 16) & 1u);
  return orc_bits_to_float(u & 0xffff0000u);
}

/* bf16_round_f over an array (exported so tests can pin it against torch). */
void orc_bf16_round_n(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = bf16_round_f(x[i]);
}

int orc_packed_decode_float_state(const float* mixed, int64_t stride_mixed,
                                  const float* a, int64_t stride_a, const float* b, int64_t stride_b,
                                  const float* A_log, const float* dt_bias, float scale,
                                  float* state, int64_t stride_state, int bf16,
                                  float* out, const int32_t* idx, int64_t num_slots,
                                  int B, int H, int HV, int K, int V, int l2norm) {
  if (K % 16 != 0 || K > 256 || (K / 16 & (K / 16 - 1)) != 0 || HV % H != 0) return 1;
  float* q = (float*)malloc(sizeof(float) * K);
  float* k = (float*)malloc(sizeof(float) * K);
  for (int64_t w = 0; w < (int64_t)B * HV; ++w) {
    const int n = (int)(w / HV), hv = (int)(w % HV);
    const int64_t slot = idx[n];
    float* o = out + ((int64_t)n * HV + hv) * V;
    if (slot <= 0 || slot >= num_slots) {
      for (int r = 0; r < V; ++r) o[r] = slot <= 0 ? 0.0f : NAN;
      continue;
    }
    const int hq = hv / (HV / H);
    const float* m = mixed + (int64_t)n * stride_mixed;
    for (int j = 0; j < K; ++j) {
      q[j] = m[(int64_t)hq * K + j];
      k[j] = m[(int64_t)H * K + (int64_t)hq * K + j];
    }
    if (l2norm) {
      const float dq = sqrtf(dot_k(q, 1, q, 1, K) + 1e-6f);
      const float dk = sqrtf(dot_k(k, 1, k, 1, K) + 1e-6f);
      for (int j = 0; j < K; ++j) {
        q[j] = q[j] / dq;
        k[j] = k[j] / dk;
      }
    }
    for (int j = 0; j < K; ++j) q[j] = q[j] * scale;
    float alpha, beta;
    orc_gates(a[(int64_t)n * stride_a + hv], b[(int64_t)n * stride_b + hv], A_log[hv], dt_bias[hv], &alpha, &beta);
    float* st = state + slot * stride_state + (int64_t)hv * V * K;
    const float* vv = m + 2 * (int64_t)H * K + (int64_t)hv * V;
    for (int r = 0; r < V; ++r) {
      float* h = st + (int64_t)r * K;
      for (int j = 0; j < K; ++j) h[j] = h[j] * alpha;
      const float dv = beta * (vv[r] - dot_k(h, 1, k, 1, K));
      for (int j = 0; j < K; ++j) h[j] = fmaf(k[j], dv, h[j]);
      o[r] = dot_k(h, 1, q, 1, K);
      if (bf16)
        for (int j = 0; j < K; ++j) h[j] = bf16_round_f(h[j]);
    }
  }
  free(q);
  free(k);
  return 0;
}

/*
 * Checker for the HIP kernels' scale division (not part of the step): the
 * kernels compute RN(a / q) for a small integer q as Markstein's correction
 * of the reciprocal product, q0 = RN(a * rq), r = fma(-q0, q, a),
 * RN(fma(r, rq, q0)) with rq = RN(1 / q). Counts, over every mantissa of a at
 * biased exponents e_lo..e_hi, the cases where that differs from the IEEE
 * quotient a / q.
 */
int64_t orc_count_div_small_int_mismatches(float q, int e_lo, int e_hi) {
  const float rq = 1.0f / q;
  int64_t bad = 0;
  for (int e = e_lo; e <= e_hi; ++e) {
#pragma omp parallel for reduction(+ : bad)
    for (int64_t m = 0; m < (1 << 23); ++m) {
      const float a = orc_bits_to_float(((uint32_t)e << 23) | (uint32_t)m);
      const float q0 = a * rq;
      const float r = fmaf(-q0, q, a);
      const float got = fmaf(r, rq, q0);
      bad += orc_float_to_bits(got) != orc_float_to_bits(a / q);
    }
  }
  return bad;
}
