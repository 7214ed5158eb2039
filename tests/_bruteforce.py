"""Independent scalar restatement of the decode step for tiny shapes.

Pure Python over np.float32 scalars (each +, *, /, sqrt rounds to fp32 as
IEEE requires) with an exact fused multiply-add (Fraction arithmetic, one
round-to-nearest-even to fp32). It follows the reference lines directly,
element by element, with none of the C oracle's code structure, so that a
mistake in either (an index, a dropped term, a swapped nibble, a reduction
order) shows up as a disagreement:
  vllm_integration/quantized_packed_decode.py:129-239  (vLLM layout)
  statequant/kernel.py:149-178, :296-341               (statequant layout)
The fp32 evaluation order of the K-sums is the one the kernels define:
chunks of 16 (vLLM layout) or slices of consecutive rows (statequant layout:
8 slices of K/8 rows up to K = 128, 16 rows each above), each a sequential
fma chain, combined as a balanced pairwise tree.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np

import oracle

F = np.float32
MAGIC = F(12582912.0)


def f32_round(x: Fraction) -> np.float32:
    """Round an exact rational to the nearest fp32 (ties to even)."""
    if x == 0:
        return F(0.0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)                       # subnormals share the 2^-149 grid
    ulp = Fraction(2) ** (e - 23)
    q = a / ulp
    m = q.numerator // q.denominator
    rem = q - m
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and m % 2 == 1):
        m += 1
    val = m * ulp
    if val >= Fraction(2) ** 128:
        return F(sign * np.inf)
    return F(sign * float(val))


def fma(a, b, c) -> np.float32:
    return f32_round(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def chunk_dot(x, y, chunk):
    """sum x*y: sequential fma chains of `chunk` elements, balanced tree over chunks."""
    parts = []
    for s in range(0, len(x), chunk):
        acc = F(x[s] * y[s])
        for j in range(s + 1, s + chunk):
            acc = fma(x[j], y[j], acc)
        parts.append(acc)
    while len(parts) > 1:
        parts = [F(parts[i] + parts[i + 1]) for i in range(0, len(parts), 2)]
    return parts[0]


def quant(t, s, inv, qmax, exact):
    c = np.rint(F(t / s)) if exact else F(fma(t, inv, MAGIC) - MAGIC)
    return F(min(max(c, -qmax), qmax))


def resid(t, c, s, exact):
    return F(t - F(c * s)) if exact else fma(-c, s, t)


def madd(x, y, a, exact):
    return F(a + F(x * y)) if exact else fma(x, y, a)


def nibble(byte, j):
    """quantized_packed_decode.py:196-199."""
    v = (int(byte) & 0xFF) >> (4 * (j % 2)) & 0xF
    return v - 16 if v > 7 else v


def packed_decode(mixed, a, b, A_log, dt_bias, scale, sc, ss, rc, rs, idx, H, *, l2norm, resid_fmt,
                  per_head, bits, exact):
    """One vLLM-layout step on copies of the pool; returns (out, sc, ss, rc, rs)."""
    sc, ss, rc, rs = sc.copy(), ss.copy(), rc.copy(), rs.copy()
    S, HV, V, K = sc.shape
    # quantized_packed_decode.py:123-127,158,165-166,196-202: lanes o_k < BK
    # load 0 past K; the sums run over KP = max(16, next_pow2(K)) values
    KP = 16
    while KP < K:
        KP *= 2
    Z = [F(0.0)] * (KP - K)
    B = mixed.shape[0]
    qmax = F(2 ** (bits - 1) - 1)
    qe = F(7.0 if resid_fmt == oracle.RESID_INT4 else 127.0)
    alpha_all, beta_all = oracle.gates(a, b, A_log[None, :], dt_bias[None, :])
    out = np.zeros((B, HV, V), F)
    for n in range(B):
        slot = int(idx[n])
        for hv in range(HV):
            if slot <= 0:
                continue
            hq = hv // (HV // H)
            q = [F(mixed[n, hq * K + j]) for j in range(K)] + Z
            k = [F(mixed[n, H * K + hq * K + j]) for j in range(K)] + Z
            if l2norm:
                dq = F(np.sqrt(F(chunk_dot(q, q, 16) + F(1e-6))))
                dk = F(np.sqrt(F(chunk_dot(k, k, 16) + F(1e-6))))
                q = [F(x / dq) for x in q]
                k = [F(x / dk) for x in k]
            q = [F(x * F(scale)) for x in q]
            al, be = F(alpha_all[n, hv]), F(beta_all[n, hv])
            es_head = F(rs[slot, hv]) if per_head else None
            eall = []
            for r in range(V):
                codes_in = [int(sc[slot, hv, r, j]) for j in range(K)] + [0] * (KP - K)
                if exact:
                    h = [F(F(F(x) * ss[slot, hv, r]) * al) for x in codes_in]
                else:
                    sa = F(ss[slot, hv, r] * al)
                    h = [F(F(x) * sa) for x in codes_in]
                rd = chunk_dot(h, k, 16)
                dv = F(be * F(F(mixed[n, 2 * H * K + hv * V + r]) - rd))
                h = [madd(k[j], dv, h[j], exact) for j in range(KP)]
                out[n, hv, r] = chunk_dot(h, q, 16)
                es_in = es_head if per_head else F(rs[slot, hv, r])
                if resid_fmt == oracle.RESID_INT4:
                    ec = [nibble(rc[slot, hv, r, j // 2], j) for j in range(K)]
                else:
                    ec = [int(rc[slot, hv, r, j]) for j in range(K)]
                ec += [0] * (KP - K)
                t = [madd(F(ec[j]), es_in, h[j], exact) for j in range(KP)]
                am = max(abs(x) for x in t)
                s = F(max(F(am / qmax), F(1e-12)))
                inv = F(F(1.0) / s)
                codes = [quant(x, s, inv, qmax, exact) for x in t]
                e = [resid(t[j], codes[j], s, exact) for j in range(KP)]
                sc[slot, hv, r, :] = np.array(codes[:K], np.int8)
                ss[slot, hv, r] = s
                eall.append(e)
            rows = range(V)
            if per_head:
                ea = max(abs(x) for e in eall for x in e)
                es_rows = [F(max(F(ea / qe), F(1e-12)))] * V
            else:
                es_rows = [F(max(F(max(abs(x) for x in eall[r]) / qe), F(1e-12))) for r in rows]
            for r in rows:
                es = es_rows[r]
                inv_e = F(F(1.0) / es)
                ecodes = [int(quant(x, es, inv_e, qe, exact)) for x in eall[r][:K]]
                if resid_fmt == oracle.RESID_INT4:
                    for j in range(0, K, 2):        # quantized_packed_decode.py:226-230
                        byte = (ecodes[j] & 0xF) | ((ecodes[j + 1] & 0xF) << 4)
                        rc[slot, hv, r, j // 2] = np.uint8(byte).view(np.int8)
                else:
                    rc[slot, hv, r, :] = np.array(ecodes, np.int8)
                if not per_head:
                    rs[slot, hv, r] = es
            if per_head:
                rs[slot, hv] = es_rows[0]
    return out, sc, ss, rc, rs


def quant_step_kv(h_int8, scale, e, e_scale, q, k, v, alpha, beta, *, bits, res_fmt, exact):
    """One statequant-layout step; residual storage as in oracle.quant_step_kv.
    Any K: the sums run over KP = max(16, next_pow2(K)) rows, zero past K, as
    the reference's Triton kernel masks its BK = next_pow2(K) rows
    (statequant/kernel.py:277-279)."""
    B, HV, K, V = h_int8.shape
    KP = 16
    while KP < K:
        KP *= 2
    rows = KP // 8 if KP <= 128 else 16        # rows per K-slice
    Z = [F(0.0)] * (KP - K)
    qmax = F(2 ** (bits - 1) - 1)
    o = np.zeros((B, HV, V), F)
    h_out = np.zeros_like(h_int8)
    s_out = np.zeros((B, HV, V), F)
    e_out = np.zeros_like(e)
    es_out = np.zeros((B, HV, V), F) if res_fmt == oracle.RES_INT8 else None
    for bb in range(B):
        for hv in range(HV):
            al, be = F(alpha[bb, hv]), F(beta[bb, hv])
            kk = [F(x) for x in k[bb, hv]] + Z
            qq = [F(x) for x in q[bb, hv]] + Z
            for c in range(V):
                sc = F(scale[bb, hv, c])
                if exact:
                    h = [F(F(F(int(h_int8[bb, hv, r, c])) * sc) * al) for r in range(K)]
                else:
                    h = [F(F(int(h_int8[bb, hv, r, c])) * F(sc * al)) for r in range(K)]
                dv = F(be * F(F(v[bb, hv, c]) - chunk_dot(h + Z, kk, rows)))
                h = [madd(kk[r], dv, h[r], exact) for r in range(K)]
                o[bb, hv, c] = chunk_dot(h + Z, qq, rows)
                if res_fmt == oracle.RES_INT8:
                    t = [madd(F(int(e[bb, hv, r, c])), F(e_scale[bb, hv, c]), h[r], exact) for r in range(K)]
                elif res_fmt == oracle.RES_FP16:
                    t = [F(h[r] + F(np.uint16(e[bb, hv, r, c]).view(np.float16))) for r in range(K)]
                elif res_fmt == oracle.RES_FP8:
                    t = [F(h[r] + oracle.e5m2_bits_to_f32(np.uint8(e[bb, hv, r, c]))[()]) for r in range(K)]
                else:
                    t = [F(h[r] + F(e[bb, hv, r, c])) for r in range(K)]
                s = F(max(F(max(abs(x) for x in t) / qmax), F(1e-12)))
                inv = F(F(1.0) / s)
                codes = [quant(x, s, inv, qmax, exact) for x in t]
                ee = [resid(t[r], codes[r], s, exact) for r in range(K)]
                h_out[bb, hv, :, c] = np.array(codes, np.int8)
                s_out[bb, hv, c] = s
                if res_fmt == oracle.RES_INT8:
                    es = F(max(F(max(abs(x) for x in ee) / qmax), F(1e-12)))
                    inv_e = F(F(1.0) / es)
                    e_out[bb, hv, :, c] = np.array([quant(x, es, inv_e, qmax, exact) for x in ee], np.int8)
                    es_out[bb, hv, c] = es
                elif res_fmt == oracle.RES_FP16:
                    e_out[bb, hv, :, c] = np.array(ee, F).astype(np.float16).view(np.uint16)
                elif res_fmt == oracle.RES_FP8:
                    e_out[bb, hv, :, c] = oracle.f32_to_e5m2_bits(np.array(ee, F))
                else:
                    e_out[bb, hv, :, c] = np.array(ee, F)
    return o, h_out, s_out, e_out, es_out
