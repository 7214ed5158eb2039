"""CPU tests that pin the oracle (no GPU): closed forms, the reference's own
known-answer constructions, an independent brute-force restatement on tiny
shapes, float64 comparisons and invariants of error feedback."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from tests import _bruteforce as bf
from tests._helpers import make_packed_inputs, make_pool, rel

F = np.float32


# ---------------------------------------------------------------------------
# gate transcendentals (quantized_packed_decode.py:179-182)
# ---------------------------------------------------------------------------

def _ulp_err(got, ref64):
    got = got.astype(np.float64)
    ulp = np.spacing(np.abs(ref64).astype(np.float32)).astype(np.float64)
    return np.abs(got - ref64) / ulp


def test_expf_accuracy_and_special_values():
    x = np.concatenate([np.linspace(-103.9, 88.7, 400001, dtype=np.float32),
                        np.float32([0.0, -0.0, 1e-30, -1e-30, 0.5, -0.5, 88.72283, -87.3])])
    y = oracle.expf(x)
    ref = np.exp(x.astype(np.float64))
    finite = ref > 1.2e-38   # normal results
    assert _ulp_err(y[finite], ref[finite]).max() <= 2.0
    sub = (ref <= 1.2e-38) & (ref > 0)
    assert np.abs(y[sub] - ref[sub]).max() <= 2 * 2.0 ** -149
    assert oracle.expf([89.0])[0] == np.inf and oracle.expf([-110.0])[0] == 0.0
    assert np.isnan(oracle.expf([np.nan])[0])
    assert oracle.expf([0.0])[0] == 1.0


def test_logf_accuracy_and_special_values():
    x = np.concatenate([np.geomspace(1e-38, 3e38, 400001).astype(np.float32),
                        np.float32([1.0, 2.0, 0.5, 1.0000001, 0.9999999, 1e-44])])
    y = oracle.logf(x)
    ref = np.log(x.astype(np.float64))
    nz = np.abs(ref) > 1e-6
    assert _ulp_err(y[nz], ref[nz]).max() <= 2.0
    assert np.abs(y[~nz] - ref[~nz]).max() <= 2e-7
    assert oracle.logf([1.0])[0] == 0.0
    assert oracle.logf([0.0])[0] == -np.inf and np.isnan(oracle.logf([-1.0])[0])


def test_gates_match_closed_form():
    """test_quantized_packed_decode.py:54-62 in float64, same threshold rule."""
    rng = np.random.default_rng(0)
    a = rng.normal(0, 3, 20000).astype(F)
    b = rng.normal(0, 3, 20000).astype(F)
    A_log = rng.normal(0, 0.5, 20000).astype(F)
    dt = rng.normal(0, 0.5, 20000).astype(F)
    al, be = oracle.gates(a, b, A_log, dt)
    x = a.astype(np.float64) + dt
    sp = np.where(x <= 20.0, np.log1p(np.exp(x)), x)
    al64 = np.exp(-np.exp(A_log.astype(np.float64)) * sp)
    be64 = 1 / (1 + np.exp(-b.astype(np.float64)))
    assert np.abs(al - al64).max() / al64.max() < 1e-6
    assert np.max(np.abs(al - al64) / np.maximum(al64, 1e-30)) < 1e-5
    assert np.max(np.abs(be - be64) / be64) < 1e-6
    # neutral gates of the reference's tie test: a = b = -60 -> alpha = 1, beta ~ 0
    al1, be1 = oracle.gates([-60.0], [-60.0], [0.0], [0.0])
    assert al1[0] == 1.0 and be1[0] < 1e-25


# ---------------------------------------------------------------------------
# scale division of the kernels (amax / qmax without an IEEE divide)
# ---------------------------------------------------------------------------

def test_small_int_division_is_correctly_rounded():
    """The kernels' RN(amax / qmax) (a Markstein-corrected reciprocal product)
    equals the IEEE quotient for every qmax the kernels use (1..127) over all
    mantissas at exponents from the 1e-12 eps floor to the top of the range."""
    bad = sum(oracle.count_div_small_int_mismatches(q, e, e) for q in range(1, 128) for e in (87, 127, 200, 254))
    assert bad == 0
    # the checker discriminates: the uncorrected product RN(a * RN(1/q)) is wrong often
    a = ((np.uint32(127) << 23) | np.arange(1 << 23, dtype=np.uint32)).view(F)
    assert np.count_nonzero(a * (F(1) / F(3)) != a / F(3)) > 1000


# ---------------------------------------------------------------------------
# storage codecs
# ---------------------------------------------------------------------------

def test_int4_pack_roundtrip_all_codes():
    """quantized_packed_decode.py:196-199 / :226-230: every (even, odd) pair of
    codes -7..7 packs into one byte and unpacks to itself."""
    codes = np.array([[e, o] for e in range(-7, 8) for o in range(-7, 8)], np.int32).reshape(1, -1)
    packed = oracle.pack_int4(codes)
    assert packed.shape[-1] == codes.shape[-1] // 2
    np.testing.assert_array_equal(oracle.unpack_int4(packed), codes)
    # the layout itself: even element in the low nibble
    assert oracle.pack_int4(np.array([[3, -2]]))[0, 0] == np.int8(np.uint8(0xE3).view(np.int8))


def test_fp16_and_e5m2_codecs():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(F) * F(1e-3),
                        rng.standard_normal(1000).astype(F) * F(1e4),
                        F([0.0, -0.0, 65504, 65519.99, 65520, 2 ** -24, 2 ** -25, 3 * 2 ** -25, 57344, 61439,
                           61440, 2 ** -16, 2 ** -17, 3 * 2 ** -17, 1.5e-5])]).astype(F)
    with np.errstate(over="ignore"):
        np.testing.assert_array_equal(oracle.f32_to_f16_bits(x), x.astype(np.float16).view(np.uint16))
    t = torch.from_numpy(x).to(torch.float8_e5m2)
    np.testing.assert_array_equal(oracle.f32_to_e5m2_bits(x), t.view(torch.uint8).numpy())
    allb = np.arange(256, dtype=np.uint8)
    dec = oracle.e5m2_bits_to_f32(allb)
    ref = torch.from_numpy(allb).view(torch.float8_e5m2).float().numpy()
    same = (dec == ref) | (np.isnan(dec) & np.isnan(ref))
    assert same.all()


# ---------------------------------------------------------------------------
# brute-force restatement on tiny shapes (bit-exact)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("resid_fmt", [oracle.RESID_INT8, oracle.RESID_INT4])
@pytest.mark.parametrize("per_head", [False, True])
@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("l2norm,bits", [(True, 8), (False, 6)])
def test_packed_decode_matches_bruteforce(resid_fmt, per_head, exact, l2norm, bits):
    B, H, HV, K, V = 2, 1, 2, 32, 3
    pool = make_pool(4, HV, V, K, resid_fmt, per_head, seed=11, bits=bits)
    mixed, a, b, A_log, dt = (x.numpy() for x in make_packed_inputs(B, H, HV, K, V, seed=3))
    idx = np.array([2, 3], np.int32)
    ref = bf.packed_decode(mixed, a, b, A_log, dt, 0.25, *pool, idx, H, l2norm=l2norm, resid_fmt=resid_fmt,
                           per_head=per_head, bits=bits, exact=exact)
    got_pool = [x.copy() for x in pool]
    out = oracle.packed_decode(mixed, a, b, A_log, dt, 0.25, *got_pool, idx, H, use_qk_l2norm=l2norm,
                               resid_fmt=resid_fmt, per_head=per_head, state_bits=bits,
                               mode=oracle.MODE_EXACT if exact else oracle.MODE_FAST)
    np.testing.assert_array_equal(out, ref[0])
    for g, r in zip(got_pool, ref[1:]):
        np.testing.assert_array_equal(g, r)


@pytest.mark.parametrize("K,resid_fmt,exact", [(7, oracle.RESID_INT8, False), (24, oracle.RESID_INT4, True),
                                               (24, oracle.RESID_INT8, False), (2, oracle.RESID_INT4, False),
                                               (100, oracle.RESID_INT8, True), (200, oracle.RESID_INT4, False),
                                               (300, oracle.RESID_INT8, True), (512, oracle.RESID_INT4, False),
                                               (1000, oracle.RESID_INT4, True)])
@pytest.mark.parametrize("per_head", [False, True])
def test_packed_decode_any_k_matches_bruteforce(K, resid_fmt, exact, per_head):
    """K that is not a power of two from 16: the brute force pads q, k and
    every row with zeros to the reference's power-of-two lane count, as its
    masked loads do (quantized_packed_decode.py:123-127,158,165-166)."""
    B, H, HV, V = 2, 1, 2, 3
    pool = make_pool(4, HV, V, K, resid_fmt, per_head, seed=K, bits=8)
    mixed, a, b, A_log, dt = (x.numpy() for x in make_packed_inputs(B, H, HV, K, V, seed=K + 1))
    idx = np.array([3, 1], np.int32)
    ref = bf.packed_decode(mixed, a, b, A_log, dt, 0.5, *pool, idx, H, l2norm=True, resid_fmt=resid_fmt,
                           per_head=per_head, bits=8, exact=exact)
    got_pool = [x.copy() for x in pool]
    out = oracle.packed_decode(mixed, a, b, A_log, dt, 0.5, *got_pool, idx, H, use_qk_l2norm=True,
                               resid_fmt=resid_fmt, per_head=per_head,
                               mode=oracle.MODE_EXACT if exact else oracle.MODE_FAST)
    np.testing.assert_array_equal(out, ref[0])
    for g, r in zip(got_pool, ref[1:]):
        np.testing.assert_array_equal(g, r)


def _pad_k(pool, mixed, H, HV, V, K, KP, resid_fmt):
    """The same step posed on rows of KP columns: zero state and residual
    codes past K, q and k of every head zero-padded to KP."""
    sc, ss, rc, rs = pool
    scp = np.zeros(sc.shape[:3] + (KP,), np.int8)
    scp[..., :K] = sc
    rk, rkp = (K // 2, KP // 2) if resid_fmt == oracle.RESID_INT4 else (K, KP)
    rcp = np.zeros(rc.shape[:3] + (rkp,), np.int8)
    rcp[..., :rk] = rc
    B = mixed.shape[0]
    q = np.zeros((B, H, KP), np.float32)
    k = np.zeros((B, H, KP), np.float32)
    q[..., :K] = mixed[:, :H * K].reshape(B, H, K)
    k[..., :K] = mixed[:, H * K:2 * H * K].reshape(B, H, K)
    mixed_p = np.concatenate([q.reshape(B, -1), k.reshape(B, -1), mixed[:, 2 * H * K:]], axis=1)
    return (scp, ss.copy(), rcp, rs.copy()), np.ascontiguousarray(mixed_p)


@pytest.mark.parametrize("K,KP", [(7, 16), (24, 32), (100, 128), (130, 256)])
@pytest.mark.parametrize("resid_fmt", [oracle.RESID_INT8, oracle.RESID_INT4])
@pytest.mark.parametrize("per_head", [False, True])
@pytest.mark.parametrize("mode", [oracle.MODE_FAST, oracle.MODE_EXACT])
def test_any_k_step_equals_zero_padded_power_of_two(K, KP, resid_fmt, per_head, mode):
    """The oracle's any-K step against its power-of-two path on the same rows
    padded with zero columns (the reference's masked lanes): identical
    outputs, scales and first K codes, and the padding columns stay zero."""
    if resid_fmt == oracle.RESID_INT4 and K % 2:
        pytest.skip("the int4 residual needs an even K")
    B, H, HV, V = 3, 2, 4, 20
    pool = make_pool(5, HV, V, K, resid_fmt, per_head, seed=K, bits=8)
    mixed, a, b, A_log, dt = (x.numpy() for x in make_packed_inputs(B, H, HV, K, V, seed=KP))
    padded, mixed_p = _pad_k(pool, mixed, H, HV, V, K, KP, resid_fmt)
    idx = np.array([4, 0, 2], np.int32)
    for l2norm in (False, True):
        out = oracle.packed_decode(mixed, a, b, A_log, dt, 0.3, *pool, idx, H, use_qk_l2norm=l2norm,
                                   resid_fmt=resid_fmt, per_head=per_head, mode=mode)
        out_p = oracle.packed_decode(mixed_p, a, b, A_log, dt, 0.3, *padded, idx, H, use_qk_l2norm=l2norm,
                                     resid_fmt=resid_fmt, per_head=per_head, mode=mode)
        np.testing.assert_array_equal(out, out_p)
        rk = K // 2 if resid_fmt == oracle.RESID_INT4 else K
        np.testing.assert_array_equal(pool[0], padded[0][..., :K])
        np.testing.assert_array_equal(pool[2], padded[2][..., :rk])
        assert not padded[0][..., K:].any() and not padded[2][..., rk:].any()
        np.testing.assert_array_equal(pool[1], padded[1])
        np.testing.assert_array_equal(pool[3], padded[3])


@pytest.mark.parametrize("res_fmt", [oracle.RES_FP32, oracle.RES_FP16, oracle.RES_FP8, oracle.RES_INT8])
@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("HV,K,V", [(2, 16, 4), (1, 64, 5), (1, 256, 3), (2, 7, 4), (1, 100, 3), (1, 200, 2)])
def test_quant_step_kv_matches_bruteforce(res_fmt, exact, HV, K, V):
    """Every residual format and mode; K = 256 takes 16 slices of 16 rows,
    smaller K 8 slices of K/8; V not a multiple of 4. K = 7, 100, 200: the
    sums over the rows zero-padded to 16, 128 and 256."""
    B = 1
    rng = np.random.default_rng(res_fmt + K)
    h0 = (rng.standard_normal((B, HV, K, V)) * 0.1).astype(F)
    codes, scale = oracle.quantize_cols(h0)
    res = (rng.standard_normal((B, HV, K, V)) * 1e-3).astype(F)
    es = None
    if res_fmt == oracle.RES_INT8:
        es = (np.abs(res).max(axis=-2) / 127).astype(F)
        e = np.clip(np.rint(res / es[:, :, None, :]), -127, 127).astype(np.int8)
    elif res_fmt == oracle.RES_FP16:
        e = res.astype(np.float16).view(np.uint16)
    elif res_fmt == oracle.RES_FP8:
        e = oracle.f32_to_e5m2_bits(res)
    else:
        e = res
    q = rng.standard_normal((B, HV, K)).astype(F)
    k = rng.standard_normal((B, HV, K)).astype(F)
    v = rng.standard_normal((B, HV, V)).astype(F)
    alpha = F(rng.uniform(0.9, 1.0, (B, HV)))
    beta = F(rng.uniform(0.1, 0.9, (B, HV)))
    ref = bf.quant_step_kv(codes, scale, e, es, q, k, v, alpha, beta, bits=8, res_fmt=res_fmt, exact=exact)
    got = oracle.quant_step_kv(codes, scale, e, es, q, k, v, alpha, beta, bits=8, res_fmt=res_fmt,
                               mode=oracle.MODE_EXACT if exact else oracle.MODE_FAST)
    for g, r in zip(got, ref):
        if r is None:
            assert g is None
        else:
            np.testing.assert_array_equal(g, r)


@pytest.mark.parametrize("res_fmt", [oracle.RES_FP32, oracle.RES_FP16, oracle.RES_FP8, oracle.RES_INT8])
@pytest.mark.parametrize("K,KP", [(5, 16), (48, 64), (100, 128), (130, 256)])
def test_statequant_any_k_equals_zero_padded_power_of_two(res_fmt, K, KP):
    """An any-K statequant step equals the KP step on the same rows followed
    by zero rows (zero codes, residual, q and k): o, scales and the first K
    rows of codes and residual agree bit for bit, and the padding rows come
    out zero."""
    B, HV, V = 2, 2, 6
    rng = np.random.default_rng(K + res_fmt)
    h0 = (rng.standard_normal((B, HV, K, V)) * 0.1).astype(F)
    codes, scale = oracle.quantize_cols(h0)
    res = (rng.standard_normal((B, HV, K, V)) * 1e-3).astype(F)
    es = None
    if res_fmt == oracle.RES_INT8:
        es = (np.abs(res).max(axis=-2) / 127).astype(F)
        e = np.clip(np.rint(res / es[:, :, None, :]), -127, 127).astype(np.int8)
    elif res_fmt == oracle.RES_FP16:
        e = res.astype(np.float16).view(np.uint16)
    elif res_fmt == oracle.RES_FP8:
        e = oracle.f32_to_e5m2_bits(res)
    else:
        e = res
    q = rng.standard_normal((B, HV, K)).astype(F)
    k = rng.standard_normal((B, HV, K)).astype(F)
    v = rng.standard_normal((B, HV, V)).astype(F)
    alpha = F(rng.uniform(0.9, 1.0, (B, HV)))
    beta = F(rng.uniform(0.1, 0.9, (B, HV)))

    def pad_rows(x):
        z = np.zeros(x.shape[:2] + (KP - K,) + x.shape[3:], x.dtype)
        return np.ascontiguousarray(np.concatenate([x, z], axis=2))

    for mode in (oracle.MODE_FAST, oracle.MODE_EXACT):
        got = oracle.quant_step_kv(codes, scale, e, es, q, k, v, alpha, beta, bits=8, res_fmt=res_fmt, mode=mode)
        ref = oracle.quant_step_kv(pad_rows(codes), scale, pad_rows(e), es, pad_rows(q), pad_rows(k), v, alpha, beta,
                                   bits=8, res_fmt=res_fmt, mode=mode)
        o, h_out, s_out, e_out, es_out = got
        o_p, h_p, s_p, e_p, es_p = ref
        np.testing.assert_array_equal(o, o_p)
        np.testing.assert_array_equal(s_out, s_p)
        np.testing.assert_array_equal(h_out, h_p[:, :, :K])
        np.testing.assert_array_equal(e_out, e_p[:, :, :K])
        assert not h_p[:, :, K:].any() and not np.asarray(e_p[:, :, K:]).view(np.uint8).any()
        if es_out is not None:
            np.testing.assert_array_equal(es_out, es_p)
    h, o = oracle.fp32_step_kv(h0, q, k, v, alpha, beta)
    h_p, o_p = oracle.fp32_step_kv(pad_rows(h0), pad_rows(q), pad_rows(k), v, alpha, beta)
    np.testing.assert_array_equal(o, o_p)
    np.testing.assert_array_equal(h, h_p[:, :, :K])
    assert not h_p[:, :, K:].any()


def _slice_order_case(K, V, rows):
    """Inputs whose h^T q is exact per product: beta = 0 (h is its dequantized
    codes), alpha = scale = 1, code 1 in each listed row with q carrying the
    value; every other code and q is 0."""
    codes = np.zeros((1, 1, K, V), np.int8)
    q = np.zeros((1, 1, K), F)
    for r, val in rows:
        codes[0, 0, r, :] = 1
        q[0, 0, r] = val
    z = np.zeros
    return (codes, np.ones((1, 1, V), F), z((1, 1, K, V), F), None, q, z((1, 1, K), F), z((1, 1, V), F),
            np.ones((1, 1), F), z((1, 1), F))


def statequant_slices(K):
    return 8 if K <= 128 else K // 16


@pytest.mark.parametrize("K", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("mode", [oracle.MODE_FAST, oracle.MODE_EXACT])
def test_statequant_reduction_order_known_answer(K, mode):
    """Closed forms that fix the K-sum order of the statequant step.
    (a) 2^24 at row 0 and 1 at rows R and R+1 (R = rows per slice): the slice
    holding rows R, R+1 sums them to 2 before meeting 2^24, giving 2^24 + 2;
    slices twice as long, or one sequential chain, would add each 1 to 2^24
    separately and round back to 2^24. (b) 2^24 at row 0 and 1 at the first
    row of every other slice: a balanced tree over S slices loses only the 1
    paired with 2^24 at its first level, giving 2^24 + S - 2; a sequential
    pass over the slices would give 2^24."""
    S = statequant_slices(K)
    R = K // S
    big = F(2.0 ** 24)
    for rows, want in (([(0, big), (R, 1.0), (R + 1, 1.0)], big + 2),
                       ([(0, big)] + [(s * R, 1.0) for s in range(1, S)], big + S - 2)):
        o = oracle.quant_step_kv(*_slice_order_case(K, 3, rows), mode=mode)[0]
        assert np.all(o == want), (K, rows[:3], o.ravel(), want)
        ref = bf.quant_step_kv(*_slice_order_case(K, 1, rows), bits=8, res_fmt=oracle.RES_FP32,
                               exact=mode == oracle.MODE_EXACT)[0]
        assert np.all(ref == want)


# ---------------------------------------------------------------------------
# known-answer constructions of the reference's tests
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("mode", [oracle.MODE_FAST, oracle.MODE_EXACT])
def test_round_half_to_even_vllm_layout(mode, H=1, HV=1, K=32, V=4):
    """vllm_integration/test_quantized_packed_decode.py:211-286."""
    odd = (np.arange(K) % 8) * 2 - 7
    rcodes = np.tile(odd, (HV, V, 1)).astype(np.int8)
    rcodes[..., 0] = 0
    scodes = np.zeros((HV, V, K), np.int8)
    scodes[..., 0] = 1
    target = scodes.astype(np.float64) * 127 + rcodes * 0.5
    expected = np.clip(np.round(target), -127, 127)            # numpy round is half-to-even
    assert ((np.abs(target) % 1) == 0.5).sum() > 0 and (np.floor(target + 0.5) != expected).sum() > 0
    sc = np.zeros((2, HV, V, K), np.int8)
    ss = np.zeros((2, HV, V), F)
    rc = np.zeros((2, HV, V, K), np.int8)
    rs = np.zeros((2, HV, V), F)
    sc[1], ss[1], rc[1], rs[1] = scodes, 127.0, rcodes, 0.5
    mixed = np.zeros((1, 2 * H * K + HV * V), F)
    oracle.packed_decode(mixed, np.full((1, HV), -60, F), np.full((1, HV), -60, F), np.zeros(HV, F),
                         np.zeros(HV, F), K ** -0.5, sc, ss, rc, rs, np.array([1], np.int32), H, mode=mode)
    np.testing.assert_array_equal(sc[1].astype(np.float64), expected)


@pytest.mark.parametrize("mode", [oracle.MODE_FAST, oracle.MODE_EXACT])
def test_round_half_to_even_statequant_layout(mode):
    """experiments/test_cuda_kernel.py:64-118 (alpha = beta = 0, target == e)."""
    K, V = 32, 8
    codes = (np.arange(K, dtype=F) % 8) - F(3.5)
    target = np.tile(codes[:, None], (1, V)).astype(F)
    target[0, :] = 127
    expected = np.clip(np.round(target), -127, 127)
    z = np.zeros
    o, h_out, s_out, _, _ = oracle.quant_step_kv(z((1, 1, K, V), np.int8), np.ones((1, 1, V), F),
                                                 target[None, None], None, z((1, 1, K), F), z((1, 1, K), F),
                                                 z((1, 1, V), F), z((1, 1), F), z((1, 1), F), mode=mode)
    np.testing.assert_array_equal(h_out[0, 0], expected)
    assert np.all(s_out == 1.0)


def test_null_block_and_paging_isolation():
    """test_quantized_packed_decode.py:153-208 on the oracle."""
    H, HV, K, V = 8, 16, 64, 64
    pool = make_pool(5, HV, V, K, oracle.RESID_INT8, False, seed=2)
    mixed, a, b, A_log, dt = (x.numpy() for x in make_packed_inputs(2, H, HV, K, V, seed=11))
    before = [x.copy() for x in pool]
    out = oracle.packed_decode(mixed, a, b, A_log, dt, 0.125, *pool, np.array([3, 0], np.int32), H)
    assert np.all(out[1] == 0)
    for slot in (0, 1, 2, 4):
        for now, was in zip(pool, before):
            np.testing.assert_array_equal(now[slot], was[slot])
    assert not np.array_equal(pool[0][3], before[0][3])
    # batched == sequential
    together = [x.copy() for x in before]
    o_t = oracle.packed_decode(mixed, a, b, A_log, dt, 0.125, *together, np.array([3, 1], np.int32), H)
    seq = [x.copy() for x in before]
    for r, slot in ((0, 3), (1, 1)):
        o1 = oracle.packed_decode(mixed[r:r + 1], a[r:r + 1], b[r:r + 1], A_log, dt, 0.125, *seq,
                                  np.array([slot], np.int32), H)
        np.testing.assert_array_equal(o1[0], o_t[r])
    for x, y in zip(seq, together):
        np.testing.assert_array_equal(x, y)


# ---------------------------------------------------------------------------
# float64 comparisons and error-feedback invariants
# ---------------------------------------------------------------------------

def _one_step_f64(mixed, a, b, A_log, dt, scale, sc, ss, rc, rs, idx, H, resid_fmt, per_head, l2norm=False):
    """The reference algorithm (quantized_packed_decode.py:158-209) in float64
    up to the quantization target; returns (out, target) per live request."""
    S, HV, V, K = sc.shape
    B = mixed.shape[0]
    al, be = oracle.gates(a, b, A_log[None], dt[None])
    q = mixed[:, :H * K].reshape(B, H, K).astype(np.float64)
    k = mixed[:, H * K:2 * H * K].reshape(B, H, K).astype(np.float64)
    v = mixed[:, 2 * H * K:].reshape(B, HV, V).astype(np.float64)
    if l2norm:
        q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6)
        k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    q = np.repeat(q * scale, HV // H, axis=1)
    k = np.repeat(k, HV // H, axis=1)
    slots = idx[:B]
    h = sc[slots].astype(np.float64) * ss[slots][..., None]            # [B, HV, V, K]
    h = h * al[..., None, None]
    rd = np.einsum("bhvk,bhk->bhv", h, k)
    dv = be[..., None] * (v - rd)
    h = h + dv[..., None] * k[:, :, None, :]
    o = np.einsum("bhvk,bhk->bhv", h, q)
    codes = oracle.unpack_int4(rc[slots]) if resid_fmt == oracle.RESID_INT4 else rc[slots].astype(np.int32)
    es = rs[slots][..., None, None] if per_head else rs[slots][..., None]
    return o, h + codes * es


@pytest.mark.parametrize("resid_fmt", [oracle.RESID_INT8, oracle.RESID_INT4])
@pytest.mark.parametrize("per_head", [False, True])
def test_one_step_vs_float64_and_ef_invariants(resid_fmt, per_head):
    B, H, HV, K, V = 4, 8, 16, 128, 128
    pool = make_pool(B + 1, HV, V, K, resid_fmt, per_head, seed=4)
    mixed, a, b, A_log, dt = (x.numpy() for x in make_packed_inputs(B, H, HV, K, V, seed=8))
    idx = np.arange(1, B + 1, dtype=np.int32)
    o64, target = _one_step_f64(mixed, a, b, A_log, dt, 0.1, *pool, idx, H, resid_fmt, per_head)
    new = [x.copy() for x in pool]
    out = oracle.packed_decode(mixed, a, b, A_log, dt, 0.1, *new, idx, H, resid_fmt=resid_fmt,
                               per_head=per_head)
    sc, ss, rc, rs = (x[1:] for x in new)
    # o and dequantized state within 1e-3 relative of the float64 algorithm
    assert rel(out, o64) < 1e-5
    deq = sc.astype(np.float64) * ss[..., None]
    assert rel(deq, target) < 1e-2      # int8 quantization noise of the state itself
    # error feedback: codes * scale + residual reconstructs the target
    codes_e = oracle.unpack_int4(rc) if resid_fmt == oracle.RESID_INT4 else rc.astype(np.int32)
    es = rs[..., None, None] if per_head else rs[..., None]
    recon = deq + codes_e * es
    assert rel(recon, target) < (2e-2 if resid_fmt == oracle.RESID_INT4 else 2e-3)
    # every row is scaled so that its largest |code| is exactly qmax
    assert np.all(np.abs(sc).max(axis=-1) == 127)
    # |e'| <= s/2 before residual quantization: |residual dequant| <= s/2 + es/2
    lim = ss[..., None] * 0.5 + np.broadcast_to(es, deq.shape) * 0.5
    assert np.all(np.abs(codes_e * es) <= lim * (1 + 1e-5))
    # codes equal rounding of the float64 target except within 1e-4 of a .5 tie
    r64 = target / ss[..., None]
    diff = sc.astype(np.float64) != np.clip(np.round(r64), -127, 127)
    assert np.all(np.abs(np.abs(r64[diff]) % 1 - 0.5) < 1e-4)
    assert diff.mean() < 1e-4


@pytest.mark.parametrize("resid_fmt", [oracle.RESID_INT8, oracle.RESID_INT4])
def test_fast_vs_exact_mode(resid_fmt):
    """FAST (rne of t * RN(1/s), fma residual, scale*alpha folded) against
    EXACT (rne of the IEEE quotient, op-by-op rounding): two legal fp32
    evaluation orders of the same algorithm. Codes differ by at most one on
    <= 0.01% of elements. On these inputs (q, k not normalised, so h + k dv
    cancels strongly) state scales differ by more than one ulp on about a
    fifth of the rows, by at most 32 ulp (about 2e-6 relative); the
    reference's own torch path differs from EXACT by more on the same
    inputs (tests/test_torch_path_cpu.py). Bit-identical scales hold only
    against an oracle with the same order, which the GPU parity tests use."""
    B, H, HV, K, V = 8, 32, 32, 128, 128
    pool = make_pool(B + 1, HV, V, K, resid_fmt, True, seed=6)
    mixed, a, b, A_log, dt = (x.numpy() for x in make_packed_inputs(B, H, HV, K, V, seed=9))
    idx = np.arange(1, B + 1, dtype=np.int32)
    pf = [x.copy() for x in pool]
    pe = [x.copy() for x in pool]
    of = oracle.packed_decode(mixed, a, b, A_log, dt, 1.0, *pf, idx, H, resid_fmt=resid_fmt, per_head=True)
    oe = oracle.packed_decode(mixed, a, b, A_log, dt, 1.0, *pe, idx, H, resid_fmt=resid_fmt, per_head=True,
                              mode=oracle.MODE_EXACT)
    assert rel(of, oe) < 1e-5
    d = np.abs(pf[0].astype(np.int32) - pe[0].astype(np.int32))
    assert d.max() <= 1 and d.mean() <= 1e-4
    su = np.abs(pf[1][1:].view(np.int32).astype(np.int64) - pe[1][1:].view(np.int32).astype(np.int64))
    print(f"state scales: {np.mean(su > 1):.3f} of rows > 1 ulp apart, max {su.max()} ulp")
    assert su.max() <= 32 and np.mean(su > 1) <= 0.25
    # residual codes: off by one, except where the state code flipped at a tie
    # (then the residual absorbs that state LSB; both pairs reconstruct the
    # same target)
    ef = oracle.unpack_int4(pf[2]) if resid_fmt == oracle.RESID_INT4 else pf[2].astype(np.int32)
    ee = oracle.unpack_int4(pe[2]) if resid_fmt == oracle.RESID_INT4 else pe[2].astype(np.int32)
    ce = np.abs(ef - ee)
    assert np.all((ce <= 1) | (d > 0))
    assert (ce > 0).mean() <= (1e-4 if resid_fmt == oracle.RESID_INT4 else 2e-3)
    es_f = pf[3][1:, :, None, None]
    recon_f = pf[0][1:] * pf[1][1:, ..., None].astype(np.float64) + ef[1:] * es_f
    recon_e = pe[0][1:] * pe[1][1:, ..., None].astype(np.float64) + ee[1:] * pe[3][1:, :, None, None]
    assert rel(recon_f, recon_e) < 1e-3


def _ef_reference_decode(h0_vk, steps, H, scale, l2norm):
    """test_quantized_packed_decode.py:80-98 in float64: the exact recurrence
    composed with ErrorFeedback (fp32-like residual) and per-V-row quantization."""
    h = h0_vk.astype(np.float64)
    e = np.zeros_like(h)
    outs = []
    for mixed, a, b, A_log, dt in steps:
        B = mixed.shape[0]
        HV, V, K = h.shape[1:]
        al, be = oracle.gates(a, b, A_log[None], dt[None])
        q = mixed[:, :H * K].reshape(B, H, K).astype(np.float64)
        k = mixed[:, H * K:2 * H * K].reshape(B, H, K).astype(np.float64)
        v = mixed[:, 2 * H * K:].reshape(B, HV, V).astype(np.float64)
        if l2norm:
            q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6)
            k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
        q = np.repeat(q * scale, HV // H, axis=1)
        k = np.repeat(k, HV // H, axis=1)
        hh = h * al[..., None, None]
        dv = be[..., None] * (v - np.einsum("bhvk,bhk->bhv", hh, k))
        hh = hh + dv[..., None] * k[:, :, None, :]
        outs.append(np.einsum("bhvk,bhk->bhv", hh, q))
        target = hh + e
        s = np.maximum(np.abs(target).max(-1, keepdims=True), 1e-12) / 127
        h = np.clip(np.round(target / s), -127, 127) * s
        e = target - h
    return np.stack(outs), h


@pytest.mark.parametrize("resid_fmt,bound", [(oracle.RESID_INT8, 5e-2), (oracle.RESID_INT4, 8e-2)])
def test_decode_vs_ef_reference(resid_fmt, bound, B=1, H=8, HV=16, K=64, V=64, T=32):
    """test_quantized_packed_decode.py:108-150 and :310-354 bounds, on the oracle."""
    rng = np.random.default_rng(0)
    h0 = (rng.standard_normal((B, HV, V, K)) * 0.1).astype(F)
    c0, s0 = oracle.quantize_rows(h0)
    sc = np.concatenate([np.zeros((1, HV, V, K), np.int8), c0])
    ss = np.concatenate([np.zeros((1, HV, V), F), s0])
    rk = K // 2 if resid_fmt == oracle.RESID_INT4 else K
    rc = np.zeros((B + 1, HV, V, rk), np.int8)
    rs = np.zeros((B + 1, HV, V), F)
    steps = [tuple(x.numpy() for x in make_packed_inputs(B, H, HV, K, V, seed=100 + t)) for t in range(T)]
    idx = np.arange(1, B + 1, dtype=np.int32)
    outs = [oracle.packed_decode(*s_, K ** -0.5, sc, ss, rc, rs, idx, H, use_qk_l2norm=True,
                                 resid_fmt=resid_fmt) for s_ in steps]
    o_ref, h_ref = _ef_reference_decode(c0.astype(np.float64) * s0[..., None], steps, H, K ** -0.5, True)
    assert rel(np.stack(outs), o_ref) < bound
    assert rel(sc[1:] * ss[1:, ..., None].astype(np.float64), h_ref) < bound


def test_statequant_decode_vs_oracle_decode():
    """experiments/test_kernel.py:115-141: fused decode (fp32 residual) against
    the recurrence + ErrorFeedback + per-V-column quantization, rel < 5e-3."""
    T, B, HV, K, V = 64, 1, 32, 128, 128
    g = torch.Generator().manual_seed(0)
    q = torch.randn(T, B, HV, K, generator=g)
    k = torch.randn(T, B, HV, K, generator=g)
    k = k / k.norm(dim=-1, keepdim=True).clamp(min=1e-8)
    v = torch.randn(T, B, HV, V, generator=g)
    alpha = torch.full((T, B, HV), 0.995)
    beta = torch.rand(T, B, HV, generator=g).sigmoid()
    h0 = (torch.randn(B, HV, K, V, generator=g) * 0.1).numpy()
    codes, scale = oracle.quantize_cols(h0)
    e = np.zeros(h0.shape, F)
    os_ = []
    for t in range(T):
        o, codes, scale, e, _ = oracle.quant_step_kv(codes, scale, e, None, q[t].numpy(), k[t].numpy(),
                                                     v[t].numpy(), alpha[t].numpy(), beta[t].numpy())
        os_.append(o)
    # float64 oracle_decode
    def per_v(x):
        s = np.maximum(np.abs(x).max(axis=-2, keepdims=True), 1e-12) / 127
        return np.clip(np.round(x / s), -127, 127) * s
    h = per_v(h0.astype(np.float64))
    ef = np.zeros_like(h)
    o_ref = []
    for t in range(T):
        h, o = oracle.gdn_step_f64(h, q[t].numpy(), k[t].numpy(), v[t].numpy(), alpha[t].numpy(), beta[t].numpy())
        target = h + ef
        h = per_v(target)
        ef = target - h
        o_ref.append(o)
    assert rel(np.stack(os_), np.stack(o_ref)) < 5e-3
    assert rel(codes * scale[..., None, :].astype(np.float64), h) < 5e-3


def test_quantize_rows_cols_match_torch_round():
    """init_quantized_state (quantized_packed_decode.py:347-351) and
    per_v_channel_quantize (statequant/kernel.py:99-113)."""
    x = torch.randn(4, 8, 32, 16, generator=torch.Generator().manual_seed(2)) * 0.3
    x[0, 0, 0] = 0.0                                           # an all-zero row
    c, s = oracle.quantize_rows(x.numpy())
    s_t = x.abs().amax(dim=-1).clamp(min=1e-12) / 127
    np.testing.assert_array_equal(s, s_t.numpy())
    np.testing.assert_array_equal(c, torch.round(x / s_t[..., None]).clamp(-127, 127).to(torch.int8).numpy())
    c2, s2 = oracle.quantize_cols(x.numpy())
    s_t2 = x.abs().amax(dim=-2).clamp(min=1e-12) / 127
    np.testing.assert_array_equal(s2, s_t2.numpy())
    np.testing.assert_array_equal(c2, torch.round(x / s_t2[..., None, :]).clamp(-127, 127).to(torch.int8).numpy())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float64, torch.float32])
@pytest.mark.parametrize("qmax", [127, 31])
def test_quantize_rows_in_dtype_matches_torch_formula(dtype, qmax):
    """oracle.quantize_rows_in_dtype against the reference's expression
    (quantized_packed_decode.py:347-351: clamp(amax, 1e-12) / qmax, then
    torch.round(h0 / scale).clamp(-qmax, qmax)) evaluated by torch in h0's own
    dtype, bit for bit, on rows that exercise the dtype's corners: all-zero
    rows (fp16: 1e-12 rounds to 0, so 0 / 0), one dominant value, tiny
    magnitudes (fp16 subnormal scales, and fp16 scales that round to 0 under
    nonzero values, whose quotients are +-inf and clamp to +-qmax) and many
    rows whose bf16 quotient rounds past qmax (the clamp binds). For the
    16-bit dtypes the in-dtype codes differ from quantizing the same values
    in fp32, so the check has teeth."""
    g = torch.Generator().manual_seed(qmax)
    x = torch.randn(64, 4, 128, generator=g, dtype=torch.float64) * 0.3
    x[0, 0] = 0.0
    x[1, 1, 5] = 50.0
    x[2] *= 3e-3
    x[3, :, ::2] *= 1e-30
    x[4] *= 1e-6
    x = x.to(dtype)
    name = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float64: "float64",
            torch.float32: "float32"}[dtype]
    vals = x.numpy() if dtype == torch.float64 else x.float().numpy()
    c, s = oracle.quantize_rows_in_dtype(vals, name, float(qmax))
    s_t = x.abs().amax(dim=-1).clamp(min=1e-12) / qmax
    c_t = torch.round(x / s_t[..., None]).clamp(-qmax, qmax).to(torch.int8).numpy()
    np.testing.assert_array_equal(s, s_t.float().numpy())
    np.testing.assert_array_equal(c, c_t)
    if dtype in (torch.bfloat16, torch.float16):
        c32, s32 = oracle.quantize_rows(x.float().numpy(), float(qmax))
        assert not np.array_equal(c, c32) and not np.array_equal(s, s32)
    if dtype == torch.bfloat16 and qmax == 127:
        q = (x / s_t[..., None]).float()
        assert int((torch.round(q).abs() > qmax).sum()) > 0   # the clamp binds
    if dtype == torch.float16:
        assert float(s_t[0, 0]) == 0.0 and np.all(c[0, 0] == 0)
        assert np.any((s > 0) & (s < 6.1e-5))                 # subnormal fp16 scales
        assert np.any(np.abs(c[4][s[4] == 0]) == qmax)        # scale 0 under nonzero values


@pytest.mark.parametrize("K,V", [(64, 32), (256, 130)])
def test_fp32_step_vs_float64(K, V):
    rng = np.random.default_rng(3)
    h = (rng.standard_normal((2, 4, K, V)) * 0.1).astype(F)
    q, k = (rng.standard_normal((2, 4, K)).astype(F) for _ in range(2))
    v = rng.standard_normal((2, 4, V)).astype(F)
    al, be = F(rng.uniform(0.9, 1, (2, 4))), F(rng.uniform(0, 1, (2, 4)))
    h1, o1 = oracle.fp32_step_kv(h, q, k, v, al, be)
    h2, o2 = oracle.gdn_step_f64(h, q, k, v, al, be)
    assert np.abs(h1 - h2).max() < 1e-5 and np.abs(o1 - o2).max() < 1e-4


def test_float_state_oracle_matches_quantized_free_recurrence():
    """The fp32-state arm of the vLLM layout is the plain recurrence."""
    B, H, HV, K, V = 2, 2, 4, 32, 16
    rng = np.random.default_rng(5)
    state = (rng.standard_normal((3, HV, V, K)) * 0.1).astype(F)
    mixed, a, b, A_log, dt = (x.numpy() for x in make_packed_inputs(B, H, HV, K, V, seed=1))
    idx = np.array([2, 1], np.int32)
    ref_state = state.copy()
    out = oracle.packed_decode_float_state(mixed, a, b, A_log, dt, 0.5, state, idx, H)
    al, be = oracle.gates(a, b, A_log[None], dt[None])
    q = np.repeat(mixed[:, :H * K].reshape(B, H, K) * 0.5, HV // H, axis=1)
    k = np.repeat(mixed[:, H * K:2 * H * K].reshape(B, H, K), HV // H, axis=1)
    v = mixed[:, 2 * H * K:].reshape(B, HV, V)
    h_kv = ref_state[idx].transpose(0, 1, 3, 2)                  # [B, HV, K, V]
    h2, o2 = oracle.gdn_step_f64(h_kv, q, k, v, al, be)
    assert np.abs(out - o2).max() < 1e-4
    assert np.abs(state[idx] - h2.transpose(0, 1, 3, 2)).max() < 1e-5


def test_memory_claim():
    """vllm_integration/test_quantized_packed_decode.py:289-307, on the product's
    closed form (pure Python, no GPU)."""
    from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd
    HV, V, K = 32, 128, 128
    fp32 = qpd.state_bytes_per_slot(HV, V, K, quantized=False, base_dtype_size=4)
    bf16 = qpd.state_bytes_per_slot(HV, V, K, quantized=False, base_dtype_size=2)
    q8 = qpd.state_bytes_per_slot(HV, V, K, quantized=True, resid_fmt=qpd.RESID_INT8)
    q4 = qpd.state_bytes_per_slot(HV, V, K, quantized=True, resid_fmt=qpd.RESID_INT4)
    q4h = qpd.state_bytes_per_slot(HV, V, K, quantized=True, resid_fmt=qpd.RESID_INT4,
                                   per_head_resid_scale=True)
    assert (fp32, bf16, q8, q4) == (2097152, 1048576, 1081344, 819200)
    assert q4h == 819200 - HV * V * 4 + HV * 4
    assert 1.9 < fp32 / q8 < 2.05 and bf16 / q8 < 1.1
    assert 2.5 < fp32 / q4 < 2.75 and bf16 / q4 > 1.25
    assert math.isclose(bf16 / q4, 1.28, abs_tol=0.005)


def test_bf16_round_matches_torch():
    """The oracle's fp32 -> bf16 rounding (numpy oracle.bf16_round and the C
    bf16_round_f behind the bf16-state arm), which sets the expected values of
    every bf16-state and bf16-output test, against torch's own
    .to(torch.bfloat16): random values over the whole exponent range, exact
    ties with an odd and an even kept bit, values just below and above the
    point where rounding overflows to inf, subnormals, +-0, +-inf and NaN."""
    import torch
    rng = np.random.default_rng(12)
    rand = rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32)
    hi = rng.integers(0, 2 ** 16, 4000, dtype=np.uint64).astype(np.uint32) << 16
    ties = np.concatenate([hi | 0x8000, hi | 0x7FFF, hi | 0x8001])          # exact ties and their neighbours
    edges = np.array([0x7F7F7FFF, 0x7F7F8000, 0x7F7FFFFF, 0x7F7F0000,      # FLT_MAX region: stays / overflows
                      0xFF7F8000, 0x00000001, 0x00008000, 0x00018000,       # subnormals, ties among them
                      0x807FFFFF, 0x00000000, 0x80000000, 0x7F800000,       # +-0, +-inf
                      0xFF800000, 0x7FC00000, 0x7F800001, 0xFFC12345], np.uint32)
    x = np.concatenate([rand, ties, edges]).view(np.float32)
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).float().numpy()
    for got in (oracle.bf16_round(x), oracle.bf16_round_c(x)):
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # the ties really are ties, and both rounding directions occur
    t = (hi | 0x8000).view(np.float32)
    r = oracle.bf16_round(t).view(np.uint32)
    assert np.any(r == hi) and np.any(r == hi + 0x10000)
