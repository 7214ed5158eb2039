"""Randomised GPU parity of the fused decode: many small configurations drawn
from fixed seeds, each run for two steps on the GPU (through the C ABI) and in
the oracle from the same pool, compared bit for bit (the outputs and all four
pool tensors). A draw picks K, V, the GQA ratio, the batch, the residual format
and scale granularity, the quant mode, the activation / gate / output dtypes,
the L2-norm flag, the state bits, NULL and out-of-range slot ids and (FAST mode)
out-of-place destinations; the fixed cases in test_packed_decode_gpu.py cover
each axis alone."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd
from tests._helpers import make_packed_inputs, make_pool, to_dev

pytestmark = pytest.mark.gpu

DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _draw(seed, any_k=False, k_max=256):
    """A random decode configuration. any_k: K anywhere in 1..k_max (even with
    the int4 residual; 257..k_max when k_max > 256), the masked kernel's
    shapes."""
    rng = np.random.default_rng(seed)
    if any_k:
        resid_fmt = int(rng.choice([qpd.RESID_INT8, qpd.RESID_INT4]))
        K = int(rng.integers(1 if k_max <= 256 else 257, k_max + 1))
        if resid_fmt == qpd.RESID_INT4 and K % 2:
            K += 1 if K < k_max else -1
    else:
        K = int(rng.choice([16, 32, 64, 128, 256]))
    KP = 16
    while KP < K:
        KP *= 2
    per_head = bool(rng.integers(2))
    rows_per_inst = 64 // (KP // 16)
    # the per-head shapes hold the head in one workgroup: 32 rows per lane-row
    # group up to KP = 256 (8 waves x 4 rows), 64 from 512 (16 waves x 4 rows)
    v_max = rows_per_inst * (64 if KP >= 512 else 32) if per_head else 300
    V = int(rng.integers(1, min(v_max, 300) + 1))
    H = int(rng.choice([1, 2, 4]))
    HV = H * int(rng.choice([1, 2, 3]))
    B = int(rng.integers(1, 25))
    if not any_k:
        resid_fmt = int(rng.choice([qpd.RESID_INT8, qpd.RESID_INT4]))
    mode = "exact" if rng.random() < 0.3 else "fast"
    act = DTYPES[int(rng.integers(3))]
    out_dt = DTYPES[int(rng.integers(3))]
    return dict(K=K, V=V, H=H, HV=HV, B=B, resid_fmt=resid_fmt, per_head=per_head, mode=mode, act=act,
                out_dt=out_dt, l2norm=bool(rng.integers(2)), bits=int(rng.integers(2, 9)),
                dst=mode == "fast" and rng.random() < 0.35, rng=rng)


def _expected_out(o_ref, out_dt):
    if out_dt == torch.bfloat16:
        return oracle.bf16_round(o_ref)
    if out_dt == torch.float16:
        return o_ref.astype(np.float16).astype(np.float32)
    return o_ref


@pytest.mark.parametrize("seed", range(48))
def test_random_configuration_bit_exact(device, seed):
    _run_decode(device, seed, _draw(1000 + seed))


@pytest.mark.parametrize("seed", range(24))
def test_random_any_k_configuration_bit_exact(device, seed):
    """K drawn from 1..256: the masked kernel (and, when the draw is a power
    of two from 16, the bandwidth kernel)."""
    _run_decode(device, seed, _draw(7000 + seed, any_k=True))


@pytest.mark.parametrize("seed", range(8))
def test_random_large_k_configuration_bit_exact(device, seed):
    """K drawn from 257..1024: rows padded to 512 or 1024 lanes."""
    _run_decode(device, seed, _draw(7500 + seed, any_k=True, k_max=1024))


def _run_decode(device, seed, c):
    rng = c.pop("rng")
    B, H, HV, K, V = c["B"], c["H"], c["HV"], c["K"], c["V"]
    S = 2 * B + 3 if c["dst"] else B + 3
    pool = make_pool(S, HV, V, K, c["resid_fmt"], c["per_head"], seed=seed, bits=c["bits"])
    dpool = to_dev(pool, device)
    perm = (rng.permutation(S - 1) + 1).astype(np.int32)
    src = perm[:B].copy()
    nulls = rng.random(B) < 0.15                      # NULL requests: zeros out, nothing touched
    src[nulls] = 0
    if B > 2 and rng.random() < 0.3:                  # one out-of-range id: NaN out, nothing touched
        src[int(rng.integers(B))] = S + int(rng.integers(3))
    dst = perm[B:2 * B].copy() if c["dst"] else None
    print(f"case seed={seed} {({k: (str(v) if isinstance(v, torch.dtype) else v) for k, v in c.items()})}",
          flush=True)
    for t in range(2):
        mixed, a, b, A_log, dt_bias = make_packed_inputs(B, H, HV, K, V, seed=7 * seed + t, dtype=c["act"])
        # gates in the activation dtype or in fp32, independently
        if rng.random() < 0.5:
            a, b = a.float(), b.float()
        out = torch.empty(B, 1, HV, V, dtype=c["out_dt"], device=device)
        qpd.quantized_gated_delta_rule_packed_decode(
            mixed.to(device), a.to(device), b.to(device), A_log.to(device), dt_bias.to(device), K ** -0.5,
            *dpool, out, torch.from_numpy(src).to(device), use_qk_l2norm_in_kernel=c["l2norm"],
            resid_fmt=c["resid_fmt"], state_bits=c["bits"], quant_mode=c["mode"],
            dst_state_indices=None if dst is None else torch.from_numpy(dst).to(device))
        torch.cuda.synchronize()
        o_ref = oracle.packed_decode(
            mixed.float().numpy(), a.float().numpy(), b.float().numpy(), A_log.float().numpy(),
            dt_bias.float().numpy(), K ** -0.5, *pool, src, H, use_qk_l2norm=c["l2norm"],
            resid_fmt=c["resid_fmt"], per_head=c["per_head"], state_bits=c["bits"],
            mode=oracle.MODE_EXACT if c["mode"] == "exact" else oracle.MODE_FAST, dst_indices=dst)
        np.testing.assert_array_equal(out[:, 0].float().cpu().numpy(), _expected_out(o_ref, c["out_dt"]),
                                      err_msg=f"out differs at step {t}")
        for name, d, h in zip(("state_codes", "state_scale", "resid_codes", "resid_scale"), dpool, pool):
            np.testing.assert_array_equal(d.cpu().numpy(), h, err_msg=f"{name} differs at step {t}")
        if dst is not None:
            src, dst = dst, src                       # read back what was written (NULL / bad ids stay put)
            src = np.where((src > 0) & (src < S), src, 0).astype(np.int32)
            dst = np.where((dst > 0) & (dst < S), dst, 0).astype(np.int32)


@pytest.mark.parametrize("seed", range(24))
def test_random_statequant_step_bit_exact(device, seed):
    """The statequant-layout step (ck_gdn_quant_step through gdn_quant_step_fused)
    on random shapes, residual formats, quant modes and state bits; from seed
    16 on, K anywhere in 1..256 (rows zero-padded to a power of two)."""
    from carrykernel_amd.statequant import kernel as sq
    from tests.test_statequant_gpu import _random_state, _storage, make_inputs

    rng = np.random.default_rng(5000 + seed)
    K = int(rng.choice([16, 32, 64, 128, 256]))
    if seed >= 16:
        K = int(rng.integers(1, 257))
    # half the draws a multiple of 4 (vector column groups), half any V
    V = 4 * int(rng.integers(1, 50)) if rng.random() < 0.5 else int(rng.integers(1, 200))
    B, HV = int(rng.integers(1, 4)), int(rng.integers(1, 9))
    res_fmt = int(rng.integers(4))
    mode = "exact" if rng.random() < 0.4 else "fast"
    bits = int(rng.integers(2, 9))
    print(f"case seed={seed} K={K} V={V} B={B} HV={HV} res={res_fmt} mode={mode} bits={bits}", flush=True)
    h_int8, scale, e, es = _random_state(B, HV, K, V, res_fmt, seed=seed, bits=bits)
    _, q, k, v, alpha, beta = make_inputs(1, B, HV, K, V, seed=100 + seed)
    got = sq.gdn_quant_step_fused(h_int8.to(device), scale.to(device), e.to(device),
                                  None if es is None else es.to(device), q[0].to(device), k[0].to(device),
                                  v[0].to(device), alpha[0].to(device), beta[0].to(device), bits=bits,
                                  res_fmt=res_fmt, quant_mode=mode)
    torch.cuda.synchronize()
    ref = oracle.quant_step_kv(h_int8.numpy(), scale.numpy(), _storage(e, res_fmt),
                               None if es is None else es.numpy(), q[0].numpy(), k[0].numpy(), v[0].numpy(),
                               alpha[0].numpy(), beta[0].numpy(), bits=bits, res_fmt=res_fmt,
                               mode=oracle.MODE_EXACT if mode == "exact" else oracle.MODE_FAST)
    for name, g_, r_ in zip(("o", "h_int8", "scale", "e", "e_scale"), got, ref):
        if r_ is None:
            assert g_ is None
            continue
        g_np = _storage(g_, res_fmt) if name == "e" else g_.cpu().numpy()
        np.testing.assert_array_equal(g_np, r_, err_msg=f"{name} differs")


@pytest.mark.parametrize("seed", range(16))
def test_random_float_state_arm_bit_exact(device, seed):
    """The unquantized-state comparison arm (ck_gdn_packed_decode_float_state)
    on random shapes, fp32 or bf16 state, fp32 or bf16 activations, the L2-norm
    flag and NULL ids, two steps against the oracle."""
    from carrykernel_amd import _native

    rng = np.random.default_rng(9000 + seed)
    K = int(rng.choice([16, 32, 64, 128, 256]))
    V = int(rng.integers(1, 200))
    H = int(rng.choice([1, 2, 4]))
    HV = H * int(rng.choice([1, 2]))
    B = int(rng.integers(1, 40))
    sdt = torch.bfloat16 if rng.random() < 0.5 else torch.float32
    act = torch.bfloat16 if rng.random() < 0.5 else torch.float32
    l2 = bool(rng.integers(2))
    S = B + 2
    print(f"case seed={seed} K={K} V={V} H={H} HV={HV} B={B} state={sdt} act={act} l2={l2}", flush=True)
    state = (torch.from_numpy(rng.standard_normal((S, HV, V, K)).astype(np.float32)) * 0.1).to(sdt)
    ref_state = state.float().numpy().copy()
    idx = (rng.permutation(S - 1)[:B] + 1).astype(np.int32)
    idx[rng.random(B) < 0.15] = 0
    dstate = state.to(device)
    L = _native.lib()
    for t in range(2):
        mixed, a, b, A_log, dt_bias = make_packed_inputs(B, H, HV, K, V, seed=31 * seed + t, dtype=act)
        code = _native.dtype_code(mixed, "mixed")
        dm, da, db, dA, dd = (x.to(device) for x in (mixed, a, b, A_log, dt_bias))
        out = torch.empty(B, 1, HV, V, device=device)
        didx = torch.from_numpy(idx).to(device)
        rc = L.ck_gdn_packed_decode_float_state(
            dm.data_ptr(), code, dm.stride(0), da.data_ptr(), code, da.stride(0), db.data_ptr(), code, db.stride(0),
            dA.data_ptr(), code, dd.data_ptr(), code, K ** -0.5, dstate.data_ptr(), 0 if sdt == torch.float32 else 1,
            dstate.stride(0), out.data_ptr(), 0, didx.data_ptr(), 1, S, B, H, HV, K, V, int(l2),
            _native.stream_handle(device))
        _native.check(rc, "float_state")
        torch.cuda.synchronize()
        o_ref = oracle.packed_decode_float_state(mixed.float().numpy(), a.float().numpy(), b.float().numpy(),
                                                 A_log.float().numpy(), dt_bias.float().numpy(), K ** -0.5,
                                                 ref_state, idx, H, bf16=sdt == torch.bfloat16, use_qk_l2norm=l2)
        np.testing.assert_array_equal(out[:, 0].cpu().numpy(), o_ref, err_msg=f"out differs at step {t}")
        np.testing.assert_array_equal(dstate.float().cpu().numpy(), ref_state, err_msg=f"state differs at step {t}")


@pytest.mark.parametrize("seed", range(16))
def test_random_slot_copy_and_reset(device, seed):
    """ck_pool_copy_slots / ck_pool_reset_slots on random pool shapes, residual
    formats and scale granularities, within one pool and between two, with
    NULL and out-of-range ids (skipped pairs) and, for a third of the draws,
    slots with padding between them (the 4-byte path); checked byte for byte
    against the same copies on the host."""
    rng = np.random.default_rng(12000 + seed)
    K = int(rng.choice([16, 32, 64, 128, 256]))
    HV, V = int(rng.integers(1, 9)), int(rng.integers(1, 80))
    resid_fmt = int(rng.choice([qpd.RESID_INT8, qpd.RESID_INT4]))
    per_head = bool(rng.integers(2))
    S, S2 = int(rng.integers(4, 20)), int(rng.integers(3, 12))
    padded = rng.random() < 0.33
    print(f"case seed={seed} K={K} HV={HV} V={V} resid={resid_fmt} per_head={per_head} S={S} S2={S2} padded={padded}",
          flush=True)

    def dev_pool(h):
        if not padded:
            return to_dev(h, device)
        out = []
        for x in h:
            n = x[0].size
            back = torch.zeros((x.shape[0], n + 4), dtype=torch.from_numpy(x[:1]).dtype, device=device)
            v = back[:, :n].view(x.shape)
            v.copy_(torch.from_numpy(x).to(device))
            out.append(v)
        return out

    a_h = make_pool(S, HV, V, K, resid_fmt, per_head, seed=seed)
    b_h = make_pool(S2, HV, V, K, resid_fmt, per_head, seed=seed + 100)
    a_d, b_d = dev_pool(a_h), dev_pool(b_h)
    n = int(rng.integers(1, 6))
    src = rng.integers(-1, S + 2, size=n).astype(np.int32)          # some ids out of range or NULL
    dst = rng.choice(np.arange(1, S2), size=min(n, S2 - 1), replace=False).astype(np.int32)
    src = src[:len(dst)]
    qpd.copy_quantized_state(a_d, torch.from_numpy(src).to(device), b_d, torch.from_numpy(dst).to(device))
    for s_, d_ in zip(src, dst):
        if 0 < s_ < S:
            for x, y in zip(a_h, b_h):
                y[d_] = x[s_]
    # within one pool: disjoint source and destination sets
    perm = rng.permutation(S - 1) + 1
    m = int(rng.integers(1, (S - 1) // 2 + 1))
    s2, d2 = perm[:m].astype(np.int32), perm[m:2 * m].astype(np.int32)
    qpd.copy_quantized_state(a_d, torch.from_numpy(s2).to(device), a_d, torch.from_numpy(d2).to(device))
    for s_, d_ in zip(s2, d2):
        for x in a_h:
            x[d_] = x[s_]
    r = rng.integers(0, S + 2, size=3).astype(np.int32)
    qpd.reset_quantized_state(a_d, torch.from_numpy(r).to(device))
    for i in r:
        if 0 < i < S:
            for x in a_h:
                x[i] = 0
    torch.cuda.synchronize()
    for pool_d, pool_h, tag in ((a_d, a_h, "pool a"), (b_d, b_h, "pool b")):
        for name, d, h in zip(("state_codes", "state_scale", "resid_codes", "resid_scale"), pool_d, pool_h):
            np.testing.assert_array_equal(d.cpu().numpy(), h, err_msg=f"{tag} {name}")
