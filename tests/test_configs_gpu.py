"""The configs' long runs on the GPU, through the product entry points:
C1 (2000-step statequant trajectory), C2 (B=8, int8 residual per head, 1000
steps), C4 (1024-slot pool, B=128 random gathers, 512 steps) and a shortened
C5 (multi-layer drift against the fp32 state arm). Each checks chosen steps
bit for bit against the oracle, restarted from the GPU's own state, and bounds
the drift against the unquantized recurrence."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import bench
import oracle
from carrykernel_amd.statequant import kernel as sq
from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd
from tests._helpers import rel
from tests.test_configs_cpu import c1_inputs

pytestmark = pytest.mark.gpu

H = HV = 32
K = V = 128


def test_c1_trajectory_bit_exact(device):
    """gdn_quant_decode_fused over C1's 2000 steps (fp32 residual) equals the
    oracle's trajectory bit for bit: every output and the final state."""
    q, k, v, h0, alpha, beta = c1_inputs()
    T = q.shape[0]
    al = np.broadcast_to(alpha, (T, 1, 1)).copy()
    be = np.broadcast_to(beta, (T, 1, 1)).copy()
    print("case C1 T=2000 res=fp32", flush=True)
    o, h_int8, scale, e, _ = sq.gdn_quant_decode_fused(
        *(torch.from_numpy(x).to(device) for x in (h0, q, k, v, al, be)), T, bits=8, res_fmt=sq.RES_FP32)
    torch.cuda.synchronize()
    codes, sc = oracle.quantize_cols(h0)
    ee = np.zeros_like(h0)
    outs = []
    for t in range(T):
        ot, codes, sc, ee, _ = oracle.quant_step_kv(codes, sc, ee, None, q[t], k[t], v[t], alpha, beta)
        outs.append(ot)
    np.testing.assert_array_equal(o.cpu().numpy(), np.stack(outs))
    np.testing.assert_array_equal(h_int8.cpu().numpy(), codes)
    np.testing.assert_array_equal(scale.cpu().numpy(), sc)
    np.testing.assert_array_equal(e.cpu().numpy(), ee)


def _config_inputs(B, gen, device, alpha=None):
    """One step of the configs' activations on the GPU: q, k, v ~ N(0,1) (q, k
    L2-normalised in the kernel), alpha = exp(g) with g ~ U(log 0.9, log 0.995)
    per (request, head) unless given per head, beta = sigmoid(U(-2, 2))."""
    mixed = torch.randn(B, 2 * H * K + HV * V, generator=gen, device=device)
    if alpha is None:
        lg = torch.rand(B, HV, generator=gen, device=device) * (math.log(0.995) - math.log(0.9)) + math.log(0.9)
    else:
        lg = torch.log(alpha.to(device)).expand(B, HV)
    a = torch.log(torch.expm1(-lg)).contiguous()
    b = (torch.rand(B, HV, generator=gen, device=device) * 4.0 - 2.0).contiguous()
    return mixed, a, b


def _host(t):
    return t.detach().cpu().numpy().copy()


def _oracle_step_on(pool_host, idx_host, inputs, resid_fmt, per_head, l2norm=True, bits=8):
    mixed, a, b, A_log, dt_bias = (_host(x) for x in inputs)
    out = oracle.packed_decode(mixed, a, b, A_log, dt_bias, 1.0, *pool_host, idx_host, H,
                               use_qk_l2norm=l2norm, resid_fmt=resid_fmt, per_head=per_head, state_bits=bits)
    return out


def test_c2_thousand_steps(device):
    """C2: B=8, int8 state + int8 residual with a per-head scale, state from
    64 fp32 warm-up steps, 1000 steps. Steps 0 and 999 are checked bit for bit
    against the oracle; the trajectory's drift against the fp32 state arm
    (same inputs) is bounded."""
    B, T = 8, 1000
    S = B + 1
    fmt = qpd.RESID_INT8
    state = bench.warm_state(S, device, seed=2)
    pool = list(qpd.init_quantized_state(S, HV, V, K, device, h0=state, resid_fmt=fmt,
                                         per_head_resid_scale=True))
    ref = state.clone()
    idx = torch.arange(1, S, dtype=torch.int32, device=device)
    A_log = torch.zeros(HV, device=device)
    dt_bias = torch.zeros(HV, device=device)
    out = torch.empty(B, 1, HV, V, device=device)
    out_r = torch.empty(B, 1, HV, V, device=device)
    gen = torch.Generator(device=device).manual_seed(2)
    o_err = []
    for t in range(T):
        mixed, a, b = _config_inputs(B, gen, device)
        check = t in (0, T - 1)
        if check:
            torch.cuda.synchronize()
            before = [_host(x) for x in pool]
            print(f"case C2 step {t}", flush=True)
        qpd.quantized_gated_delta_rule_packed_decode(mixed, a, b, A_log, dt_bias, 1.0, *pool, out, idx,
                                                     use_qk_l2norm_in_kernel=True, resid_fmt=fmt)
        bench.float_state_step(ref, mixed, a, b, A_log, dt_bias, 1.0, out_r, idx, True)
        if check:
            torch.cuda.synchronize()
            o_ref = _oracle_step_on(before, _host(idx), (mixed, a, b, A_log, dt_bias), fmt, True)
            np.testing.assert_array_equal(_host(out[:, 0]), o_ref, err_msg=f"out at step {t}")
            for name, d, h in zip(("state_codes", "state_scale", "resid_codes", "resid_scale"), pool, before):
                np.testing.assert_array_equal(_host(d), h, err_msg=f"{name} at step {t}")
        if t % 100 == 99:
            o_err.append(rel(_host(out), _host(out_r)))
    h_err = rel(_host(bench.dequant_pool(pool, fmt, True)[1:]), _host(ref[1:]))
    print(f"C2 after {T} steps: state rel err {h_err:.2e}; o rel err every 100 steps {['%.1e' % x for x in o_err]}")
    assert h_err < 2e-2
    assert max(o_err) < 2e-2


def test_c4_pool_gather_scatter(device):
    """C4: 1024-slot pool (slot 0 the NULL block) of int8 state + int4
    residual with per-V-row scales; each step gathers 128 random distinct ids
    from 1..1023 and scatters the update back, 512 steps. At steps 0, 255 and
    511 the gathered slots match the oracle bit for bit and every other slot
    is untouched."""
    S, B, T = 1024, 128, 512
    fmt = qpd.RESID_INT4
    g = torch.Generator().manual_seed(4)
    h0 = torch.randn(S, HV, V, K, generator=g).mul_(0.1).to(device)
    pool = list(qpd.init_quantized_state(S, HV, V, K, device, h0=h0, resid_fmt=fmt))
    del h0
    A_log = torch.zeros(HV, device=device)
    dt_bias = torch.zeros(HV, device=device)
    out = torch.empty(B, 1, HV, V, device=device)
    gen = torch.Generator(device=device).manual_seed(4)
    for t in range(T):
        ids = (torch.randperm(S - 1, generator=g)[:B] + 1).to(torch.int32)
        idx = ids.to(device)
        mixed, a, b = _config_inputs(B, gen, device)
        check = t in (0, T // 2 - 1, T - 1)
        if check:
            torch.cuda.synchronize()
            print(f"case C4 step {t}", flush=True)
            full_before = [x.clone() for x in pool]
            li = ids.long()
            compact = [np.concatenate([np.zeros_like(_host(x[:1])), _host(x[li.to(device)])]) for x in pool]
        qpd.quantized_gated_delta_rule_packed_decode(mixed, a, b, A_log, dt_bias, 1.0, *pool, out, idx,
                                                     use_qk_l2norm_in_kernel=True, resid_fmt=fmt)
        if check:
            torch.cuda.synchronize()
            cidx = np.arange(1, B + 1, dtype=np.int32)
            o_ref = _oracle_step_on(compact, cidx, (mixed, a, b, A_log, dt_bias), fmt, False)
            np.testing.assert_array_equal(_host(out[:, 0]), o_ref, err_msg=f"out at step {t}")
            touched = torch.zeros(S, dtype=torch.bool, device=device)
            touched[li.to(device)] = True
            for name, d, before, h in zip(("state_codes", "state_scale", "resid_codes", "resid_scale"),
                                          pool, full_before, compact):
                np.testing.assert_array_equal(_host(d[li.to(device)]), h[1:], err_msg=f"{name} at step {t}")
                assert torch.equal(d[~touched], before[~touched]), f"{name}: untouched slots changed at step {t}"
            del full_before


@pytest.mark.parametrize("bits,bound", [(8, 2e-2), (6, 8e-2)])
def test_c5_drift_shortened(device, bits, bound):
    """C5 at 4 layers x B=16 x 256 tokens (the full 24 x 64 x 2048 run is
    bench.py --drift): drift of the dequantized state and outputs against the
    fp32 state arm stays bounded, and the residual reduces the state error."""
    print(f"case C5 bits={bits}", flush=True)
    rows = bench.drift_c5(device, bits, tokens=256, layers=4, B=16, every=64)
    print(f"C5 int{bits}: {rows}")
    for r in rows:
        assert r["state_rel"] < bound and r["o_rel"] < bound
        assert r["state_plus_residual_rel"] < r["state_rel"]
