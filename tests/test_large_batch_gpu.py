"""GPU runs at the configs' full sizes and at serving batches large enough
that a workgroup takes more than 64 items (its gates are staged in LDS by
more than one wave) or that the step is split over consecutive launches
(more items than a launch may hold):

* C3 at B=256 (HV=32, K=V=128, int4 residual with a per-head scale), two
  steps bit for bit against the oracle;
* B=1100 through the quantized decode (per-head int8 FAST on the
  persistent kernel, chosen through ck_set_decode_kernel: one launch, more
  than 64 items per workgroup; per-head int4 FAST and per-row int8 EXACT on
  the one-item kernel, the automatic choice: one launch of 35,200 / 70,400
  workgroups) and through the bf16-state arm (two launches): every item is
  checked bit for bit;
* small steps split into launches of a few items (a limit lowered through
  ck_set_max_items_per_launch) with bf16 activations and output,
  strided ids and out-of-place destinations;
* C5 at full size (24 layers x B=64 x 2048 tokens, int8 and int6 state,
  mixed alpha), its drift against the fp32 state arm bounded and the
  residual lowering the state error at every report.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
import oracle
from carrykernel_amd import _native
from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd
from tests._helpers import make_packed_inputs, make_pool

pytestmark = pytest.mark.gpu

H = HV = 32
K = V = 128


def _host(t):
    return t.detach().cpu().numpy().copy()


def _check_step(device, pool, ids, inputs, resid_fmt, per_head, mode, l2norm, tag):
    """One GPU step through the drop-in front end, compared bit for bit with
    the oracle on host copies of the same pool."""
    mixed, a, b, A_log, dt_bias = inputs
    B = mixed.shape[0]
    torch.cuda.synchronize()
    host = [_host(x) for x in pool]
    out = torch.empty(B, 1, HV, V, device=device)
    print(f"case {tag}", flush=True)
    qpd.quantized_gated_delta_rule_packed_decode(
        mixed, a, b, A_log, dt_bias, 1.0 if not l2norm else K ** -0.5, *pool, out, ids,
        use_qk_l2norm_in_kernel=l2norm, resid_fmt=resid_fmt,
        quant_mode="exact" if mode == oracle.MODE_EXACT else "fast")
    torch.cuda.synchronize()
    ref = oracle.packed_decode(*(_host(x) for x in inputs), 1.0 if not l2norm else K ** -0.5, *host, _host(ids), H,
                               use_qk_l2norm=l2norm, resid_fmt=resid_fmt, per_head=per_head, mode=mode)
    np.testing.assert_array_equal(_host(out[:, 0]), ref, err_msg=f"out ({tag})")
    for name, d, h in zip(("state_codes", "state_scale", "resid_codes", "resid_scale"), pool, host):
        np.testing.assert_array_equal(_host(d), h, err_msg=f"{name} ({tag})")


def test_c3_b256_bit_exact(device):
    """C3's largest batch: B=256 random slots of a 513-slot pool, state from
    64 fp32 warm-up steps, the configs' activation distributions (q, k
    normalised on the host, kernel flag off), two consecutive steps."""
    B, S = 256, 513
    state = bench.warm_state(S, device, seed=3)
    pool = list(qpd.init_quantized_state(S, HV, V, K, device, h0=state, resid_fmt=qpd.RESID_INT4,
                                         per_head_resid_scale=True))
    del state
    sets, A_log, dt_bias = bench.make_step_inputs(B, 2, device, seed=5)
    perm = torch.randperm(S - 1, generator=torch.Generator().manual_seed(3))[:B] + 1
    ids = perm.to(torch.int32).to(device)
    for t in range(2):
        mixed, a, b = sets[t]
        _check_step(device, pool, ids, (mixed, a, b, A_log, dt_bias), qpd.RESID_INT4, True, oracle.MODE_FAST,
                    False, f"C3 B=256 step {t}")


@pytest.mark.parametrize("resid_fmt,per_head,mode,decode_kernel", [
    (oracle.RESID_INT8, True, oracle.MODE_FAST, "persistent"),
    (oracle.RESID_INT4, True, oracle.MODE_FAST, "auto"),
    (oracle.RESID_INT8, False, oracle.MODE_EXACT, "auto")], indirect=["decode_kernel"])
def test_more_than_64_items_per_workgroup(device, resid_fmt, per_head, mode, decode_kernel):
    """B=1100 requests x 32 heads. The int8 per-head step runs the
    persistent kernel (chosen for the test; two workgroups per CU on 256 CUs
    with the int8 residual's LDS table), which gives every workgroup more
    than 64 items, so a second wave stages the gates of items 64..; the int4
    per-head and the per-row int8 steps run the automatic choice, the
    one-item kernel, over 35,200 and 70,400 workgroups in one launch (it has
    no gate table, so no per-launch item limit). GQA (H=16), the in-kernel L2
    norm, every item checked bit for bit."""
    B = 1100
    S = B + 1
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    # per-head: one 8-wave workgroup per head item, two per CU; per-row:
    # 64-row items, four 4-wave workgroups per CU
    items, per_cu = (B * HV, 2) if per_head else (B * HV * (V // 64), 4)
    assert items / (per_cu * cus) > 64, "batch too small for more than 64 items per workgroup on this device"
    Hq = 16
    pool = [torch.from_numpy(x).to(device) for x in make_pool(S, HV, V, K, resid_fmt, per_head, seed=8)]
    inputs = [x.to(device) for x in make_packed_inputs(B, Hq, HV, K, V, seed=8)]
    ids = (torch.randperm(S - 1, generator=torch.Generator().manual_seed(8)) + 1).to(torch.int32).to(device)
    mixed, a, b, A_log, dt_bias = inputs
    torch.cuda.synchronize()
    host = [_host(x) for x in pool]
    out = torch.empty(B, 1, HV, V, device=device)
    print(f"case B=1100 resid={resid_fmt} per_head={per_head} mode={mode} kernel={decode_kernel}", flush=True)
    qpd.quantized_gated_delta_rule_packed_decode(
        mixed, a, b, A_log, dt_bias, K ** -0.5, *pool, out, ids, use_qk_l2norm_in_kernel=True,
        resid_fmt=resid_fmt, quant_mode="exact" if mode == oracle.MODE_EXACT else "fast")
    torch.cuda.synchronize()
    ref = oracle.packed_decode(*(_host(x) for x in inputs), K ** -0.5, *host, _host(ids), Hq, use_qk_l2norm=True,
                               resid_fmt=resid_fmt, per_head=per_head, mode=mode)
    np.testing.assert_array_equal(_host(out[:, 0]), ref)
    for name, d, h in zip(("state_codes", "state_scale", "resid_codes", "resid_scale"), pool, host):
        np.testing.assert_array_equal(_host(d), h, err_msg=name)


def test_float_state_more_than_64_items_per_workgroup(device):
    """The bf16-state arm at B=1100 (two 64-row items per head, 70,400 items:
    two launches), every output and state row bit for bit."""
    B = 1100
    S = B + 1
    g = torch.Generator().manual_seed(9)
    state = (torch.randn(S, HV, V, K, generator=g) * 0.1).to(torch.bfloat16)
    ref_state = state.float().numpy().copy()
    dstate = state.to(device)
    del state
    mixed, a, b, A_log, dt_bias = make_packed_inputs(B, H, HV, K, V, seed=9)
    ids = torch.randperm(S - 1, generator=torch.Generator().manual_seed(9)).to(torch.int32) + 1
    out = torch.empty(B, 1, HV, V, device=device)
    print("case float-state bf16 B=1100", flush=True)
    bench.float_state_step(dstate, mixed.to(device), a.to(device), b.to(device), A_log.to(device),
                           dt_bias.to(device), K ** -0.5, out, ids.to(device), True)
    torch.cuda.synchronize()
    o_ref = oracle.packed_decode_float_state(mixed.numpy(), a.numpy(), b.numpy(), A_log.numpy(), dt_bias.numpy(),
                                             K ** -0.5, ref_state, ids.numpy(), H, bf16=True, use_qk_l2norm=True)
    np.testing.assert_array_equal(_host(out[:, 0]), o_ref)
    np.testing.assert_array_equal(dstate.float().cpu().numpy(), ref_state)


@pytest.mark.parametrize("bits,bound", [(8, 2e-2), (6, 8e-2)])
def test_c5_full_size_drift(device, bits, bound):
    """C5 at its full size: 24 layers x B=64 x 2048 tokens, heads 0-15 at
    alpha 0.995 and 16-31 at 0.9, fresh q/k/v per layer and token, int4
    residual with a per-head scale, int8 or int6 state, against the fp32
    state arm on the same inputs. Reports every 256 tokens: state, state plus
    residual and output errors stay bounded, and the carried residual lowers
    the state error at every report."""
    print(f"case C5 full size bits={bits}", flush=True)
    rows = bench.drift_c5(device, bits, log=lambda r: print(f"C5 int{bits}", r, flush=True))
    assert len(rows) == 8 and rows[-1]["token"] == 2048
    for r in rows:
        assert r["state_rel"] < bound and r["o_rel"] < bound
        assert r["state_plus_residual_rel"] < r["state_rel"]


@pytest.mark.parametrize("per_head,resid_fmt,cap", [(True, oracle.RESID_INT4, 40), (False, oracle.RESID_INT8, 150)])
def test_split_over_launches_small_cap(device, per_head, resid_fmt, cap):
    """ck_set_max_items_per_launch lowers what one launch holds, so a
    small step runs as several launches over slices of the requests (the
    per-request pointers advanced on the host): bf16 activations and output,
    strided slot ids, an out-of-place destination, a NULL slot, against the
    oracle bit for bit, then the same step unsplit for comparison."""
    B, Hq, HVl, Kl, Vl = 23, 4, 8, 64, 100
    S = 2 * B + 3
    rng = np.random.default_rng(cap)
    pool = make_pool(S, HVl, Vl, Kl, resid_fmt, per_head, seed=cap)
    perm = (rng.permutation(S - 1) + 1).astype(np.int32)
    src, dst = perm[:B].copy(), perm[B:2 * B].copy()
    src[5] = 0
    mixed, a, b, A_log, dt_bias = make_packed_inputs(B, Hq, HVl, Kl, Vl, seed=cap, dtype=torch.bfloat16)
    ref_pool = [x.copy() for x in pool]
    o_ref = oracle.packed_decode(mixed.float().numpy(), a.float().numpy(), b.float().numpy(), A_log.float().numpy(),
                                 dt_bias.float().numpy(), Kl ** -0.5, *ref_pool, src, Hq, use_qk_l2norm=True,
                                 resid_fmt=resid_fmt, per_head=per_head, dst_indices=dst)
    try:
        for split in (True, False):
            _run_split_case(device, split, cap, per_head, resid_fmt, pool, ref_pool, o_ref, src, dst, mixed, a, b,
                            A_log, dt_bias, B, Hq, HVl, Kl, Vl)
    finally:
        _native.set_max_items_per_launch(0)


def _run_split_case(device, split, cap, per_head, resid_fmt, pool, ref_pool, o_ref, src, dst, mixed, a, b, A_log,
                    dt_bias, B, Hq, HVl, Kl, Vl):
    """One run of test_split_over_launches_small_cap's step: split into
    launches of at most `cap` items, or unsplit."""
    _native.set_max_items_per_launch(cap if split else 0)
    dpool = [torch.from_numpy(x.copy()).to(device) for x in pool]
    ids2 = torch.zeros(2 * B, dtype=torch.int32)
    ids2[::2] = torch.from_numpy(src)
    ids = ids2.to(device)[::2]
    out = torch.empty(B, 1, HVl, Vl, dtype=torch.bfloat16, device=device)
    print(f"case split={split} per_head={per_head} cap={cap}", flush=True)
    qpd.quantized_gated_delta_rule_packed_decode(
        mixed.to(device), a.to(device), b.to(device), A_log.to(device), dt_bias.to(device), Kl ** -0.5, *dpool,
        out, ids, use_qk_l2norm_in_kernel=True, resid_fmt=resid_fmt, dst_state_indices=torch.from_numpy(dst).to(device))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out[:, 0].float().cpu().numpy(), oracle.bf16_round(o_ref), err_msg=f"out split={split}")
    for name, d, h in zip(("state_codes", "state_scale", "resid_codes", "resid_scale"), dpool, ref_pool):
        np.testing.assert_array_equal(_host(d), h, err_msg=f"{name} split={split}")


def test_float_state_split_over_launches_small_cap(device):
    """The bf16-state arm split into launches of at most 30 items (B=19,
    HV=8, two 64-row items per head), bit for bit against the oracle."""
    B, Hq, HVl, Kl, Vl = 19, 8, 8, 128, 128
    S = B + 2
    g = torch.Generator().manual_seed(19)
    state = (torch.randn(S, HVl, Vl, Kl, generator=g) * 0.1).to(torch.bfloat16)
    ref_state = state.float().numpy().copy()
    dstate = state.to(device)
    mixed, a, b, A_log, dt_bias = make_packed_inputs(B, Hq, HVl, Kl, Vl, seed=19)
    ids = torch.randperm(S - 1, generator=g)[:B].to(torch.int32) + 1
    out = torch.empty(B, 1, HVl, Vl, device=device)
    _native.set_max_items_per_launch(30)
    print("case float-state split cap=30", flush=True)
    try:
        bench.float_state_step(dstate, mixed.to(device), a.to(device), b.to(device), A_log.to(device),
                               dt_bias.to(device), Kl ** -0.5, out, ids.to(device), True)
        torch.cuda.synchronize()
    finally:
        _native.set_max_items_per_launch(0)
    o_ref = oracle.packed_decode_float_state(mixed.numpy(), a.numpy(), b.numpy(), A_log.numpy(), dt_bias.numpy(),
                                             Kl ** -0.5, ref_state, ids.numpy(), Hq, bf16=True, use_qk_l2norm=True)
    np.testing.assert_array_equal(_host(out[:, 0]), o_ref)
    np.testing.assert_array_equal(dstate.float().cpu().numpy(), ref_state)
