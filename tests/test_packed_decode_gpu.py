"""GPU parity of the vLLM-layout fused decode (ck_gdn_packed_decode) against
the CPU oracle, following vllm_integration/test_quantized_packed_decode.py."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd
from tests._helpers import make_packed_inputs, make_pool, rel, to_dev

pytestmark = pytest.mark.gpu

MODES = {"fast": oracle.MODE_FAST, "exact": oracle.MODE_EXACT}


def _normalize_qk(mixed, B, H, K):
    """q and k of a packed row L2-normalised on the host (config C1-C5 inputs)."""
    x = mixed.clone()
    qk = x[:, :2 * H * K].view(B, 2 * H, K)
    x[:, :2 * H * K] = (qk / qk.norm(dim=-1, keepdim=True)).reshape(B, -1)
    return x


def _run_both(device, B, H, HV, K, V, resid_fmt, per_head, mode, l2norm, T=1, seed=0,
              act_dtype=torch.float32, out_dtype=torch.float32, bits=8, scale=None, normalize_qk=False,
              null_tail=0):
    """Run T steps on the GPU and in the oracle from the same pool; assert
    bit-exact agreement of every output after every step. The last
    `null_tail` requests read the NULL block (a batch padded to a captured
    size)."""
    S = B + 3
    scale = K ** -0.5 if scale is None else scale
    pool = make_pool(S, HV, V, K, resid_fmt, per_head, seed=seed, bits=bits)
    dpool = to_dev(pool, device)
    rng = np.random.default_rng(seed + 1)
    indices = (rng.permutation(S - 1)[:B] + 1).astype(np.int32)
    if null_tail:
        indices[B - null_tail:] = qpd.NULL_BLOCK_ID
    didx = torch.from_numpy(indices).to(device)
    for t in range(T):
        mixed, a, b, A_log, dt_bias = make_packed_inputs(B, H, HV, K, V, seed=1000 * seed + t, dtype=act_dtype)
        if normalize_qk:
            mixed = _normalize_qk(mixed.float(), B, H, K).to(act_dtype)
        out = torch.empty(B, 1, HV, V, dtype=out_dtype, device=device)
        print(f"case B={B} H={H} HV={HV} K={K} V={V} resid={resid_fmt} per_head={per_head} "
              f"mode={mode} l2={l2norm} t={t}", flush=True)
        qpd.quantized_gated_delta_rule_packed_decode(
            mixed.to(device), a.to(device), b.to(device), A_log.to(device), dt_bias.to(device), scale,
            *dpool, out, didx, use_qk_l2norm_in_kernel=l2norm, resid_fmt=resid_fmt,
            state_bits=bits, quant_mode=mode)
        torch.cuda.synchronize()
        o_ref = oracle.packed_decode(
            mixed.float().numpy(), a.float().numpy(), b.float().numpy(), A_log.float().numpy(),
            dt_bias.float().numpy(), scale, *pool, indices, H, use_qk_l2norm=l2norm,
            resid_fmt=resid_fmt, per_head=per_head, state_bits=bits, mode=MODES[mode])
        got = out[:, 0].float().cpu().numpy()
        if out_dtype == torch.bfloat16:
            o_ref = oracle.bf16_round(o_ref)
        elif out_dtype == torch.float16:
            o_ref = o_ref.astype(np.float16).astype(np.float32)
        np.testing.assert_array_equal(got, o_ref, err_msg=f"out differs at step {t}")
        names = ("state_codes", "state_scale", "resid_codes", "resid_scale")
        for name, d, h in zip(names, dpool, pool):
            np.testing.assert_array_equal(d.cpu().numpy(), h, err_msg=f"{name} differs at step {t}")


@pytest.mark.parametrize("resid_fmt", [qpd.RESID_INT8, qpd.RESID_INT4])
@pytest.mark.parametrize("per_head", [False, True])
@pytest.mark.parametrize("mode", ["fast", "exact"])
def test_bit_exact_vs_oracle_k128(device, resid_fmt, per_head, mode):
    _run_both(device, B=4, H=32, HV=32, K=128, V=128, resid_fmt=resid_fmt, per_head=per_head,
              mode=mode, l2norm=False, T=3)


@pytest.mark.parametrize("B", [1, 8])
@pytest.mark.parametrize("mode", ["fast", "exact"])
def test_c3_small_batches_bit_exact(device, B, mode):
    """Config C3 at its small batches, on the config's shape: H = HV = 32,
    K = V = 128, packed int4 residual with a per-head scale, q and k
    normalised on the host (flag off, scale 1). B=1 runs one item per
    workgroup on 32 CUs, B=8 256 items with no prefetch past the first."""
    _run_both(device, B=B, H=32, HV=32, K=128, V=128, resid_fmt=qpd.RESID_INT4, per_head=True,
              mode=mode, l2norm=False, T=3, seed=B, scale=1.0, normalize_qk=True)


@pytest.mark.parametrize("resid_fmt", [qpd.RESID_INT8, qpd.RESID_INT4])
@pytest.mark.parametrize("per_head", [False, True])
@pytest.mark.parametrize("B", [64, 37])
@pytest.mark.parametrize("decode_kernel", ["auto", "persistent"], indirect=True)
def test_bit_exact_full_occupancy(device, resid_fmt, per_head, B, decode_kernel):
    """Batches with more items than resident workgroups at K=128. The
    automatic choice runs the one-item kernel, dispatcher-balanced; the
    persistent kernel, chosen for the test, shares items unevenly between the
    workgroups of a CU (B=37: CU groups with different item counts) and
    prefetches each next item into its second register set."""
    _run_both(device, B=B, H=32, HV=32, K=128, V=128, resid_fmt=resid_fmt, per_head=per_head,
              mode="fast", l2norm=False, T=2)


@pytest.mark.parametrize("per_head,mode,act", [(True, "exact", torch.bfloat16), (True, "fast", torch.float16),
                                               (False, "exact", torch.bfloat16)])
def test_one_item_kernel_at_full_occupancy(device, per_head, mode, act):
    """More items than resident workgroups on the one-item kernel (int4 at
    K=128, per head and per row): 16-bit activations and outputs, the
    in-kernel L2 norm and both modes, B=64 at HV=32, GQA (H=8)."""
    _run_both(device, B=64, H=8, HV=32, K=128, V=128, resid_fmt=qpd.RESID_INT4, per_head=per_head, mode=mode,
              l2norm=True, T=2, seed=7 + per_head, act_dtype=act, out_dtype=act)


@pytest.mark.parametrize("K,resid_fmt,mode,act,decode_kernel", [
    (128, qpd.RESID_INT8, "exact", torch.float32, "persistent"),   # int8 per head: the residual
    (128, qpd.RESID_INT8, "fast", torch.bfloat16, "persistent"),   # waits in a 64 KB LDS table
    (128, qpd.RESID_INT8, "fast", torch.float16, "auto"),          # ... and in VGPRs (one-item)
    (64, qpd.RESID_INT4, "fast", torch.float32, "persistent"),     # per head below K=128
    (64, qpd.RESID_INT4, "exact", torch.float16, "persistent"),
    (64, qpd.RESID_INT8, "fast", torch.float32, "persistent"),
    (64, qpd.RESID_INT8, "exact", torch.bfloat16, "auto"),
    (256, qpd.RESID_INT4, "fast", torch.float32, "auto"),          # one 16-wave workgroup per CU
], indirect=["decode_kernel"])
def test_persistent_kernel_at_full_occupancy(device, K, resid_fmt, mode, act, decode_kernel):
    """Per-head shapes with more items than resident workgroups on the
    persistent kernel (items shared by workgroup age, the next item
    prefetched into the second register set): K = 256, which the automatic
    choice keeps there, and K = 64 and 128, chosen for the test (their
    automatic choice, the one-item kernel, runs the "auto" cases); HV=32,
    B=64 (B=32 at K=256, where a 16-wave workgroup holds a CU), the in-kernel
    L2 norm."""
    _run_both(device, B=64 if K < 256 else 32, H=32, HV=32, K=K, V=128, resid_fmt=resid_fmt, per_head=True,
              mode=mode, l2norm=True, T=2, seed=K + resid_fmt, act_dtype=act, out_dtype=act)


@pytest.mark.parametrize("K,V,H,HV", [(64, 64, 8, 16), (32, 8, 4, 4), (32, 4, 1, 1), (16, 40, 2, 2),
                                      (256, 128, 2, 4), (128, 200, 1, 2)])
@pytest.mark.parametrize("resid_fmt", [qpd.RESID_INT8, qpd.RESID_INT4])
@pytest.mark.parametrize("per_head", [False, True])
def test_bit_exact_shapes(device, K, V, H, HV, resid_fmt, per_head):
    _run_both(device, B=3, H=H, HV=HV, K=K, V=V, resid_fmt=resid_fmt, per_head=per_head,
              mode="fast", l2norm=True, T=2, seed=K + V)


@pytest.mark.parametrize("K,B,HV", [(64, 3, 8), (32, 3, 8), (32, 9, 32), (16, 3, 8)])
@pytest.mark.parametrize("resid_fmt", [qpd.RESID_INT8, qpd.RESID_INT4])
@pytest.mark.parametrize("mode", ["fast", "exact"])
def test_bit_exact_small_k_per_head_shapes(device, K, B, HV, resid_fmt, mode):
    """A V=128 head at K = 64 / 32 / 16 with a per-head residual scale: 2 rows
    per lane over 4 waves, 1 row over 4 waves (up to 256 items; B=9 x HV=32
    takes the one-wave shape) and 1 row over 2 waves."""
    _run_both(device, B=B, H=HV // 2, HV=HV, K=K, V=128, resid_fmt=resid_fmt, per_head=True,
              mode=mode, l2norm=True, T=2, seed=K + B)


@pytest.mark.parametrize("resid_fmt", [qpd.RESID_INT8, qpd.RESID_INT4])
@pytest.mark.parametrize("mode", ["fast", "exact"])
def test_bit_exact_k256_per_head_16_waves(device, resid_fmt, mode):
    """A V=128 head at K=256 with a per-head residual scale from one head per
    CU on (B x HV >= 256): 16 waves of 2 rows per lane."""
    _run_both(device, B=8, H=16, HV=32, K=256, V=128, resid_fmt=resid_fmt, per_head=True,
              mode=mode, l2norm=True, T=2, seed=256)


@pytest.mark.parametrize("act_dtype,out_dtype", [(torch.bfloat16, torch.bfloat16),
                                                 (torch.float16, torch.float32),
                                                 (torch.float32, torch.bfloat16)])
def test_bit_exact_dtypes(device, act_dtype, out_dtype):
    _run_both(device, B=2, H=16, HV=32, K=128, V=128, resid_fmt=qpd.RESID_INT4, per_head=False,
              mode="fast", l2norm=True, T=2, act_dtype=act_dtype, out_dtype=out_dtype, seed=7)


def test_bit_exact_int6_state(device):
    _run_both(device, B=2, H=32, HV=32, K=128, V=128, resid_fmt=qpd.RESID_INT8, per_head=True,
              mode="fast", l2norm=False, T=3, bits=6, seed=11)


@pytest.mark.parametrize("B,null_tail,resid_fmt,per_head", [
    (64, 16, qpd.RESID_INT4, True),    # whole requests dealt to the XCDs, the NULL ones last
    (40, 5, qpd.RESID_INT4, True),
    (45, 9, qpd.RESID_INT8, True),     # dealt requests and a B mod 8 tail in contiguous ranges
    (21, 6, qpd.RESID_INT4, False),
])
def test_padded_batch_bit_exact(device, B, null_tail, resid_fmt, per_head):
    """A batch padded at its end with NULL slot ids, as a captured batch size
    is: every live request bit-exact against the oracle, the NULL ones zero,
    over the one-item kernel's mapping of requests to XCDs."""
    _run_both(device, B=B, H=16, HV=32, K=128, V=128, resid_fmt=resid_fmt, per_head=per_head, mode="fast",
              l2norm=True, T=2, seed=23, null_tail=null_tail)


def test_null_block_padding(device, H=8, HV=16, K=64, V=64):
    """vllm_integration/test_quantized_packed_decode.py:153-177."""
    B = 2
    scale = K ** -0.5
    g = torch.Generator().manual_seed(3)
    pool = (torch.randn(3, HV, V, K, generator=g) * 0.1).to(device)
    sc, ss, rc, rs = qpd.init_quantized_state(3, HV, V, K, device, h0=pool)
    before = [x.clone() for x in (sc, ss, rc, rs)]
    indices = torch.tensor([2, qpd.NULL_BLOCK_ID], dtype=torch.int32, device=device)
    mixed, a, b, A_log, dt_bias = (x.to(device) for x in make_packed_inputs(B, H, HV, K, V, seed=7))
    out = torch.full((B, 1, HV, V), float("nan"), device=device)
    qpd.quantized_gated_delta_rule_packed_decode(mixed, a, b, A_log, dt_bias, scale, sc, ss, rc, rs, out, indices)
    torch.cuda.synchronize()
    assert torch.all(out[1] == 0), "NULL_BLOCK_ID request must emit zeros"
    assert not torch.any(torch.isnan(out[0])), "real request must be written"
    for slot in (0, 1):
        for now, was in zip((sc, ss, rc, rs), before):
            assert torch.equal(now[slot], was[slot]), f"slot {slot} was modified"
    assert not torch.equal(sc[2], before[0][2]), "the real slot should have advanced"


def test_out_of_range_slot_is_nan_and_untouched(device, H=4, HV=4, K=32, V=8):
    B = 2
    sc, ss, rc, rs = qpd.init_quantized_state(3, HV, V, K, device,
                                              h0=torch.randn(3, HV, V, K, device=device))
    before = [x.clone() for x in (sc, ss, rc, rs)]
    indices = torch.tensor([3, 1], dtype=torch.int32, device=device)   # 3 == num_slots
    mixed, a, b, A_log, dt_bias = (x.to(device) for x in make_packed_inputs(B, H, HV, K, V, seed=2))
    out = torch.zeros(B, 1, HV, V, device=device)
    qpd.quantized_gated_delta_rule_packed_decode(mixed, a, b, A_log, dt_bias, 1.0, sc, ss, rc, rs, out, indices)
    torch.cuda.synchronize()
    assert torch.all(torch.isnan(out[0]))
    assert not torch.any(torch.isnan(out[1]))
    for now, was in zip((sc, ss, rc, rs), before):
        assert torch.equal(now[0], was[0]) and torch.equal(now[2], was[2])


def test_paging_isolation(device, H=8, HV=16, K=64, V=64):
    """vllm_integration/test_quantized_packed_decode.py:180-208: batched == sequential."""
    scale = K ** -0.5
    g = torch.Generator().manual_seed(5)
    pool = (torch.randn(5, HV, V, K, generator=g) * 0.1).to(device)
    sc, ss, rc, rs = qpd.init_quantized_state(5, HV, V, K, device, h0=pool)
    indices = torch.tensor([3, 1], dtype=torch.int32, device=device)
    mixed, a, b, A_log, dt_bias = (x.to(device) for x in make_packed_inputs(2, H, HV, K, V, seed=11))
    out = torch.empty(2, 1, HV, V, device=device)
    qpd.quantized_gated_delta_rule_packed_decode(mixed, a, b, A_log, dt_bias, scale, sc, ss, rc, rs, out, indices)
    torch.cuda.synchronize()
    together = (sc.clone(), ss.clone(), rc.clone(), rs.clone(), out.clone())
    sc2, ss2, rc2, rs2 = qpd.init_quantized_state(5, HV, V, K, device, h0=pool)
    for r, slot in ((0, 3), (1, 1)):
        idx = torch.tensor([slot], dtype=torch.int32, device=device)
        o1 = torch.empty(1, 1, HV, V, device=device)
        qpd.quantized_gated_delta_rule_packed_decode(
            mixed[r:r + 1], a[r:r + 1], b[r:r + 1], A_log, dt_bias, scale, sc2, ss2, rc2, rs2, o1, idx)
        torch.cuda.synchronize()
        assert torch.equal(o1[0], together[4][r]), f"request {r} output differs when batched"
    for now, was in zip((sc2, ss2, rc2, rs2), together[:4]):
        assert torch.equal(now, was), "batched vs sequential state differs"


@pytest.mark.parametrize("mode", ["fast", "exact"])
def test_round_half_to_even(device, mode, H=1, HV=1, K=32, V=4):
    """vllm_integration/test_quantized_packed_decode.py:211-286: constructed .5 ties
    (odd int8 residual codes at scale 0.5, a state pin of 127 so the derived
    scale is exactly 1.0, gates neutralised with a = b = -60)."""
    RESID_SCALE = 0.5
    odd = (torch.arange(K, dtype=torch.float32) % 8) * 2 - 7
    resid_codes_in = odd[None, None, :].repeat(HV, V, 1).contiguous()
    resid_codes_in[..., 0] = 0.0
    state_codes_in = torch.zeros(HV, V, K)
    state_codes_in[..., 0] = 1.0
    target = state_codes_in * qpd.QMAX_INT8 + resid_codes_in * RESID_SCALE
    derived = target.abs().amax(dim=-1).clamp(min=qpd.EPS) / qpd.QMAX_INT8
    assert torch.all(derived == 1.0)
    ratios = target / derived[..., None]
    expected = torch.round(ratios).clamp(-127, 127)
    assert int(((ratios.abs() % 1.0) == 0.5).sum()) > 0
    assert int((torch.floor(ratios + 0.5) != expected).sum()) > 0

    sc = torch.zeros(2, HV, V, K, dtype=torch.int8, device=device)
    ss = torch.zeros(2, HV, V, device=device)
    rc = torch.zeros(2, HV, V, K, dtype=torch.int8, device=device)
    rs = torch.zeros(2, HV, V, device=device)
    sc[1] = state_codes_in.to(torch.int8).to(device)
    ss[1] = qpd.QMAX_INT8
    rc[1] = resid_codes_in.to(torch.int8).to(device)
    rs[1] = RESID_SCALE
    mixed = torch.zeros(1, 2 * H * K + HV * V, device=device)
    a = torch.full((1, HV), -60.0, device=device)
    b = torch.full((1, HV), -60.0, device=device)
    A_log = torch.zeros(HV, device=device)
    dt_bias = torch.zeros(HV, device=device)
    indices = torch.tensor([1], dtype=torch.int32, device=device)
    out = torch.empty(1, 1, HV, V, device=device)
    qpd.quantized_gated_delta_rule_packed_decode(mixed, a, b, A_log, dt_bias, K ** -0.5, sc, ss, rc, rs, out,
                                                 indices, quant_mode=mode)
    torch.cuda.synchronize()
    assert torch.equal(sc[1].float().cpu(), expected), "rounding does not match torch.round"


def _quantize_vk(h_vk):
    scale = h_vk.abs().amax(dim=-1).clamp(min=qpd.EPS) / qpd.QMAX_INT8
    codes = torch.round(h_vk / scale[..., None]).clamp(-127, 127)
    return codes.to(torch.int8), scale


def _unpack_qkv(mixed, B, H, HV, K, V, scale, l2norm):
    q = mixed[:, :H * K].reshape(B, H, K).double()
    k = mixed[:, H * K:2 * H * K].reshape(B, H, K).double()
    v = mixed[:, 2 * H * K:].reshape(B, HV, V).double()
    if l2norm:
        q = q / torch.sqrt((q * q).sum(-1, keepdim=True) + 1e-6)
        k = k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    q = q * scale
    rep = HV // H
    return q.repeat_interleave(rep, dim=1), k.repeat_interleave(rep, dim=1), v


@pytest.mark.parametrize("resid_fmt,bound", [(qpd.RESID_INT8, 5e-2), (qpd.RESID_INT4, 8e-2)])
def test_decode_vs_ef_oracle(device, resid_fmt, bound, B=2, H=8, HV=16, K=64, V=64, T=32):
    """vllm_integration/test_quantized_packed_decode.py:108-150 / :310-354: T-step
    decode against the float64 recurrence with an fp32 error-feedback residual
    (statequant/quant.py:65-80) and per-V-row quantization."""
    S = B + 1
    scale = K ** -0.5
    g = torch.Generator().manual_seed(0)
    h0 = torch.randn(B, HV, V, K, generator=g) * 0.1
    pool = torch.zeros(S, HV, V, K)
    pool[1:] = h0
    sc, ss, rc, rs = qpd.init_quantized_state(S, HV, V, K, device, h0=pool.to(device), resid_fmt=resid_fmt)
    indices = torch.arange(1, B + 1, dtype=torch.int32, device=device)
    steps = [make_packed_inputs(B, H, HV, K, V, seed=100 + t) for t in range(T)]
    outs = []
    for (mixed, a, b, A_log, dt_bias) in steps:
        out = torch.empty(B, 1, HV, V, device=device)
        qpd.quantized_gated_delta_rule_packed_decode(
            mixed.to(device), a.to(device), b.to(device), A_log.to(device), dt_bias.to(device), scale,
            sc, ss, rc, rs, out, indices, use_qk_l2norm_in_kernel=True, resid_fmt=resid_fmt)
        outs.append(out[:, 0].cpu())
    torch.cuda.synchronize()
    kernel_o = torch.stack(outs).double()

    c0, s0 = _quantize_vk(pool[1:])
    h = (c0.double() * s0.double()[..., None]).transpose(-1, -2)   # [B, HV, K, V]
    e = torch.zeros_like(h)
    o_ref = []
    for (mixed, a, b, A_log, dt_bias) in steps:
        alpha, beta = oracle.gates(a.numpy(), b.numpy(), A_log.numpy()[None], dt_bias.numpy()[None])
        q, k, v = _unpack_qkv(mixed, B, H, HV, K, V, scale, True)
        hn, o = oracle.gdn_step_f64(h.numpy(), q.numpy(), k.numpy(), v.numpy(), alpha, beta)
        target = torch.from_numpy(hn) + e
        s = target.abs().amax(dim=-2, keepdim=True).clamp(min=1e-12) / 127.0
        hq = torch.round(target / s).clamp(-127, 127) * s
        e = target - hq
        h = hq
        o_ref.append(torch.from_numpy(o))
    o_ref = torch.stack(o_ref)
    h_ref = h.transpose(-1, -2)
    h_got = sc[1:].double().cpu() * ss[1:].double().cpu()[..., None]
    o_rel = rel(kernel_o.numpy(), o_ref.numpy())
    h_rel = rel(h_got.numpy(), h_ref.numpy())
    print(f"decode T={T} resid={resid_fmt}: o rel={o_rel:.3e} h rel={h_rel:.3e}")
    assert o_rel < bound and h_rel < bound
