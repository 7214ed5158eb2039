"""GPU parity of the fused decode at batches with several items per resident
workgroup (K = V = 128, packed int4 or int8 residual, per-head or per-row scales,
B >= 32 at HV = 32), on both kernels: the automatic choice, the one-item
kernel (one workgroup per item, dispatcher-balanced), and the persistent
kernel, chosen for the test through ck_set_decode_kernel: its item loop's
register double buffer (item k computed while item k + 1 loads), the
alternating LDS staging buffers whose parity follows the count of live
items, and the collapsed prefetch past a workgroup's last item. Each case
runs consecutive steps on one pool through the drop-in front end and
compares the output and all four pool tensors bit for bit with the oracle
after every step.

Cases cover NULL and out-of-range slots between live items of one workgroup,
out-of-place destinations, GQA, the in-kernel L2 norm, 16-bit activations
and outputs, EXACT mode, 6-bit state, and ragged item counts per workgroup
(two or three items).
"""

from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

import oracle
from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd
from tests._helpers import make_packed_inputs, make_pool, to_dev

pytestmark = pytest.mark.gpu

K = V = 128
HV = 32

# name: B, H, per_head, mode, act dtype, out dtype, l2norm, NULL fraction,
#       out-of-range id, out-of-place, state bits, steps[, residual format (int4 if absent)]
CASES = {
    "c3_b64_six_steps": (64, 32, True, "fast", torch.float32, torch.float32, False, 0.0, False, False, 8, 6),
    "nulls_gqa_l2_bf16": (96, 16, True, "fast", torch.bfloat16, torch.bfloat16, True, 0.1, True, False, 8, 3),
    "per_head_exact": (64, 32, True, "exact", torch.float32, torch.float32, True, 0.05, False, False, 8, 2),
    "per_head_int6": (64, 32, True, "fast", torch.float32, torch.float32, False, 0.0, False, False, 6, 2),
    "per_head_out_of_place": (64, 32, True, "fast", torch.float32, torch.float32, True, 0.05, False, True, 8, 2),
    "ragged_b33": (33, 32, True, "fast", torch.float32, torch.float32, False, 0.0, False, False, 8, 3),
    "ragged_b40_nulls": (40, 8, True, "fast", torch.float32, torch.float16, True, 0.2, True, False, 8, 2),
    "per_row_exact_f16": (64, 32, False, "exact", torch.float16, torch.float32, True, 0.0, False, False, 8, 3),
    "per_row_nulls_bf16": (80, 16, False, "fast", torch.bfloat16, torch.bfloat16, False, 0.1, True, False, 8, 2),
    "per_row_out_of_place": (64, 32, False, "fast", torch.float32, torch.float32, True, 0.0, False, True, 8, 2),
    "int8_head_nulls_exact": (48, 16, True, "exact", torch.float32, torch.float32, True, 0.1, True, False, 8, 2,
                              qpd.RESID_INT8),
    "int8_row_out_of_place": (64, 32, False, "fast", torch.bfloat16, torch.bfloat16, False, 0.05, False, True, 8, 2,
                              qpd.RESID_INT8),
}


def _expected_out(o_ref, out_dt):
    if out_dt == torch.bfloat16:
        return oracle.bf16_round(o_ref)
    if out_dt == torch.float16:
        return o_ref.astype(np.float16).astype(np.float32)
    return o_ref


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("decode_kernel", ["auto", "persistent"], indirect=True)
def test_multi_item_decode_bit_exact(device, name, decode_kernel):
    B, H, per_head, mode, act, out_dt, l2norm, null_frac, bad_id, dst_mode, bits, steps = CASES[name][:12]
    resid_fmt = CASES[name][12] if len(CASES[name]) > 12 else qpd.RESID_INT4
    # at least two items per resident workgroup: two 8-wave workgroups per CU
    # with a per-head scale, four 4-wave (64-row tiles) per row
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    items, per_cu = (B * HV, 2) if per_head else (B * HV * (V // 64), 4)
    assert items >= 2 * per_cu * cus, f"{name}: batch too small for several items per workgroup"
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    S = 2 * B + 3 if dst_mode else B + 3
    pool = make_pool(S, HV, V, K, resid_fmt, per_head, seed=B, bits=bits)
    dpool = to_dev(pool, device)
    perm = (rng.permutation(S - 1) + 1).astype(np.int32)
    src = perm[:B].copy()
    src[rng.random(B) < null_frac] = 0
    if bad_id:
        src[int(rng.integers(B))] = S + 1
    dst = perm[B:2 * B].copy() if dst_mode else None
    print(f"case {name} kernel={decode_kernel}", flush=True)
    for t in range(steps):
        mixed, a, b, A_log, dt_bias = make_packed_inputs(B, H, HV, K, V, seed=31 * B + t, dtype=act)
        scale = K ** -0.5 if l2norm else 1.0
        out = torch.empty(B, 1, HV, V, dtype=out_dt, device=device)
        qpd.quantized_gated_delta_rule_packed_decode(
            mixed.to(device), a.to(device), b.to(device), A_log.to(device), dt_bias.to(device), scale, *dpool, out,
            torch.from_numpy(src).to(device), use_qk_l2norm_in_kernel=l2norm, resid_fmt=resid_fmt,
            state_bits=bits, quant_mode=mode,
            dst_state_indices=None if dst is None else torch.from_numpy(dst).to(device))
        torch.cuda.synchronize()
        o_ref = oracle.packed_decode(
            mixed.float().numpy(), a.float().numpy(), b.float().numpy(), A_log.float().numpy(),
            dt_bias.float().numpy(), scale, *pool, src, H, use_qk_l2norm=l2norm, resid_fmt=resid_fmt,
            per_head=per_head, state_bits=bits, mode=oracle.MODE_EXACT if mode == "exact" else oracle.MODE_FAST,
            dst_indices=dst)
        np.testing.assert_array_equal(out[:, 0].float().cpu().numpy(), _expected_out(o_ref, out_dt),
                                      err_msg=f"{name}: out differs at step {t}")
        for tname, d, h in zip(("state_codes", "state_scale", "resid_codes", "resid_scale"), dpool, pool):
            np.testing.assert_array_equal(d.cpu().numpy(), h, err_msg=f"{name}: {tname} differs at step {t}")
        if dst is not None:
            src, dst = dst, src                       # read back what was written
            src = np.where((src > 0) & (src < S), src, 0).astype(np.int32)
            dst = np.where((dst > 0) & (dst < S), dst, 0).astype(np.int32)
