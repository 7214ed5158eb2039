"""The packed decode's two host routes on the GPU: the C++ checks and launch
(``_ck_front``, csrc/front.cpp) that every usual call takes, and the Python
checks with the ctypes launch that a declined call takes. Both must launch
the same step: outputs and pools bit-identical. Parity of the step itself
against the oracle is in the other decode tests, which run through the C++
route."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from carrykernel_amd import _native
from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd
from tests._helpers import make_packed_inputs, make_pool, to_dev

pytestmark = pytest.mark.gpu


def _step(device, pool, mixed, a, b, A_log, dt_bias, ids, dst, out_dtype, **kw):
    B, HV, V = mixed.shape[0], pool[0].shape[1], pool[0].shape[2]
    out = torch.empty(B, 1, HV, V, dtype=out_dtype, device=device)
    qpd.quantized_gated_delta_rule_packed_decode(mixed, a, b, A_log, dt_bias, 0.0883, *pool, out, ids,
                                                 dst_state_indices=dst, **kw)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("case", ["int4_head", "int8_row_dst", "int4_row_bf16_wide", "int8_head_exact_l2"])
def test_cpp_and_python_routes_launch_the_same_step(device, monkeypatch, case):
    B, H, HV, K, V = 6, 4, 8, 128, 64
    resid_fmt = qpd.RESID_INT8 if "int8" in case else qpd.RESID_INT4
    per_head = "head" in case
    act = torch.bfloat16 if "bf16" in case else torch.float32
    kw = dict(resid_fmt=resid_fmt, use_qk_l2norm_in_kernel="l2" in case,
              quant_mode="exact" if "exact" in case else "fast")
    print(f"case {case}", flush=True)
    S = 2 * B + 2
    host_pool = make_pool(S, HV, V, K, resid_fmt, per_head, seed=3)
    mixed, a, b, A_log, dt_bias = make_packed_inputs(B, H, HV, K, V, seed=4, dtype=act)
    mixed, a, b, A_log, dt_bias = (t.to(device) for t in (mixed, a, b, A_log, dt_bias))
    if "wide" in case:   # rows of wider buffers: row strides above the row widths
        wide = torch.zeros(B, mixed.shape[1] + 64, dtype=act, device=device)
        wide[:, :mixed.shape[1]] = mixed
        mixed = wide[:, :mixed.shape[1]]
    ids = torch.arange(1, B + 1, dtype=torch.int32, device=device)
    dst = torch.arange(B + 1, 2 * B + 1, dtype=torch.int32, device=device) if "dst" in case else None

    _native.lib()
    front = _native._front
    assert front is not None, "the _ck_front extension is not built"
    pool_c = to_dev(host_pool, device)
    out_c = torch.empty(B, 1, HV, V, dtype=act, device=device)
    assert front.launch_args(mixed, a, b, A_log, dt_bias, 0.0883, *pool_c, out_c, ids, dst,
                             kw["use_qk_l2norm_in_kernel"], resid_fmt, 8, qpd._QUANT_MODES[kw["quant_mode"]],
                             True) is not None, "the C++ route declined a valid call"
    out_c = _step(device, pool_c, mixed, a, b, A_log, dt_bias, ids, dst, act, **kw)

    pool_p = to_dev(host_pool, device)
    monkeypatch.setattr(_native, "_front", None)          # the Python checks and the ctypes launch
    out_p = _step(device, pool_p, mixed, a, b, A_log, dt_bias, ids, dst, act, **kw)

    assert torch.equal(out_c, out_p)
    for name, x, y in zip(("state_codes", "state_scale", "resid_codes", "resid_scale"), pool_c, pool_p):
        assert torch.equal(x, y), name
    # the step changed the written slots and nothing else
    written = (dst if dst is not None else ids).cpu().numpy()
    moved = ~np.all(pool_c[0].cpu().numpy() == host_pool[0], axis=(1, 2, 3))
    assert set(np.nonzero(moved)[0]) <= set(written.tolist()) and moved.any()


def test_declined_calls_raise_the_python_errors(device):
    """On GPU tensors too, a call the C++ route declines reaches the Python
    checks, which raise the front end's errors: a destination with EXACT
    rounding, and a tensor on another device."""
    B, H, HV, K, V = 2, 2, 4, 64, 32
    pool = to_dev(make_pool(B + 3, HV, V, K, qpd.RESID_INT4, True, seed=5), device)
    mixed, a, b, A_log, dt_bias = (t.to(device) for t in make_packed_inputs(B, H, HV, K, V, seed=6))
    ids = torch.tensor([1, 2], dtype=torch.int32, device=device)
    out = torch.empty(B, 1, HV, V, device=device)
    print("case declined calls", flush=True)
    _native.lib()
    assert _native._front is not None
    with pytest.raises(ValueError, match="dst_state_indices is supported with quant_mode='fast'"):
        qpd.quantized_gated_delta_rule_packed_decode(mixed, a, b, A_log, dt_bias, 0.1, *pool, out, ids,
                                                     resid_fmt=qpd.RESID_INT4, quant_mode="exact",
                                                     dst_state_indices=ids + 2)
    with pytest.raises(_native.HipUnavailable, match="a is on cpu"):
        qpd.quantized_gated_delta_rule_packed_decode(mixed, a.cpu(), b, A_log, dt_bias, 0.1, *pool, out, ids,
                                                     resid_fmt=qpd.RESID_INT4)
