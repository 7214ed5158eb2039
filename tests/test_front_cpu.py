"""The packed decode's C++ argument checks (``_ck_front``, csrc/front.cpp)
against the Python front end's (quantized_packed_decode.py, which follows the
reference's quantized_packed_decode.py:268-309). On CPU tensors, with the
device checks left out, the C++ side must accept exactly the calls the Python
checks accept, with the same C-ABI arguments, and decline the rest (the
Python checks then raise the reference's errors)."""

from __future__ import annotations

import ctypes
import random

import pytest
import torch

from carrykernel_amd import _native
from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd


@pytest.fixture(scope="module")
def front():
    if not _native.library_available():
        pytest.skip("the HIP library is not built")
    _native.lib()
    assert _native._front is not None, "the _ck_front extension is not built (python -m carrykernel_amd.build)"
    return _native._front


def _case(B=2, H=2, HV=4, K=64, V=32, S=3, resid_fmt=qpd.RESID_INT4, per_head=False):
    rk = K // 2 if resid_fmt == qpd.RESID_INT4 else K
    return dict(mixed_qkv=torch.zeros(B, 2 * H * K + HV * V), a=torch.zeros(B, HV), b=torch.zeros(B, HV),
                A_log=torch.zeros(HV), dt_bias=torch.zeros(HV), scale=0.1,
                state_codes=torch.zeros(S, HV, V, K, dtype=torch.int8), state_scale=torch.zeros(S, HV, V),
                resid_codes=torch.zeros(S, HV, V, rk, dtype=torch.int8),
                resid_scale=torch.zeros((S, HV) if per_head else (S, HV, V)),
                out=torch.zeros(B, 1, HV, V), ssm_state_indices=torch.arange(1, B + 1, dtype=torch.int32),
                use_qk_l2norm_in_kernel=False, resid_fmt=resid_fmt, state_bits=8, quant_mode="fast",
                dst_state_indices=None)


def _python(c):
    """C-ABI arguments from the Python checks, or the exception they raise."""
    try:
        _, args = qpd._decode_call_args(**c, check_devices=False)
    except (ValueError, ZeroDivisionError) as e:
        return e
    # ck_gdn_packed_decode_to's order (no destination: 0, 0); scale as the C float
    args = list(args)
    args[13] = ctypes.c_float(args[13]).value
    if c["dst_state_indices"] is None:
        args[26:26] = [0, 0]
    return tuple(args)


def _cpp(front, c, require_cuda=False):
    return front.launch_args(
        c["mixed_qkv"], c["a"], c["b"], c["A_log"], c["dt_bias"], c["scale"], c["state_codes"],
        c["state_scale"], c["resid_codes"], c["resid_scale"], c["out"], c["ssm_state_indices"],
        c["dst_state_indices"], c["use_qk_l2norm_in_kernel"], c["resid_fmt"], c["state_bits"],
        qpd._QUANT_MODES[c["quant_mode"]], require_cuda)


def _padded(t, pad=7):
    """The same values with every slot padded by `pad` elements (slot stride
    larger than the slot)."""
    S = t.shape[0]
    back = torch.zeros(S, t[0].numel() + pad, dtype=t.dtype)
    v = back[:, :t[0].numel()].view(t.shape)
    v.copy_(t)
    return v


def _wide_rows(t, extra=5):
    """Rows of a wider buffer: row stride larger than the row."""
    back = torch.zeros(t.shape[0], t.shape[1] + extra, dtype=t.dtype)
    back[:, :t.shape[1]] = t
    return back[:, :t.shape[1]]


def test_constants_match_the_python_front_end(front):
    assert front.MAX_K == qpd.MAX_K
    assert front.RESID_INT8 == qpd.RESID_INT8 and front.RESID_INT4 == qpd.RESID_INT4
    assert front.QUANT_FAST == _native.QUANT_FAST == qpd._QUANT_MODES["fast"]
    assert front.DECLINED < 0 and min(_native.CK_OK, _native.CK_EINVAL, _native.CK_EUNSUPPORTED,
                                      _native.CK_ELAUNCH) >= 0


VALID = {
    "int4_row": {},
    "int4_head": dict(per_head=True),
    "int8_row": dict(resid_fmt=qpd.RESID_INT8),
    "int8_head": dict(resid_fmt=qpd.RESID_INT8, per_head=True),
    "k128_v128": dict(H=2, HV=8, K=128, V=128, B=5, S=9, per_head=True),
    "k7_int8": dict(K=7, resid_fmt=qpd.RESID_INT8),
    "k1024": dict(K=1024, V=4, HV=2, H=1),
    "hv_eq_h": dict(H=4, HV=4),
}
TWEAKS = {
    "plain": lambda c: None,
    "bf16": lambda c: c.update(mixed_qkv=c["mixed_qkv"].bfloat16(), a=c["a"].bfloat16(),
                               b=c["b"].bfloat16(), out=c["out"].bfloat16()),
    "fp16_gates": lambda c: c.update(A_log=c["A_log"].half(), dt_bias=c["dt_bias"].bfloat16()),
    "wide_rows": lambda c: c.update(mixed_qkv=_wide_rows(c["mixed_qkv"]), a=_wide_rows(c["a"]),
                                    b=_wide_rows(c["b"], 3)),
    "padded_slots": lambda c: c.update(**{k: _padded(c[k]) for k in
                                          ("state_codes", "state_scale", "resid_codes", "resid_scale")}),
    "options": lambda c: c.update(use_qk_l2norm_in_kernel=True, state_bits=4, quant_mode="exact"),
    "dst": lambda c: c.update(dst_state_indices=torch.arange(2, 2 + c["out"].shape[0], dtype=torch.int32)),
    "long_ids": lambda c: c.update(ssm_state_indices=torch.ones(c["out"].shape[0] + 3, dtype=torch.int32)),
    "strided_ids": lambda c: c.update(ssm_state_indices=torch.ones(2 * c["out"].shape[0], dtype=torch.int32)[::2]),
}


@pytest.mark.parametrize("tweak", list(TWEAKS))
@pytest.mark.parametrize("shape", list(VALID))
def test_accepts_valid_calls_with_the_python_arguments(front, shape, tweak):
    c = _case(**VALID[shape])
    TWEAKS[tweak](c)
    py = _python(c)
    assert isinstance(py, tuple), py
    assert _cpp(front, c) == py
    assert _cpp(front, c, require_cuda=True) is None      # CPU tensors are never launched


MUTATIONS = [
    lambda c: c.update(mixed_qkv=torch.zeros(2, 3, 4)),
    lambda c: c.update(mixed_qkv=torch.zeros(c["mixed_qkv"].shape[1], 2).t()),
    lambda c: c.update(mixed_qkv=c["mixed_qkv"][:, :-2]),
    lambda c: c.update(mixed_qkv=c["mixed_qkv"][:1]),
    lambda c: c.update(mixed_qkv=c["mixed_qkv"].to(torch.int32)),
    lambda c: c.update(state_codes=c["state_codes"][..., 0]),
    lambda c: c.update(state_codes=c["state_codes"].transpose(2, 3).contiguous().transpose(2, 3)),
    lambda c: c.update(state_codes=c["state_codes"].transpose(1, 2).contiguous().transpose(1, 2)),
    lambda c: c.update(state_codes=c["state_codes"].to(torch.uint8)),
    lambda c: c.update(resid_codes=c["resid_codes"].float()),
    lambda c: c.update(resid_codes=c["resid_codes"][..., :-1]),
    lambda c: c.update(resid_codes=c["resid_codes"][:-1]),
    lambda c: c.update(resid_fmt=1 - c["resid_fmt"]),
    lambda c: c.update(resid_fmt=2),
    lambda c: c.update(ssm_state_indices=c["ssm_state_indices"][None]),
    lambda c: c.update(ssm_state_indices=c["ssm_state_indices"].long()),
    lambda c: c.update(ssm_state_indices=c["ssm_state_indices"][:1]),
    lambda c: c.update(out=c["out"][:, 0]),
    lambda c: c.update(out=c["out"][:1]),
    lambda c: c.update(out=c["out"].transpose(2, 3).contiguous().transpose(2, 3)),
    lambda c: c.update(out=c["out"].to(torch.float64)),
    lambda c: c.update(state_scale=c["state_scale"].half()),
    lambda c: c.update(state_scale=c["state_scale"][:, :, :1]),
    lambda c: c.update(resid_scale=c["resid_scale"].double()),
    lambda c: c.update(resid_scale=torch.zeros(c["state_codes"].shape[0], 5)),
    lambda c: c.update(resid_scale=c["resid_scale"].transpose(0, 1).contiguous().transpose(0, 1)),
    lambda c: c.update(a=c["a"][:, :-1]),
    lambda c: c.update(b=c["b"].t().contiguous().t()),
    lambda c: c.update(b=c["b"].to(torch.int64)),
    lambda c: c.update(A_log=torch.zeros(2 * c["A_log"].shape[0])[::2]),
    lambda c: c.update(dt_bias=c["dt_bias"][None]),
    lambda c: c.update(state_bits=1),
    lambda c: c.update(state_bits=9),
    lambda c: c.update(state_bits=5),
    lambda c: c.update(use_qk_l2norm_in_kernel=True),
    lambda c: c.update(quant_mode="exact"),
    lambda c: c.update(dst_state_indices=torch.ones(c["out"].shape[0], dtype=torch.int32)),
    lambda c: c.update(dst_state_indices=torch.ones(c["out"].shape[0], dtype=torch.int64)),
    lambda c: c.update(dst_state_indices=torch.ones(max(c["out"].shape[0] - 1, 0), dtype=torch.int32)),
    lambda c: c.update(dst_state_indices=torch.ones(1, c["out"].shape[0], dtype=torch.int32)),
    lambda c: c.update(**{k: _padded(c[k], 3) for k in ("state_codes", "resid_codes")}),
    lambda c: c.update(mixed_qkv=_wide_rows(c["mixed_qkv"])),
]


def test_declines_the_calls_the_python_checks_reject(front):
    """Every mutation of the reference's error table and beyond, alone and in
    random combinations of up to three: declined exactly where the Python
    checks raise, and otherwise the same arguments."""
    rng = random.Random(0)
    base = [dict(), dict(per_head=True), dict(resid_fmt=qpd.RESID_INT8), dict(K=7, resid_fmt=qpd.RESID_INT8)]
    trials = [(b, (m,)) for b in range(len(base)) for m in range(len(MUTATIONS))]
    trials += [(rng.randrange(len(base)), tuple(rng.sample(range(len(MUTATIONS)), rng.randint(2, 3))))
               for _ in range(600)]
    declined = 0
    for bi, ms in trials:
        c = _case(**base[bi])
        for m in ms:
            try:
                MUTATIONS[m](c)
            except (RuntimeError, IndexError):   # does not apply to an earlier mutation's result
                pass
        py = _python(c)
        cpp = _cpp(front, c)
        if isinstance(py, tuple):
            assert cpp == py, (bi, ms)
        else:
            assert cpp is None, (bi, ms, py)
            declined += 1
    assert declined > len(trials) // 2      # the table is mostly errors


def test_python_front_end_raises_after_a_declined_call(front):
    """CPU tensors: the C++ side declines, the Python checks run and raise the
    reference's errors (or, for a valid call, the missing-GPU error)."""
    c = _case()
    c["mixed_qkv"] = torch.zeros(2, 3, 4)
    with pytest.raises(ValueError, match="mixed_qkv must be 2-D"):
        qpd.quantized_gated_delta_rule_packed_decode(**c)
    with pytest.raises(_native.HipUnavailable):
        qpd.quantized_gated_delta_rule_packed_decode(**_case())
