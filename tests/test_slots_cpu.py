"""Slot operations around the decode step, without a GPU: the oracle's
out-of-place step (read one slot, write another) against its in-place step,
and the argument checks of the C ABI and Python front ends of
ck_gdn_packed_decode_to / ck_pool_copy_slots / ck_pool_reset_slots.

The out-of-place step has no counterpart in the reference (its packed decode
is in place only, vllm_integration/quantized_packed_decode.py:217-239); it is
pinned here by composition: a chain of out-of-place steps equals the same
steps in place, every intermediate slot holding the in-place state of its
step, so whatever pins the in-place oracle pins this one."""

from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest
import torch

import oracle
from carrykernel_amd import _native
from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd
from tests._helpers import make_packed_inputs, make_pool

H, HV, K, V = 4, 8, 64, 32


def _inputs(B, seed):
    return [x.numpy() for x in make_packed_inputs(B, H, HV, K, V, seed=seed)]


@pytest.mark.parametrize("resid_fmt", [oracle.RESID_INT8, oracle.RESID_INT4])
@pytest.mark.parametrize("per_head", [False, True])
def test_dst_equal_to_src_is_the_in_place_step(resid_fmt, per_head):
    pool = make_pool(6, HV, V, K, resid_fmt, per_head, seed=3)
    twin = [x.copy() for x in pool]
    mixed, a, b, A_log, dt = _inputs(3, 4)
    idx = np.array([2, 0, 5], np.int32)
    o1 = oracle.packed_decode(mixed, a, b, A_log, dt, 0.125, *pool, idx, H, resid_fmt=resid_fmt, per_head=per_head)
    o2 = oracle.packed_decode(mixed, a, b, A_log, dt, 0.125, *twin, idx, H, resid_fmt=resid_fmt, per_head=per_head,
                              dst_indices=idx)
    np.testing.assert_array_equal(o1, o2)
    for x, y in zip(pool, twin):
        np.testing.assert_array_equal(x, y)


@pytest.mark.parametrize("resid_fmt", [oracle.RESID_INT8, oracle.RESID_INT4])
@pytest.mark.parametrize("per_head", [False, True])
def test_chain_equals_in_place_steps_and_keeps_every_state(resid_fmt, per_head):
    """Token t reads the slot token t-1 wrote (speculative decoding): the
    outputs and every intermediate state equal the in-place run's, and each
    earlier slot still holds its state (rollback target)."""
    T = 4
    chain = [1, 3, 4, 6, 7]                 # slot of the state after t tokens
    pool = make_pool(9, HV, V, K, resid_fmt, per_head, seed=5)
    inplace = [x.copy() for x in pool]
    snapshots = []
    for t in range(T):
        mixed, a, b, A_log, dt = _inputs(1, 100 + t)
        o_ref = oracle.packed_decode(mixed, a, b, A_log, dt, 0.2, *inplace, np.array([1], np.int32), H,
                                     resid_fmt=resid_fmt, per_head=per_head)
        snapshots.append([x[1].copy() for x in inplace])
        o = oracle.packed_decode(mixed, a, b, A_log, dt, 0.2, *pool, np.array([chain[t]], np.int32), H,
                                 resid_fmt=resid_fmt, per_head=per_head,
                                 dst_indices=np.array([chain[t + 1]], np.int32))
        np.testing.assert_array_equal(o, o_ref)
    for t in range(T):
        for got, want in zip(pool, snapshots[t]):
            np.testing.assert_array_equal(got[chain[t + 1]], want)
    untouched = make_pool(9, HV, V, K, resid_fmt, per_head, seed=5)
    for slot in (0, 1, 2, 5, 8):
        for got, want in zip(pool, untouched):
            np.testing.assert_array_equal(got[slot], want[slot])


@pytest.mark.parametrize("dst", [0, -3, 6])
def test_invalid_destination_discards_the_update(dst):
    pool = make_pool(6, HV, V, K, oracle.RESID_INT4, True, seed=8)
    before = [x.copy() for x in pool]
    ref = [x.copy() for x in pool]
    mixed, a, b, A_log, dt = _inputs(1, 9)
    o_ref = oracle.packed_decode(mixed, a, b, A_log, dt, 0.3, *ref, np.array([2], np.int32), H,
                                 resid_fmt=oracle.RESID_INT4, per_head=True)
    o = oracle.packed_decode(mixed, a, b, A_log, dt, 0.3, *pool, np.array([2], np.int32), H,
                             resid_fmt=oracle.RESID_INT4, per_head=True, dst_indices=np.array([dst], np.int32))
    np.testing.assert_array_equal(o, o_ref)
    for x, y in zip(pool, before):
        np.testing.assert_array_equal(x, y)


def test_batched_destinations_equal_one_request_at_a_time():
    pool = make_pool(10, HV, V, K, oracle.RESID_INT8, False, seed=12)
    seq = [x.copy() for x in pool]
    mixed, a, b, A_log, dt = _inputs(3, 13)
    src, dst = np.array([1, 4, 0], np.int32), np.array([7, 9, 8], np.int32)
    o = oracle.packed_decode(mixed, a, b, A_log, dt, 0.5, *pool, src, H, dst_indices=dst)
    for r in range(3):
        o1 = oracle.packed_decode(mixed[r:r + 1], a[r:r + 1], b[r:r + 1], A_log, dt, 0.5, *seq, src[r:r + 1], H,
                                  dst_indices=dst[r:r + 1])
        np.testing.assert_array_equal(o1[0], o[r])
    for x, y in zip(pool, seq):
        np.testing.assert_array_equal(x, y)
    assert np.all(o[2] == 0)                      # NULL source: zeros, nothing written
    untouched = make_pool(10, HV, V, K, oracle.RESID_INT8, False, seed=12)
    np.testing.assert_array_equal(pool[0][8], untouched[0][8])


# ---------------------------------------------------------------------------
# C ABI argument checks (no kernel is launched)
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def L():
    if not _native.library_available():
        pytest.skip("library not built")
    return _native.lib()


def _pool_abi(stride_state=8 * 32 * 64, stride_sscale=8 * 32, stride_resid=8 * 32 * 32, stride_rscale=8,
              num_slots=4, base=16):
    p = ctypes.c_void_p(base)
    return [p, stride_state, p, stride_sscale, p, stride_resid, p, stride_rscale, num_slots]


def test_pool_copy_argument_errors(L):
    ids = ctypes.c_void_p(16)
    shape = [8, 32, 64, qpd.RESID_INT4, _native.RSCALE_PER_HEAD, None]
    assert L.ck_pool_copy_slots(*_pool_abi(), *_pool_abi(), ids, ids, 0, *shape) == _native.CK_OK
    rc = L.ck_pool_copy_slots(*_pool_abi(), *_pool_abi(), ids, ids, 3, 8, 32, 64, 5, 1, None)
    assert rc == _native.CK_EINVAL and "resid_fmt" in L.ck_last_error().decode()
    rc = L.ck_pool_copy_slots(*_pool_abi(stride_state=100), *_pool_abi(), ids, ids, 3, *shape)
    assert rc == _native.CK_EINVAL and "smaller than a slot" in L.ck_last_error().decode()
    rc = L.ck_pool_copy_slots(*_pool_abi(), *_pool_abi(base=18), ids, ids, 3, *shape)
    assert rc == _native.CK_EINVAL and "4-byte aligned" in L.ck_last_error().decode()
    rc = L.ck_pool_copy_slots(*_pool_abi(), *_pool_abi(), None, ids, 3, *shape)
    assert rc == _native.CK_EINVAL and "slot id array" in L.ck_last_error().decode()
    rc = L.ck_pool_copy_slots(*_pool_abi(), *_pool_abi(num_slots=0), ids, ids, 3, *shape)
    assert rc == _native.CK_EINVAL and "num_slots" in L.ck_last_error().decode()
    rc = L.ck_pool_reset_slots(*_pool_abi(), ids, 3, 8, 32, 20, qpd.RESID_INT4, 0, None)
    assert rc == _native.CK_EINVAL and "multiple of 8" in L.ck_last_error().decode()
    assert L.ck_pool_reset_slots(*_pool_abi(), ids, 0, *shape) == _native.CK_OK


def test_packed_decode_to_needs_destinations(L):
    p = ctypes.c_void_p(16)
    args = [p, 0, 384, p, 0, 2, p, 0, 2, p, 0, p, 0, 1.0, p, 2 * 64 * 128, p, 128, p, 2 * 64 * 64, p, 2,
            p, 0, p, 1, None, 1, 4, 1, 1, 2, 128, 64, 0, 1, 1, 8, 0, None]
    assert L.ck_gdn_packed_decode_to(*args) == _native.CK_EINVAL
    assert "dst_state_indices" in L.ck_last_error().decode()


# ---------------------------------------------------------------------------
# Python front ends
# ---------------------------------------------------------------------------

def _cpu_pool(S=3, resid_fmt=qpd.RESID_INT4, per_head=False):
    rk = K // 2 if resid_fmt == qpd.RESID_INT4 else K
    return (torch.zeros(S, HV, V, K, dtype=torch.int8), torch.zeros(S, HV, V),
            torch.zeros(S, HV, V, rk, dtype=torch.int8), torch.zeros((S, HV) if per_head else (S, HV, V)))


def test_copy_and_reset_front_end_errors():
    ids = torch.tensor([1, 2], dtype=torch.int32)
    with pytest.raises(ValueError, match="same HV, V, K"):
        qpd.copy_quantized_state(_cpu_pool()[:3] + (torch.zeros(3, HV, V),), ids,
                                 _cpu_pool(per_head=True), ids)
    bad = list(_cpu_pool())
    bad[2] = torch.zeros(3, HV, V, 7, dtype=torch.int8)
    with pytest.raises(ValueError, match="resid_codes must be"):
        qpd.reset_quantized_state(tuple(bad), ids)
    with pytest.raises(ValueError, match=re.escape("(state_codes, state_scale, resid_codes, resid_scale)")):
        qpd.reset_quantized_state(_cpu_pool()[:3], ids)
    # valid layout on CPU tensors: no CPU fallback
    with pytest.raises(_native.HipUnavailable):
        qpd.copy_quantized_state(_cpu_pool(), ids, _cpu_pool(), ids)
    with pytest.raises(_native.HipUnavailable):
        qpd.reset_quantized_state(_cpu_pool(), ids)


def test_dst_indices_front_end_errors():
    B = 2
    c = dict(mixed_qkv=torch.zeros(B, 2 * H * K + HV * V), a=torch.zeros(B, HV), b=torch.zeros(B, HV),
             A_log=torch.zeros(HV), dt_bias=torch.zeros(HV), scale=1.0)
    pool = _cpu_pool()
    idx = torch.tensor([1, 2], dtype=torch.int32)
    out = torch.zeros(B, 1, HV, V)
    with pytest.raises(ValueError, match="dst_state_indices must be a 1-D int32"):
        qpd.quantized_gated_delta_rule_packed_decode(**c, state_codes=pool[0], state_scale=pool[1],
                                                     resid_codes=pool[2], resid_scale=pool[3], out=out,
                                                     ssm_state_indices=idx, resid_fmt=qpd.RESID_INT4,
                                                     dst_state_indices=idx.long())
    with pytest.raises(ValueError, match="at least B=2"):
        qpd.quantized_gated_delta_rule_packed_decode(**c, state_codes=pool[0], state_scale=pool[1],
                                                     resid_codes=pool[2], resid_scale=pool[3], out=out,
                                                     ssm_state_indices=idx, resid_fmt=qpd.RESID_INT4,
                                                     dst_state_indices=idx[:1])
    with pytest.raises(ValueError, match="quant_mode='fast'"):
        qpd.quantized_gated_delta_rule_packed_decode(**c, state_codes=pool[0], state_scale=pool[1],
                                                     resid_codes=pool[2], resid_scale=pool[3], out=out,
                                                     ssm_state_indices=idx, resid_fmt=qpd.RESID_INT4,
                                                     quant_mode="exact", dst_state_indices=idx)
    qpd._check_dst_indices_host(idx, torch.tensor([1, 2], dtype=torch.int32), 4)
    with pytest.raises(ValueError, match="duplicate"):
        qpd._check_dst_indices_host(idx, torch.tensor([3, 3], dtype=torch.int32), 4)
    with pytest.raises(ValueError, match="also read"):
        qpd._check_dst_indices_host(idx, torch.tensor([2, 3], dtype=torch.int32), 4)
