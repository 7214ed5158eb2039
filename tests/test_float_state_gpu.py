"""GPU parity of the unquantized-state packed decode (the fp32 / bf16 comparison
arm, ck_gdn_packed_decode_float_state) against the CPU oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from carrykernel_amd import _native
from tests._helpers import make_packed_inputs

pytestmark = pytest.mark.gpu


def _run(device, state, mixed, a, b, A_log, dt_bias, idx, out, H, l2norm, scale):
    st = state.dtype
    L = _native.lib()
    S, HV, V, K = state.shape
    rc = L.ck_gdn_packed_decode_float_state(
        mixed.data_ptr(), 0, mixed.stride(0), a.data_ptr(), 0, a.stride(0), b.data_ptr(), 0, b.stride(0),
        A_log.data_ptr(), 0, dt_bias.data_ptr(), 0, scale, state.data_ptr(), 0 if st == torch.float32 else 1,
        state.stride(0), out.data_ptr(), 0, idx.data_ptr(), 1, S, mixed.shape[0], H, HV, K, V, int(l2norm),
        _native.stream_handle(device))
    _native.check(rc, "float_state")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("K,V,H,HV", [(128, 128, 16, 32), (64, 64, 8, 16)])
def test_float_state_bit_exact(device, dtype, K, V, H, HV):
    B, S = 3, 6
    g = torch.Generator().manual_seed(K)
    state = (torch.randn(S, HV, V, K, generator=g) * 0.1).to(dtype)
    idx = torch.tensor([4, 0, 2], dtype=torch.int32)
    ref_state = state.float().numpy().copy()
    for t in range(2):
        mixed, a, b, A_log, dt_bias = make_packed_inputs(B, H, HV, K, V, seed=20 + t)
        out = torch.empty(B, 1, HV, V, device=device)
        dstate = state.to(device)
        _run(device, dstate, mixed.to(device), a.to(device), b.to(device), A_log.to(device), dt_bias.to(device),
             idx.to(device), out, H, True, K ** -0.5)
        torch.cuda.synchronize()
        o_ref = oracle.packed_decode_float_state(mixed.numpy(), a.numpy(), b.numpy(), A_log.numpy(),
                                                 dt_bias.numpy(), K ** -0.5, ref_state, idx.numpy(), H,
                                                 bf16=dtype == torch.bfloat16, use_qk_l2norm=True)
        np.testing.assert_array_equal(out[:, 0].cpu().numpy(), o_ref)
        state = dstate.cpu()
        np.testing.assert_array_equal(state.float().numpy(), ref_state)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("K,V,H,HV,B", [(16, 40, 2, 4, 5), (256, 100, 2, 2, 3), (128, 128, 4, 8, 300)])
def test_float_state_shapes_and_persistence(device, dtype, K, V, H, HV, B):
    """Tiles past V, K at both ends of the range, and a batch large enough
    that every workgroup loops over several items; one NULL and one
    out-of-range id (NaN out, state untouched)."""
    S = B + 2
    g = torch.Generator().manual_seed(K + V + B)
    state = (torch.randn(S, HV, V, K, generator=g) * 0.1).to(dtype)
    rng = np.random.default_rng(B)
    idx = (rng.permutation(S - 1)[:B] + 1).astype(np.int32)
    idx[0] = 0
    idx[-1] = S   # out of range
    ref_state = state.float().numpy().copy()
    mixed, a, b, A_log, dt_bias = make_packed_inputs(B, H, HV, K, V, seed=B)
    out = torch.empty(B, 1, HV, V, device=device)
    dstate = state.to(device)
    print(f"case float state {dtype} K={K} V={V} B={B}", flush=True)
    _run(device, dstate, mixed.to(device), a.to(device), b.to(device), A_log.to(device), dt_bias.to(device),
         torch.from_numpy(idx).to(device), out, H, True, K ** -0.5)
    torch.cuda.synchronize()
    idx_o = idx.copy()
    idx_o[-1] = 0   # the oracle treats it as NULL; the kernel writes NaN
    o_ref = oracle.packed_decode_float_state(mixed.numpy(), a.numpy(), b.numpy(), A_log.numpy(), dt_bias.numpy(),
                                             K ** -0.5, ref_state, idx_o, H, bf16=dtype == torch.bfloat16,
                                             use_qk_l2norm=True)
    got = out[:, 0].cpu().numpy()
    np.testing.assert_array_equal(got[:-1], o_ref[:-1])
    assert np.all(np.isnan(got[-1])) and np.all(got[0] == 0)
    np.testing.assert_array_equal(dstate.cpu().float().numpy(), ref_state)


def test_float_state_bf16_activations(device, K=128, V=128, H=8, HV=16):
    B, S = 4, 7
    g = torch.Generator().manual_seed(1)
    state = (torch.randn(S, HV, V, K, generator=g) * 0.1).to(torch.bfloat16)
    idx = torch.tensor([6, 2, 0, 4], dtype=torch.int32)
    ref_state = state.float().numpy().copy()
    mixed, a, b, A_log, dt_bias = make_packed_inputs(B, H, HV, K, V, seed=77, dtype=torch.bfloat16)
    out = torch.empty(B, 1, HV, V, device=device)
    dstate = state.to(device)
    L = _native.lib()
    dm, da, db, dA, ddt, didx = (x.to(device) for x in (mixed, a, b, A_log, dt_bias, idx))  # kept alive
    rc = L.ck_gdn_packed_decode_float_state(
        dm.data_ptr(), 1, dm.stride(0), da.data_ptr(), 1, da.stride(0), db.data_ptr(), 1, db.stride(0),
        dA.data_ptr(), 1, ddt.data_ptr(), 1, K ** -0.5, dstate.data_ptr(), 1, dstate.stride(0), out.data_ptr(), 0,
        didx.data_ptr(), 1, S, B, H, HV, K, V, 1, _native.stream_handle(device))
    torch.cuda.synchronize()
    _native.check(rc, "float_state")
    o_ref = oracle.packed_decode_float_state(mixed.float().numpy(), a.float().numpy(), b.float().numpy(),
                                             A_log.float().numpy(), dt_bias.float().numpy(), K ** -0.5, ref_state,
                                             idx.numpy(), H, bf16=True, use_qk_l2norm=True)
    np.testing.assert_array_equal(out[:, 0].cpu().numpy(), o_ref)
    np.testing.assert_array_equal(dstate.cpu().float().numpy(), ref_state)
