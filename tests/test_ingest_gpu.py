"""GPU parity of the state ingest (init_quantized_state seeding through
ck_quantize_rows) against the CPU oracle: fp32, bf16 and fp16 prefill states,
int8 and int6 code ranges, all-zero rows and rows with one dominant value."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bits", [8, 6])
def test_init_quantized_state_matches_oracle(device, dtype, bits, S=5, HV=4, V=24, K=128):
    g = torch.Generator().manual_seed(bits)
    h0 = torch.randn(S, HV, V, K, generator=g) * 0.3
    h0[1, 2, 3] = 0.0                       # all-zero row: scale = eps / qmax, codes 0
    h0[2, 0, 5, 17] = 40.0                  # one dominant value
    h0[3, 1, :, ::2] *= 1e-30               # tiny and subnormal magnitudes
    h0 = h0.to(dtype)
    print(f"case ingest {dtype} bits={bits}", flush=True)
    sc, ss, rc, rs = qpd.init_quantized_state(S, HV, V, K, device, h0=h0.to(device), resid_fmt=qpd.RESID_INT4,
                                              per_head_resid_scale=True, state_bits=bits)
    torch.cuda.synchronize()
    c_ref, s_ref = oracle.quantize_rows(h0.float().numpy(), float(2 ** (bits - 1) - 1))
    np.testing.assert_array_equal(sc.cpu().numpy(), c_ref)
    np.testing.assert_array_equal(ss.cpu().numpy(), s_ref)
    assert torch.all(rc == 0) and torch.all(rs == 0)
    assert rs.shape == (S, HV) and rc.shape == (S, HV, V, K // 2)
    # quantized_packed_decode.py:347-351: clamp(amax, eps) / qmax, torch.round
    qmax = 2 ** (bits - 1) - 1
    x = h0.float()
    s_t = x.abs().amax(dim=-1).clamp(min=1e-12) / qmax
    np.testing.assert_array_equal(ss.cpu().numpy(), s_t.numpy())
    np.testing.assert_array_equal(sc.cpu().numpy(),
                                  torch.round(x / s_t[..., None]).clamp(-qmax, qmax).to(torch.int8).numpy())


def test_init_from_strided_prefill_state(device, S=3, HV=2, V=16, K=64):
    """A non-contiguous h0 (a view) is seeded like its contiguous copy."""
    g = torch.Generator().manual_seed(4)
    big = torch.randn(S, HV, V, 2 * K, generator=g).to(device)
    h0 = big[..., ::2]
    assert not h0.is_contiguous()
    a = qpd.init_quantized_state(S, HV, V, K, device, h0=h0)
    b = qpd.init_quantized_state(S, HV, V, K, device, h0=h0.contiguous())
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)
