"""GPU parity of the state ingest (init_quantized_state seeding through
ck_quantize_rows) against the CPU oracle: fp32, bf16, fp16 and float64
prefill states quantized in their own precision, int8 and int6 code ranges,
all-zero rows, rows with one dominant value, tiny magnitudes and fp16 scales
that are subnormal or round to zero."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd

pytestmark = pytest.mark.gpu


DTYPE_NAMES = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16",
               torch.float64: "float64"}


def _h0_cases(S, HV, V, K, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    h0 = torch.randn(S, HV, V, K, generator=g, dtype=torch.float64) * 0.3
    h0[1, 2, 3] = 0.0                       # all-zero row: scale = eps / qmax (0 in fp16), codes 0
    h0[2, 0, 5, 17] = 40.0                  # one dominant value
    h0[3, 1, :, ::2] *= 1e-30               # tiny and subnormal magnitudes
    if dtype == torch.float16:
        h0[0, 3] *= 1e-2                    # rows whose fp16 scale is subnormal
        h0[4, 0] *= 1e-6                    # fp16 scale rounds to 0 under nonzero values: +-qmax
    return h0.to(dtype)


def _reference_formula(h0, qmax):
    """quantized_packed_decode.py:347-351 evaluated by torch on the CPU in h0's
    own dtype (with the configurable qmax of state_bits)."""
    scale = h0.abs().amax(dim=-1).clamp(min=1e-12) / qmax
    codes = torch.round(h0 / scale[..., None]).clamp(-qmax, qmax)
    return codes.to(torch.int8).numpy(), scale.float().numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
@pytest.mark.parametrize("bits", [8, 6])
def test_init_quantized_state_matches_oracle(device, dtype, bits, S=5, HV=4, V=24, K=128):
    """The pool seeded from h0 in h0's own precision equals the oracle's
    in-dtype restatement and the reference's torch expression evaluated in
    that dtype, bit for bit: codes and scales."""
    h0 = _h0_cases(S, HV, V, K, dtype, bits)
    qmax = 2 ** (bits - 1) - 1
    print(f"case ingest {dtype} bits={bits}", flush=True)
    sc, ss, rc, rs = qpd.init_quantized_state(S, HV, V, K, device, h0=h0.to(device), resid_fmt=qpd.RESID_INT4,
                                              per_head_resid_scale=True, state_bits=bits)
    torch.cuda.synchronize()
    c_ref, s_ref = oracle.quantize_rows_in_dtype(h0.double().numpy() if dtype == torch.float64
                                                 else h0.float().numpy(), DTYPE_NAMES[dtype], float(qmax))
    np.testing.assert_array_equal(sc.cpu().numpy(), c_ref)
    np.testing.assert_array_equal(ss.cpu().numpy(), s_ref)
    assert torch.all(rc == 0) and torch.all(rs == 0)
    assert rs.shape == (S, HV) and rc.shape == (S, HV, V, K // 2)
    c_t, s_t = _reference_formula(h0, qmax)
    np.testing.assert_array_equal(ss.cpu().numpy(), s_t)
    np.testing.assert_array_equal(sc.cpu().numpy(), c_t)


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


@pytest.mark.parametrize("K", [16, 32, 64, 256, 48, 7])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_init_quantized_state_every_k(device, K, dtype, S=3, HV=2, V=9):
    """Every decode K through the vectorised row kernel, with a row count
    (S * HV * V = 54) that leaves the last wave's row group partly empty, and
    two K (48, 7) that take the general row kernel; in h0's precision."""
    g = torch.Generator().manual_seed(K)
    h0 = (torch.randn(S, HV, V, K, generator=g) * 0.2).to(dtype)
    h0[0, 1, 2] = 0.0
    print(f"case ingest K={K} {dtype}", flush=True)
    sc, ss, _, _ = qpd.init_quantized_state(S, HV, V, K, device, h0=h0.to(device), resid_fmt=qpd.RESID_INT8)
    torch.cuda.synchronize()
    c_ref, s_ref = oracle.quantize_rows_in_dtype(h0.float().numpy(), DTYPE_NAMES[dtype], 127.0)
    np.testing.assert_array_equal(sc.cpu().numpy(), c_ref)
    np.testing.assert_array_equal(ss.cpu().numpy(), s_ref)


@pytest.mark.parametrize("offset", [0, 1])
def test_quantize_rows_padded_and_unaligned_rows(device, offset, rows=37, K=128):
    """ck_quantize_rows through the C ABI on rows with padding between them:
    16-byte aligned rows take the vectorised kernel, rows starting one fp32
    element (4 bytes) off alignment the general one; both give the oracle's
    codes and scales."""
    from carrykernel_amd import _native
    L = _native.lib()
    g = torch.Generator().manual_seed(offset)
    pitch = K + 12                                   # elements between row starts
    back = torch.randn(rows * pitch + offset + 16, generator=g).to(device)
    x = back[offset:offset + rows * pitch].view(rows, pitch)
    codes = torch.full((rows, K), 99, dtype=torch.int8, device=device)
    scale = torch.empty(rows, device=device)
    print(f"case quantize_rows offset={offset}", flush=True)
    st = L.ck_quantize_rows(x.data_ptr(), 0, pitch, rows, K, 127.0, codes.data_ptr(), scale.data_ptr(),
                            _native.stream_handle(device))
    _native.check(st, "ck_quantize_rows")
    torch.cuda.synchronize()
    c_ref, s_ref = oracle.quantize_rows(np.ascontiguousarray(x[:, :K].cpu().numpy()), 127.0)
    np.testing.assert_array_equal(codes.cpu().numpy(), c_ref)
    np.testing.assert_array_equal(scale.cpu().numpy(), s_ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
def test_init_from_host_and_float64_prefill_state(device, dtype, S=3, HV=2, V=16, K=128):
    """An h0 on the host seeds the pool like the same tensor on the GPU (the
    reference accepts any device, quantized_packed_decode.py:347-351), each
    in its own precision: float64 in float64 arithmetic with its scale
    rounded to fp32, which differs from quantizing the fp32-rounded values."""
    g = torch.Generator().manual_seed(7)
    h0 = (torch.randn(S, HV, V, K, generator=g, dtype=torch.float64) * 0.2).to(dtype)
    print(f"case ingest host h0 {dtype}", flush=True)
    a = qpd.init_quantized_state(S, HV, V, K, device, h0=h0, resid_fmt=qpd.RESID_INT4)
    b = qpd.init_quantized_state(S, HV, V, K, device, h0=h0.to(device), resid_fmt=qpd.RESID_INT4)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    vals = h0.numpy() if dtype == torch.float64 else h0.float().numpy()
    c_ref, s_ref = oracle.quantize_rows_in_dtype(vals, DTYPE_NAMES[dtype], 127.0)
    np.testing.assert_array_equal(a[0].cpu().numpy(), c_ref)
    np.testing.assert_array_equal(a[1].cpu().numpy(), s_ref)
    c_t, s_t = _reference_formula(h0, 127)
    np.testing.assert_array_equal(a[0].cpu().numpy(), c_t)
    np.testing.assert_array_equal(a[1].cpu().numpy(), s_t)
