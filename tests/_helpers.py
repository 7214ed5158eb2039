"""Shared input builders for the tests (seeded on the CPU, so the GPU and the
oracle see the same values)."""

from __future__ import annotations

import numpy as np
import torch

import oracle


def make_packed_inputs(B, H, HV, K, V, seed=0, dtype=torch.float32):
    """Packed [B, 2HK + HV V] activations and gates, as
    vllm_integration/test_quantized_packed_decode.py:38-51 builds them."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, K, generator=g)
    k = torch.randn(B, H, K, generator=g)
    v = torch.randn(B, HV, V, generator=g)
    mixed = torch.cat([q.reshape(B, -1), k.reshape(B, -1), v.reshape(B, -1)], dim=1).contiguous()
    a = torch.randn(B, HV, generator=g) * 0.5
    b = torch.randn(B, HV, generator=g)
    A_log = torch.randn(HV, generator=g) * 0.2
    dt_bias = torch.randn(HV, generator=g) * 0.1
    return mixed.to(dtype), a.to(dtype), b.to(dtype), A_log.to(dtype), dt_bias.to(dtype)


def make_pool(S, HV, V, K, resid_fmt, per_head, seed=0, h_scale=0.1, bits=8):
    """A non-trivial quantized pool on the host: state from quantizing
    h_scale * N(0,1) per V-row, residual codes uniform over the format's range
    with scales about half a state LSB."""
    rng = np.random.default_rng(seed)
    qmax = float(2 ** (bits - 1) - 1)
    h0 = (rng.standard_normal((S, HV, V, K)) * h_scale).astype(np.float32)
    sc, ss = oracle.quantize_rows(h0, qmax)
    if resid_fmt == oracle.RESID_INT4:
        codes = rng.integers(-7, 8, size=(S, HV, V, K))
        rc = oracle.pack_int4(codes)
        qe = 7.0
    else:
        rc = rng.integers(-127, 128, size=(S, HV, V, K)).astype(np.int8)
        qe = 127.0
    if per_head:
        rs = (ss.max(axis=-1) * 0.5 / qe).astype(np.float32)
    else:
        rs = (ss * 0.5 / qe * rng.uniform(0.5, 1.0, size=ss.shape)).astype(np.float32)
    return (np.ascontiguousarray(sc), np.ascontiguousarray(ss),
            np.ascontiguousarray(rc), np.ascontiguousarray(rs))


def to_dev(arrs, device):
    return [torch.from_numpy(np.array(x, copy=True)).to(device) for x in arrs]


def rel(x, y):
    x = np.asarray(x, np.float64)
    y = np.asarray(y, np.float64)
    return float(np.linalg.norm(x - y) / (np.linalg.norm(y) + 1e-12))
