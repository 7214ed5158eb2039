"""GPU parity of the statequant-layout step (ck_gdn_quant_step, ck_gdn_fp32_step)
against the CPU oracle, following experiments/test_kernel.py and
experiments/test_cuda_kernel.py."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from carrykernel_amd.hip import binding
from carrykernel_amd.statequant import kernel as sq
from tests._helpers import rel

pytestmark = pytest.mark.gpu

MODES = {"fast": oracle.MODE_FAST, "exact": oracle.MODE_EXACT}


def make_inputs(T, B, HV, K, V, seed=0):
    """experiments/test_kernel.py:28-37: k L2-normalised, alpha 0.995, beta sigmoid(rand)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(T, B, HV, K, generator=g)
    k = torch.randn(T, B, HV, K, generator=g)
    k = k / k.norm(dim=-1, keepdim=True).clamp(min=1e-8)
    v = torch.randn(T, B, HV, V, generator=g)
    alpha = torch.full((T, B, HV), 0.995)
    beta = torch.rand(T, B, HV, generator=g).sigmoid()
    h0 = torch.randn(B, HV, K, V, generator=g) * 0.1
    return h0, q, k, v, alpha, beta


def _storage(e: torch.Tensor, res_fmt: int) -> np.ndarray:
    """Residual tensor -> the oracle's storage convention."""
    e = e.cpu()
    if res_fmt == sq.RES_FP16:
        return e.view(torch.int16).numpy().view(np.uint16)
    if res_fmt == sq.RES_FP8:
        return e.view(torch.uint8).numpy()
    return e.numpy()


def _random_state(B, HV, K, V, res_fmt, seed, bits=8):
    """A non-trivial state: quantized h0 plus a residual of realistic size."""
    g = torch.Generator().manual_seed(seed)
    h0 = torch.randn(B, HV, K, V, generator=g) * 0.1
    qmax = 2 ** (bits - 1) - 1
    codes, scale = oracle.quantize_cols(h0.numpy(), qmax)
    resid = torch.randn(B, HV, K, V, generator=g) * torch.from_numpy(scale)[:, :, None, :] * 0.3
    if res_fmt == sq.RES_INT8:
        es = (resid.abs().amax(dim=-2) / qmax).clamp(min=1e-12)
        e = torch.round(resid / es[:, :, None, :]).clamp(-qmax, qmax).to(torch.int8)
    else:
        e, es = resid.to(sq.residual_dtype(res_fmt)), None
    return torch.from_numpy(codes), torch.from_numpy(scale), e, es


@pytest.mark.parametrize("res_fmt", [sq.RES_FP32, sq.RES_FP16, sq.RES_FP8, sq.RES_INT8])
@pytest.mark.parametrize("mode", ["fast", "exact"])
@pytest.mark.parametrize("K,V,B,HV", [(128, 128, 2, 32), (64, 64, 1, 4), (32, 8, 1, 1), (16, 136, 2, 3),
                                     (256, 128, 1, 4), (128, 130, 1, 3), (256, 130, 2, 2), (16, 3, 2, 2),
                                     (64, 67, 1, 2), (16, 1, 3, 1), (48, 128, 2, 4), (100, 67, 1, 3),
                                     (7, 8, 2, 2), (200, 128, 1, 2), (1, 5, 2, 2)])
def test_step_bit_exact_vs_oracle(device, res_fmt, mode, K, V, B, HV):
    """K = 256 runs 16 slices of 16 rows; V not a multiple of 4 (130, 3, 67,
    and a single column) takes the per-column access path with a partial last
    column group. K = 48, 100, 7, 200, 1: rows zero-padded to 64, 128, 16,
    256, 16 (the oracle pads the same way)."""
    h_int8, scale, e, es = _random_state(B, HV, K, V, res_fmt, seed=K + V + res_fmt)
    _, q, k, v, alpha, beta = make_inputs(1, B, HV, K, V, seed=5)
    beta = beta[0] * 0 + torch.rand(B, HV, generator=torch.Generator().manual_seed(9))
    print(f"case K={K} V={V} B={B} HV={HV} res={res_fmt} mode={mode}", flush=True)
    got = sq.gdn_quant_step_fused(h_int8.to(device), scale.to(device), e.to(device),
                                  None if es is None else es.to(device), q[0].to(device), k[0].to(device),
                                  v[0].to(device), alpha[0].to(device), beta.to(device), bits=8,
                                  res_fmt=res_fmt, quant_mode=mode)
    torch.cuda.synchronize()
    ref = oracle.quant_step_kv(h_int8.numpy(), scale.numpy(), _storage(e, res_fmt),
                               None if es is None else es.numpy(), q[0].numpy(), k[0].numpy(), v[0].numpy(),
                               alpha[0].numpy(), beta.numpy(), bits=8, res_fmt=res_fmt, mode=MODES[mode])
    names = ("o", "h_int8", "scale", "e", "e_scale")
    for name, g_, r_ in zip(names, got, ref):
        if r_ is None:
            assert g_ is None
            continue
        g_np = _storage(g_, res_fmt) if name == "e" else g_.cpu().numpy()
        np.testing.assert_array_equal(g_np, r_, err_msg=f"{name} differs")


def test_int6_state_int8_residual(device):
    B, HV, K, V = 2, 8, 128, 128
    h_int8, scale, e, es = _random_state(B, HV, K, V, sq.RES_INT8, seed=3, bits=6)
    _, q, k, v, alpha, beta = make_inputs(1, B, HV, K, V, seed=6)
    got = sq.gdn_quant_step_fused(h_int8.to(device), scale.to(device), e.to(device), es.to(device),
                                  q[0].to(device), k[0].to(device), v[0].to(device), alpha[0].to(device),
                                  beta[0].to(device), bits=6, res_fmt=sq.RES_INT8)
    ref = oracle.quant_step_kv(h_int8.numpy(), scale.numpy(), e.numpy(), es.numpy(), q[0].numpy(), k[0].numpy(),
                               v[0].numpy(), alpha[0].numpy(), beta[0].numpy(), bits=6, res_fmt=sq.RES_INT8)
    for g_, r_ in zip(got, ref):
        np.testing.assert_array_equal(g_.cpu().numpy(), r_)
    assert int(got[1].abs().max()) <= 31 and int(got[3].abs().max()) <= 31


@pytest.mark.parametrize("K,V", [(128, 128), (32, 8), (256, 128), (256, 130), (64, 3), (48, 128), (100, 67),
                                 (200, 130), (3, 4)])
def test_fp32_step_bit_exact(device, K, V):
    h0, q, k, v, alpha, beta = make_inputs(1, 2, 4, K, V, seed=7)
    h_g, o_g = binding.gdn_fp32_step_hip(h0.to(device), q[0].to(device), k[0].to(device), v[0].to(device),
                                         alpha[0].to(device), beta[0].to(device))
    h_r, o_r = oracle.fp32_step_kv(h0.numpy(), q[0].numpy(), k[0].numpy(), v[0].numpy(), alpha[0].numpy(),
                                   beta[0].numpy())
    np.testing.assert_array_equal(h_g.cpu().numpy(), h_r)
    np.testing.assert_array_equal(o_g.cpu().numpy(), o_r)
    # and against the float64 recurrence (experiments/test_kernel.py:89-94 bound 1e-3)
    h64, o64 = oracle.gdn_step_f64(h0.numpy(), q[0].numpy(), k[0].numpy(), v[0].numpy(), alpha[0].numpy(),
                                   beta[0].numpy())
    assert np.abs(h_g.cpu().numpy() - h64).max() < 1e-3 and np.abs(o_g.cpu().numpy() - o64).max() < 1e-3


def _shifted(t: torch.Tensor) -> torch.Tensor:
    """A contiguous copy of t that starts one element into its allocation, so
    its address is not 16-byte aligned."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    out = buf[1:].view(t.shape)
    out.copy_(t)
    return out


@pytest.mark.parametrize("res_fmt", [sq.RES_FP32, sq.RES_FP16, sq.RES_FP8, sq.RES_INT8])
def test_step_unaligned_tensors(device, res_fmt):
    """V = 128 but every input starts one element past an aligned address:
    the host picks the per-column access path, which must match the oracle."""
    B, HV, K, V = 2, 3, 64, 128
    h_int8, scale, e, es = _random_state(B, HV, K, V, res_fmt, seed=40 + res_fmt)
    _, q, k, v, alpha, beta = make_inputs(1, B, HV, K, V, seed=11)
    args = [h_int8, scale, e, es, q[0], k[0], v[0], alpha[0], beta[0]]
    dev_args = [None if a is None else _shifted(a.to(device)) for a in args]
    assert all(a is None or a.data_ptr() % 16 for a in dev_args)
    print(f"case unaligned res={res_fmt}", flush=True)
    got = sq.gdn_quant_step_fused(*dev_args, bits=8, res_fmt=res_fmt)
    torch.cuda.synchronize()
    ref = oracle.quant_step_kv(h_int8.numpy(), scale.numpy(), _storage(e, res_fmt),
                               None if es is None else es.numpy(), q[0].numpy(), k[0].numpy(), v[0].numpy(),
                               alpha[0].numpy(), beta[0].numpy(), bits=8, res_fmt=res_fmt)
    for name, g_, r_ in zip(("o", "h_int8", "scale", "e", "e_scale"), got, ref):
        if r_ is not None:
            g_np = _storage(g_, res_fmt) if name == "e" else g_.cpu().numpy()
            np.testing.assert_array_equal(g_np, r_, err_msg=f"{name} differs")


@pytest.mark.parametrize("K", [16, 64, 128, 256])
@pytest.mark.parametrize("V", [4, 5])
def test_reduction_order_known_answer(device, K, V):
    """The closed forms that fix the K-sum order (the oracle's CPU test holds
    the derivation): beta = 0 and alpha = scale = 1 make o = sum over rows of
    code * q exactly per product. 2^24 at row 0 with 1 at rows R, R+1 of the
    next slice gives 2^24 + 2; 2^24 at row 0 with 1 at the first row of every
    other slice gives 2^24 + S - 2 (S slices of R rows: 8 up to K = 128, K/16
    at K = 256)."""
    S = 8 if K <= 128 else K // 16
    R = K // S
    big = 2.0 ** 24
    z = dict(device=device)
    for rows, want in (([(0, big), (R, 1.0), (R + 1, 1.0)], big + 2),
                       ([(0, big)] + [(s * R, 1.0) for s in range(1, S)], big + S - 2)):
        codes = torch.zeros(1, 1, K, V, dtype=torch.int8, **z)
        q = torch.zeros(1, 1, K, **z)
        for r, val in rows:
            codes[0, 0, r, :] = 1
            q[0, 0, r] = val
        for mode in ("fast", "exact"):
            o = sq.gdn_quant_step_fused(codes, torch.ones(1, 1, V, **z), torch.zeros(1, 1, K, V, **z), None, q,
                                        torch.zeros(1, 1, K, **z), torch.zeros(1, 1, V, **z),
                                        torch.ones(1, 1, **z), torch.zeros(1, 1, **z), quant_mode=mode)[0]
            assert torch.all(o.cpu() == want), (K, V, mode, o.cpu().ravel().tolist(), want)


def test_per_v_channel_quantize(device):
    x = torch.randn(3, 128, 128, generator=torch.Generator().manual_seed(1)) * 0.7
    codes, scale, deq = sq.per_v_channel_quantize(x.to(device), 8)
    c_ref, s_ref = oracle.quantize_cols(x.numpy(), 127.0)
    np.testing.assert_array_equal(codes.cpu().numpy(), c_ref)
    np.testing.assert_array_equal(scale.cpu().numpy(), s_ref)
    # statequant/quant.py:37-42 semantics with torch.round
    s_t = x.abs().amax(dim=-2, keepdim=True).clamp(min=1e-12) / 127
    np.testing.assert_array_equal(codes.cpu().numpy(), torch.round(x / s_t).clamp(-127, 127).numpy())
    assert torch.equal(deq.cpu(), codes.cpu().float() * scale.cpu()[..., None, :])


def test_round_half_to_even(device):
    """experiments/test_cuda_kernel.py:64-118: alpha=beta=0 so target == e; codes
    (arange%8)-3.5 with row 0 pinned at qmax make exact .5 ties at scale 1.0."""
    B, HV, K, V = 1, 1, 32, 8
    qmax = 127.0
    codes = (torch.arange(K, dtype=torch.float32) % 8) - 3.5
    target = codes[:, None].repeat(1, V).contiguous()
    target[0, :] = qmax
    scale = target.abs().amax(dim=0).clamp(min=1e-12) / qmax
    assert torch.all(scale == 1.0)
    expected = torch.round(target / scale[None, :]).clamp(-qmax, qmax)
    assert int(((target.abs() % 1.0) == 0.5).sum()) > 0
    assert int((torch.floor(target + 0.5) != expected).sum()) > 0
    z = dict(device=device)
    for mode in ("fast", "exact"):
        _, h_out, s_out, _, _ = binding.gdn_quant_step_hip(
            torch.zeros(B, HV, K, V, dtype=torch.int8, **z), torch.ones(B, HV, V, **z),
            target[None, None].to(device), None, torch.zeros(B, HV, K, **z), torch.zeros(B, HV, K, **z),
            torch.zeros(B, HV, V, **z), torch.zeros(B, HV, **z), torch.zeros(B, HV, **z), 8, sq.RES_FP32,
            quant_mode=mode)
        assert torch.equal(h_out[0, 0].float().cpu(), expected), mode
        assert torch.all(s_out.cpu() == 1.0)


def _oracle_decode_f64(h0, q, k, v, alpha, beta, bits=8):
    """experiments/test_kernel.py:40-55: float64 recurrence + ErrorFeedback with
    an fp32-precision residual and per-V-column quantization (amax over K)."""
    qmax = 2 ** (bits - 1) - 1

    def per_v(x):
        s = np.maximum(np.abs(x).max(axis=-2, keepdims=True), 1e-12) / qmax
        return np.clip(np.round(x / s), -qmax, qmax) * s

    h = per_v(h0.numpy().astype(np.float64))
    e = np.zeros_like(h)
    os_ = []
    for t in range(q.shape[0]):
        h, o = oracle.gdn_step_f64(h, q[t].numpy(), k[t].numpy(), v[t].numpy(), alpha[t].numpy(), beta[t].numpy())
        target = h + e
        h = per_v(target)
        e = target - h
        os_.append(o)
    return np.stack(os_), h


@pytest.mark.parametrize("res_fmt,bound", [(sq.RES_FP32, 5e-3), (sq.RES_FP16, 5e-3), (sq.RES_FP8, 1.5e-1),
                                           (sq.RES_INT8, 1.5e-1)])
def test_decode_vs_oracle(device, res_fmt, bound):
    """experiments/test_cuda_kernel.py:158-190 bounds: T=64, B=1, HV=32, K=V=128."""
    T, B, HV, K, V = 64, 1, 32, 128, 128
    h0, q, k, v, alpha, beta = make_inputs(T, B, HV, K, V)
    o_g, h_g, s_g, _, _ = binding.gdn_quant_decode_hip(h0.to(device), q.to(device), k.to(device), v.to(device),
                                                       alpha.to(device), beta.to(device), T, 8, res_fmt)
    o_ref, h_ref = _oracle_decode_f64(h0, q, k, v, alpha, beta)
    h_deq = (h_g.float() * s_g[..., None, :]).cpu().numpy()
    o_rel, h_rel = rel(o_g.cpu().numpy(), o_ref), rel(h_deq, h_ref)
    print(f"res_fmt={res_fmt}: o rel={o_rel:.3e} h rel={h_rel:.3e}")
    assert o_rel < bound and h_rel < bound


def test_batch8_step(device):
    """experiments/test_cuda_kernel.py:230-233: batch-8 coverage."""
    h0, q, k, v, alpha, beta = make_inputs(1, 8, 32, 128, 128, seed=1)
    h_int8, scale, e, es = sq.init_quant_state(h0.to(device), 8, sq.RES_INT8)
    got = sq.gdn_quant_step_fused(h_int8, scale, e, es, q[0].to(device), k[0].to(device), v[0].to(device),
                                  alpha[0].to(device), beta[0].to(device), 8, sq.RES_INT8)
    ref = oracle.quant_step_kv(h_int8.cpu().numpy(), scale.cpu().numpy(), e.cpu().numpy(), es.cpu().numpy(),
                               q[0].numpy(), k[0].numpy(), v[0].numpy(), alpha[0].numpy(), beta[0].numpy(),
                               res_fmt=sq.RES_INT8)
    for g_, r_ in zip(got, ref):
        np.testing.assert_array_equal(g_.cpu().numpy(), r_)


@pytest.mark.parametrize("K", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("V", [4, 36, 200, 7])
def test_per_v_channel_quantize_shapes_and_ties(device, K, V):
    """Every K of the vectorised column kernel, V below and above one
    workgroup's 128 columns and not a multiple of 32 (idle lanes), and V = 7
    (the general kernel); column 0 holds exact .5 ties at scale 1.0 (amax 127),
    which round to even as torch.round does."""
    g = torch.Generator().manual_seed(K * 1000 + V)
    x = torch.randn(5, K, V, generator=g) * 0.7
    ties = torch.tensor([2.5, -3.5, 0.5, -0.5, 1.5, 126.5])
    x[:, :len(ties), 0] = ties
    x[:, len(ties), 0] = 127.0
    x[:, len(ties) + 1:, 0] = 0.25
    print(f"case per_v_channel_quantize K={K} V={V}", flush=True)
    codes, scale, _ = sq.per_v_channel_quantize(x.to(device), 8)
    torch.cuda.synchronize()
    c_ref, s_ref = oracle.quantize_cols(x.numpy(), 127.0)
    np.testing.assert_array_equal(codes.cpu().numpy(), c_ref)
    np.testing.assert_array_equal(scale.cpu().numpy(), s_ref)
    assert torch.all(scale.cpu()[:, 0] == 1.0)
    assert codes.cpu()[0, :len(ties), 0].tolist() == [2, -4, 0, 0, 2, 126]


@pytest.mark.parametrize("res_fmt", [sq.RES_FP32, sq.RES_INT8])
def test_native_module_boundary(device, res_fmt):
    """The extension module's launchers (cuda/gdn_state_kernel.cu:310-371) as
    binding.load_extension() exposes them: outputs owned by the caller, bytes
    equal to the wrapper's, TORCH_CHECK failures as RuntimeError."""
    B, HV, K, V = 2, 4, 32, 64
    codes, scale, e, es = _random_state(B, HV, K, V, res_fmt, seed=21)
    _, q, k, v, alpha, beta = make_inputs(1, B, HV, K, V, seed=22)
    d = [t.to(device) if t is not None else None for t in (codes, scale, e, es, q[0], k[0], v[0], alpha[0], beta[0])]
    want = binding.gdn_quant_step_hip(*d, 8, res_fmt)
    ext = binding.load_extension()
    es_in = d[3] if d[3] is not None else torch.zeros(B, HV, V, device=device)
    outs = (torch.empty(B, HV, V, device=device), torch.empty(B, HV, K, V, dtype=torch.int8, device=device),
            torch.empty(B, HV, V, device=device), torch.empty_like(d[2]), torch.empty(B, HV, V, device=device))
    ext.gdn_quant_step(d[0], d[1], d[2], es_in, *d[4:], *outs, 127.0, res_fmt, 128)
    torch.cuda.synchronize()
    for got, ref in zip(outs, want):
        if ref is not None:
            assert torch.equal(got.view(torch.uint8) if got.dtype == torch.int8 else got,
                               ref.view(torch.uint8) if ref.dtype == torch.int8 else ref)
    with pytest.raises(RuntimeError, match="block_v must be in"):
        ext.gdn_quant_step(d[0], d[1], d[2], es_in, *d[4:], *outs, 127.0, res_fmt, 0)
    with pytest.raises(RuntimeError, match="h_in must be int8"):
        ext.gdn_quant_step(d[1], d[1], d[2], es_in, *d[4:], *outs, 127.0, res_fmt, 128)
    with pytest.raises(RuntimeError, match="q must be"):
        ext.gdn_quant_step(d[0], d[1], d[2], es_in, d[4][:1], *d[5:], *outs, 127.0, res_fmt, 128)
    with pytest.raises(RuntimeError, match="unknown res_fmt"):
        ext.gdn_quant_step(d[0], d[1], d[2], es_in, *d[4:], *outs, 127.0, 9, 128)
    h32 = torch.randn(B, HV, K, V, device=device)
    o, h_out = torch.empty(B, HV, V, device=device), torch.empty_like(h32)
    ext.gdn_fp32_step(h32, *d[4:], o, h_out, 128)
    ref_h, ref_o = binding.gdn_fp32_step_hip(h32, *d[4:])
    torch.cuda.synchronize()
    assert torch.equal(h_out, ref_h) and torch.equal(o, ref_o)
    with pytest.raises(RuntimeError, match="h_in must be fp32"):
        ext.gdn_fp32_step(d[0], *d[4:], o, h_out, 128)


@pytest.mark.parametrize("res_fmt", [sq.RES_FP32, sq.RES_INT8])
def test_empty_batch(device, res_fmt):
    """B = 0: the fused step (front end and binding) and the fp32 step return
    empty outputs of the right shapes without launching anything."""
    HV, K, V = 4, 32, 64
    codes = torch.zeros(0, HV, K, V, dtype=torch.int8, device=device)
    scale = torch.zeros(0, HV, V, device=device)
    e = torch.zeros(0, HV, K, V, dtype=sq.residual_dtype(res_fmt), device=device)
    es = torch.zeros(0, HV, V, device=device) if res_fmt == sq.RES_INT8 else None
    q, k = torch.zeros(0, HV, K, device=device), torch.zeros(0, HV, K, device=device)
    v = torch.zeros(0, HV, V, device=device)
    alpha, beta = torch.zeros(0, HV, device=device), torch.zeros(0, HV, device=device)
    for step in (sq.gdn_quant_step_fused, binding.gdn_quant_step_hip):
        o, h, s, e_new, es_new = step(codes, scale, e, es, q, k, v, alpha, beta, 8, res_fmt)
        assert o.shape == (0, HV, V) and s.shape == (0, HV, V)
        assert h.shape == (0, HV, K, V) and h.dtype == torch.int8
        assert e_new.shape == (0, HV, K, V) and e_new.dtype == e.dtype
        assert (es_new is None) == (res_fmt != sq.RES_INT8)
    h_out, o = sq.gdn_step_fused_fp32(torch.zeros(0, HV, K, V, device=device), q, k, v, alpha, beta)
    assert h_out.shape == (0, HV, K, V) and o.shape == (0, HV, V)
    torch.cuda.synchronize()
