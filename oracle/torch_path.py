"""The reference's CPU path, restated in PyTorch for the vLLM layout.

TEST INFRASTRUCTURE ONLY (like the rest of ``oracle/``): used by ``tests/`` as
an independent cross-check of the C oracle and by ``bench.py``'s CPU-baseline
leg as the CPU path that is timed beside the GPU. The product never imports it.

``packed_decode_torch`` is one decode step with the arithmetic of
``gdn_quant_step_torch`` (statequant/kernel.py:149-178): dequantize as
``codes.float() * scale``, decay by a separate multiply, ``torch.einsum`` for the
three K-reductions (in whatever order torch's CPU kernels sum), ``h + k dv`` as
a rounded product then a rounded add, IEEE division by the new scale and
``torch.round`` (half to even), and the residual ``target - codes * scale``.
Around it sit the vLLM-layout parts of
vllm_integration/quantized_packed_decode.py: the slot gather and NULL block
(:129-136), q/k/v unpacking with GQA (:121,160-167), the optional L2 norm and
q scale (:169-172), the gates (:174-182), the per-V-row residual
(:195-215; per-head scale as configs C2/C3 define it), the int4 nibble layout
(:196-199, :221-237) and the in-place stores. Scales are
``max(amax / qmax, 1e-12)`` as the kernels compute them (:206, :213).
"""

from __future__ import annotations

import torch

EPS = 1e-12
SOFTPLUS_THRESHOLD = 20.0
RESID_INT8 = 0
RESID_INT4 = 1


def unpack_int4_torch(packed: torch.Tensor) -> torch.Tensor:
    """[..., K/2] int8 bytes -> [..., K] int32 codes: even K in the low nibble,
    odd K in the high one, nibbles above 7 are negative (qpd:196-199)."""
    p = packed.to(torch.int32) & 0xFF
    lo = p & 0xF
    hi = (p >> 4) & 0xF
    lo = torch.where(lo > 7, lo - 16, lo)
    hi = torch.where(hi > 7, hi - 16, hi)
    return torch.stack([lo, hi], dim=-1).reshape(*p.shape[:-1], 2 * p.shape[-1])


def pack_int4_torch(codes: torch.Tensor) -> torch.Tensor:
    """[..., K] integer codes in -7..7 -> [..., K/2] int8 bytes (qpd:226-237)."""
    c = codes.to(torch.int32) & 0xF
    return (c[..., 0::2] | (c[..., 1::2] << 4)).to(torch.uint8).view(torch.int8)


def gates_torch(a, b, A_log, dt_bias):
    """alpha = exp(-exp(A_log) * softplus(a + dt_bias)), beta = sigmoid(b)
    (qpd:174-182), in fp32 with torch's CPU exp / log."""
    x = a.float() + dt_bias.float()
    sp = torch.where(x <= SOFTPLUS_THRESHOLD, torch.log(1.0 + torch.exp(x)), x)
    g = -torch.exp(A_log.float()) * sp
    return torch.exp(g), torch.sigmoid(b.float())


def packed_decode_torch(mixed_qkv, a, b, A_log, dt_bias, scale,
                        state_codes, state_scale, resid_codes, resid_scale,
                        indices, H, *, use_qk_l2norm=False, resid_fmt=RESID_INT8,
                        per_head=False, state_bits=8, gates=None):
    """One step on CPU tensors, updating the four pool tensors in place.

    ``gates`` (optional): precomputed ``(alpha, beta)`` of shape [B, HV], used
    instead of ``gates_torch`` so that a comparison can isolate the step's
    arithmetic. Returns ``out [B, HV, V]`` fp32 (zeros for NULL-block ids,
    NaN for ids at or past the pool size).
    """
    B = mixed_qkv.shape[0]
    S, HV, V, K = state_codes.shape
    mixed = mixed_qkv.float()
    q = mixed[:, :H * K].reshape(B, H, K)
    k = mixed[:, H * K:2 * H * K].reshape(B, H, K)
    v = mixed[:, 2 * H * K:2 * H * K + HV * V].reshape(B, HV, V)
    if use_qk_l2norm:
        q = q / torch.sqrt((q * q).sum(-1, keepdim=True) + 1e-6)
        k = k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    q = q * scale
    rep = HV // H
    q = q.repeat_interleave(rep, dim=1)
    k = k.repeat_interleave(rep, dim=1)
    alpha, beta = gates if gates is not None else gates_torch(a, b, A_log, dt_bias)

    slots = indices.to(torch.int64)
    out = torch.zeros(B, HV, V, dtype=torch.float32)
    out[slots >= S] = float("nan")
    live = (slots > 0) & (slots < S)
    if not bool(live.any()):
        return out
    ls = slots[live]
    qmax = float(2 ** (state_bits - 1) - 1)
    qmax_e = 7.0 if resid_fmt == RESID_INT4 else 127.0

    h = state_codes[ls].float() * state_scale[ls][..., None]          # [n, HV, V, K]
    h = alpha[live][..., None, None] * h
    read = torch.einsum("nhvk,nhk->nhv", h, k[live])
    dv = beta[live][..., None] * (v[live] - read)
    h = h + torch.einsum("nhv,nhk->nhvk", dv, k[live])
    out[live] = torch.einsum("nhvk,nhk->nhv", h, q[live])

    if resid_fmt == RESID_INT4:
        ecodes = unpack_int4_torch(resid_codes[ls]).float()
    else:
        ecodes = resid_codes[ls].float()
    rs = resid_scale[ls]
    e = ecodes * (rs[..., None, None] if per_head else rs[..., None])
    target = h + e

    s_new = (target.abs().amax(dim=-1) / qmax).clamp(min=EPS)          # [n, HV, V]
    codes = torch.round(target / s_new[..., None]).clamp(-qmax, qmax)
    e_new = target - codes * s_new[..., None]
    if per_head:
        es = (e_new.abs().amax(dim=(-2, -1)) / qmax_e).clamp(min=EPS)  # [n, HV]
        ec = torch.round(e_new / es[..., None, None]).clamp(-qmax_e, qmax_e)
    else:
        es = (e_new.abs().amax(dim=-1) / qmax_e).clamp(min=EPS)        # [n, HV, V]
        ec = torch.round(e_new / es[..., None]).clamp(-qmax_e, qmax_e)

    state_codes[ls] = codes.to(torch.int8)
    state_scale[ls] = s_new
    resid_codes[ls] = pack_int4_torch(ec) if resid_fmt == RESID_INT4 else ec.to(torch.int8)
    resid_scale[ls] = es
    return out
