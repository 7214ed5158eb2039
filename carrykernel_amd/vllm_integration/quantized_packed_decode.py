"""INT8 + error-feedback recurrent state for vLLM's GDN packed decode, on MI355X.

Drop-in for ``vllm_integration/quantized_packed_decode.py`` of
tomalmog/carrykernel: same public names, constants, call signature, argument
meaning, in-place semantics and ``ValueError`` messages
(quantized_packed_decode.py:73-83, :242-369). The device work is a
hand-written gfx950 HIP kernel reached through the C ABI in
``include/carrykernel_gdn.h`` (``ck_gdn_packed_decode``).

State pool per slot, per value-head (vLLM's ``[num_slots, HV, V, K]``, K
contiguous):
  * ``state_codes`` int8 ``[S, HV, V, K]`` and ``state_scale`` fp32 ``[S, HV, V]``
  * ``resid_codes`` int8 ``[S, HV, V, K]`` (RESID_INT8) or packed nibbles
    ``[S, HV, V, K/2]`` (RESID_INT4, even K in the low nibble)
  * ``resid_scale`` fp32 ``[S, HV, V]`` (one scale per V-row, the reference's
    layout) or ``[S, HV]`` (one scale per head; the per-head residual scale of
    the benchmark's configs 2 and 3). The shape selects the mode.

Per step (one launch): dequantize, decay, delta-rule rank-1 write, output
read, add the carried residual, requantize with round-half-to-even, store
codes, scales and residual in place. Slot ids <= 0 are ``NULL_BLOCK_ID``
padding: ``out`` gets zeros and no state is touched.

Differences from the reference, all additive:
  * ``state_bits`` (default 8) sets the state code range to
    +-(2^(bits-1) - 1) (int6 for the long-horizon config).
  * ``quant_mode="fast"`` (default) rounds ``t * (1/s)``; ``"exact"`` rounds
    the correctly rounded quotient ``t / s`` with op-by-op rounding.
  * Slot ids >= num_slots make the kernel emit NaN and skip the state, where
    the reference would access memory out of bounds.
  * ``dst_state_indices`` writes the updated state to other slots than the
    ones read (speculative-decode chains, decoding from a shared prefix slot).
  * ``copy_quantized_state`` / ``reset_quantized_state`` move or clear whole
    slots (codes, scales and the EF residual together), the cache operations
    the reference leaves to the engine (its "Stage B", CLAUDE.md:235-239).
  * Tensors must be on a GPU; there is no CPU fallback.
"""

from __future__ import annotations

import os

import torch

from .. import _native

QMAX_INT8 = 127.0
QMAX_INT4 = 7.0
EPS = 1e-12
SOFTPLUS_THRESHOLD = 20.0
NULL_BLOCK_ID = 0

RESID_INT8 = 0
RESID_INT4 = 1

HAS_HIP = _native.library_available()

# The reference takes any K (its BK = next_pow2(K) lanes are masked past K);
# here K up to 1024. Power-of-two K from 16 to 256 with 16-byte aligned pool
# rows run the bandwidth kernel, every other K or row alignment the masked
# kernel (rows padded to 512 or 1024 lanes above 256; a per-head residual
# scale there needs V <= 128 at K <= 512 and V <= 64 above).
MAX_K = 1024

_QUANT_MODES = {"fast": _native.QUANT_FAST, "exact": _native.QUANT_EXACT}

# CARRYKERNEL_DEBUG=1 adds host-side checks of ssm_state_indices (range and
# duplicate slot ids, which would race on the in-place update). They copy the
# indices to the host, so they synchronise the stream.
_DEBUG = os.environ.get("CARRYKERNEL_DEBUG", "0") not in ("", "0")


def _check_indices_host(ssm_state_indices: torch.Tensor, num_slots: int) -> None:
    ids = ssm_state_indices.detach().to("cpu").tolist()
    live = [i for i in ids if i > NULL_BLOCK_ID]
    if any(i >= num_slots for i in live):
        raise ValueError(f"ssm_state_indices has slot ids >= num_slots ({num_slots})")
    if len(set(live)) != len(live):
        raise ValueError("ssm_state_indices has duplicate slot ids (in-place update would race)")


def _slot_contiguous(t: torch.Tensor) -> bool:
    """Every dim but the slot dim is densely packed (row-major)."""
    return _dense_after_slot(t.shape, t.stride())


def _dense_after_slot(sh, st) -> bool:
    """_slot_contiguous on a tensor's shape and strides."""
    n = len(sh)
    # the usual dense layouts, without the general loop (this runs per call)
    if n == 4 and st[3] == 1 and st[2] == sh[3] and st[1] == sh[2] * sh[3]:
        return True
    if n == 3 and st[2] == 1 and st[1] == sh[2]:
        return True
    if n == 2 and st[1] == 1:
        return True
    expect = 1
    for i in range(n - 1, 0, -1):
        if sh[i] != 1 and st[i] != expect:
            return False
        expect *= sh[i]
    return True


def quantized_gated_delta_rule_packed_decode(
    mixed_qkv: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    A_log: torch.Tensor,
    dt_bias: torch.Tensor,
    scale: float,
    state_codes: torch.Tensor,
    state_scale: torch.Tensor,
    resid_codes: torch.Tensor,
    resid_scale: torch.Tensor,
    out: torch.Tensor,
    ssm_state_indices: torch.Tensor,
    use_qk_l2norm_in_kernel: bool = False,
    resid_fmt: int = RESID_INT8,
    *,
    state_bits: int = 8,
    quant_mode: str = "fast",
    dst_state_indices: torch.Tensor | None = None,
):
    """INT8 + error-feedback drop-in for ``fused_recurrent_gated_delta_rule_packed_decode``.

    Signature of quantized_packed_decode.py:242-257. Updates the four pool
    tensors and ``out`` in place, asynchronously on the current stream, and
    returns ``out``.

    ``dst_state_indices`` (int32 ``[>= B]``, optional): request n reads slot
    ``ssm_state_indices[n]`` and writes its updated state to slot
    ``dst_state_indices[n]`` of the same pool; an id outside
    ``[1, num_slots)`` discards the update (``out`` is still written).
    """
    front = _native._front
    if front is not None and not _DEBUG:
        # the usual call: the checks below and the launch, in C++ over the
        # tensors' metadata (csrc/front.cpp); a call it declines takes the
        # checks below, which raise the reference's errors
        try:
            dev = state_codes.get_device()
            status = front.DECLINED if dev < 0 else front.packed_decode(
                mixed_qkv, a, b, A_log, dt_bias, scale, state_codes, state_scale, resid_codes,
                resid_scale, out, ssm_state_indices, dst_state_indices, use_qk_l2norm_in_kernel,
                resid_fmt, state_bits, _QUANT_MODES[quant_mode], _native.stream_handle(dev))
        except Exception:   # an argument of another type: the checks below name it
            status = front.DECLINED
        if status != front.DECLINED:
            _native.check(status, "quantized_gated_delta_rule_packed_decode")
            return out

    if not _native.library_available():
        raise RuntimeError("The HIP library is required for the quantized packed decode "
                           "(build it with `python -m carrykernel_amd.build`)")
    dev, args = _decode_call_args(mixed_qkv, a, b, A_log, dt_bias, scale, state_codes, state_scale,
                                  resid_codes, resid_scale, out, ssm_state_indices,
                                  use_qk_l2norm_in_kernel, resid_fmt, state_bits, quant_mode,
                                  dst_state_indices)
    L = _native.lib()
    fn = L.ck_gdn_packed_decode if dst_state_indices is None else L.ck_gdn_packed_decode_to
    _native.check(fn(*args, _native.stream_handle(dev)), "quantized_gated_delta_rule_packed_decode")
    return out


def _decode_call_args(mixed_qkv, a, b, A_log, dt_bias, scale, state_codes, state_scale,
                      resid_codes, resid_scale, out, ssm_state_indices, use_qk_l2norm_in_kernel,
                      resid_fmt, state_bits, quant_mode, dst_state_indices, check_devices=True):
    """The packed decode's checks; returns (device index, the arguments of
    ck_gdn_packed_decode, or of ck_gdn_packed_decode_to with
    dst_state_indices, without the stream). ``check_devices=False`` leaves
    out the device checks (tests on CPU tensors)."""
    # validation and messages follow quantized_packed_decode.py:268-309
    m_sh, m_st = mixed_qkv.shape, mixed_qkv.stride()
    sc_sh, sc_st = state_codes.shape, state_codes.stride()
    rc_sh = resid_codes.shape
    if len(m_sh) != 2:
        raise ValueError(f"mixed_qkv must be 2-D, got {tuple(m_sh)}")
    if m_st[-1] != 1:
        raise ValueError("mixed_qkv must be contiguous in its last dimension")
    if len(sc_sh) != 4:
        raise ValueError(f"state_codes must be 4-D, got {tuple(sc_sh)}")
    if sc_st[-1] != 1:
        raise ValueError("state_codes must be contiguous in its last dimension")
    if state_codes.dtype != torch.int8 or resid_codes.dtype != torch.int8:
        raise ValueError("state_codes and resid_codes must be int8 storage")
    if resid_fmt == RESID_INT4 and rc_sh[-1] * 2 != sc_sh[-1]:
        raise ValueError(
            "int4 residual must be packed two codes per byte: expected last dim "
            f"{sc_sh[-1] // 2}, got {rc_sh[-1]}")
    if resid_fmt == RESID_INT8 and rc_sh != sc_sh:
        raise ValueError("int8 residual must have the same shape as the state")
    if resid_fmt not in (RESID_INT8, RESID_INT4):
        raise ValueError(f"resid_fmt must be RESID_INT8 or RESID_INT4, got {resid_fmt}")
    if ssm_state_indices.dim() != 1:
        raise ValueError("ssm_state_indices must be 1-D")
    if ssm_state_indices.dtype != torch.int32:
        raise ValueError("ssm_state_indices must be int32")

    B = m_sh[0]
    num_slots, HV, V, K = sc_sh
    o_sh = out.shape
    if o_sh != (B, 1, HV, V):
        raise ValueError(f"out must be {(B, 1, HV, V)}, got {tuple(o_sh)}")
    if not out.is_contiguous():
        raise ValueError("out must be contiguous")

    # H is inferred from the packed width, exactly as upstream does.
    qkv_dim = m_sh[1]
    qk_dim = qkv_dim - HV * V
    if qk_dim <= 0 or qk_dim % 2 != 0:
        raise ValueError(f"cannot infer H from mixed_qkv width {qkv_dim}")
    H = (qk_dim // 2) // K
    if H <= 0 or 2 * H * K != qk_dim or HV % H != 0:
        raise ValueError(f"cannot infer H from mixed_qkv width {qkv_dim}")
    if resid_fmt == RESID_INT4 and K % 2 != 0:
        raise ValueError(f"int4 residual packing needs an even K, got {K}")
    if K > MAX_K:
        raise ValueError(f"packed decode supports K <= {MAX_K}, got K={K}")

    # checks the reference leaves implicit
    ss_sh, rs_sh = state_scale.shape, resid_scale.shape
    if ss_sh != (num_slots, HV, V) or state_scale.dtype != torch.float32:
        raise ValueError(f"state_scale must be float32 {(num_slots, HV, V)}, "
                         f"got {state_scale.dtype} {tuple(ss_sh)}")
    if resid_scale.dtype != torch.float32:
        raise ValueError("resid_scale must be float32")
    if rs_sh == (num_slots, HV, V):
        rscale_mode = _native.RSCALE_PER_ROW
    elif rs_sh == (num_slots, HV):
        rscale_mode = _native.RSCALE_PER_HEAD
    else:
        raise ValueError(f"resid_scale must be {(num_slots, HV, V)} (per V-row) or "
                         f"{(num_slots, HV)} (per head), got {tuple(rs_sh)}")
    if rc_sh[:3] != (num_slots, HV, V):
        raise ValueError("resid_codes must have the state's slot, head and V dims")
    ss_st, rc_st, rs_st = state_scale.stride(), resid_codes.stride(), resid_scale.stride()
    for name, sh, st in (("state_codes", sc_sh, sc_st), ("state_scale", ss_sh, ss_st),
                         ("resid_codes", rc_sh, rc_st), ("resid_scale", rs_sh, rs_st)):
        if not _dense_after_slot(sh, st):
            raise ValueError(f"{name} must be contiguous within a slot")
    a_st, b_st = a.stride(), b.stride()
    for name, t, st in (("a", a, a_st), ("b", b, b_st)):
        if t.shape != (B, HV) or st[-1] != 1:   # the shape test also rejects other ranks
            raise ValueError(f"{name} must be [B, HV] = {(B, HV)} with a contiguous last dim")
    for name, t in (("A_log", A_log), ("dt_bias", dt_bias)):
        if t.shape != (HV,) or t.stride(0) != 1:
            raise ValueError(f"{name} must be a contiguous [HV] = ({HV},) tensor")
    if ssm_state_indices.shape[0] < B:
        raise ValueError(f"ssm_state_indices must have at least B={B} entries")
    if quant_mode not in _QUANT_MODES:
        raise ValueError(f"quant_mode must be one of {tuple(_QUANT_MODES)}, got {quant_mode!r}")
    if not 2 <= int(state_bits) <= 8:
        raise ValueError(f"state_bits must be in 2..8, got {state_bits}")
    if dst_state_indices is not None:
        if dst_state_indices.dim() != 1 or dst_state_indices.dtype != torch.int32:
            raise ValueError("dst_state_indices must be a 1-D int32 tensor")
        if quant_mode != "fast":
            raise ValueError("dst_state_indices is supported with quant_mode='fast'")
        if dst_state_indices.shape[0] < B:
            raise ValueError(f"dst_state_indices must have at least B={B} entries")

    dev = state_codes.get_device()   # -1 for a CPU tensor
    if check_devices:
        tensors = (("mixed_qkv", mixed_qkv), ("a", a), ("b", b), ("A_log", A_log),
                   ("dt_bias", dt_bias), ("state_codes", state_codes), ("state_scale", state_scale),
                   ("resid_codes", resid_codes), ("resid_scale", resid_scale), ("out", out),
                   ("ssm_state_indices", ssm_state_indices))
        if dst_state_indices is not None:
            tensors += (("dst_state_indices", dst_state_indices),)
        for name, t in tensors:
            if t.get_device() != dev or dev < 0:
                _native.require_gpu(t, name)
                _native.require_gpu(state_codes, "state_codes")
                raise ValueError(f"{name} is on {t.device}, the state pool on {state_codes.device}")
    if _DEBUG:
        _check_indices_host(ssm_state_indices[:B], num_slots)
        if dst_state_indices is not None:
            _check_dst_indices_host(ssm_state_indices[:B], dst_state_indices[:B], num_slots)

    head = (mixed_qkv.data_ptr(), _native.dtype_code(mixed_qkv, "mixed_qkv"), m_st[0],
            a.data_ptr(), _native.dtype_code(a, "a"), a_st[0],
            b.data_ptr(), _native.dtype_code(b, "b"), b_st[0],
            A_log.data_ptr(), _native.dtype_code(A_log, "A_log"),
            dt_bias.data_ptr(), _native.dtype_code(dt_bias, "dt_bias"),
            float(scale),
            state_codes.data_ptr(), sc_st[0],
            state_scale.data_ptr(), ss_st[0],
            resid_codes.data_ptr(), rc_st[0],
            resid_scale.data_ptr(), rs_st[0],
            out.data_ptr(), _native.dtype_code(out, "out"),
            ssm_state_indices.data_ptr(), ssm_state_indices.stride(0))
    if dst_state_indices is not None:
        head += (dst_state_indices.data_ptr(), dst_state_indices.stride(0))
    tail = (num_slots, B, H, HV, K, V,
            int(bool(use_qk_l2norm_in_kernel)), int(resid_fmt), rscale_mode,
            int(state_bits), _QUANT_MODES[quant_mode])
    return dev, head + tail


def _check_dst_indices_host(src: torch.Tensor, dst: torch.Tensor, num_slots: int) -> None:
    s = src.detach().to("cpu").tolist()
    d = dst.detach().to("cpu").tolist()
    live_d = [j for i, j in zip(s, d) if 0 < i < num_slots and 0 < j < num_slots]
    if len(set(live_d)) != len(live_d):
        raise ValueError("dst_state_indices has duplicate slot ids (the writes would race)")
    read = {i for i in s if 0 < i < num_slots}
    if any(j in read and j != i for i, j in zip(s, d) if 0 < i < num_slots and 0 < j < num_slots):
        raise ValueError("a destination slot is also read by another request of the call (race)")


def _pool_layout(pool, name: str):
    """(HV, V, K, resid_fmt, rscale_mode) of a quantized pool tuple, validated."""
    if len(pool) != 4:
        raise ValueError(f"{name} must be (state_codes, state_scale, resid_codes, resid_scale)")
    sc, ss, rc, rs = pool
    if sc.dim() != 4 or sc.dtype != torch.int8 or rc.dtype != torch.int8:
        raise ValueError(f"{name}: state_codes / resid_codes must be int8 [S, HV, V, K] / [S, HV, V, K or K/2]")
    S, HV, V, K = sc.shape
    if rc.shape == sc.shape:
        resid_fmt = RESID_INT8
    elif K % 2 == 0 and rc.shape == (S, HV, V, K // 2):
        resid_fmt = RESID_INT4
    else:
        raise ValueError(f"{name}: resid_codes must be {(S, HV, V, K)} or {(S, HV, V, K // 2)}, "
                         f"got {tuple(rc.shape)}")
    if ss.dtype != torch.float32 or ss.shape != (S, HV, V):
        raise ValueError(f"{name}: state_scale must be float32 {(S, HV, V)}")
    if rs.dtype != torch.float32 or rs.shape not in ((S, HV, V), (S, HV)):
        raise ValueError(f"{name}: resid_scale must be float32 {(S, HV, V)} or {(S, HV)}")
    rscale_mode = _native.RSCALE_PER_HEAD if rs.dim() == 2 else _native.RSCALE_PER_ROW
    for tname, t in zip(("state_codes", "state_scale", "resid_codes", "resid_scale"), pool):
        if not _slot_contiguous(t):
            raise ValueError(f"{name}: {tname} must be contiguous within a slot")
    return HV, V, K, resid_fmt, rscale_mode


def _require_pool_gpu(pool, name: str):
    for tname, t in zip(("state_codes", "state_scale", "resid_codes", "resid_scale"), pool):
        _native.require_gpu(t, f"{name}.{tname}")
        if t.device != pool[0].device:
            raise ValueError(f"{name}: {tname} is on {t.device}, state_codes on {pool[0].device}")


def _pool_args(pool):
    sc, ss, rc, rs = pool
    return (sc.data_ptr(), sc.stride(0), ss.data_ptr(), ss.stride(0), rc.data_ptr(), rc.stride(0),
            rs.data_ptr(), rs.stride(0), sc.shape[0])


def _slot_ids(ids: torch.Tensor, name: str, device) -> torch.Tensor:
    if ids.dim() != 1 or ids.dtype != torch.int32:
        raise ValueError(f"{name} must be a 1-D int32 tensor")
    if ids.device != device:
        raise ValueError(f"{name} is on {ids.device}, the pool on {device}")
    return ids.contiguous()


def copy_quantized_state(src_pool, src_ids: torch.Tensor, dst_pool, dst_ids: torch.Tensor):
    """Copy whole slots between quantized pools of the same layout: slot
    ``src_ids[i]`` of ``src_pool`` -> slot ``dst_ids[i]`` of ``dst_pool``, state
    codes and scales together with the error-feedback residual and its
    scales (prefix-cache fork, speculative-decode checkpoint, moving a
    preempted request's state to and from a staging pool). Pools are the
    4-tuples ``init_quantized_state`` returns and may be the same; a slot must
    not be both read and written by one call. Ids outside ``[1, S)`` of their
    pool skip the pair. Asynchronous on the current stream."""
    layout = _pool_layout(src_pool, "src_pool")
    if _pool_layout(dst_pool, "dst_pool") != layout:
        raise ValueError("src_pool and dst_pool must have the same HV, V, K, residual format and scale layout")
    _require_pool_gpu(src_pool, "src_pool")
    _require_pool_gpu(dst_pool, "dst_pool")
    dev = src_pool[0].device
    if dst_pool[0].device != dev:
        raise ValueError("src_pool and dst_pool must be on the same GPU")
    src_ids = _slot_ids(src_ids, "src_ids", dev)
    dst_ids = _slot_ids(dst_ids, "dst_ids", dev)
    if src_ids.shape != dst_ids.shape:
        raise ValueError("src_ids and dst_ids must have the same length")
    HV, V, K, resid_fmt, rscale_mode = layout
    status = _native.lib().ck_pool_copy_slots(
        *_pool_args(src_pool), *_pool_args(dst_pool), src_ids.data_ptr(), dst_ids.data_ptr(), src_ids.shape[0],
        HV, V, K, resid_fmt, rscale_mode, _native.stream_handle(dev))
    _native.check(status, "copy_quantized_state")


def reset_quantized_state(pool, ids: torch.Tensor):
    """Zero the listed slots (codes, scales, residual and residual scales):
    the state of a new request, as ``init_quantized_state`` without ``h0``
    gives (quantized_packed_decode.py:341-345). Ids outside ``[1, S)`` are
    skipped. Asynchronous on the current stream."""
    HV, V, K, resid_fmt, rscale_mode = _pool_layout(pool, "pool")
    _require_pool_gpu(pool, "pool")
    dev = pool[0].device
    ids = _slot_ids(ids, "ids", dev)
    status = _native.lib().ck_pool_reset_slots(
        *_pool_args(pool), ids.data_ptr(), ids.shape[0], HV, V, K, resid_fmt, rscale_mode,
        _native.stream_handle(dev))
    _native.check(status, "reset_quantized_state")


def init_quantized_state(num_slots: int, HV: int, V: int, K: int, device,
                         h0: torch.Tensor | None = None,
                         resid_fmt: int = RESID_INT8,
                         *,
                         per_head_resid_scale: bool = False,
                         state_bits: int = 8):
    """Allocate the quantized state pool, optionally seeding slot contents.

    quantized_packed_decode.py:330-352. ``h0``, when given, is
    ``[num_slots, HV, V, K]`` in a floating dtype on any device (a host
    tensor is copied to ``device``) and is quantized into the pool on the GPU
    (``ck_quantize_rows``: scale = max(amax_K, eps) / qmax, codes =
    clamp(rne(h0 / scale))) in h0's own precision, as the reference's torch
    expression computes it: fp32 and float64 as such (a float64 scale is
    stored rounded to fp32), bf16 and fp16 with every operation rounded to
    that dtype; other floating dtypes are read as fp32. The residual starts at
    zero. Returns ``(state_codes, state_scale, resid_codes, resid_scale)``.
    ``per_head_resid_scale`` allocates ``resid_scale`` as ``[num_slots, HV]``.
    """
    device = torch.device(device)
    if h0 is not None:
        if tuple(h0.shape) != (num_slots, HV, V, K):
            raise ValueError(f"h0 must be {(num_slots, HV, V, K)}, got {tuple(h0.shape)}")
        if not h0.is_floating_point():
            raise ValueError(f"h0 must be a floating-point tensor, got {h0.dtype}")
    if device.type != "cuda":
        raise _native.HipUnavailable(f"the quantized pool lives on a GPU, got device {device}")
    resid_k = K // 2 if resid_fmt == RESID_INT4 else K
    state_codes = torch.zeros((num_slots, HV, V, K), dtype=torch.int8, device=device)
    state_scale = torch.zeros((num_slots, HV, V), dtype=torch.float32, device=device)
    resid_codes = torch.zeros((num_slots, HV, V, resid_k), dtype=torch.int8, device=device)
    rs_shape = (num_slots, HV) if per_head_resid_scale else (num_slots, HV, V)
    resid_scale = torch.zeros(rs_shape, dtype=torch.float32, device=device)

    if h0 is not None:
        # h0 may come from any device and in any float dtype, as the
        # reference's (quantized_packed_decode.py:347-351 quantizes in h0's
        # precision and copy_()s into the pool): move it to the pool's GPU;
        # the kernel reads fp32, bf16, fp16 and float64 in their own
        # precision, other floating dtypes are read as fp32.
        if h0.dtype == torch.float64:
            code = _native.DTYPE_F64
        else:
            if h0.dtype not in (torch.float32, torch.bfloat16, torch.float16):
                h0 = h0.to(torch.float32)
            code = _native.dtype_code(h0, "h0")
        h0 = h0.to(device).contiguous()
        qmax = float(2 ** (int(state_bits) - 1) - 1)
        L = _native.lib()
        status = L.ck_quantize_rows(h0.data_ptr(), code, K,
                                    num_slots * HV * V, K, qmax,
                                    state_codes.data_ptr(), state_scale.data_ptr(),
                                    _native.stream_handle(device))
        _native.check(status, "init_quantized_state")
    return state_codes, state_scale, resid_codes, resid_scale


def state_bytes_per_slot(HV: int, V: int, K: int, quantized: bool,
                         base_dtype_size: int = 4, resid_fmt: int = RESID_INT8,
                         *, per_head_resid_scale: bool = False):
    """Bytes of recurrent state per request slot (quantized_packed_decode.py:355-369).

    ``per_head_resid_scale`` counts one fp32 residual scale per head instead of
    one per V-row.
    """
    if not quantized:
        return HV * V * K * base_dtype_size
    codes = HV * V * K
    resid = HV * V * (K // 2 if resid_fmt == RESID_INT4 else K)
    scales = HV * V * 4 + (HV * 4 if per_head_resid_scale else HV * V * 4)
    return codes + resid + scales
