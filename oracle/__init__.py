"""CPU oracle for the fused GDN decode step with EF state quantization.

TEST INFRASTRUCTURE ONLY. Imported by ``tests/``, ``__graft_entry__.smoke()``
and the CPU-baseline leg of ``bench.py``, always as the checker. The product
package (``carrykernel_amd``) never imports it.

The arithmetic lives in ``gdn_oracle.c`` (built by ``oracle/Makefile`` into
``oracle/lib/libgdn_oracle.so``); this module is its numpy front end plus a few
pure-numpy restatements used to pin the C code (nibble packing, the
float64 GDN recurrence, bf16 rounding). Each function cites the reference
file:line it restates.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ORACLE_DIR, "lib", "libgdn_oracle.so")

MODE_FAST = 0
MODE_EXACT = 1

RESID_INT8 = 0
RESID_INT4 = 1

_lock = threading.Lock()
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float


def build() -> str:
    """Compile the C oracle with its Makefile (always rebuilds)."""
    subprocess.run(["make", "-B", "-s", "-C", ORACLE_DIR], check=True,
                   capture_output=True, text=True)
    return LIB_PATH


def lib():
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                build()
            L = ctypes.CDLL(LIB_PATH)
            L.orc_expf_n.argtypes = [_f32p, _f32p, _i64]
            L.orc_logf_n.argtypes = [_f32p, _f32p, _i64]
            L.orc_gates_n.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i64]
            L.orc_packed_decode.restype = _int
            L.orc_packed_decode.argtypes = [
                _f32p, _i64, _f32p, _i64, _f32p, _i64, _f32p, _f32p, _flt,
                _i8p, _i64, _f32p, _i64, _i8p, _i64, _f32p, _i64,
                _f32p, _i32p, ctypes.c_void_p, _i64,
                _int, _int, _int, _int, _int,
                _int, _int, _int, _int, _int, _int]
            L.orc_quantize_rows.argtypes = [_f32p, _i64, _int, _flt, _i8p, _f32p]
            _vp = ctypes.c_void_p
            L.orc_quant_step_kv.restype = _int
            L.orc_quant_step_kv.argtypes = [_i8p, _f32p, _vp, _vp, _f32p, _f32p, _f32p, _f32p, _f32p,
                                            _f32p, _i8p, _f32p, _vp, _vp,
                                            _int, _int, _int, _int, _flt, _int, _int, _int]
            L.orc_fp32_step_kv.restype = _int
            L.orc_fp32_step_kv.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                           _int, _int, _int, _int]
            L.orc_packed_decode_float_state.restype = _int
            L.orc_packed_decode_float_state.argtypes = [
                _f32p, _i64, _f32p, _i64, _f32p, _i64, _f32p, _f32p, _flt,
                _f32p, _i64, _int, _f32p, _i32p, _i64, _int, _int, _int, _int, _int, _int]
            _u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
            _u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
            L.orc_f32_to_f16_n.argtypes = [_f32p, _u16p, _i64]
            L.orc_f32_to_e5m2_n.argtypes = [_f32p, _u8p, _i64]
            L.orc_e5m2_to_f32_n.argtypes = [_u8p, _f32p, _i64]
            L.orc_quantize_cols.argtypes = [_f32p, _i64, _int, _int, _flt, _i8p, _f32p]
            L.orc_bf16_round_n.argtypes = [_f32p, _f32p, _i64]
            L.orc_count_div_small_int_mismatches.restype = _i64
            L.orc_count_div_small_int_mismatches.argtypes = [_flt, _int, _int]
            _lib = L
    return _lib


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


# ---------------------------------------------------------------------------
# Gate math
# ---------------------------------------------------------------------------

def expf(x) -> np.ndarray:
    x = _f32(x).ravel()
    y = np.empty_like(x)
    lib().orc_expf_n(x, y, x.size)
    return y


def logf(x) -> np.ndarray:
    x = _f32(x).ravel()
    y = np.empty_like(x)
    lib().orc_logf_n(x, y, x.size)
    return y


def gates(a, b, A_log, dt_bias):
    """alpha, beta per quantized_packed_decode.py:179-182 (arrays broadcast)."""
    a, b, A_log, dt_bias = np.broadcast_arrays(_f32(a), _f32(b), _f32(A_log), _f32(dt_bias))
    shape = a.shape
    a, b, A_log, dt_bias = (_f32(x).ravel() for x in (a, b, A_log, dt_bias))
    alpha = np.empty_like(a)
    beta = np.empty_like(a)
    lib().orc_gates_n(a, b, A_log, dt_bias, alpha, beta, a.size)
    return alpha.reshape(shape), beta.reshape(shape)


# ---------------------------------------------------------------------------
# vLLM-layout step
# ---------------------------------------------------------------------------

def packed_decode(mixed_qkv, a, b, A_log, dt_bias, scale,
                  state_codes, state_scale, resid_codes, resid_scale,
                  indices, H, *, use_qk_l2norm=False, resid_fmt=RESID_INT8,
                  per_head=False, state_bits=8, mode=MODE_FAST, nthreads=0, dst_indices=None):
    """One step of quantized_packed_decode.py:116-239 on host arrays.

    The pool arrays (``state_codes [S,HV,V,K]`` int8, ``state_scale [S,HV,V]``,
    ``resid_codes [S,HV,V,K or K/2]`` int8, ``resid_scale [S,HV,V]`` or
    ``[S,HV]`` when ``per_head``) are updated in place and must be
    C-contiguous numpy arrays. Returns ``out [B, HV, V]`` fp32.
    ``dst_indices`` (optional): request n's updated state goes to slot
    ``dst_indices[n]`` (outside ``[1, S)``: discarded) instead of the slot
    it was read from.
    """
    mixed = _f32(mixed_qkv)
    a = _f32(a)
    b = _f32(b)
    A_log = _f32(A_log)
    dt_bias = _f32(dt_bias)
    idx = np.ascontiguousarray(np.asarray(indices, dtype=np.int32))
    for arr, dt in ((state_codes, np.int8), (resid_codes, np.int8),
                    (state_scale, np.float32), (resid_scale, np.float32)):
        if arr.dtype != dt or not arr.flags.c_contiguous:
            raise ValueError("pool arrays must be C-contiguous with the right dtype")
    S, HV, V, K = state_codes.shape
    B = mixed.shape[0]
    out = np.empty((B, HV, V), dtype=np.float32)
    didx = None if dst_indices is None else np.ascontiguousarray(np.asarray(dst_indices, dtype=np.int32))
    rc = lib().orc_packed_decode(
        mixed, mixed.shape[1], a, a.shape[1], b, b.shape[1], A_log, dt_bias, float(scale),
        state_codes, state_codes[0].size, state_scale, state_scale[0].size,
        resid_codes, resid_codes[0].size, resid_scale, resid_scale[0].size,
        out, idx, None if didx is None else didx.ctypes.data_as(ctypes.c_void_p), S, B, H, HV, K, V,
        int(bool(use_qk_l2norm)), int(resid_fmt), int(bool(per_head)), int(state_bits),
        int(mode), int(nthreads))
    if rc != 0:
        raise ValueError("oracle: unsupported shape")
    return out


def quantize_rows(x, qmax=127.0):
    """init_quantized_state seeding (quantized_packed_decode.py:347-351), last dim."""
    x = _f32(x)
    K = x.shape[-1]
    rows = x.size // K
    codes = np.empty(x.shape, dtype=np.int8)
    scale = np.empty(x.shape[:-1], dtype=np.float32)
    lib().orc_quantize_rows(x, rows, K, float(qmax), codes, scale)
    return codes, scale


def quantize_rows_in_dtype(x, dtype: str, qmax=127.0):
    """init_quantized_state seeding (quantized_packed_decode.py:347-351) of an
    h0 of dtype "float32", "bfloat16", "float16" or "float64", in that dtype's
    precision as torch evaluates ``scale = h0.abs().amax(-1).clamp(min=1e-12)
    / qmax; codes = torch.round(h0 / scale).clamp(-qmax, qmax).to(int8)``:
    for the 16-bit dtypes each operation in fp32, rounded to nearest even to
    the dtype (numpy float16 for fp16, ``bf16_round`` for bf16); float64 in
    float64, its scale then rounded to fp32 as ``state_scale.copy_`` does.
    ``x`` holds the h0 values (exactly representable in ``dtype``). NaN
    quotients (0 / 0 when an fp16 scale rounds to 0) become code 0, as the
    int8 conversion gives them. Pure numpy."""
    if dtype == "float32":
        return quantize_rows(x, qmax)
    if dtype == "float64":
        xd = np.asarray(x, np.float64)
        s = np.maximum(np.abs(xd).max(axis=-1), 1e-12) / float(qmax)
        with np.errstate(invalid="ignore", divide="ignore"):
            q = np.clip(np.rint(xd / s[..., None]), -qmax, qmax)
        return q.astype(np.int8), s.astype(np.float32)
    if dtype == "bfloat16":
        r16 = bf16_round
    elif dtype == "float16":
        def r16(v):
            return np.asarray(v, np.float32).astype(np.float16).astype(np.float32)
    else:
        raise ValueError(f"unsupported dtype {dtype}")
    xf = np.asarray(x, np.float32)
    assert np.array_equal(r16(xf), xf), "x must hold values of the dtype"
    eps = r16(np.float32(1e-12))
    s = r16(np.maximum(np.abs(xf).max(axis=-1), eps) / np.float32(qmax))
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        q = r16(xf / s[..., None])
    q = np.where(np.isnan(q), np.float32(0), q)
    codes = np.clip(np.rint(q), -qmax, qmax).astype(np.int8)
    return codes, s.astype(np.float32)


def quantize_cols(x, qmax=127.0):
    """per_v_channel_quantize (statequant/kernel.py:99-113): [..., K, V], amax over K."""
    x = _f32(x)
    K, V = x.shape[-2:]
    M = x.size // (K * V)
    codes = np.empty(x.shape, dtype=np.int8)
    scale = np.empty(x.shape[:-2] + (V,), dtype=np.float32)
    lib().orc_quantize_cols(x, M, K, V, float(qmax), codes, scale)
    return codes, scale


# ---------------------------------------------------------------------------
# statequant layout ([B, HV, K, V], V contiguous)
# ---------------------------------------------------------------------------

RES_FP32, RES_FP16, RES_FP8, RES_INT8 = 0, 1, 2, 3


def f32_to_f16_bits(x) -> np.ndarray:
    x = _f32(x)
    y = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_n(x.ravel(), y.ravel(), x.size)
    return y


def f32_to_e5m2_bits(x) -> np.ndarray:
    x = _f32(x)
    y = np.empty(x.shape, np.uint8)
    lib().orc_f32_to_e5m2_n(x.ravel(), y.ravel(), x.size)
    return y


def e5m2_bits_to_f32(b) -> np.ndarray:
    b = np.asarray(b, np.uint8)
    shape = b.shape
    flat = np.ascontiguousarray(b.ravel())
    y = np.empty(flat.shape, np.float32)
    lib().orc_e5m2_to_f32_n(flat, y, flat.size)
    return y.reshape(shape)


def quant_step_kv(h_int8, scale, e, e_scale, q, k, v, alpha, beta, bits=8, res_fmt=RES_FP32,
                  mode=MODE_FAST, nthreads=0):
    """One out-of-place step of statequant/kernel.py:149-178 / :260-341.

    ``e`` is the residual's storage: float32 values (RES_FP32), uint16 fp16
    bits (RES_FP16), uint8 e5m2 bits (RES_FP8) or int8 codes (RES_INT8, with
    ``e_scale``). Returns ``(o, h_int8_new, scale_new, e_new, e_scale_new)``
    in the same storage conventions.
    """
    h_int8 = np.ascontiguousarray(h_int8, np.int8)
    B, HV, K, V = h_int8.shape
    store = {RES_FP32: np.float32, RES_FP16: np.uint16, RES_FP8: np.uint8, RES_INT8: np.int8}[res_fmt]
    e = np.ascontiguousarray(e, store)
    o = np.empty((B, HV, V), np.float32)
    h_out = np.empty_like(h_int8)
    s_out = np.empty((B, HV, V), np.float32)
    e_out = np.empty_like(e)
    es_in = _f32(e_scale) if res_fmt == RES_INT8 else None
    es_out = np.empty((B, HV, V), np.float32) if res_fmt == RES_INT8 else None
    rc = lib().orc_quant_step_kv(
        h_int8, _f32(scale), e.ctypes.data, None if es_in is None else es_in.ctypes.data,
        _f32(q), _f32(k), _f32(v), _f32(alpha), _f32(beta),
        o, h_out, s_out, e_out.ctypes.data, None if es_out is None else es_out.ctypes.data,
        B, HV, K, V, float(2 ** (bits - 1) - 1), int(res_fmt), int(mode), int(nthreads))
    if rc != 0:
        raise ValueError("oracle: unsupported shape")
    return o, h_out, s_out, e_out, es_out


def fp32_step_kv(h, q, k, v, alpha, beta):
    """statequant/kernel.py:116-123 in the fixed reduction order. Returns (h, o)."""
    h = _f32(h)
    B, HV, K, V = h.shape
    o = np.empty((B, HV, V), np.float32)
    h_out = np.empty_like(h)
    rc = lib().orc_fp32_step_kv(h, _f32(q), _f32(k), _f32(v), _f32(alpha), _f32(beta), o, h_out, B, HV, K, V)
    if rc != 0:
        raise ValueError("oracle: unsupported shape")
    return h_out, o


def packed_decode_float_state(mixed_qkv, a, b, A_log, dt_bias, scale, state, indices, H, *,
                              bf16=False, use_qk_l2norm=False):
    """vLLM-layout step on an unquantized state pool ``[S, HV, V, K]`` (fp32
    values; rounded to bf16 after the update when ``bf16``), in place.
    Returns ``out [B, HV, V]``."""
    mixed = _f32(mixed_qkv)
    if state.dtype != np.float32 or not state.flags.c_contiguous:
        raise ValueError("state must be a C-contiguous float32 array")
    S, HV, V, K = state.shape
    B = mixed.shape[0]
    out = np.empty((B, HV, V), np.float32)
    a, b = _f32(a), _f32(b)
    rc = lib().orc_packed_decode_float_state(
        mixed, mixed.shape[1], a, a.shape[1], b, b.shape[1], _f32(A_log), _f32(dt_bias), float(scale),
        state, state[0].size, int(bool(bf16)), out, np.ascontiguousarray(indices, np.int32), S,
        B, H, HV, K, V, int(bool(use_qk_l2norm)))
    if rc != 0:
        raise ValueError("oracle: unsupported shape")
    return out


# ---------------------------------------------------------------------------
# numpy restatements used to pin the C code
# ---------------------------------------------------------------------------

def pack_int4(codes: np.ndarray) -> np.ndarray:
    """quantized_packed_decode.py:226-230: byte = (c_even & 0xF) | (c_odd & 0xF) << 4."""
    c = np.asarray(codes).astype(np.int32)
    lo = c[..., 0::2] & 0xF
    hi = (c[..., 1::2] & 0xF) << 4
    return (lo | hi).astype(np.uint8).view(np.int8)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """quantized_packed_decode.py:196-199: even K low nibble, odd K high, >7 -> -16."""
    p = np.asarray(packed).astype(np.int32) & 0xFF
    lo = p & 0xF
    hi = (p >> 4) & 0xF
    lo = np.where(lo > 7, lo - 16, lo)
    hi = np.where(hi > 7, hi - 16, hi)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.int32)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (round to nearest even) -> fp32; NaN stays NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    r = (u & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, r)


def bf16_round_c(x: np.ndarray) -> np.ndarray:
    """The C oracle's bf16 rounding (bf16_round_f in gdn_oracle.c)."""
    x = _f32(x)
    y = np.empty_like(x)
    lib().orc_bf16_round_n(x.ravel(), y.ravel(), x.size)
    return y


def gdn_step_f64(h, q, k, v, alpha, beta):
    """statequant/reference.py:20-34 in float64 on a [.., K, V] state."""
    h = np.asarray(h, np.float64) * np.asarray(alpha, np.float64)[..., None, None]
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    read = np.einsum("...kv,...k->...v", h, k)
    dv = np.asarray(beta, np.float64)[..., None] * (np.asarray(v, np.float64) - read)
    h = h + k[..., :, None] * dv[..., None, :]
    o = np.einsum("...kv,...k->...v", h, q)
    return h, o


def count_div_small_int_mismatches(q: float, e_lo: int, e_hi: int) -> int:
    """Mismatches of the kernels' Markstein quotient RN(a/q) against IEEE a/q
    over every mantissa of a at biased exponents e_lo..e_hi."""
    return int(lib().orc_count_div_small_int_mismatches(float(q), int(e_lo), int(e_hi)))
