"""Native-binding layer of the statequant-layout step.

Counterpart of ``cuda/binding.py`` of tomalmog/carrykernel (binding.py:27-156)
and of the extension module it builds (cuda/gdn_state_kernel.cu:299-377). The
reference JIT-builds ``carrykernel_gdn_cuda`` once under a lock; the module's
two host launchers write into caller-owned tensors on the current stream and
raise ``RuntimeError`` from ``TORCH_CHECK``; the binding's wrappers cast the
inputs, allocate the outputs, pass a zero ``e_scale`` when there is none and
call the launchers. Here the module is the prebuilt in-tree HIP library
(``python -m carrykernel_amd.build``): :func:`load_extension` loads it once
under a lock and returns a :class:`HipModule` whose ``gdn_quant_step`` and
``gdn_fp32_step`` keep the launchers' signatures (.cu:310-315, :350-352) and
checks, over the C ABI (``ck_gdn_quant_step``, ``ck_gdn_fp32_step``). The
``*_hip`` wrappers keep the binding's argument preparation and return values;
``*_cuda`` aliases let callers of the reference module run unchanged.
"""

from __future__ import annotations

import threading

import torch

from .. import _native
from ..statequant import kernel as sq

HipUnavailable = _native.HipUnavailable
CudaUnavailable = HipUnavailable  # the reference's exception name (binding.py:31)

_QUANT_MODES = {"fast": _native.QUANT_FAST, "exact": _native.QUANT_EXACT}
_RES_DTYPES = {sq.RES_FP32: torch.float32, sq.RES_FP16: torch.float16, sq.RES_FP8: torch.float8_e5m2,
               sq.RES_INT8: torch.int8}


def _check(cond: bool, msg: str) -> None:
    """TORCH_CHECK: a failed check is a RuntimeError (.cu:299-302, 316-323)."""
    if not cond:
        raise RuntimeError(msg)


def _check_state(t: torch.Tensor, name: str) -> None:
    """check_state of .cu:299-302."""
    _check(t.is_cuda, f"{name} must be a CUDA tensor")
    _check(t.is_contiguous(), f"{name} must be contiguous")


def _check_operands(device: torch.device, operands) -> None:
    """The reference's launchers take every other operand's data pointer as
    is; over a C ABI a wrong shape, dtype, device or layout would be read or
    written out of bounds, so each is checked here (RuntimeError, like the
    launchers' own checks)."""
    for name, t, dtype, shape in operands:
        _check(t.device == device, f"{name} must be on {device}, got {t.device}")
        _check(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")
        _check(tuple(t.shape) == shape, f"{name} must be {shape}, got {tuple(t.shape)}")
        _check(t.is_contiguous(), f"{name} must be contiguous")


class HipModule:
    """The extension module's two host launchers (.cu:310-371, pybind
    :373-377), asynchronous on the current stream of the state's device."""

    def __init__(self, lib):
        self._lib = lib

    def gdn_quant_step(self, h_in, scale_in, e_in, e_scale_in, q, k, v, alpha, beta,
                       o, h_out, scale_out, e_out, e_scale_out,
                       qmax: float, res_fmt: int, block_v: int, quant_mode: str = "fast") -> None:
        """Fused GDN + INT8 quantize + error feedback into the caller's
        ``o, h_out, scale_out, e_out, e_scale_out`` (.cu:310-348).
        ``e_scale_in`` / ``e_scale_out`` are read / written for the int8
        residual only, and always passed, as in the reference.

        K is any of 1..256: the CUDA launcher loops over any K at run time
        (.cu:161-166, :185-190); here rows past K are zero-padded to the next
        power of two (at least 16), whose K-slices fix the reduction order.
        K above 256 raises ``RuntimeError`` ("K must be in 1..256")."""
        _check_state(h_in, "h_in")
        _check_state(e_in, "e_in")
        _check(h_in.dtype == torch.int8, "h_in must be int8")
        _check(h_in.dim() == 4, "h_in must be [B, HV, K, V]")
        _check(0 < int(block_v) <= 1024, "block_v must be in (0, 1024]")
        _check(int(res_fmt) in _RES_DTYPES, f"unknown res_fmt {res_fmt}")
        _check(quant_mode in _QUANT_MODES, f"unknown quant_mode {quant_mode!r}")
        B, HV, K, V = h_in.shape
        col = (B, HV, V)
        f32 = torch.float32
        _check_operands(h_in.device, (
            ("scale_in", scale_in, f32, col), ("e_in", e_in, _RES_DTYPES[int(res_fmt)], (B, HV, K, V)),
            ("e_scale_in", e_scale_in, f32, col), ("q", q, f32, (B, HV, K)), ("k", k, f32, (B, HV, K)),
            ("v", v, f32, col), ("alpha", alpha, f32, (B, HV)), ("beta", beta, f32, (B, HV)),
            ("o", o, f32, col), ("h_out", h_out, torch.int8, (B, HV, K, V)), ("scale_out", scale_out, f32, col),
            ("e_out", e_out, e_in.dtype, (B, HV, K, V)), ("e_scale_out", e_scale_out, f32, col)))
        st = self._lib.ck_gdn_quant_step(
            h_in.data_ptr(), scale_in.data_ptr(), e_in.data_ptr(), e_scale_in.data_ptr(), q.data_ptr(),
            k.data_ptr(), v.data_ptr(), alpha.data_ptr(), beta.data_ptr(), o.data_ptr(), h_out.data_ptr(),
            scale_out.data_ptr(), e_out.data_ptr(), e_scale_out.data_ptr(), B, HV, K, V, float(qmax),
            int(res_fmt), _QUANT_MODES[quant_mode], _native.stream_handle(h_in.device))
        _check(st == _native.CK_OK, f"gdn_quant_step: {_last_error(self._lib, st)}")

    def gdn_fp32_step(self, h_in, q, k, v, alpha, beta, o, h_out, block_v: int) -> None:
        """Fused FP32 GDN step into the caller's ``o, h_out`` (.cu:350-371).
        K in 1..256, as for gdn_quant_step."""
        _check_state(h_in, "h_in")
        _check(h_in.dtype == torch.float32, "h_in must be fp32")
        _check(h_in.dim() == 4, "h_in must be [B, HV, K, V]")
        _check(0 < int(block_v) <= 1024, "block_v must be in (0, 1024]")
        B, HV, K, V = h_in.shape
        f32 = torch.float32
        _check_operands(h_in.device, (
            ("q", q, f32, (B, HV, K)), ("k", k, f32, (B, HV, K)), ("v", v, f32, (B, HV, V)),
            ("alpha", alpha, f32, (B, HV)), ("beta", beta, f32, (B, HV)), ("o", o, f32, (B, HV, V)),
            ("h_out", h_out, f32, (B, HV, K, V))))
        st = self._lib.ck_gdn_fp32_step(h_in.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                        alpha.data_ptr(), beta.data_ptr(), o.data_ptr(), h_out.data_ptr(),
                                        B, HV, K, V, _native.stream_handle(h_in.device))
        _check(st == _native.CK_OK, f"gdn_fp32_step: {_last_error(self._lib, st)}")


def _last_error(lib, status: int) -> str:
    return f"status {status}: " + lib.ck_last_error().decode(errors="replace")


_module: HipModule | None = None
_module_lock = threading.Lock()


def load_extension(verbose: bool = False) -> HipModule:
    """Load (once, under a lock) and return the native module (binding.py:42-68
    builds and loads). Raises :class:`CudaUnavailable` (``HipUnavailable``)
    without a GPU or without the built library."""
    global _module
    if _module is not None:
        return _module
    with _module_lock:
        if _module is None:
            if not torch.cuda.is_available():
                raise CudaUnavailable("no GPU device available")
            if verbose:
                print(f"loading {_native.LIB_PATH}")
            _module = HipModule(_native.lib())
    return _module


def gdn_quant_step_hip(h_int8, scale, e, e_scale, q, k, v, alpha, beta,
                       bits: int = 8, res_fmt: int = sq.RES_FP32, BLOCK_V: int = 128,
                       *, quant_mode: str = "fast"):
    """One fused GDN + INT8-quantize + error-feedback step (binding.py:81-123):
    inputs cast to contiguous fp32 (the residual kept in its storage dtype), a
    zero ``e_scale`` when none is given, outputs allocated on the state's
    device. Returns ``(o, h_int8_new, scale_new, e_new, e_scale_new)``;
    ``e_scale_new`` is ``None`` for every residual format except int8."""
    ext = load_extension()
    assert h_int8.dtype == torch.int8, f"h_int8 must be int8, got {h_int8.dtype}"
    assert h_int8.dim() == 4, f"expected [B, HV, K, V], got {tuple(h_int8.shape)}"
    B, HV, K, V = h_int8.shape
    dev = h_int8.device
    scale, q, k, v, alpha, beta = (t.contiguous().float() for t in (scale, q, k, v, alpha, beta))
    e_scale = (torch.zeros((B, HV, V), device=dev, dtype=torch.float32) if e_scale is None
               else e_scale.contiguous().float())
    o = torch.empty((B, HV, V), device=dev, dtype=torch.float32)
    h_out = torch.empty((B, HV, K, V), device=dev, dtype=torch.int8)
    scale_out = torch.empty((B, HV, V), device=dev, dtype=torch.float32)
    e_out = torch.empty((B, HV, K, V), device=dev, dtype=e.dtype)
    e_scale_out = torch.empty((B, HV, V), device=dev, dtype=torch.float32)
    ext.gdn_quant_step(h_int8.contiguous(), scale, e.contiguous(), e_scale, q, k, v, alpha, beta,
                       o, h_out, scale_out, e_out, e_scale_out, float(2 ** (int(bits) - 1) - 1), int(res_fmt),
                       int(BLOCK_V), quant_mode=quant_mode)
    return o, h_out, scale_out, e_out, e_scale_out if res_fmt == sq.RES_INT8 else None


def gdn_fp32_step_hip(h, q, k, v, alpha, beta, BLOCK_V: int = 128):
    """Fused FP32 GDN step (baseline), binding.py:126-143. Returns ``(h_out, o)``."""
    ext = load_extension()
    assert h.dim() == 4, f"expected [B, HV, K, V], got {tuple(h.shape)}"
    B, HV, K, V = h.shape
    dev = h.device
    h, q, k, v, alpha, beta = (t.contiguous().float() for t in (h, q, k, v, alpha, beta))
    o = torch.empty((B, HV, V), device=dev, dtype=torch.float32)
    h_out = torch.empty((B, HV, K, V), device=dev, dtype=torch.float32)
    ext.gdn_fp32_step(h, q, k, v, alpha, beta, o, h_out, int(BLOCK_V))
    return h_out, o


def gdn_quant_decode_hip(h0, q, k, v, alpha, beta, T, bits: int = 8,
                         res_fmt: int = sq.RES_FP32, BLOCK_V: int = 128, *, quant_mode: str = "fast"):
    """T-step decode over ``[T, B, HV, *]`` inputs (binding.py:146-156):
    init_quant_state, then one step per token, outputs stacked."""
    state = sq.init_quant_state(h0, bits, res_fmt)
    outs = []
    for t in range(T):
        o, *state = gdn_quant_step_hip(*state, q[t], k[t], v[t], alpha[t], beta[t], bits=bits,
                                       res_fmt=res_fmt, BLOCK_V=BLOCK_V, quant_mode=quant_mode)
        outs.append(o)
    return (torch.stack(outs), *state)


gdn_quant_step_cuda = gdn_quant_step_hip
gdn_fp32_step_cuda = gdn_fp32_step_hip
gdn_quant_decode_cuda = gdn_quant_decode_hip
