"""Loader for the gfx950 HIP library behind the C ABI (``include/carrykernel_gdn.h``).

The library is linked against ``libamdhip64.so.7``. ``torch`` is imported
first so that the dynamic loader binds the library to the HIP runtime torch
already loaded: device pointers and ``hipStream_t`` handles taken from torch
tensors and streams are then valid in the library.

There is no CPU fallback: if the library is missing or no GPU is visible the
entry points raise ``HipUnavailable`` (a ``RuntimeError``).

Loading the library also loads ``_ck_front`` (``csrc/front.cpp``), the host
C++ argument checks and launch of the packed decode for its Python front end,
and binds it to the loaded library's entry points.
"""

from __future__ import annotations

import ctypes
import importlib.util
import os
import sysconfig
import threading

import torch

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "lib", "libcarrykernel_gdn.so")
# measurement build of the same sources with per-workgroup timestamps
# (CK_TIMELINE); loaded only by use_timeline_build()
TIMELINE_LIB_PATH = os.path.join(PKG_DIR, "lib", "libcarrykernel_gdn_timeline.so")
FRONT_PATH = os.path.join(PKG_DIR, "lib", "_ck_front" + sysconfig.get_config_var("EXT_SUFFIX"))

ABI_VERSION = 2

# enum ck_status
CK_OK = 0
CK_EINVAL = 1
CK_EUNSUPPORTED = 2
CK_ELAUNCH = 3

# enum ck_dtype
DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
DTYPE_F64 = 3  # CK_DTYPE_F64: ck_quantize_rows only

# enum ck_res_fmt / ck_resid_fmt / ck_rscale_mode / ck_quant_mode
QUANT_FAST = 0
QUANT_EXACT = 1
RSCALE_PER_ROW = 0
RSCALE_PER_HEAD = 1


class HipUnavailable(RuntimeError):
    """The HIP library or a GPU is not available."""


_lock = threading.Lock()
_lib = None
# _ck_front bound to _lib's packed decode entry points; set with _lib (None
# until the library is loaded or when the extension is not built)
_front = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float

_SIGNATURES = {
    "ck_last_error": (ctypes.c_char_p, []),
    "ck_abi_version": (_int, []),
    "ck_set_max_items_per_launch": (_int, [_i64]),
    "ck_set_decode_kernel": (_int, [_int]),
    "ck_gdn_packed_decode": (_int, [
        _vp, _int, _i64,          # mixed_qkv, dtype, stride
        _vp, _int, _i64,          # a
        _vp, _int, _i64,          # b
        _vp, _int,                # A_log
        _vp, _int,                # dt_bias
        _flt,                     # scale
        _vp, _i64, _vp, _i64,     # state codes / scale
        _vp, _i64, _vp, _i64,     # resid codes / scale
        _vp, _int,                # out
        _vp, _i64,                # indices
        _i64,                     # num_slots
        _int, _int, _int, _int, _int,   # B H HV K V
        _int, _int, _int, _int, _int,   # l2norm resid_fmt rscale_mode bits quant_mode
        _vp]),
    "ck_gdn_packed_decode_to": (_int, [
        _vp, _int, _i64, _vp, _int, _i64, _vp, _int, _i64, _vp, _int, _vp, _int, _flt,
        _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64,
        _vp, _int,
        _vp, _i64,                # indices
        _vp, _i64,                # destination indices
        _i64,
        _int, _int, _int, _int, _int,
        _int, _int, _int, _int, _int,
        _vp]),
    "ck_pool_copy_slots": (_int, [
        _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64,   # source pool
        _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64,   # destination pool
        _vp, _vp, _int, _int, _int, _int, _int, _int, _vp]),
    "ck_pool_reset_slots": (_int, [
        _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _vp, _int, _int, _int, _int, _int, _int, _vp]),
    "ck_gdn_packed_decode_float_state": (_int, [
        _vp, _int, _i64, _vp, _int, _i64, _vp, _int, _i64, _vp, _int, _vp, _int, _flt,
        _vp, _int, _i64, _vp, _int, _vp, _i64, _i64,
        _int, _int, _int, _int, _int, _int, _vp]),
    "ck_gdn_quant_step": (_int, [
        _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
        _vp, _vp, _vp, _vp, _vp,
        _int, _int, _int, _int, _flt, _int, _int, _vp]),
    "ck_gdn_fp32_step": (_int, [
        _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _int, _int, _int, _int, _vp]),
    "ck_quantize_rows": (_int, [_vp, _int, _i64, _i64, _int, _flt, _vp, _vp, _vp]),
    "ck_quantize_cols": (_int, [_vp, _i64, _int, _int, _flt, _vp, _vp, _vp]),
    "ck_hbm_copy": (_int, [_vp, _vp, _i64, _int, _vp]),
}


def library_available() -> bool:
    return _lib is not None or os.path.exists(LIB_PATH)


def lib():
    """Load (once) and return the ctypes handle; raises HipUnavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise HipUnavailable(
                    f"{LIB_PATH} is missing: build it with `python -m carrykernel_amd.build`")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(L, name, None)
                if fn is None:   # a library built from older sources
                    raise HipUnavailable(f"{LIB_PATH} does not export {name}; rebuild it "
                                         "with `python -m carrykernel_amd.build`")
                fn.restype = res
                fn.argtypes = args
            if L.ck_abi_version() != ABI_VERSION:
                raise HipUnavailable("libcarrykernel_gdn.so ABI version mismatch; rebuild it")
            _bind_front(L)
            _lib = L
    return _lib


def _bind_front(L) -> None:
    """Load ``_ck_front`` (when built) and give it the addresses of ``L``'s
    ck_gdn_packed_decode and ck_gdn_packed_decode_to."""
    global _front
    if not os.path.exists(FRONT_PATH):
        _front = None
        return
    spec = importlib.util.spec_from_file_location("_ck_front", FRONT_PATH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    addr = lambda fn: ctypes.cast(fn, ctypes.c_void_p).value
    mod.bind(addr(L.ck_gdn_packed_decode), addr(L.ck_gdn_packed_decode_to))
    _front = mod


def use_timeline_build():
    """Measurement only: load the timeline build instead of the product
    library (must come before anything else loads the library). Its decode
    launches write per-workgroup timestamps to the buffer given to
    ``ck_timeline_set`` (see packed_decode_impl.h)."""
    global LIB_PATH
    with _lock:
        if _lib is not None and LIB_PATH != TIMELINE_LIB_PATH:
            raise RuntimeError("the product library is already loaded in this process")
        LIB_PATH = TIMELINE_LIB_PATH
    L = lib()
    L.ck_timeline_set.restype = _int
    L.ck_timeline_set.argtypes = [_vp]
    return L


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def require_gpu(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise HipUnavailable(
            f"{name} is on {t.device}; the HIP kernels need GPU tensors (there is no CPU path)")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device) -> int:
    """hipStream_t of torch's current stream on `device` (a torch.device or
    a device index)."""
    if isinstance(device, int):
        index = device
    else:
        index = torch.device(device).index
        if index is None:
            index = torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


def check(status: int, what: str) -> None:
    if status == CK_OK:
        return
    msg = lib().ck_last_error().decode(errors="replace")
    if status in (CK_EINVAL, CK_EUNSUPPORTED):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def dtype_code(t: torch.Tensor, name: str) -> int:
    try:
        return DTYPE_CODES[t.dtype]
    except KeyError:
        raise ValueError(f"{name} must be float32, bfloat16 or float16, got {t.dtype}") from None


def set_max_items_per_launch(cap: int) -> None:
    """Lower, process-wide, the work items of one decode launch (0: no lower
    limit): larger steps then run as consecutive launches over slices of
    their requests (``ck_set_max_items_per_launch``; used by the tests of the
    split)."""
    check(lib().ck_set_max_items_per_launch(int(cap)), "set_max_items_per_launch")


DECODE_KERNEL_AUTO = 0
DECODE_KERNEL_PERSISTENT = 1
DECODE_KERNEL_ONE_ITEM = 2


def set_decode_kernel(which: int) -> None:
    """Choose, process-wide, the kernel of the quantized decode steps issued
    afterwards: DECODE_KERNEL_AUTO (the default), DECODE_KERNEL_PERSISTENT or
    DECODE_KERNEL_ONE_ITEM for every batch (``ck_set_decode_kernel``; used by
    the tests to run each kernel on shapes the automatic choice gives to the
    other). Both give the same bits."""
    check(lib().ck_set_decode_kernel(int(which)), "set_decode_kernel")
