"""Native-binding entry points of the statequant-layout step.

Mirror of ``cuda/binding.py`` of tomalmog/carrykernel (binding.py:27-156):
``load_extension``, ``gdn_quant_step_*``, ``gdn_fp32_step_*``,
``gdn_quant_decode_*`` with the reference's argument meaning and return
values, and the reference's ``BLOCK_V=128`` default. The reference JIT-builds
a CUDA extension; here the library is prebuilt in-tree
(``python -m carrykernel_amd.build``) and loaded through ctypes, so
``load_extension`` only loads it. The ``*_cuda`` names are kept as aliases so
callers of the reference module run unchanged.
"""

from __future__ import annotations

from .. import _native
from ..statequant import kernel as sq

HipUnavailable = _native.HipUnavailable
CudaUnavailable = HipUnavailable  # the reference's exception name (binding.py:31)


def load_extension(verbose: bool = False):
    """Load the prebuilt HIP library (binding.py:42-68 builds-and-loads)."""
    if verbose:
        print(f"loading {_native.LIB_PATH}")
    return _native.lib()


def gdn_quant_step_hip(h_int8, scale, e, e_scale, q, k, v, alpha, beta,
                       bits: int = 8, res_fmt: int = sq.RES_FP32, BLOCK_V: int = 128,
                       *, quant_mode: str = "fast"):
    """One fused GDN + INT8-quantize + error-feedback step (binding.py:81-123).

    Returns ``(o, h_int8_new, scale_new, e_new, e_scale_new)``; ``e_scale_new``
    is ``None`` for every residual format except int8.
    """
    load_extension()
    return sq.gdn_quant_step_fused(h_int8, scale, e, e_scale, q, k, v, alpha, beta, bits=bits,
                                   res_fmt=res_fmt, BLOCK_V=BLOCK_V, quant_mode=quant_mode)


def gdn_fp32_step_hip(h, q, k, v, alpha, beta, BLOCK_V: int = 128):
    """Fused FP32 GDN step (baseline), binding.py:126-143. Returns ``(h_out, o)``."""
    load_extension()
    return sq.gdn_step_fused_fp32(h, q, k, v, alpha, beta, BLOCK_V=BLOCK_V)


def gdn_quant_decode_hip(h0, q, k, v, alpha, beta, T, bits: int = 8,
                         res_fmt: int = sq.RES_FP32, BLOCK_V: int = 128, *, quant_mode: str = "fast"):
    """T-step decode (binding.py:146-156)."""
    load_extension()
    return sq.gdn_quant_decode_fused(h0, q, k, v, alpha, beta, T, bits=bits, res_fmt=res_fmt,
                                     BLOCK_V=BLOCK_V, quant_mode=quant_mode)


gdn_quant_step_cuda = gdn_quant_step_hip
gdn_fp32_step_cuda = gdn_fp32_step_hip
gdn_quant_decode_cuda = gdn_quant_decode_hip
