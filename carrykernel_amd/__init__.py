"""MI355X-native fused Gated DeltaNet decode step with error-feedback state quantization.

Hand-written gfx950 HIP kernels behind a C ABI (``include/carrykernel_gdn.h``),
with Python front ends that keep the call signatures of tomalmog/carrykernel:

* ``carrykernel_amd.vllm_integration.quantized_packed_decode`` - vLLM paged
  ``[slots, HV, V, K]`` layout, in place (the engine drop-in);
* ``carrykernel_amd.statequant.kernel`` - ``[B, HV, K, V]`` layout, out of place;
* ``carrykernel_amd.hip.binding`` - the native-binding entry points.
"""

__version__ = "0.1.0"
