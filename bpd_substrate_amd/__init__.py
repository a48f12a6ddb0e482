"""bpd_substrate_amd — MI355X (gfx950) implementation of bpd-substrate's
quantized-inference hot path: Q4_K dequant, Q8_K / Q8_0 activation
quantization, the Q4_K x Q8_K and Q8_0 x Q8_0 GEMVs, behind the reference's
C ABI (include/bpdq.h, libbpdq_hip.so).

Modules:
  formats  GGUF block layouts and byte counts
  gpu      host mirror of the reference GPU entry points (ctypes over the C ABI)
  synth    deterministic synthetic tensors for the benchmark configurations
  build    in-tree build of the native libraries
"""
from . import formats  # noqa: F401

__all__ = ["formats", "gpu", "synth", "build"]
