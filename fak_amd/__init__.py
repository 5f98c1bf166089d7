"""fak_amd — an MI355X-native (gfx950) HIP backend for fak's GGUF Q4_K / Q8_0 matmul path.

Layers:
  include/fakhip.h        the flat C ABI (the cgo / ctypes boundary)
  fak_amd/csrc/*.hip      runtime shim, tiled weight layouts, GEMV / MFMA GEMM kernels
  fak_amd/fakhip.py       ctypes declarations of the C ABI
  fak_amd/backend.py      host mirror of compute.Backend for the quantized matmul
  fak_amd/synth.py        seeded synthetic GGUF blocks / activations for benchmarks
"""
__all__ = ["fakhip", "backend", "synth", "build"]
