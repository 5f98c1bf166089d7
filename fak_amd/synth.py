"""Seeded synthetic GGUF weights and activations for the benchmark and test shapes.

No model files exist in this environment, so every workload runs on synthetic data with the
statistics the workloads specify:

* Q4_K super-block (256 weights, 144 B): f16 ``d`` and ``dmin`` drawn as |N(0,1)|*1e-3 (rounded
  to nearest-even f16, so ~5% of them are f16 subnormals), 16 six-bit (scale, min) fields uniform
  in [0, 63] packed into the 12-byte field by the inverse of ``GetScaleMinK4``
  (internal/model/quantbits.go:42-47), and 128 uniform nibble bytes.
* Q8_0 block (32 weights, 34 B): f16 ``d`` = |N(0,1)|*0.002, 32 int8 codes uniform in
  [-127, 127].
* Activations: f32 N(0,1).

Byte layouts follow internal/model/quant_q4k.go:22-26 and internal/ggufload/gguf.go:24.
"""
from __future__ import annotations

import numpy as np

Q4K_BLOCK = 144
Q8_0_BLOCK = 34


def pack_scale_min_k4(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Pack 8 six-bit scales and 8 six-bit mins per row into the 12-byte k-quant field.

    The inverse of GetScaleMinK4 (internal/model/quantbits.go:42-47): pairs 0..3 keep their low
    six bits in bytes j / j+4 and donate their top two bits to pairs 4..7, whose low nibbles sit
    in bytes 8..11. ``sc``/``mn`` have shape [..., 8] with values in [0, 63].
    """
    sc = np.asarray(sc, np.uint8)
    mn = np.asarray(mn, np.uint8)
    q = np.zeros(sc.shape[:-1] + (12,), np.uint8)
    for j in range(4):
        q[..., j] = (sc[..., j] & 63) | ((sc[..., j + 4] >> 4) << 6)
        q[..., j + 4] = (mn[..., j] & 63) | ((mn[..., j + 4] >> 4) << 6)
    for j in range(4, 8):
        q[..., j + 4] = (sc[..., j] & 0xF) | ((mn[..., j] & 0xF) << 4)
    return q


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(v.astype(np.float16)).view(np.uint8).reshape(v.shape + (2,))


def q4k_weights(out: int, in_: int, seed: int) -> np.ndarray:
    """Row-major raw Q4_K bytes for an [out, in] weight: out*(in/256) super-blocks of 144 B."""
    if in_ % 256:
        raise ValueError("Q4_K reduction dim must be a multiple of 256")
    rng = np.random.default_rng(seed)
    nb = out * (in_ // 256)
    blk = np.empty((nb, Q4K_BLOCK), np.uint8)
    dd = np.abs(rng.standard_normal((nb, 2), dtype=np.float32)) * np.float32(1e-3)
    blk[:, 0:4] = _f16_bytes(dd).reshape(nb, 4)
    fields = rng.integers(0, 64, size=(nb, 16), dtype=np.uint8)
    blk[:, 4:16] = pack_scale_min_k4(fields[:, :8], fields[:, 8:])
    blk[:, 16:] = rng.integers(0, 256, size=(nb, 128), dtype=np.uint8)
    return blk.reshape(-1)


def q8_0_weights(out: int, in_: int, seed: int) -> np.ndarray:
    """Row-major raw Q8_0 bytes for an [out, in] weight: out*(in/32) blocks of 34 B."""
    if in_ % 32:
        raise ValueError("Q8_0 reduction dim must be a multiple of 32")
    rng = np.random.default_rng(seed)
    nb = out * (in_ // 32)
    blk = np.empty((nb, Q8_0_BLOCK), np.uint8)
    d = np.abs(rng.standard_normal(nb, dtype=np.float32)) * np.float32(0.002)
    blk[:, 0:2] = _f16_bytes(d)
    blk[:, 2:] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    return blk.reshape(-1)


def activations(m: int, k: int, seed: int) -> np.ndarray:
    """f32 N(0,1) activations of shape [m, k]."""
    rng = np.random.default_rng(seed)
    return rng.standard_normal((m, k), dtype=np.float32)
