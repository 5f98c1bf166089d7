"""Input generators restated from the reference's own Go tests (pure integer recurrences, so
they reproduce the reference's fixtures exactly without Go's math/rand).

* lcg_bytes            internal/model/quant_kquant_test.go:9-15
* pin_q8_0_scales      internal/model/quant_kquant_test.go:90-106 (f16One = 0x3C00 into d)
* LCG (.f())           internal/compute/compute_test.go:10-15
* f32_to_f16_bits_test internal/compute/cuda_quant_test.go:188-204 (round-half-up, flush tiny)
* rand_q4k_bytes       internal/compute/cuda_quant_test.go:212-227
* rscale               internal/compute/cuda_test.go:42-48
"""
from __future__ import annotations

import numpy as np

MASK64 = (1 << 64) - 1
LCG_A = 6364136223846793005
LCG_C = 1442695040888963407
F16_ONE = 0x3C00


def lcg_bytes(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.uint8)
    s = seed
    for i in range(n):
        s = (s * LCG_A + LCG_C) & MASK64
        out[i] = (s >> 33) & 0xFF
    return out


class LCG:
    def __init__(self, seed: int):
        self.s = seed & MASK64

    def f(self) -> np.float32:
        self.s = (self.s * LCG_A + LCG_C) & MASK64
        v = (self.s >> 32) & 0xFFFFFFFF
        if v >= 1 << 31:
            v -= 1 << 32  # int32(s >> 32)
        return np.float32(np.float32(v) / np.float32(1 << 31)) - np.float32(0.5)


def f32_to_f16_bits_test(f: np.float32) -> int:
    b = int(np.float32(f).view(np.uint32))
    sign = (b >> 16) & 0x8000
    exp = ((b >> 23) & 0xFF) - 127 + 15
    mant = b & 0x7FFFFF
    if exp <= 0:
        return sign
    if exp >= 0x1F:
        return sign | 0x7C00
    half = ((exp << 10) | (mant >> 13)) & 0xFFFF
    if mant & 0x1000:
        half = (half + 1) & 0xFFFF
    return sign | half


def rand_q4k_bytes(g: LCG, out: int, in_: int) -> np.ndarray:
    nsb = in_ // 256
    raw = np.empty(out * nsb * 144, np.uint8)
    for blk in range(out * nsb):
        base = blk * 144
        d = np.float32(0.01) + np.float32(abs(g.f())) * np.float32(0.03)
        dmin = np.float32(0.004) + np.float32(abs(g.f())) * np.float32(0.012)
        hd, hm = f32_to_f16_bits_test(d), f32_to_f16_bits_test(dmin)
        raw[base:base + 4] = [hd & 0xFF, hd >> 8, hm & 0xFF, hm >> 8]
        for i in range(140):
            v = np.float32((g.f() + np.float32(0.5)) * np.float32(255.0))
            raw[base + 4 + i] = int(v) & 0xFF  # byte(int32(...) & 0xff)
    return raw


def rscale(g: LCG, n: int, scale: float) -> np.ndarray:
    return np.array([g.f() * np.float32(scale) for _ in range(n)], np.float32)


def pin_f16_scale(raw: np.ndarray, nblocks: int, block_bytes: int, d_bits: int = F16_ONE,
                  dmin_bits=None) -> np.ndarray:
    """Write d (and optionally dmin) into every block, like pinResidentQuantScales /
    benchQ4KFixture."""
    raw = raw.copy().reshape(nblocks, block_bytes)
    raw[:, 0] = d_bits & 0xFF
    raw[:, 1] = d_bits >> 8
    if dmin_bits is not None:
        raw[:, 2] = dmin_bits & 0xFF
        raw[:, 3] = dmin_bits >> 8
    return raw.reshape(-1)
