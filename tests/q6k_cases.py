"""Q6_K inputs shared by the oracle's pinning tests and the GPU parity tests: an independent
vectorised decode of the GGUF Q6_K layout, the reference's integer fixture, and a hand-built
order-revealing row."""
import numpy as np

from tests import fixtures as fx

Q6K = 210


def numpy_decode(raw: np.ndarray) -> np.ndarray:
    """Decode raw Q6_K super-blocks from the layout description (ql[128] | qh[64] | int8
    scales[16] | f16 d): weight 128 h + l + 32 i uses nibble (i >= 2) of ql[64 h + l + 32 (i & 1)],
    bits 2i..2i+1 of qh[32 h + l] and scale[8 h + l // 16 + 2 i]; w = (d * scale) * (q - 32)."""
    blk = np.asarray(raw, np.uint8).reshape(-1, Q6K)
    nb = blk.shape[0]
    d = blk[:, 208:210].copy().view(np.float16).astype(np.float32).reshape(nb)
    sc = blk[:, 192:208].view(np.int8).astype(np.float32)
    out = np.empty((nb, 256), np.float32)
    l = np.arange(32)
    for h in range(2):
        for i in range(4):
            ql = blk[:, 64 * h + l + 32 * (i & 1)].astype(np.int32)
            lo = (ql >> 4) if i >= 2 else (ql & 0x0F)
            hi = (blk[:, 128 + 32 * h + l].astype(np.int32) >> (2 * i)) & 3
            q = (lo | (hi << 4)) - 32
            s = sc[:, 8 * h + l // 16 + 2 * i]
            out[:, 128 * h + l + 32 * i] = (d[:, None] * s) * q.astype(np.float32)
    return out


def pin_d(raw: np.ndarray, d_bits: int) -> np.ndarray:
    r = np.array(raw, np.uint8).reshape(-1, Q6K).copy()
    r[:, 208] = d_bits & 0xFF
    r[:, 209] = d_bits >> 8
    return r.reshape(-1)


def reference_fixture():
    """TestKQuantMatRowsMatchesDequantRef for Q6_K (internal/model/quant_kquant_test.go:51-88):
    lcgBytes(seed 0x9e3779b97f4a7c15) over out = 9, in = 512, d pinned to 1.0, x[i] = (7i % 23)
    - 11. Every weight is an integer scale * code, so the exact dot is an integer."""
    out, in_ = 9, 512
    raw = pin_d(fx.lcg_bytes(out * (in_ // 256) * Q6K, 0x9E3779B97F4A7C15), fx.F16_ONE)
    x = (np.arange(in_) * 7 % 23 - 11).astype(np.float32)
    return raw, x, out, in_


def order_row():
    """One row, one super-block, d = 1, every scale 1 and every code 32 (weight 0) except
    weights 0, 1, 4, 8 with code 33 (weight 1); x[0] = 2^24, x[1] = 1, x[4] = 1, x[8] = -2^24.
    The reference's four accumulators take i % 4: s0 = (2^24 + 1) - 2^24 = 0 (2^24 + 1 rounds to
    2^24), s1 = 1, so y = (s0 + s1) + (s2 + s3) = 1. A single running sum gives 0."""
    blk = np.zeros(Q6K, np.uint8)
    blk[128:192] = 0xAA  # high bits 2 for every weight: code 32 + low nibble
    blk[192:208] = 1
    blk[208], blk[209] = fx.F16_ONE & 0xFF, fx.F16_ONE >> 8
    for j in (0, 1, 4, 8):  # weights 0..31 (h = 0, i = 0): low nibble of ql[j]
        blk[j] |= 1
    x = np.zeros(256, np.float32)
    x[0], x[1], x[4], x[8] = 2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)
    return blk, x, np.float32(1.0)
