"""Hand-built inputs for the int8 Q4_K route (q4kMatRowsRangeInt8,
internal/model/quant_q4k_int8.go:72-142), shared by the oracle's pinning tests and the GPU parity
tests. Each builder returns raw GGUF Q4_K bytes [out, in] and, where it matters, the activation
and the expected result derived by hand in the docstring."""
import numpy as np

from fak_amd import synth

F16_ONE = 0x3C00


def q4k_block(d_bits: int, dmin_bits: int, sc, mn, nib: dict) -> np.ndarray:
    """One 144-byte super-block: f16 bit patterns d/dmin, 8 scales, 8 mins, and the nibble
    values {weight index j: n} (all others 0) placed in the GGUF order (chunk j // 64, low nibble
    of byte 32c + (j % 64) for j % 64 < 32, else the high nibble of byte 32c + j % 64 - 32)."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([d_bits & 0xFF, d_bits >> 8], np.uint8)
    b[2:4] = np.array([dmin_bits & 0xFF, dmin_bits >> 8], np.uint8)
    b[4:16] = synth.pack_scale_min_k4(np.array(sc, np.uint8)[None], np.array(mn, np.uint8)[None])[0]
    for j, n in nib.items():
        c, w = divmod(j, 64)
        if w < 32:
            b[16 + 32 * c + w] |= n & 0xF
        else:
            b[16 + 32 * c + w - 32] |= (n & 0xF) << 4
    return b


def identity_headers(raw: np.ndarray, out: int, in_: int) -> np.ndarray:
    """The same nibbles with d = 1, dmin = 0, every scale 1 and min 0: the dequantized weight is
    then the nibble value itself (w = 1*1*n - 0)."""
    blk = np.array(raw, np.uint8).reshape(out * (in_ // 256), 144).copy()
    hdr = q4k_block(F16_ONE, 0, [1] * 8, [0] * 8, {})[:16]
    blk[:, :16] = hdr
    return blk.reshape(-1)


def order_cases():
    """Three rows over one super-block whose reference results are fixed by the order of the
    float chain acc += T1_s; acc -= T2_s (s = 0..7), T1 = (I*ws)*dx, T2 = (S*wm)*dx.

    Activation (K = 256; quantizeVecQ8 keeps these exact):
      block 0: x[0] = 127, x[1] = 101          -> dx = 1,     qx[0] = 127, qx[1] = 101
      block 1: x[32] = 127 * 2^20              -> dx = 2^20,  qx[32] = 127
      block 2: x[64] = 127 * 2^20              -> dx = 2^20,  qx[64] = 127
      block 3: x[96] = 127, x[97] = 101        -> dx = 1,     qx[96] = 127, qx[97] = 101
      block 4: x[128] = -127 * 2^20            -> dx = 2^20,  qx[128] = -127
      blocks 5-7: zero                         -> dx = 0, codes 0
    A = 127 * 2^20 = 133169152 lies in [2^26, 2^27), where the f32 spacing is 8.

    row 0 (d = dmin = 1; sc0 = sc1 = 1, m1 = 1; n[0] = n[32] = 1):
      s0: T1 = 127, T2 = 0 -> 127;  s1: T1 = A -> round(A + 127) = A + 128, T2 = A -> 128.
      Result 128. Adding T1 - T2 as one term would give 127.
    row 1 (d = 1, dmin = 0; sc2 = sc3 = sc4 = 1; n[64] = n[97] = n[128] = 1):
      s2: A;  s3: + 101 -> round(A + 101) = A + 104;  s4: - A -> 104.
      Result 104. Taking low-nibble sub-blocks first (0, 2, 4, 6, 1, 3, 5, 7) would give 101.
    row 2 (d = 1, dmin = 0; sc0 = sc1 = sc4 = 1; n[1] = n[32] = n[128] = 1):
      s0: 101;  s1: + A -> A + 104;  s4: - A -> 104.
      Result 104. Walking the sub-blocks backwards would give (-A + A) + 101 = 101.
    """
    A = np.float32(127 * 2.0 ** 20)
    x = np.zeros(256, np.float32)
    x[0], x[1], x[32], x[64], x[96], x[97], x[128] = 127, 101, A, A, 127, 101, -A
    z = [0] * 8
    rows = [
        q4k_block(F16_ONE, F16_ONE, [1, 1, 0, 0, 0, 0, 0, 0], [0, 1, 0, 0, 0, 0, 0, 0],
                  {0: 1, 32: 1}),
        q4k_block(F16_ONE, 0, [0, 0, 1, 1, 1, 0, 0, 0], z, {64: 1, 97: 1, 128: 1}),
        q4k_block(F16_ONE, 0, [1, 1, 0, 0, 1, 0, 0, 0], z, {1: 1, 32: 1, 128: 1}),
    ]
    return np.concatenate(rows), x, np.array([128, 104, 104], np.float32)


def integer_exact_case(out: int, in_: int, seed: int):
    """d = dmin = 1 with random 6-bit scales/mins and nibbles, and an integer activation whose
    every 32-block has max |x| = 127: quantizeVecQ8 then gives dx = 1 and qx = x, every term and
    partial sum is an integer, and while they stay below 2^24 the f32 chain is exact in any order.
    Returns raw, x, and the exact per-row values sum_k w_k x_k with w = sc*n - m (Python ints),
    plus the largest partial sum magnitude of the chain (the caller checks it is < 2^24)."""
    rng = np.random.default_rng(seed)
    nblk = in_ // 256
    blocks, exact, peak = [], [], 0
    x = rng.integers(-60, 61, size=in_).astype(np.int64)
    for b in range(in_ // 32):
        i = b * 32 + int(rng.integers(0, 32))
        x[i] = 127 if rng.integers(0, 2) else -127
    for o in range(out):
        acc = 0
        for b in range(nblk):
            sc = rng.integers(0, 64, 8)
            mn = rng.integers(0, 64, 8)
            n = rng.integers(0, 16, 256)
            blk = q4k_block(F16_ONE, F16_ONE, sc, mn, {j: int(n[j]) for j in range(256)})
            blocks.append(blk)
            for s in range(8):
                xs = x[b * 256 + 32 * s: b * 256 + 32 * s + 32]
                ns = n[32 * s: 32 * s + 32]
                acc += int(sc[s]) * int(np.dot(ns, xs))
                peak = max(peak, abs(acc))
                acc -= int(mn[s]) * int(xs.sum())
                peak = max(peak, abs(acc))
        exact.append(acc)
    return np.concatenate(blocks), x.astype(np.float32), exact, peak
