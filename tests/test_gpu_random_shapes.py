"""Seeded random shapes across every route of the Q4_K and Q6_K matmuls (the 1..4-token int8
GEMV, the 5..16-token kernel, its 17..32-token f16 form, the prefill GEMM on 128- and 256-row
workgroups with and without K ranges), each against the oracle at its bound: max|dY|/RMS <= 1e-3
up to 16 tokens, 1e-2 beyond. Activations are N(0,1) times a per-case power of ten in
[1e-3, 1e3]; outputs are checked on every row, or on rows spread over every row block for the
largest products."""
import numpy as np
import pytest

from fak_amd import synth
from tests import q6k_cases as qc
from tests.gpu_util import q4k_matmul, rel_err, spread_rows
from tests.test_gpu_q6k import dev_matmul as q6k_matmul

pytestmark = pytest.mark.gpu

TOKENS = [1, 2, 3, 4, 5, 7, 8, 12, 16, 17, 23, 32, 33, 64, 100, 127, 128, 129, 200, 255, 300,
          511, 600, 897, 1000, 1100, 1500, 2100]
BLOCKS = [1, 2, 3, 4, 7, 9, 14, 20, 37, 74]
ROWS = [1, 7, 16, 33, 100, 255, 256, 300, 1000, 1024, 2049, 3000, 3584, 5000, 9000]


def cases(seed: int, n: int):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        fmt = "q6k" if rng.random() < 0.35 else "q4k"
        K = 256 * int(rng.choice(BLOCKS))
        N = int(rng.choice(ROWS))
        M = int(rng.choice(TOKENS))
        if N * K * M > 3_000_000_000:
            M = max(1, 3_000_000_000 // (N * K))
        out.append((i, fmt, N, K, M, float(f"{10.0 ** rng.uniform(-3, 3):.3g}")))
    return out


@pytest.mark.parametrize("i,fmt,N,K,M,scale", cases(2026, 48))
def test_random_shape(hip, oracle_mod, i, fmt, N, K, M, scale):
    print(f"[case] {i} {fmt} N={N} K={K} M={M} scale={scale:.3g}", flush=True)
    rng = np.random.default_rng(1000 + i)
    X = (rng.standard_normal((M, K)) * scale).astype(np.float32)
    if fmt == "q4k":
        raw = synth.q4k_weights(N, K, seed=i)
        Y = q4k_matmul(raw, N, K, X, M)
        rb = (K // 256) * 144
        rows = spread_rows(N, per_block=1) if N * K * M > 200_000_000 else np.arange(N)
        sub = np.concatenate([raw[o * rb:(o + 1) * rb] for o in rows])
        ref = oracle_mod.q4k_gemm(sub, len(rows), K, X, M, workers=16)
    else:
        raw = qc.pin_d(rng.integers(0, 256, size=N * (K // 256) * 210, dtype=np.uint8), 0x1400)
        Y = q6k_matmul(raw, N, K, X, M)
        rb = (K // 256) * 210
        rows = spread_rows(N, per_block=1) if N * K * M > 50_000_000 else np.arange(N)
        sub = np.concatenate([raw[o * rb:(o + 1) * rb] for o in rows])
        ref = oracle_mod.q6k_gemm(sub, len(rows), K, X, M)
    assert np.all(np.isfinite(Y))
    e = rel_err(Y[:, rows], ref)
    print(f"    max|d|/RMS = {e:.2e}", flush=True)
    assert e <= (1e-3 if M <= 16 else 1e-2)
