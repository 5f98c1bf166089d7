"""Launch-shape coverage: the small-M kernels pick their workgroup shape from the tile count and
the K length (one tile per workgroup up to one tile per CU, balanced tile counts per CU up to
eight, the tall-matrix rule beyond, shorter K parts when K is short). These shapes sit on both
sides of each of those boundaries for Q4_K, Q6_K and Q8_0 and check every output against the
oracle at the GEMV bound (max|dY|/RMS <= 1e-3)."""
import numpy as np
import pytest

from fak_amd import synth
from tests import q6k_cases as qc
from tests.gpu_util import Dev, q4k_matmul, q8_0_matmul, rel_err
from fak_amd import fakhip

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3

# 16-row tiles per shape: 1, 7, 100, 200, 256, 257, 300, 512, 513, 1100, 2048 (= 8 x 256 CUs),
# 2100; K from one super-block to 36.
Q4K_SHAPES = [(7, 256, 1), (1600, 512, 1), (3205, 1280, 1), (4096, 768, 1), (4112, 2304, 1),
              (4800, 256, 1), (8192, 1024, 1), (8208, 512, 1), (17600, 1024, 1), (32768, 256, 1),
              (33600, 256, 1), (520, 9216, 1), (1000, 2560, 2), (5000, 1536, 3), (700, 4096, 4),
              (4112, 768, 4)]
Q6K_SHAPES = [(7, 256), (1600, 512), (4096, 768), (4112, 2304), (4800, 256), (8208, 512),
              (17600, 1024), (33600, 256), (520, 9216), (2000, 6400)]
Q8_SHAPES = [(1, 32), (50, 96), (16, 64), (4000, 1024), (4112, 576), (300, 4096),
             (20000, 512), (3, 11008)]


@pytest.mark.parametrize("out,in_,P", Q4K_SHAPES)
def test_q4k_small_m_shapes(hip, oracle_mod, out, in_, P):
    print(f"[case] q4k sweep out={out} in={in_} P={P}", flush=True)
    raw = synth.q4k_weights(out, in_, seed=out + in_ + P)
    X = synth.activations(P, in_, seed=out + 7)
    Y = q4k_matmul(raw, out, in_, X, P)
    e = rel_err(Y, oracle_mod.q4k_gemm(raw, out, in_, X, P, workers=16))
    print(f"    max|d|/RMS = {e:.3e}", flush=True)
    assert e <= GEMV_TOL, e


def _q6k_matmul(raw, out, in_, X, P):
    lib = fakhip.load()
    w = fakhip.alloc_call("fhip_q6k_upload", np.ascontiguousarray(raw).ctypes.data, out, in_)
    try:
        with Dev.from_host(np.ascontiguousarray(X, np.float32)) as dx, Dev(P * out * 4) as dy:
            fakhip.call("fhip_q6k_matmul_f32", w, dx.ptr, dy.ptr, out, in_, P)
            return dy.to_host(np.float32).reshape(P, out)
    finally:
        lib.fhip_free(w)


@pytest.mark.parametrize("out,in_", Q6K_SHAPES)
def test_q6k_one_token_shapes(hip, oracle_mod, out, in_):
    print(f"[case] q6k sweep out={out} in={in_}", flush=True)
    rng = np.random.default_rng(out * 3 + in_)
    raw = qc.pin_d(rng.integers(0, 256, size=out * (in_ // 256) * 210, dtype=np.uint8), 0x1400)
    X = rng.standard_normal((1, in_)).astype(np.float32)
    Y = _q6k_matmul(raw, out, in_, X, 1)
    e = rel_err(Y, oracle_mod.q6k_gemm(raw, out, in_, X, 1))
    print(f"    max|d|/RMS = {e:.3e}", flush=True)
    assert e <= GEMV_TOL, e


@pytest.mark.parametrize("out,in_", Q8_SHAPES)
def test_q8_0_one_token_shapes(hip, oracle_mod, out, in_):
    print(f"[case] q8_0 sweep out={out} in={in_}", flush=True)
    raw = synth.q8_0_weights(out, in_, seed=out + 2 * in_)
    X = synth.activations(1, in_, seed=out + 3)
    Y = q8_0_matmul(raw, out, in_, X, 1)
    e = rel_err(Y, oracle_mod.q8_0_gemm(raw, out, in_, X, 1))
    print(f"    max|d|/RMS = {e:.3e}", flush=True)
    assert e <= GEMV_TOL, e
