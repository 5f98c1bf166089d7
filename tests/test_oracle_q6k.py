"""Pin the oracle's Q6_K functions: q6kDequantSuperBlock (internal/model/quant_kquant.go:139-163)
and kQuantMatRowsRange with kind Q6_K (:210-232).

  * the hand golden of TestKQuantDequantGolden (quant_kquant_test.go:113-129);
  * bit-identity with an independent vectorised numpy decode of the layout on random bytes
    (every (ql, qh, scale) combination occurs) and with f16-subnormal / negative d;
  * the reference's integer fixture (TestKQuantMatRowsMatchesDequantRef, quant_kquant_test.go:
    51-88) against the exact integer dot;
  * a hand-derived row whose result (1.0) only the four-accumulator order gives;
  * f64 brute force on random rows.
"""
import numpy as np

from tests import fixtures as fx
from tests import q6k_cases as qc


def test_dequant_golden(oracle_mod):
    blk = np.zeros(210, np.uint8)
    blk[192:208] = 1
    blk[208:210] = np.frombuffer(np.float16(2.0).tobytes(), np.uint8)
    np.testing.assert_array_equal(oracle_mod.q6k_dequant(blk, 1, 256)[0], np.full(256, -64.0, np.float32))


def test_dequant_matches_numpy_decode(oracle_mod):
    rng = np.random.default_rng(6)
    raw = rng.integers(0, 256, size=64 * 210, dtype=np.uint8)
    # d: normal, subnormal and negative f16 values
    ds = np.concatenate([rng.standard_normal(48).astype(np.float16) * np.float16(0.01),
                         np.array([6e-8, -6e-8, 3e-5, -2.0] * 4, np.float16)])
    r = raw.reshape(64, 210)
    r[:, 208:210] = ds.view(np.uint8).reshape(64, 2)
    got = oracle_mod.q6k_dequant(r.reshape(-1), 1, 64 * 256).reshape(64, 256)
    want = qc.numpy_decode(r.reshape(-1))
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_matrows_reference_fixture_exact(oracle_mod):
    raw, x, out, in_ = qc.reference_fixture()
    w = qc.numpy_decode(raw).reshape(out, in_).astype(np.int64)
    exact = w @ x.astype(np.int64)
    assert np.abs(exact).max() < 2 ** 24
    y = oracle_mod.q6k_matrows(raw, out, in_, x)
    np.testing.assert_array_equal(y, exact.astype(np.float32))


def test_matrows_order(oracle_mod):
    blk, x, want = qc.order_row()
    assert oracle_mod.q6k_matrows(blk, 1, 256, x)[0] == want


def test_matrows_vs_f64(oracle_mod):
    rng = np.random.default_rng(7)
    out, in_ = 24, 1024
    raw = qc.pin_d(rng.integers(0, 256, size=out * 4 * 210, dtype=np.uint8), 0x1400)  # d ~ 1e-3
    x = rng.standard_normal(in_).astype(np.float32)
    w = qc.numpy_decode(raw).reshape(out, in_).astype(np.float64)
    ref = w @ x.astype(np.float64)
    y = oracle_mod.q6k_matrows(raw, out, in_, x)
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.sqrt(np.mean(ref ** 2))
