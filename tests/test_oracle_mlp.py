"""Pins the oracle's silu / SwiGLU (internal/model/forward.go:452, moe.go:111-136) against an
evaluation that shares none of its code: e^-z from Python's 50-digit decimal arithmetic,
rounded to f64 (the precision math.Exp returns) and then to f32 as float32(math.Exp(..)) does,
followed by 1 + t and z / s in numpy's IEEE f32 arithmetic. A dropped sign, an f32 exp, or a
reordered formula fails the dense sweep."""
import decimal
import math

import numpy as np
import pytest

decimal.getcontext().prec = 50


def silu_decimal(z: np.float32) -> np.float32:
    if np.isnan(z):
        return np.float32(np.nan)
    if np.isinf(z):
        return np.float32(np.inf) if z > 0 else np.float32(np.nan)
    t64 = float((-decimal.Decimal(float(z))).exp()) if -float(z) < 709 else math.inf
    with np.errstate(over="ignore"):
        t = np.float32(t64)
        s = np.float32(1) + t
        return np.float32(z) / s


def sweep():
    rng = np.random.default_rng(3)
    v = [rng.standard_normal(3000).astype(np.float32) * np.float32(s) for s in (0.1, 2, 20, 60)]
    edges = np.array([0, -0.0, 1e-30, -1e-30, 1e-45, 88, -88, 89, -89, 100, -100, 103, -104,
                      1e30, -1e30, 3.4e38, -3.4e38], np.float32)
    return np.concatenate(v + [edges])


def test_silu_bit_exact_against_decimal(oracle_mod):
    for z in sweep():
        got, want = oracle_mod.silu(z), silu_decimal(z)
        assert np.array_equal(np.float32(got).view(np.uint32), np.float32(want).view(np.uint32)) \
            or (np.isnan(got) and np.isnan(want)), (z, got, want)


@pytest.mark.parametrize("z,want", [
    (0.0, 0.0), (-0.0, -0.0), (np.inf, np.inf), (-100.0, -0.0), (-1e30, -0.0), (1e30, 1e30),
])
def test_silu_special_values(oracle_mod, z, want):
    got = oracle_mod.silu(z)
    assert got == want and np.signbit(got) == np.signbit(np.float32(want))


def test_silu_nan(oracle_mod):
    assert np.isnan(oracle_mod.silu(np.nan)) and np.isnan(oracle_mod.silu(-np.inf))


def test_swiglu_is_silu_times_up(oracle_mod):
    rng = np.random.default_rng(9)
    g = rng.standard_normal(777).astype(np.float32) * 5
    u = rng.standard_normal(777).astype(np.float32)
    got = oracle_mod.swiglu(g, u)
    want = np.array([silu_decimal(a) for a in g], np.float32) * u
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_mlp_composition_small(oracle_mod):
    """The MLP oracle is the composition of already-pinned pieces; on an integer-exact case
    (d = 1, dmin = 0, small codes) the gate/up stage is exact, so the chain is checked against
    float64 matrix products of the dequantized weights."""
    from fak_amd import synth
    H, I = 256, 512
    gate, up, down = (synth.q4k_weights(I, H, 1), synth.q4k_weights(I, H, 2),
                      synth.q4k_weights(H, I, 3))
    X = synth.activations(2, H, 4)
    Y = oracle_mod.q4k_mlp(gate, up, down, H, I, X, 2)
    Wg = oracle_mod.q4k_dequant(gate, I, H).astype(np.float64)
    Wu = oracle_mod.q4k_dequant(up, I, H).astype(np.float64)
    Wd = oracle_mod.q4k_dequant(down, H, I).astype(np.float64)
    g, u = X @ Wg.T, X @ Wu.T
    ref = ((g / (1 + np.exp(-g))) * u) @ Wd.T
    err = np.max(np.abs(Y - ref)) / np.sqrt(np.mean(ref ** 2))
    assert err < 1e-4
