"""Pin the oracle's int8 Q4_K route (FAK_KQ_INT8): q4kReduceRowScalar, q4kCombineRow and
q4kMatRowsRangeInt8 (internal/model/quant_q4k_int8.go:72-142) with the activation quantized by
quantizeRowQ8scalar (internal/model/quant_quantize.go:16-43).

  * the integer reduction against the pinned f32 dequant path (identity headers make the
    dequantized weight equal the nibble) and an exhaustive-range extreme case;
  * the combine against a closed form on integer-exact inputs (d = dmin = 1, dx = 1);
  * the float chain's order against hand-derived cancellation cases (tests/int8_cases.py);
  * TestQ4KInt8DotMatchesF32 (internal/model/quant_q4k_int8_test.go:16-60): max|int8 - f32| / RMS
    <= 0.05 against the f32 route on random blocks, out = 48, in = 768;
  * the association inside one term, (f32(I) * ws) * dx (quant_q4k_int8.go:122: Go evaluates
    left to right and never fuses on amd64), on a term where the other association rounds to a
    different f32, the expected value derived with exact rational arithmetic.
"""
import fractions
import struct
import numpy as np
import pytest

from fak_amd import synth
from tests import int8_cases as ic


def test_reduce_row_matches_dequant_path(oracle_mod):
    out, in_ = 6, 768
    nblk = in_ // 256
    raw = synth.q4k_weights(out, in_, 21)
    w = oracle_mod.q4k_dequant(ic.identity_headers(raw, out, in_), out, in_)  # == nibbles
    assert np.all(w == np.round(w)) and w.min() >= 0 and w.max() <= 15
    rng = np.random.default_rng(5)
    qx = rng.integers(-127, 128, size=in_, dtype=np.int8)
    for o in range(out):
        row = raw[o * nblk * 144:(o + 1) * nblk * 144]
        IS, SS = oracle_mod.q4k_reduce_row(row, nblk, qx)
        want_i = (w[o].astype(np.int64) * qx).reshape(-1, 32).sum(1)
        want_s = qx.astype(np.int64).reshape(-1, 32).sum(1)
        np.testing.assert_array_equal(IS, want_i)
        np.testing.assert_array_equal(SS, want_s)


def test_reduce_row_extremes(oracle_mod):
    """All nibbles 15 against all-127 and all-(-127) codes: |I_s| reaches 32*15*127 = 60960."""
    blk = np.zeros(144, np.uint8)
    blk[16:] = 0xFF
    for v in (127, -127):
        IS, SS = oracle_mod.q4k_reduce_row(blk, 1, np.full(256, v, np.int8))
        np.testing.assert_array_equal(IS, np.full(8, 32 * 15 * v))
        np.testing.assert_array_equal(SS, np.full(8, 32 * v))


@pytest.mark.parametrize("out,in_,seed", [(5, 256, 1), (4, 768, 2), (3, 2048, 3)])
def test_combine_closed_form(oracle_mod, out, in_, seed):
    raw, x, exact, peak = ic.integer_exact_case(out, in_, seed)
    assert peak < 2 ** 24, "test inputs must keep every partial sum exact in f32"
    q, d = oracle_mod.quantize_vec_q8(x, 32)
    np.testing.assert_array_equal(q, x.astype(np.int8))
    np.testing.assert_array_equal(d, np.ones(in_ // 32, np.float32))
    y = oracle_mod.q4k_matrows_int8(raw, out, in_, x)
    np.testing.assert_array_equal(y, np.array(exact, np.float32))
    # the two halves alone give the same rows
    nblk = in_ // 256
    for o in range(out):
        row = raw[o * nblk * 144:(o + 1) * nblk * 144]
        IS, SS = oracle_mod.q4k_reduce_row(row, nblk, q)
        assert oracle_mod.q4k_combine_row(row, nblk, d, IS, SS) == float(exact[o])


def test_combine_order_cases(oracle_mod):
    raw, x, want = ic.order_cases()
    y = oracle_mod.q4k_matrows_int8(raw, 3, 256, x)
    np.testing.assert_array_equal(y, want)


def _round_f32(q: fractions.Fraction) -> float:
    """The f32 nearest to the rational q (ties to even), for normal-range q."""
    if q == 0:
        return 0.0
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while fractions.Fraction(2) ** e > a:
        e -= 1
    while fractions.Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = fractions.Fraction(2) ** (e - 23)  # 24-bit significand
    n, r = divmod(a, ulp)
    if r * 2 > ulp or (r * 2 == ulp and n % 2 == 1):
        n += 1
    return sign * float(n * ulp)


def test_combine_term_association(oracle_mod):
    """One sub-block term, I = 7305, d = f16 0x3EE5 (1.7236328125), sc = 59, dx = 0x3AA69B6D
    (dmin = 0, so the min term is zero): (f32(I) * ws) * dx rounds to 944.27966..., the other
    association f32(I) * (ws * dx) to 944.27972...; the oracle must give the first."""
    d_bits, sc, I = 0x3EE5, 59, 7305
    dx = struct.unpack("<f", struct.pack("<I", 0x3AA69B6D))[0]
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(struct.pack("<H", d_bits), np.uint8)
    scm = np.zeros(8, np.uint8)
    scm[0] = sc
    blk[4:16] = synth.pack_scale_min_k4(scm[None, :], np.zeros((1, 8), np.uint8))[0]
    F = fractions.Fraction
    d = F(struct.unpack("<e", struct.pack("<H", d_bits))[0])
    ws = _round_f32(d * sc)
    go = _round_f32(F(_round_f32(F(I) * F(ws))) * F(dx))
    alt = _round_f32(F(I) * F(_round_f32(F(ws) * F(dx))))
    assert go != alt  # the case separates the two associations
    IS = np.zeros(8, np.int32)
    IS[0] = I
    got = oracle_mod.q4k_combine_row(blk, 1, np.full(8, dx, np.float32), IS, np.zeros(8, np.int32))
    assert got == go, (got, go, alt)


def test_int8_route_close_to_f32(oracle_mod):
    """TestQ4KInt8DotMatchesF32's gate on this oracle (random blocks, gaussian activation)."""
    out, in_ = 48, 768
    raw = synth.q4k_weights(out, in_, 23)
    x = np.random.default_rng(23).standard_normal(in_).astype(np.float32)
    y8 = oracle_mod.q4k_matrows_int8(raw, out, in_, x)
    yf = oracle_mod.q4k_matrows(raw, out, in_, x)
    rms = float(np.sqrt(np.mean(yf.astype(np.float64) ** 2)))
    assert rms > 1e-9
    rel = float(np.max(np.abs(y8.astype(np.float64) - yf))) / rms
    print(f"int8 vs f32 max-abs/RMS = {rel:.4e}")
    assert rel <= 0.05
    assert rel > 0  # the int8 route really quantizes the activation


def test_gemm_int8_is_per_token_gemv(oracle_mod):
    """q4kGemmRangeInt8 (internal/model/quant_q4k.go:359-372): each token on its own."""
    out, in_, P = 7, 512, 3
    raw = synth.q4k_weights(out, in_, 4)
    X = np.random.default_rng(4).standard_normal((P, in_)).astype(np.float32)
    Y = oracle_mod.q4k_gemm_int8(raw, out, in_, X, P)
    for t in range(P):
        np.testing.assert_array_equal(Y[t], oracle_mod.q4k_matrows_int8(raw, out, in_, X[t]))


def test_q8round_nan_and_overflow(oracle_mod):
    """amd64's int32(NaN) / int32(|x| >= 2^31) is 0x80000000 and Go's int32 t-- wraps: NaN and
    3e9 end at -127 (the fraction is NaN, or positive so t++ stays negative), -3e9 at +127
    (0x80000000 - 1 wraps to 2^31 - 1)."""
    assert oracle_mod.q8round(float("nan")) == -127
    assert oracle_mod.q8round(3e9) == -127
    assert oracle_mod.q8round(-3e9) == 127
    assert oracle_mod.q8round(126.5) == 127 and oracle_mod.q8round(-0.5) == -1
