"""Pin the oracle (the C restatement of fak's Go Q4_K / Q8_0 path) against things other than
itself: IEEE conversions, hand-derived goldens from the reference's tests, integer-exact closed
forms, order-revealing adversarial sums, f64 brute force, and the reference's own invariants.

Reference tests mirrored here (internal/...):
  model/quant_kquant_test.go:112-203  TestKQuantDequantGolden (Q8_0 golden; Q5_K packing case)
  model/quant_kquant_test.go:51-88    TestKQuantMatRowsMatchesDequantRef (lcgBytes fixture)
  model/quant_q4k_test.go:79-96       TestQ4KDequantSuperBlockMatchesRef
  model/quant_q4k_test.go:105-161     TestQ4KMatRowsMatchesF32 (max|d|/RMS <= 1e-3)
  model/prefill_q4k_test.go:75-110    TestQ4KGemmMatchesMatRows (bit-identical)
  model/quant_q4k_test.go:234-241     TestQ4KFromRawGuards
  model/quant_test.go:53-78           TestQ8RoundMatchesMathRound
  model/quant_q4k_int8_bench_test.go:13-31  benchQ4KFixture
"""
import numpy as np
import pytest

from fak_amd import synth
from tests import fixtures as fx


# ---- a1: F16BitsToF32Bits --------------------------------------------------------------------

def test_f16_to_f32_exhaustive(oracle_mod):
    """All 65,536 half patterns: finite and infinite values equal numpy's IEEE conversion; NaNs
    keep sign and payload unquieted (quantbits.go:31-32)."""
    L = oracle_mod.lib()
    h = np.arange(65536, dtype=np.uint32)
    got = np.array([L.fr_f16_bits_to_f32_bits(int(v)) for v in h], np.uint32)
    ieee = h.astype(np.uint16).view(np.float16).astype(np.float32).view(np.uint32)
    exp = (h >> 10) & 0x1F
    frac = h & 0x3FF
    nan = (exp == 0x1F) & (frac != 0)
    np.testing.assert_array_equal(got[~nan], ieee[~nan])
    want_nan = ((h & 0x8000) << 16) | 0x7F800000 | (frac << 13)
    np.testing.assert_array_equal(got[nan], want_nan[nan])
    # the subnormal branch really is exercised and lands on exact powers of two
    assert got[0x0001] == np.float32(2.0 ** -24).view(np.uint32)
    assert got[0x03FF] == np.float32(1023 * 2.0 ** -24).view(np.uint32)


# ---- a2: GetScaleMinK4 and its inverse -------------------------------------------------------

def test_scale_min_packer_roundtrip_exhaustive(oracle_mod):
    """Every value 0..63 in every one of the 16 six-bit fields survives pack -> unpack, so the
    12-byte field is a bijection of 16 uniform six-bit fields."""
    for pos in range(16):
        for v in range(64):
            fields = np.random.default_rng(pos * 64 + v).integers(0, 64, 16, dtype=np.uint8)
            fields[pos] = v
            q = synth.pack_scale_min_k4(fields[:8][None], fields[8:][None])[0]
            for j in range(8):
                assert oracle_mod.get_scale_min_k4(j, q) == (fields[j], fields[8 + j])


def test_scale_min_hand_cases(oracle_mod):
    # quant_kquant_test.go:136-141: bytes 1,1,1,1,0,0,0,0,1,1,1,1 -> (scale,min) = (1,0) for all j
    q = np.array([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1], np.uint8)
    for j in range(8):
        assert oracle_mod.get_scale_min_k4(j, q) == (1, 0)
    # high-pair splice by hand: q[0]=0xC0 (top bits 3 -> scale4 bits 4-5), q[8]=0x5A
    q = np.zeros(12, np.uint8)
    q[0], q[4], q[8] = 0xC0 | 5, 0x80 | 7, 0x5A
    assert oracle_mod.get_scale_min_k4(0, q) == (5, 7)
    assert oracle_mod.get_scale_min_k4(4, q) == (0xA | (3 << 4), 0x5 | (2 << 4))


# ---- a3: q4kDequantSuperBlock ----------------------------------------------------------------

def _block(d_bits, dmin_bits, sc, mn, qs) -> np.ndarray:
    b = np.zeros(144, np.uint8)
    b[0:2] = [d_bits & 0xFF, d_bits >> 8]
    b[2:4] = [dmin_bits & 0xFF, dmin_bits >> 8]
    b[4:16] = synth.pack_scale_min_k4(np.array(sc, np.uint8)[None], np.array(mn, np.uint8)[None])[0]
    b[16:] = qs
    return b


def test_q4k_dequant_golden_constant(oracle_mod):
    """d=2, dmin=0, every (scale,min)=(1,0), every nibble 3 -> w = 6 (the Q5_K golden of
    quant_kquant_test.go:132-153, restated for Q4_K)."""
    b = _block(0x4000, 0, [1] * 8, [0] * 8, np.full(128, 0x33, np.uint8))
    w = oracle_mod.q4k_dequant(b, 1, 256)
    assert np.all(w == 6.0)


def test_q4k_dequant_golden_index_map(oracle_mod):
    """Distinct scales/mins/nibbles: w[64k+l] = d*sc[2k]*lo(qs[32k+l]) - dmin*m[2k] and
    w[64k+32+l] = d*sc[2k+1]*hi(qs[32k+l]) - dmin*m[2k+1] (exact dyadic arithmetic)."""
    sc = [1, 2, 3, 5, 8, 13, 21, 34]
    mn = [0, 1, 4, 9, 16, 25, 36, 49]
    qs = np.array([(7 * i + 3) & 0xFF for i in range(128)], np.uint8)
    b = _block(0x3800, 0x3400, sc, mn, qs)  # d = 0.5, dmin = 0.25
    w = oracle_mod.q4k_dequant(b, 1, 256)[0]
    for k in range(4):
        for l in range(32):
            q = int(qs[32 * k + l])
            assert w[64 * k + l] == 0.5 * sc[2 * k] * (q & 15) - 0.25 * mn[2 * k]
            assert w[64 * k + 32 + l] == 0.5 * sc[2 * k + 1] * (q >> 4) - 0.25 * mn[2 * k + 1]


def _numpy_q4k_dequant(raw: np.ndarray, nb: int) -> np.ndarray:
    """Independent vectorised restatement of the GGML Q4_K formula (numpy float32, no fusion)."""
    blk = raw.reshape(nb, 144)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dm = blk[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    q = blk[:, 4:16].astype(np.uint32)
    sc = np.empty((nb, 8), np.uint32)
    mn = np.empty((nb, 8), np.uint32)
    sc[:, :4] = q[:, 0:4] & 63
    mn[:, :4] = q[:, 4:8] & 63
    sc[:, 4:] = (q[:, 8:12] & 0xF) | ((q[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (q[:, 8:12] >> 4) | ((q[:, 4:8] >> 6) << 4)
    d1 = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
    m1 = (dm[:, None] * mn.astype(np.float32)).astype(np.float32)
    nib = blk[:, 16:].reshape(nb, 4, 32)
    lo = (nib & 15).astype(np.float32)
    hi = (nib >> 4).astype(np.float32)
    w = np.empty((nb, 4, 2, 32), np.float32)
    w[:, :, 0, :] = (d1[:, 0::2, None] * lo) - m1[:, 0::2, None]
    w[:, :, 1, :] = (d1[:, 1::2, None] * hi) - m1[:, 1::2, None]
    return w.reshape(nb, 256)


def test_q4k_dequant_random_vs_numpy(oracle_mod):
    """Random blocks from the benchmark generator (incl. f16-subnormal d/dmin) plus fully random
    bytes with finite d/dmin: bit-identical to an independent numpy restatement."""
    nb = 2000
    raw = synth.q4k_weights(nb, 256, seed=42)
    d = raw.reshape(nb, 144)[:, 0:2].copy().view(np.float16)[:, 0]
    assert np.any(np.abs(d) < np.float16(6.1e-5)) and np.any(d != 0)  # subnormals present
    got = oracle_mod.q4k_dequant(raw, nb, 256)
    np.testing.assert_array_equal(got.view(np.uint32), _numpy_q4k_dequant(raw, nb).view(np.uint32))
    rnd = np.random.default_rng(7).integers(0, 256, (nb, 144), dtype=np.uint8)
    rnd[:, 1] = (rnd[:, 1] & 0x83) | (15 << 2)  # finite exponent, like randQ4KBlock
    rnd[:, 3] = (rnd[:, 3] & 0x83) | (14 << 2)
    got = oracle_mod.q4k_dequant(rnd.reshape(-1), nb, 256)
    np.testing.assert_array_equal(got.view(np.uint32),
                                  _numpy_q4k_dequant(rnd.reshape(-1), nb).view(np.uint32))


# ---- a4 / a5: q4kMatRowsRange / q4kGemmRange -------------------------------------------------

def test_q4k_gemv_integer_exact_fixture(oracle_mod):
    """benchQ4KFixture (seed 0xfeedface12345678, d=1, dmin=0, x=(i*13)%29-14) at in=1024: every
    weight is the integer sc*n and every partial sum stays below 2^24, so the f32 result must
    equal the exact integer dot product."""
    out, in_ = 48, 1024
    nb = out * in_ // 256
    raw = fx.pin_f16_scale(fx.lcg_bytes(nb * 144, 0xFEEDFACE12345678), nb, 144, fx.F16_ONE, 0)
    x = np.array([(i * 13) % 29 - 14 for i in range(in_)], np.float32)
    w = _numpy_q4k_dequant(raw, nb).reshape(out, in_).astype(np.int64)
    want = (w * x.astype(np.int64)).sum(axis=1)
    got = oracle_mod.q4k_matrows(raw, out, in_, x)
    np.testing.assert_array_equal(got, want.astype(np.float32))


def test_q4k_gemv_accumulation_order(oracle_mod):
    """Order-revealing sums: with every weight 1, x[0]=2^24, x[1]=x[2]=x[3]=1 the reference's
    4-accumulator dot gives ((2^24+1)+(1+1)) = 2^24+2 (s0+s1 rounds to even), while a sequential
    or 8-lane sum gives 2^24. A second super-block of x=1 then adds 256 in one step."""
    ones = np.full(128, 0x11, np.uint8)
    b = _block(F16(1.0), 0, [1] * 8, [0] * 8, ones)
    raw = np.concatenate([b, b])
    x = np.zeros(512, np.float32)
    x[0] = 2.0 ** 24
    x[1:4] = 1.0
    got = oracle_mod.q4k_matrows(raw, 1, 512, x)
    assert got[0] == np.float32(2.0 ** 24 + 2)
    x[256:] = 1.0
    got = oracle_mod.q4k_matrows(raw, 1, 512, x)
    assert got[0] == np.float32(2.0 ** 24 + 2) + np.float32(256)
    # lanes: x[4] lands in s0 (lost against 2^24), x[5] in s1 (kept)
    x = np.zeros(512, np.float32)
    x[0], x[4], x[5] = 2.0 ** 24, 1.0, 1.0
    assert oracle_mod.q4k_matrows(raw, 1, 512, x)[0] == np.float32(2.0 ** 24)


def F16(v: float) -> int:
    return int(np.array([v], np.float16).view(np.uint16)[0])


def test_q4k_gemv_vs_f64_bruteforce(oracle_mod):
    """TestQ4KMatRowsMatchesF32 shape [32,768] with benchmark-statistics blocks: max|d|/RMS vs an
    f64 dot over the dequantized weights is at f32 rounding level (<< 1e-3)."""
    out, in_ = 32, 768
    raw = synth.q4k_weights(out, in_, seed=7)
    x = synth.activations(1, in_, seed=8)[0]
    w = _numpy_q4k_dequant(raw, out * in_ // 256).reshape(out, in_)
    ref = w.astype(np.float64) @ x.astype(np.float64)
    got = oracle_mod.q4k_matrows(raw, out, in_, x)
    rel = np.max(np.abs(got - ref)) / np.sqrt(np.mean(ref ** 2))
    assert rel < 1e-5, rel


@pytest.mark.parametrize("P", [1, 3, 8])
def test_q4k_gemm_bit_identical_to_gemv(oracle_mod, P):
    """TestQ4KGemmMatchesMatRows: Y[t,o] == q4kMatRows(X[t])[o] bitwise."""
    out, in_ = 32, 768
    raw = synth.q4k_weights(out, in_, seed=11)
    X = synth.activations(P, in_, seed=12)
    Y = oracle_mod.q4k_gemm(raw, out, in_, X, P)
    for t in range(P):
        np.testing.assert_array_equal(Y[t].view(np.uint32),
                                      oracle_mod.q4k_matrows(raw, out, in_, X[t]).view(np.uint32))


def test_parallel_split_is_bit_identical(oracle_mod):
    """parFor row split (parallel.go:266-330) computes each row serially: any worker count gives
    the same bits, including the ragged tail (odd out)."""
    out, in_ = 97, 512
    raw = synth.q4k_weights(out, in_, seed=3)
    x = synth.activations(1, in_, seed=4)[0]
    y1 = oracle_mod.q4k_matrows(raw, out, in_, x, workers=1)
    for w in (2, 5, 8):
        np.testing.assert_array_equal(y1.view(np.uint32),
                                      oracle_mod.q4k_matrows(raw, out, in_, x, workers=w).view(np.uint32))
    X = synth.activations(4, in_, seed=5)
    np.testing.assert_array_equal(oracle_mod.q4k_gemm(raw, out, in_, X, 4, workers=1),
                                  oracle_mod.q4k_gemm(raw, out, in_, X, 4, workers=7))


# ---- a7: Q8_0 ----------------------------------------------------------------------------------

def test_q8_0_dequant_golden(oracle_mod):
    """quant_kquant_test.go:154-167: d=2, code[i]=(i%5)-2 -> w = 2*((i%5)-2)."""
    b = np.zeros(34, np.uint8)
    b[0:2] = [0x00, 0x40]
    b[2:] = np.array([(i % 5) - 2 for i in range(32)], np.int8).view(np.uint8)
    w = oracle_mod.q8_0_dequant(b, 1, 32)[0]
    np.testing.assert_array_equal(w, np.array([2.0 * ((i % 5) - 2) for i in range(32)], np.float32))


def test_q8_0_gemv_lcg_fixture_integer_exact(oracle_mod):
    """TestKQuantMatRowsMatchesDequantRef's Q8_0 case: out=9, in=512, lcgBytes seed
    0x9e3779b97f4a7c15, d pinned to 1.0, x=(i*7)%23-11. All products and partial sums are small
    integers, so the result is the exact integer dot."""
    out, in_ = 9, 512
    nb = out * in_ // 32
    raw = fx.pin_f16_scale(fx.lcg_bytes(nb * 34, 0x9E3779B97F4A7C15), nb, 34)
    x = np.array([(i * 7) % 23 - 11 for i in range(in_)], np.float32)
    codes = raw.reshape(nb, 34)[:, 2:].view(np.int8).reshape(out, in_).astype(np.int64)
    want = (codes * x.astype(np.int64)).sum(axis=1).astype(np.float32)
    np.testing.assert_array_equal(oracle_mod.q8_0_matrows(raw, out, in_, x), want)
    np.testing.assert_array_equal(oracle_mod.q8_0_matrows(raw, out, in_, x, workers=4), want)


def test_q8_0_gemv_accumulation_order(oracle_mod):
    """Per 32-block the same 4-lane dot: x[0]=2^24, x[1..3]=1 with unit weights -> 2^24+2."""
    b = np.zeros(34, np.uint8)
    b[0:2] = [0x00, 0x3C]
    b[2:] = 1
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2], x[3] = 2.0 ** 24, 1, 1, 1
    assert oracle_mod.q8_0_matrows(b, 1, 32, x)[0] == np.float32(2.0 ** 24 + 2)


def test_q8_0_vs_f64_bruteforce(oracle_mod):
    out, in_ = 64, 576
    raw = synth.q8_0_weights(out, in_, seed=1)
    x = synth.activations(1, in_, seed=2)[0]
    w = oracle_mod.q8_0_dequant(raw, out, in_)
    blk = raw.reshape(-1, 34)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    w64 = blk[:, 2:].view(np.int8).astype(np.float64) * d[:, None]
    np.testing.assert_array_equal(w.reshape(-1, 32), w64.astype(np.float32))
    ref = w64.reshape(out, in_) @ x.astype(np.float64)
    got = oracle_mod.q8_0_matrows(raw, out, in_, x)
    assert np.max(np.abs(got - ref)) / np.sqrt(np.mean(ref ** 2)) < 1e-5


# ---- a8: the HAL Q8 lane -----------------------------------------------------------------------

def test_q8round_matches_round_half_away(oracle_mod):
    """TestQ8RoundMatchesMathRound over a dense sweep incl. exact .5 ties and clamping."""
    xs = np.concatenate([np.arange(-140, 140, 0.25, dtype=np.float32),
                         np.random.default_rng(0).uniform(-130, 130, 20000).astype(np.float32)])
    for v in xs:
        want = int(np.clip(np.sign(v) * np.floor(np.abs(np.float64(v)) + 0.5), -127, 127))
        assert oracle_mod.q8round(float(v)) == want, v


def test_quantize_and_qdot8_closed_form(oracle_mod):
    """Activations that are exact multiples of amax/127 quantize exactly; the int8 dot is then
    the exact integer sum times the two scales (powers of two here, so no rounding)."""
    codes = np.random.default_rng(1).integers(-127, 128, 64).astype(np.int8)
    codes[0], codes[32] = 127, -127  # amax = 127 * 2^-3 in each block
    x = codes.astype(np.float32) * np.float32(0.125)
    q, d = oracle_mod.quantize_vec_q8(x)
    np.testing.assert_array_equal(q, codes)
    np.testing.assert_array_equal(d, np.float32(0.125))
    qw = np.random.default_rng(2).integers(-127, 128, 64).astype(np.int8)
    dw = np.array([0.5, 0.25], np.float32)
    got = oracle_mod.qdot8(qw, dw, q, d)
    i0 = int((qw[:32].astype(np.int64) * codes[:32]).sum())
    i1 = int((qw[32:].astype(np.int64) * codes[32:]).sum())
    assert got == np.float32(i0 * 0.5 * 0.125 + i1 * 0.25 * 0.125)
    assert oracle_mod.qgemm8cell(qw, dw, q, d) == got  # both exact here


def test_qgemm8cell_lane_tree(oracle_mod):
    """qgemm8cell keeps 16 float lanes per block and reduces them 8->4->2->1 at the end, unlike
    qdot8's per-block float combine: 2^24 in lane 0 swallows later +1s in that lane only."""
    qw = np.zeros(64, np.int8)
    qx = np.zeros(64, np.int8)
    qw[0], qx[0] = 64, 64     # block 0, lane 0: 4096 * s
    qw[32], qx[32] = 1, 1     # block 1, lane 0: +1 * s
    qw[34], qx[34] = 1, 1     # block 1, lane 1: +1 * s
    dw = np.array([4096.0, 1.0], np.float32)  # block 0 lane 0 -> 2^24
    dx = np.array([1.0, 1.0], np.float32)
    # lane 0: 2^24 + 1 rounds to 2^24 (ties to even); lane 1 holds 1; the tree's final
    # acc[0] + acc[1] = 2^24 + 1 rounds to 2^24 again.
    assert oracle_mod.qgemm8cell(qw, dw, qx, dx) == np.float32(2.0 ** 24)
    # qdot8 sums block 1's integers first (isum = 2), then adds 2 to 2^24 exactly.
    assert oracle_mod.qdot8(qw, dw, qx, dx) == np.float32(2.0 ** 24 + 2)


# ---- the CUDA witness fixture (cuda_quant_test.go:212-227, 278-316) ---------------------------

def test_cuda_witness_fixture_reference_side(oracle_mod):
    """Reproduce the CUDA Q4_K witness inputs (lcg seed 0x4b4b, out=320, in=256, non-IEEE
    f32ToF16Bits) and check the reference side of that gate on the CPU: the Q4_K GEMV against
    an f64 product of the dequantized weights, argmax-exact on the dominant row."""
    g = fx.LCG(0x4B4B)
    out, in_ = 320, 256
    raw = fx.rand_q4k_bytes(g, out, in_)
    w = oracle_mod.q4k_dequant(raw, out, in_)
    target = int(np.argmax((w.astype(np.float64) ** 2).sum(axis=1)))
    x = w[target].copy()
    y = oracle_mod.q4k_matrows(raw, out, in_, x)
    ref = w.astype(np.float64) @ x.astype(np.float64)
    assert int(np.argmax(y)) == target == int(np.argmax(ref))
    cos = np.dot(y, ref) / (np.linalg.norm(y) * np.linalg.norm(ref))
    assert cos > 0.9999999


def test_guards(oracle_mod):
    """TestQ4KFromRawGuards: a non-multiple-of-256 reduction dim is rejected."""
    with pytest.raises(AssertionError):
        oracle_mod.q4k_matrows(np.zeros(144, np.uint8), 1, 255, np.zeros(255, np.float32))
    with pytest.raises(ValueError):
        synth.q4k_weights(1, 255, 0)
