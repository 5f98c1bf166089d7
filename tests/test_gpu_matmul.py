"""Device matmul parity against the oracle (fak's Go CPU path restated in C) on the same seeded
inputs, at the reference's tolerances (metric of internal/model/quant_q4k_test.go:140-158):

  GEMV (P <= 16, f32-accumulate)  max|dY|/RMS(Y_ref) <= 1e-3
  P > 16 (f16 MFMA: 17..32 on the small-M kernel's f16 form, more on the prefill GEMM)
                                  max|dY|/RMS(Y_ref) <= 1e-2

Shapes: the five workloads (Q8_0 576->1536; Q4_K 3584->18944 and 18944->3584; prefill
M=128/512/2048 at 3584->18944; 27B-class 5120<->25600 at M=1,4,8,16) plus small/ragged shapes
and the reference's witness shapes. Full-size GEMMs are checked on sampled output rows spread
over every 128-row block (the oracle cost is per row), everything else on every output.
"""
import numpy as np
import pytest

from fak_amd import synth
from tests.gpu_util import cosine, knobs, q4k_matmul, q8_0_matmul, rel_err, spread_rows

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3
GEMM_TOL = 1e-2


def _check_q4k(oracle_mod, out, in_, P, seed, tol, workers=16, rows=None):
    print(f"[case] q4k out={out} in={in_} P={P} seed={seed}", flush=True)
    raw = synth.q4k_weights(out, in_, seed=seed)
    X = synth.activations(P, in_, seed=seed + 1)
    Y = q4k_matmul(raw, out, in_, X, P)
    assert np.all(np.isfinite(Y))
    if rows is None:
        ref = oracle_mod.q4k_gemm(raw, out, in_, X, P, workers=workers)
        got = Y
    else:
        # `rows` is a budget: at least two rows in every 128-row block
        rb = (in_ // 256) * 144
        sel = spread_rows(out, per_block=max(2, rows // -(-out // 128)))
        sub = np.concatenate([raw[o * rb:(o + 1) * rb] for o in sel])
        ref = oracle_mod.q4k_gemm(sub, len(sel), in_, X, P, workers=workers)
        got = Y[:, sel]
    e = rel_err(got, ref)
    print(f"    max|d|/RMS = {e:.3e}  cosine = {cosine(got, ref):.9f}", flush=True)
    assert e <= tol, e
    return e


@pytest.mark.parametrize("out,in_,P", [
    (16, 256, 1), (1, 256, 1), (9, 512, 1), (33, 768, 3), (320, 256, 8), (100, 1024, 16),
    (64, 2560, 5), (17, 4096, 13)])
def test_q4k_gemv_small_shapes(hip, oracle_mod, out, in_, P):
    _check_q4k(oracle_mod, out, in_, P, seed=out * 31 + in_ + P, tol=GEMV_TOL)


@pytest.mark.parametrize("out,in_", [(18944, 3584), (3584, 18944)])
def test_q4k_gemv_7b_ffn(hip, oracle_mod, out, in_):
    """Decode GEMV at the Qwen2.5-7B FFN shapes (gate/up and down)."""
    _check_q4k(oracle_mod, out, in_, 1, seed=2024 + out, tol=GEMV_TOL)


def test_q4k_lm_head_7b(hip, oracle_mod):
    """The largest matmul of a Qwen2.5-7B decode token, a Q4_K lm_head 3584 -> 152064 (306 MB),
    every output checked."""
    _check_q4k(oracle_mod, 152064, 3584, 1, seed=152064, tol=GEMV_TOL)


@pytest.mark.parametrize("P", [2, 3, 4])
def test_q4k_gemv_7b_gateup_2_to_4_tokens(hip, oracle_mod, P):
    """Two to four tokens on the 7B gate/up shape: one-wave tiles streaming 14 records each, the
    ring refilled unconditionally so every ring wait counts exactly; every output checked."""
    _check_q4k(oracle_mod, 18944, 3584, P, seed=4096 + P, tol=GEMV_TOL)


@pytest.mark.parametrize("out,in_,P", [(5120, 25600, 2), (3584, 18944, 3), (3584, 18944, 4)])
def test_q4k_gemv_global_operands_natural(hip, oracle_mod, out, in_, P):
    """Shapes whose activation operands do not fit in LDS, so the GEMV takes its global-operand
    path by itself: the 27B down projection at 2 tokens, the 7B one at 3 and 4."""
    _check_q4k(oracle_mod, out, in_, P, seed=out + in_ + 7 * P, tol=GEMV_TOL)


@pytest.mark.parametrize("P", [1, 2, 4])
@pytest.mark.parametrize("out,in_", [(18944, 3584), (3584, 18944)])
def test_q4k_gemv_global_operands_forced(hip, oracle_mod, monkeypatch, out, in_, P):
    """FAK_HIP_GEMV_GLOBALX=1 forces the global-operand path on the C2 shapes; it is also
    bit-identical to the LDS path (same operands, same order)."""
    raw = synth.q4k_weights(out, in_, seed=out + P)
    X = synth.activations(P, in_, seed=in_ + P)
    lds = q4k_matmul(raw, out, in_, X, P)
    with knobs(monkeypatch, FAK_HIP_GEMV_GLOBALX=1):
        glob = q4k_matmul(raw, out, in_, X, P)
    ref = oracle_mod.q4k_gemm(raw, out, in_, X, P, workers=16)
    assert rel_err(glob, ref) <= GEMV_TOL
    assert np.array_equal(glob.view(np.uint32), lds.view(np.uint32))
    assert np.array_equal(lds.view(np.uint32), glob.view(np.uint32))


def test_q4k_gemv16_from_knob_is_clamped(hip, oracle_mod, monkeypatch):
    """FAK_HIP_GEMV16_FROM names the first width on the 5..16-token kernel; values the int8
    kernel cannot take (it holds 1..4 tokens) are ignored, so 6 tokens still get every row."""
    out, in_, P = 512, 2048, 6
    raw = synth.q4k_weights(out, in_, seed=66)
    X = synth.activations(P, in_, seed=67)
    with knobs(monkeypatch, FAK_HIP_GEMV16_FROM=8):
        Y = q4k_matmul(raw, out, in_, X, P)
    assert rel_err(Y, oracle_mod.q4k_gemm(raw, out, in_, X, P)) <= GEMV_TOL


@pytest.mark.parametrize("pattern", ["big", "tiny", "wee", "mixed", "outlier"])
@pytest.mark.parametrize("out,in_,P", [(1024, 3584, 1), (512, 2048, 4), (512, 2048, 8),
                                       (1024, 5120, 16), (512, 2048, 64)])
def test_q4k_activation_scales(hip, oracle_mod, out, in_, P, pattern):
    """Activations far outside f16 (x 1e5, a lone 7e4), far below it (x 1e-20, x 1e-35) and
    mixed within a row: every token row within its route's bound of the oracle, judged per row."""
    from tests.gpu_util import rel_err_rows, scaled_activations
    print(f"[case] q4k scales out={out} in={in_} P={P} {pattern}", flush=True)
    raw = synth.q4k_weights(out, in_, seed=out + P)
    X = scaled_activations(P, in_, 3 * P + 1, pattern)
    Y = q4k_matmul(raw, out, in_, X, P)
    ref = oracle_mod.q4k_gemm(raw, out, in_, X, P, workers=16)
    e = rel_err_rows(Y, ref)
    print(f"    per-row max|d|/RMS = {e:.3e}", flush=True)
    tol = GEMV_TOL if P <= 16 else GEMM_TOL
    assert e <= tol, e


@pytest.mark.parametrize("P", [1, 2, 3, 4])
@pytest.mark.parametrize("out,in_", [(18944, 3584), (3584, 18944), (512, 2048)])
def test_q4k_decode_outlier_rows(hip, oracle_mod, out, in_, P):
    """The 1..4-token GEMV on rows where one activation dominates (a lone 7e4 among N(0,1)
    values, the pattern of models with massive activations): each 32-value block is carried as
    three int8 digits under a power-of-two scale, so the block-mates of the outlier keep ~22 bits
    and every token row stays within the GEMV bound, at the 7B FFN shapes and a small one (full
    output checked)."""
    from tests.gpu_util import rel_err_rows, scaled_activations
    print(f"[case] q4k decode outlier out={out} in={in_} P={P}", flush=True)
    raw = synth.q4k_weights(out, in_, seed=out + in_ + P)
    X = scaled_activations(P, in_, 5 * P + 2, "outlier")
    Y = q4k_matmul(raw, out, in_, X, P)
    e = rel_err_rows(Y, oracle_mod.q4k_gemm(raw, out, in_, X, P, workers=16))
    print(f"    per-row max|d|/RMS = {e:.3e}", flush=True)
    assert e <= GEMV_TOL, e


@pytest.mark.parametrize("P", [8, 16])
@pytest.mark.parametrize("out,in_", [(3584, 18944), (5120, 25600)])
def test_q4k_verify_widths_large_activations(hip, oracle_mod, out, in_, P):
    """The 5..16-token kernel on the down projections with rows of x 1e5, x 1e-20, mixed blocks
    and a lone 7e4: the f16 operands never overflow or flush (full output checked)."""
    from tests.gpu_util import rel_err_rows, scaled_activations
    print(f"[case] q4k verify widths, large activations out={out} in={in_} P={P}", flush=True)
    raw = synth.q4k_weights(out, in_, seed=out + 2 * P)
    X = scaled_activations(P, in_, P + 3, "all")
    Y = q4k_matmul(raw, out, in_, X, P)
    e = rel_err_rows(Y, oracle_mod.q4k_gemm(raw, out, in_, X, P, workers=16))
    print(f"    per-row max|d|/RMS = {e:.3e}", flush=True)
    assert e <= GEMV_TOL, e


def test_q4k_verify_matches_decode_argmax(hip, oracle_mod):
    """Speculative verify runs 2..16 tokens through kernels whose arithmetic differs from the
    one-token decode GEMV (int8 digits for 1..4 tokens, hi/lo f16 for 5..16), so a token's
    output is not bit-identical across widths; the property verify needs is that greedy picks
    agree. On the reference's CUDA witness weights (lcg 0x4b4b, randQ4KBytes) with every token's
    activation aligned to a different row (alignActToRow, internal/compute/cuda_quant_test.go:
    48-84, plus noise), each token's argmax at widths 2..16 equals its argmax decoded alone, and
    the outputs agree within twice the GEMV bound."""
    from tests import fixtures as fx
    g = fx.LCG(0x4B4B)
    out, in_ = 320, 256
    raw = fx.rand_q4k_bytes(g, out, in_)
    w = oracle_mod.q4k_dequant(raw, out, in_)
    rng = np.random.default_rng(17)
    targets = rng.choice(out, 16, replace=False)
    X = np.stack([w[t] + 0.05 * rng.standard_normal(in_).astype(np.float32) * np.abs(w[t]).mean()
                  for t in targets]).astype(np.float32)
    Y1 = np.concatenate([q4k_matmul(raw, out, in_, X[t:t + 1], 1) for t in range(16)])
    for k in (2, 3, 4, 5, 8, 16):
        Yk = q4k_matmul(raw, out, in_, X[:k], k)
        for t in range(k):
            assert int(np.argmax(Yk[t])) == int(np.argmax(Y1[t])), (k, t)
        assert rel_err(Yk, Y1[:k]) <= 2 * GEMV_TOL, k


@pytest.mark.parametrize("pattern", ["big", "tiny", "mixed", "outlier", "all"])
@pytest.mark.parametrize("P", [1, 4, 8, 16, 40])
def test_q8_0_activation_scales(hip, oracle_mod, P, pattern):
    from tests.gpu_util import rel_err_rows, scaled_activations
    out, in_ = 1536, 576
    print(f"[case] q8_0 scales P={P} {pattern}", flush=True)
    raw = synth.q8_0_weights(out, in_, seed=P + 9)
    X = scaled_activations(P, in_, P, pattern)
    Y = q8_0_matmul(raw, out, in_, X, P)
    e = rel_err_rows(Y, oracle_mod.q8_0_gemm(raw, out, in_, X, P))
    print(f"    per-row max|d|/RMS = {e:.3e}", flush=True)
    assert e <= GEMV_TOL, e


@pytest.mark.parametrize("P", [1, 3, 4, 8, 16])
@pytest.mark.parametrize("out,in_", [(25600, 5120), (5120, 25600)])
def test_q4k_small_m_27b(hip, oracle_mod, out, in_, P):
    """Speculative-verify widths on the 27B-class FFN."""
    _check_q4k(oracle_mod, out, in_, P, seed=77 + P + out, tol=GEMV_TOL)


@pytest.mark.parametrize("out,in_,P", [(256, 512, 33), (300, 768, 40), (512, 1024, 128),
                                       (1000, 2048, 200), (64, 256, 1000)])
def test_q4k_gemm_small_shapes(hip, oracle_mod, out, in_, P):
    _check_q4k(oracle_mod, out, in_, P, seed=out + in_ + P, tol=GEMM_TOL)


@pytest.mark.parametrize("out,in_,P", [(18944, 3584, 17), (18944, 3584, 24), (3584, 18944, 32),
                                       (5120, 25600, 20), (1000, 2048, 19), (300, 768, 32),
                                       (16, 256, 31), (100, 1024, 25)])
def test_q4k_small_prefill_17_to_32(hip, oracle_mod, out, in_, P):
    """17..32 tokens on the 32x32 small-M kernel with one f16 operand row per token (K split in
    ranges at the long shapes): every output against the oracle at the GEMM bound."""
    rows = 256 if out * in_ > 4096 * 4096 else None
    e = _check_q4k(oracle_mod, out, in_, P, seed=3 * out + in_ + P, tol=GEMM_TOL, rows=rows)
    assert e <= 2e-3, e  # f16 activations under a per-token power-of-two scale: ~1e-3


@pytest.mark.parametrize("pattern", ["big", "tiny", "mixed", "outlier"])
def test_q4k_small_prefill_activation_scales(hip, oracle_mod, pattern):
    from tests.gpu_util import rel_err_rows, scaled_activations
    out, in_, P = 512, 2048, 24
    print(f"[case] q4k 17..32 scales out={out} in={in_} P={P} {pattern}", flush=True)
    raw = synth.q4k_weights(out, in_, seed=out + P)
    X = scaled_activations(P, in_, 3 * P + 1, pattern)
    Y = q4k_matmul(raw, out, in_, X, P)
    ref = oracle_mod.q4k_gemm(raw, out, in_, X, P, workers=16)
    e = rel_err_rows(Y, ref)
    print(f"    per-row max|d|/RMS = {e:.3e}", flush=True)
    assert e <= GEMM_TOL, e


@pytest.mark.parametrize("P", [128, 512, 2048])
def test_q4k_gemm_prefill_7b(hip, oracle_mod, P):
    """Prefill GEMM at M=128/512/2048, K=3584, N=18944, checked on two output rows in every
    one of the 148 row blocks (296 rows)."""
    _check_q4k(oracle_mod, 18944, 3584, P, seed=512 + P, tol=GEMM_TOL, rows=256)


@pytest.mark.parametrize("out,in_,P", [(300, 768, 600), (1000, 2048, 520), (64, 256, 1000),
                                       (18944, 3584, 512)])
def test_q4k_gemm_forms_bit_identical(hip, oracle_mod, monkeypatch, out, in_, P):
    """The staged GEMM (the default: four waves of 32 rows, weights loaded straight to the
    registers of the lanes that use them) and the four-wave 2x2 GEMM (records staged through LDS)
    share the tile, the K order and each accumulator's MFMA sequence: their outputs agree bit
    for bit, on whole and ragged row / token tiles, and the staged result meets the GEMM bound
    against the oracle (sampled rows at the 7B shape)."""
    print(f"[case] gemm forms out={out} in={in_} P={P}", flush=True)
    raw = synth.q4k_weights(out, in_, seed=out + 3 * P)
    X = synth.activations(P, in_, seed=P + 5)
    # without a K split, and with the K ranges the launch rule picks (the same for both forms,
    # added by the same ordered reduce)
    with knobs(monkeypatch, FAK_HIP_GEMM32_FORM=1, FAK_HIP_GEMM32_SK=1):
        Y1 = q4k_matmul(raw, out, in_, X, P)
    with knobs(monkeypatch, FAK_HIP_GEMM32_SK=1):
        Y3 = q4k_matmul(raw, out, in_, X, P)
    assert np.array_equal(Y1.view(np.uint32), Y3.view(np.uint32))
    with knobs(monkeypatch, FAK_HIP_GEMM32_FORM=1):
        Y2 = q4k_matmul(raw, out, in_, X, P)
    Y4 = q4k_matmul(raw, out, in_, X, P)
    assert np.array_equal(Y2.view(np.uint32), Y4.view(np.uint32))
    if out > 4096:
        rb = (in_ // 256) * 144
        sel = spread_rows(out)
        sub = np.concatenate([raw[o * rb:(o + 1) * rb] for o in sel])
        ref = oracle_mod.q4k_gemm(sub, len(sel), in_, X, P, workers=16)
        got = Y3[:, sel]
    else:
        ref = oracle_mod.q4k_gemm(raw, out, in_, X, P, workers=16)
        got = Y3
    assert rel_err(got, ref) <= GEMM_TOL


@pytest.mark.parametrize("out,in_,P", [(18944, 3584, 2048), (18900, 1024, 2100)])
def test_q4k_gemm_wide_tiles(hip, oracle_mod, monkeypatch, out, in_, P):
    """From eight token tiles (M > 896) the staged kernel takes 256-row workgroups (four waves of
    64 rows). Every output keeps the 128-row kernel's MFMA sequence, so the result is
    bit-identical to the unsplit four-wave 2x2 form, on whole and ragged row and token tiles, and
    meets the GEMM bound on rows spread over every row tile."""
    print(f"[case] gemm wide tiles out={out} in={in_} P={P}", flush=True)
    raw = synth.q4k_weights(out, in_, seed=out + 5 * P)
    X = synth.activations(P, in_, seed=P + 19)
    Y = q4k_matmul(raw, out, in_, X, P)
    with knobs(monkeypatch, FAK_HIP_GEMM32_FORM=1, FAK_HIP_GEMM32_SK=1):
        Y1 = q4k_matmul(raw, out, in_, X, P)
    assert np.array_equal(Y.view(np.uint32), Y1.view(np.uint32))
    rb = (in_ // 256) * 144
    sel = spread_rows(out, per_block=1)
    sub = np.concatenate([raw[o * rb:(o + 1) * rb] for o in sel])
    assert rel_err(Y[:, sel], oracle_mod.q4k_gemm(sub, len(sel), in_, X, P, workers=16)) <= GEMM_TOL


@pytest.mark.parametrize("out,in_,P", [(3584, 18944, 512), (1000, 2048, 520), (18944, 3584, 128),
                                       (300, 4096, 40), (3584, 18944, 1024), (3000, 18944, 1000)])
def test_q4k_gemm_k_split(hip, oracle_mod, out, in_, P):
    """Grids too small for the GPU split K and add the ranges' partial sums in range order: the
    result meets the GEMM bound against the oracle (sampled rows for the 7B shapes) and is the
    same bits call after call. From eight token tiles the split tiles are the 256-row ones (the
    7B down projection at 1024 tokens: 112 tiles in 4 ranges; 3000 rows and 1000 tokens: ragged
    row and token tiles in 5 ranges)."""
    print(f"[case] gemm k split out={out} in={in_} P={P}", flush=True)
    raw = synth.q4k_weights(out, in_, seed=out + 7 * P)
    X = synth.activations(P, in_, seed=P + 11)
    Y = q4k_matmul(raw, out, in_, X, P)
    assert np.array_equal(Y.view(np.uint32), q4k_matmul(raw, out, in_, X, P).view(np.uint32))
    if out * in_ > 4_000_000:
        rb = (in_ // 256) * 144
        sel = spread_rows(out, per_block=1)
        sub = np.concatenate([raw[o * rb:(o + 1) * rb] for o in sel])
        ref = oracle_mod.q4k_gemm(sub, len(sel), in_, X, P, workers=16)
        got = Y[:, sel]
    else:
        ref = oracle_mod.q4k_gemm(raw, out, in_, X, P, workers=16)
        got = Y
    assert rel_err(got, ref) <= GEMM_TOL


@pytest.mark.parametrize("out,in_,P", [(18900, 3584, 500), (18900, 1024, 500), (18944, 3584, 256),
                                       (18944, 3584, 2048)])
def test_q4k_gemm_tail_split(hip, oracle_mod, monkeypatch, out, in_, P):
    """Grids of more tiles than CUs run whole tiles in rounds of one per CU and split only the
    last, partial round's tiles into K ranges (range 0 in Y, the rest added in range order). On
    ragged row and token tiles: the first row block (whole tiles) is bit-identical to the
    unsplit kernel, the last rows (split tiles) meet the GEMM bound against the oracle, and the
    result is the same bits call after call. (128-row workgroups throughout: from eight token
    tiles the default takes 256-row ones, whose 1184 tiles at 2048 tokens need no split.)"""
    print(f"[case] gemm tail split out={out} in={in_} P={P}", flush=True)
    raw = synth.q4k_weights(out, in_, seed=out + 13 * P)
    X = synth.activations(P, in_, seed=P + 17)
    with knobs(monkeypatch, FAK_HIP_GEMM32_NT=1):
        Y = q4k_matmul(raw, out, in_, X, P)
        assert np.array_equal(Y.view(np.uint32), q4k_matmul(raw, out, in_, X, P).view(np.uint32))
    with knobs(monkeypatch, FAK_HIP_GEMM32_SK=1):
        Y1 = q4k_matmul(raw, out, in_, X, P)
    assert np.array_equal(Y[:, :128].view(np.uint32), Y1[:, :128].view(np.uint32))
    rb = (in_ // 256) * 144
    sel = np.concatenate([np.arange(0, 16), np.arange(out - 112, out)])
    sub = np.concatenate([raw[o * rb:(o + 1) * rb] for o in sel])
    ref = oracle_mod.q4k_gemm(sub, len(sel), in_, X, P, workers=16)
    assert rel_err(Y[:, sel], ref) <= GEMM_TOL
    assert rel_err(Y[:, out - 112:], Y1[:, out - 112:]) <= GEMM_TOL


@pytest.mark.parametrize("out,in_,P", [(18944, 3584, 1024), (18900, 3584, 1000)])
def test_q4k_gemm_tail_split_wide(hip, oracle_mod, monkeypatch, out, in_, P):
    """The tail split on 256-row workgroups (eight token tiles, 592 tiles: 512 whole, the last 80
    in 3 K ranges), on whole and ragged row and token tiles: the first row block is
    bit-identical to the unsplit 128-row kernel, sampled rows of every row block and the last
    rows meet the GEMM bound against the oracle, and the result is the same bits call after
    call."""
    print(f"[case] gemm tail split wide out={out} in={in_} P={P}", flush=True)
    raw = synth.q4k_weights(out, in_, seed=out + 3 * P)
    X = synth.activations(P, in_, seed=P + 23)
    Y = q4k_matmul(raw, out, in_, X, P)
    assert np.array_equal(Y.view(np.uint32), q4k_matmul(raw, out, in_, X, P).view(np.uint32))
    with knobs(monkeypatch, FAK_HIP_GEMM32_SK=1):
        Y1 = q4k_matmul(raw, out, in_, X, P)
    assert np.array_equal(Y[:, :256].view(np.uint32), Y1[:, :256].view(np.uint32))
    rb = (in_ // 256) * 144
    sel = np.unique(np.concatenate([spread_rows(out, per_block=1), np.arange(out - 64, out)]))
    sub = np.concatenate([raw[o * rb:(o + 1) * rb] for o in sel])
    ref = oracle_mod.q4k_gemm(sub, len(sel), in_, X, P, workers=16)
    assert rel_err(Y[:, sel], ref) <= GEMM_TOL


def test_q4k_gemm_equals_gemv_per_token_within_tolerance(hip, oracle_mod):
    """The reference pins GEMM(o,t) == GEMV(X_t)(o) bitwise on the CPU; on the device the two
    kernels use different precisions, so each is held to its own bound against the same oracle
    and to each other at the GEMM bound."""
    out, in_, P = 256, 1024, 24
    raw = synth.q4k_weights(out, in_, seed=9)
    X = synth.activations(P, in_, seed=10)
    Yg = q4k_matmul(raw, out, in_, X, P)
    Yv = np.concatenate([q4k_matmul(raw, out, in_, X[t:t + 1], 1) for t in range(P)])
    assert rel_err(Yg, Yv) <= GEMM_TOL


@pytest.mark.parametrize("out,in_,P", [(1536, 576, 1), (9, 512, 1), (17, 96, 3), (64, 1056, 16),
                                       (100, 256, 40), (37, 96, 1), (300, 1056, 1)])
def test_q8_0_matmul(hip, oracle_mod, out, in_, P):
    print(f"[case] q8_0 out={out} in={in_} P={P}", flush=True)
    raw = synth.q8_0_weights(out, in_, seed=out * 3 + in_)
    X = synth.activations(P, in_, seed=out + 1)
    Y = q8_0_matmul(raw, out, in_, X, P)
    ref = oracle_mod.q8_0_gemm(raw, out, in_, X, P)
    e = rel_err(Y, ref)
    print(f"    max|d|/RMS = {e:.3e}", flush=True)
    assert e <= GEMV_TOL, e


def test_q8_0_lcg_fixture_integer_exact(hip, oracle_mod):
    """The reference's Q8_0 GEMV fixture (lcgBytes, d=1, integer x): every product and partial
    sum is a small integer, so the device result must equal the oracle exactly."""
    from tests import fixtures as fx
    out, in_ = 9, 512
    nb = out * in_ // 32
    raw = fx.pin_f16_scale(fx.lcg_bytes(nb * 34, 0x9E3779B97F4A7C15), nb, 34)
    x = np.array([(i * 7) % 23 - 11 for i in range(in_)], np.float32)
    Y = q8_0_matmul(raw, out, in_, x[None], 1)[0]
    np.testing.assert_array_equal(Y, oracle_mod.q8_0_matrows(raw, out, in_, x))


def test_q4k_integer_fixture_exact(hip, oracle_mod):
    """benchQ4KFixture-style inputs (d=1, dmin=0, integer x): the device GEMV is exact."""
    from tests import fixtures as fx
    out, in_ = 48, 1024
    nb = out * in_ // 256
    raw = fx.pin_f16_scale(fx.lcg_bytes(nb * 144, 0xFEEDFACE12345678), nb, 144, fx.F16_ONE, 0)
    x = np.array([(i * 13) % 29 - 14 for i in range(in_)], np.float32)
    Y = q4k_matmul(raw, out, in_, x[None], 1)[0]
    np.testing.assert_array_equal(Y, oracle_mod.q4k_matrows(raw, out, in_, x))


@pytest.mark.parametrize("P", [1, 3, 4, 8, 40])
def test_q4k_group_qkv(hip, oracle_mod, P):
    """A layer's q/k/v sharing one activation (3584 -> 3584, 512, 512) through the group entry:
    every member within the GEMV (P <= 16) or GEMM bound of its own oracle result, and within
    the same bound of the single-matrix entry."""
    from tests.gpu_util import q4k_matmul_group
    in_, outs = 3584, [3584, 512, 512]
    print(f"[case] q4k group qkv in={in_} outs={outs} P={P}", flush=True)
    raws = [synth.q4k_weights(o, in_, seed=300 + i) for i, o in enumerate(outs)]
    X = synth.activations(P, in_, seed=399)
    Ys = q4k_matmul_group(raws, outs, in_, X, P)
    tol = GEMV_TOL if P <= 16 else GEMM_TOL
    for raw, o, Y in zip(raws, outs, Ys):
        ref = oracle_mod.q4k_gemm(raw, o, in_, X, P, workers=16)
        e = rel_err(Y, ref)
        single = q4k_matmul(raw, o, in_, X, P)
        print(f"    out={o}: max|d|/RMS = {e:.3e}, vs single call {rel_err(Y, single):.3e}",
              flush=True)
        assert e <= tol
        assert rel_err(Y, single) <= tol


def test_q4k_group_ragged_members(hip, oracle_mod):
    """Members whose row counts are not multiples of 16 (tile padding inside the group)."""
    from tests.gpu_util import q4k_matmul_group
    in_, outs = 512, [17, 33, 100, 1]
    raws = [synth.q4k_weights(o, in_, seed=500 + i) for i, o in enumerate(outs)]
    X = synth.activations(2, in_, seed=599)
    Ys = q4k_matmul_group(raws, outs, in_, X, 2)
    for raw, o, Y in zip(raws, outs, Ys):
        assert rel_err(Y, oracle_mod.q4k_gemm(raw, o, in_, X, 2)) <= GEMV_TOL
