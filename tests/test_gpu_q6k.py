"""GGUF Q6_K on the device (fhip_q6k_upload / fhip_q6k_dequant_f32 / fhip_q6k_matmul_f32)
against the oracle's q6kDequantSuperBlock and kQuantMatRowsRange(kind Q6_K)
(internal/model/quant_kquant.go:139-163,210-232): dequant bit-identical, the GEMV within
max|dY|/RMS <= 1e-3 (exact on the reference's integer fixture)."""
import numpy as np
import pytest

from fak_amd import fakhip
from tests import q6k_cases as qc
from tests.gpu_util import Dev, knobs, rel_err, spread_rows

pytestmark = pytest.mark.gpu


def upload(raw, out, in_):
    return fakhip.alloc_call("fhip_q6k_upload", np.ascontiguousarray(raw).ctypes.data, out, in_)


def dev_dequant(raw, out, in_):
    lib = fakhip.load()
    w = upload(raw, out, in_)
    try:
        with Dev(out * in_ * 4) as dw:
            fakhip.call("fhip_q6k_dequant_f32", dw.ptr, w, out, in_)
            return dw.to_host(np.float32).reshape(out, in_)
    finally:
        lib.fhip_free(w)


def dev_matmul(raw, out, in_, X, P):
    lib = fakhip.load()
    w = upload(raw, out, in_)
    try:
        with Dev.from_host(np.ascontiguousarray(X, np.float32)) as dx, Dev(P * out * 4) as dy:
            fakhip.call("fhip_q6k_matmul_f32", w, dx.ptr, dy.ptr, out, in_, P)
            return dy.to_host(np.float32).reshape(P, out)
    finally:
        lib.fhip_free(w)


def test_dequant_bit_exact(hip, oracle_mod):
    print("[case] q6k dequant: random blocks, every finite f16 exponent of d", flush=True)
    rng = np.random.default_rng(3)
    nb = 256
    raw = rng.integers(0, 256, size=nb * 210, dtype=np.uint8).reshape(nb, 210)
    d = (np.arange(nb, dtype=np.uint32) * 0x79 + 0x0401) & 0x7BFF  # spread over finite patterns
    d[::7] |= 0x8000
    d[5], d[6] = 0x0001, 0x03FF  # subnormals
    raw[:, 208] = d & 0xFF
    raw[:, 209] = d >> 8
    got = dev_dequant(raw.reshape(-1), 1, nb * 256)
    want = oracle_mod.q6k_dequant(raw.reshape(-1), 1, nb * 256)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_gemv_reference_fixture_exact(hip, oracle_mod):
    raw, x, out, in_ = qc.reference_fixture()
    y = dev_matmul(raw, out, in_, x, 1)[0]
    np.testing.assert_array_equal(y, oracle_mod.q6k_matrows(raw, out, in_, x))


@pytest.mark.parametrize("out,in_,P", [(1536, 3584, 1), (3584, 18944, 1), (152, 4096, 5),
                                       (4096, 512, 3), (37, 256, 8), (17, 66048, 1),
                                       (152064, 3584, 1), (3584, 18944, 2), (3584, 18944, 16),
                                       (1000, 2048, 13), (300, 768, 16), (18944, 3584, 1),
                                       (5120, 4096, 1), (14336, 1024, 1), (8192, 768, 1)])
def test_gemv_matches_oracle(hip, oracle_mod, out, in_, P):
    print(f"[case] q6k gemv out={out} in={in_} P={P}", flush=True)
    rng = np.random.default_rng(out + in_ + P)
    raw = qc.pin_d(rng.integers(0, 256, size=out * (in_ // 256) * 210, dtype=np.uint8), 0x1400)
    X = rng.standard_normal((P, in_)).astype(np.float32)
    Y = dev_matmul(raw, out, in_, X, P)
    ref = oracle_mod.q6k_gemm(raw, out, in_, X, P)
    err = rel_err(Y, ref)
    print(f"    max|d|/RMS = {err:.2e}", flush=True)
    assert err <= 1e-3


@pytest.mark.parametrize("pattern", ["big", "tiny", "wee", "mixed", "outlier"])
@pytest.mark.parametrize("out,in_,P", [(1024, 2048, 1), (3584, 18944, 1), (1024, 2048, 4),
                                       (1024, 2048, 16), (512, 2048, 40)])
def test_activation_scales(hip, oracle_mod, out, in_, P, pattern):
    """Q6_K on activations far outside f16 (x 1e5, a lone 7e4), far below it (x 1e-20, x 1e-35)
    and mixed within a row: every token row within its route's bound of the oracle (1e-3 up to
    16 tokens, 1e-2 on the GEMM), judged per row."""
    from tests.gpu_util import rel_err_rows, scaled_activations
    print(f"[case] q6k scales out={out} in={in_} P={P} {pattern}", flush=True)
    rng = np.random.default_rng(out + in_ + P)
    raw = qc.pin_d(rng.integers(0, 256, size=out * (in_ // 256) * 210, dtype=np.uint8), 0x1400)
    X = scaled_activations(P, in_, 7 * P + 3, pattern)
    Y = dev_matmul(raw, out, in_, X, P)
    e = rel_err_rows(Y, oracle_mod.q6k_gemm(raw, out, in_, X, P))
    print(f"    per-row max|d|/RMS = {e:.3e}", flush=True)
    assert e <= (1e-3 if P <= 16 else 1e-2), e


@pytest.mark.parametrize("out,in_", [(1, 256), (16, 512), (37, 768), (300, 1024)])
def test_repack_round_trip(hip, out, in_):
    """The tiled layout is a byte permutation: repack then unpack returns the raw rows, and
    the padding rows of the last tile are zero."""
    lib = fakhip.load()
    rng = np.random.default_rng(out + in_)
    raw = rng.integers(0, 256, size=out * (in_ // 256) * 210, dtype=np.uint8)
    nb = lib.fhip_q6k_packed_bytes(out, in_)
    assert nb == -(-out // 16) * (in_ // 256) * 3360
    with Dev.from_host(raw) as dr, Dev(nb) as dp, Dev(raw.nbytes) as back:
        fakhip.call("fhip_q6k_repack", dp.ptr, dr.ptr, out, in_)
        fakhip.call("fhip_q6k_unpack", back.ptr, dp.ptr, out, in_)
        np.testing.assert_array_equal(back.to_host(np.uint8), raw)
        packed = dp.to_host(np.uint8).reshape(-1, in_ // 256, 3360)
        if out % 16:
            tail = packed[-1]  # every record of the last tile: rows out%16.. are zero
            r0 = out % 16
            assert not tail[:, 16 * r0:256].any()        # scales
            assert not tail[:, 256 + 2 * r0:288].any()   # d


def test_argument_errors(hip):
    lib = fakhip.load()
    with Dev(4096) as a:
        assert lib.fhip_q6k_matmul_f32(a.ptr, a.ptr, a.ptr, 4, 300, 1) == -1
        assert lib.fhip_q6k_dequant_f32(a.ptr, a.ptr, 0, 256) == -1
        assert lib.fhip_q6k_matmul_f32(a.ptr, a.ptr, a.ptr, 4, 256, 0) == 0
    assert lib.fhip_q6k_bytes(3, 512) == 3 * 2 * 210
    assert lib.fhip_q6k_bytes(3, 500) == 0


@pytest.mark.parametrize("out,in_,P,rows", [(256, 512, 17, None), (300, 768, 40, None),
                                            (3584, 18944, 24, 48), (152, 4096, 32, None),
                                            (37, 256, 19, None), (1000, 2048, 28, None),
                                            (1000, 2048, 200, 64), (18944, 3584, 512, 64),
                                            (3584, 18944, 128, 48), (3584, 18944, 1024, 48),
                                            (3000, 18944, 1000, 48), (18944, 3584, 1024, 64)])
def test_gemm_prefill_matches_oracle(hip, oracle_mod, out, in_, P, rows):
    """More than 16 tokens (17..32 on the small-M kernel's f16 form, more on the f16 MFMA prefill
    GEMM, its 256-row workgroups with K ranges from eight token tiles on the long rows) on the
    Q6_K records: max|dY|/RMS <= 1e-2 (the GEMM bound), checked on every output or on a sample
    of rows at full shape."""
    print(f"[case] q6k gemm out={out} in={in_} P={P}", flush=True)
    rng = np.random.default_rng(out + 7 * in_ + P)
    raw = qc.pin_d(rng.integers(0, 256, size=out * (in_ // 256) * 210, dtype=np.uint8), 0x1400)
    X = rng.standard_normal((P, in_)).astype(np.float32)
    Y = dev_matmul(raw, out, in_, X, P)
    assert np.all(np.isfinite(Y))
    if rows is None:
        ref, got = oracle_mod.q6k_gemm(raw, out, in_, X, P), Y
    else:
        rb = (in_ // 256) * 210
        sel = spread_rows(out, per_block=max(1, rows // max(1, out // 128)))
        sub = np.concatenate([raw[o * rb:(o + 1) * rb] for o in sel])
        ref, got = oracle_mod.q6k_gemm(sub, len(sel), in_, X, P), Y[:, sel]
    err = rel_err(got, ref)
    print(f"    max|d|/RMS = {err:.2e}", flush=True)
    assert err <= 1e-2


@pytest.mark.parametrize("out,in_,P", [(300, 768, 40), (1000, 2048, 200), (152, 4096, 131),
                                       (3584, 18944, 128), (18944, 3584, 512)])
def test_gemm_forms_bit_identical(hip, oracle_mod, monkeypatch, out, in_, P):
    """The staged prefill GEMM (the default: weights loaded straight to the registers of the
    lanes that use them) and the four-wave 2x2 form (records staged through LDS) share the tile,
    the K order, the dequantized f16 weights and each accumulator's MFMA sequence: on Q6_K their
    outputs agree bit for bit (ragged row and token tiles, K-split and whole tiles), and the
    staged result meets the GEMM bound against the oracle on rows spread over every row tile."""
    print(f"[case] q6k gemm forms out={out} in={in_} P={P}", flush=True)
    rng = np.random.default_rng(out + 3 * P)
    raw = qc.pin_d(rng.integers(0, 256, size=out * (in_ // 256) * 210, dtype=np.uint8), 0x1400)
    X = rng.standard_normal((P, in_)).astype(np.float32)
    with knobs(monkeypatch, FAK_HIP_GEMM32_FORM=1):
        Y1 = dev_matmul(raw, out, in_, X, P)
    Y2 = dev_matmul(raw, out, in_, X, P)
    assert np.array_equal(Y1.view(np.uint32), Y2.view(np.uint32))
    rb = (in_ // 256) * 210
    sel = spread_rows(out, per_block=1) if out > 1024 else np.arange(out)
    sub = np.concatenate([raw[o * rb:(o + 1) * rb] for o in sel])
    err = rel_err(Y2[:, sel], oracle_mod.q6k_gemm(sub, len(sel), in_, X, P))
    print(f"    max|d|/RMS = {err:.2e}", flush=True)
    assert err <= 1e-2


@pytest.mark.parametrize("out,in_,P", [(18944, 3584, 2048), (18900, 1024, 1100)])
def test_gemm_wide_tiles(hip, oracle_mod, monkeypatch, out, in_, P):
    """From eight token tiles (M > 896) the staged Q6_K kernel takes 256-row workgroups (four
    waves of 64 rows). Each output keeps the 128-row kernel's MFMA sequence: on grids that the
    plan leaves without a K split (1184 and 666 workgroups on 256 CUs), bit-identical to the
    unsplit four-wave 2x2 form on whole and ragged row and token tiles, and within the GEMM bound
    of the oracle on rows spread over every row tile."""
    print(f"[case] q6k gemm wide tiles out={out} in={in_} P={P}", flush=True)
    rng = np.random.default_rng(out + 5 * P)
    raw = qc.pin_d(rng.integers(0, 256, size=out * (in_ // 256) * 210, dtype=np.uint8), 0x1400)
    X = rng.standard_normal((P, in_)).astype(np.float32)
    Y = dev_matmul(raw, out, in_, X, P)
    with knobs(monkeypatch, FAK_HIP_GEMM32_FORM=1, FAK_HIP_GEMM32_SK=1):
        Y1 = dev_matmul(raw, out, in_, X, P)
    assert np.array_equal(Y.view(np.uint32), Y1.view(np.uint32))
    rb = (in_ // 256) * 210
    sel = spread_rows(out, per_block=1)
    sub = np.concatenate([raw[o * rb:(o + 1) * rb] for o in sel])
    err = rel_err(Y[:, sel], oracle_mod.q6k_gemm(sub, len(sel), in_, X, P))
    print(f"    max|d|/RMS = {err:.2e}", flush=True)
    assert err <= 1e-2
