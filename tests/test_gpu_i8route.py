"""The int8 Q4_K route on the device (fhip_q4k_matmul_int8_f32) against the oracle's
q4kMatRowsRangeInt8 / q4kGemmRangeInt8 restatement (internal/model/quant_q4k_int8.go:72-142,
internal/model/quant_q4k.go:359-372): every output bit-identical, on random weights, on the
hand-built order and closed-form cases, on non-finite activations, and through windows of
records (long rows) and groups of 16 tokens."""
import numpy as np
import pytest

from fak_amd import fakhip, synth
from tests import int8_cases as ic
from tests.gpu_util import Dev, knobs, q4k_matmul_int8, rel_err

pytestmark = pytest.mark.gpu


def same_bits(got: np.ndarray, want: np.ndarray):
    """Bit-identical, except that any NaN matches any NaN (x86 and the GPU make different
    default NaN patterns)."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    both_nan = np.isnan(got) & np.isnan(want)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(got.view(np.uint32)[~both_nan], want.view(np.uint32)[~both_nan])


def test_order_cases(hip, oracle_mod):
    print("[case] int8 route: hand-built order cases", flush=True)
    raw, x, want = ic.order_cases()
    y = q4k_matmul_int8(raw, 3, 256, x, 1)[0]
    np.testing.assert_array_equal(y, want)


@pytest.mark.parametrize("out,in_,seed", [(5, 256, 1), (40, 2048, 3)])
def test_closed_form(hip, oracle_mod, out, in_, seed):
    print(f"[case] int8 route: closed form out={out} in={in_}", flush=True)
    raw, x, exact, peak = ic.integer_exact_case(out, in_, seed)
    assert peak < 2 ** 24
    y = q4k_matmul_int8(raw, out, in_, x, 1)[0]
    np.testing.assert_array_equal(y, np.array(exact, np.float32))


@pytest.mark.parametrize("out,in_,P", [(48, 768, 1), (4096, 4096, 1), (37, 1024, 3),
                                       (100, 512, 16), (64, 18944, 1), (48, 18944, 17),
                                       (1536, 2304, 4), (16, 256, 33)])
def test_matches_oracle(hip, oracle_mod, out, in_, P):
    print(f"[case] int8 route out={out} in={in_} P={P}", flush=True)
    raw = synth.q4k_weights(out, in_, out + in_ + P)
    X = synth.activations(P, in_, P * 7 + 1)
    Y = q4k_matmul_int8(raw, out, in_, X, P)
    ref = oracle_mod.q4k_gemm_int8(raw, out, in_, X, P)
    same_bits(Y, ref)


@pytest.mark.parametrize("out,in_,P,tw", [(16400, 512, 5, 0), (16400, 512, 16, 0),
                                          (100, 512, 16, 4), (100, 2304, 9, 8), (37, 1024, 3, 2),
                                          (48, 18944, 17, 4), (64, 768, 1, 3)])
def test_multi_tile_workgroups(hip, oracle_mod, monkeypatch, out, in_, P, tw):
    """Several one-wave tiles per workgroup sharing its staged activations (the launch's choice
    for wide matrices beyond four tokens, tw = 0: 16400 rows = 1025 tiles, the last workgroup
    with one real tile; forced elsewhere with FAK_HIP_I8R_TW, ragged last workgroups, fused and
    staged activations, windows of records): every output still bit-identical to the oracle."""
    print(f"[case] int8 route tiles/wg={tw} out={out} in={in_} P={P}", flush=True)
    raw = synth.q4k_weights(out, in_, out + 3 * in_ + P)
    X = synth.activations(P, in_, P * 5 + 2)
    if tw:
        with knobs(monkeypatch, FAK_HIP_I8R_TW=tw):
            Y = q4k_matmul_int8(raw, out, in_, X, P)
    else:
        Y = q4k_matmul_int8(raw, out, in_, X, P)
    if out > 4096:
        rb = (in_ // 256) * 144
        sel = np.r_[0:80, out - 400:out]
        sub = np.concatenate([raw[o * rb:(o + 1) * rb] for o in sel])
        same_bits(Y[:, sel], oracle_mod.q4k_gemm_int8(sub, len(sel), in_, X, P))
    else:
        same_bits(Y, oracle_mod.q4k_gemm_int8(raw, out, in_, X, P))


def test_reference_tolerance_vs_f32(hip, oracle_mod):
    """TestQ4KInt8DotMatchesF32 (internal/model/quant_q4k_int8_test.go:16-60) on the device."""
    out, in_ = 48, 768
    raw = synth.q4k_weights(out, in_, 23)
    x = np.random.default_rng(23).standard_normal(in_).astype(np.float32)
    y = q4k_matmul_int8(raw, out, in_, x, 1)[0]
    assert rel_err(y, oracle_mod.q4k_matrows(raw, out, in_, x)) <= 0.05


def test_non_finite_and_zero_blocks(hip, oracle_mod):
    print("[case] int8 route: NaN / Inf / zero activation blocks", flush=True)
    out, in_ = 32, 1024
    raw = synth.q4k_weights(out, in_, 9)
    X = synth.activations(3, in_, 9).reshape(3, in_)
    X[0, 32:64] = 0.0                     # zero block: dx = 0, codes 0
    X[1, 5] = np.nan                      # NaN code -127, amax ignores it
    X[2, 300] = np.inf                    # Inf scale: the block's terms are Inf/NaN
    X[2, 672:704] = 0.0                   # a block whose only value is subnormal: d is
    X[2, 700] = np.float32(1e-40)         # subnormal, 1/d overflows to Inf, 0 * Inf is NaN
    Y = q4k_matmul_int8(raw, out, in_, X, 3)
    same_bits(Y, oracle_mod.q4k_gemm_int8(raw, out, in_, X, 3))


def test_argument_errors(hip):
    lib = fakhip.load()
    with Dev(4096) as a:
        assert lib.fhip_q4k_matmul_int8_f32(a.ptr, a.ptr, a.ptr, 16, 300, 1) == -1   # in % 256
        assert lib.fhip_q4k_matmul_int8_f32(a.ptr, a.ptr + 4, a.ptr, 16, 256, 1) == -1  # align
        assert lib.fhip_q4k_matmul_int8_f32(a.ptr, a.ptr, a.ptr, 16, 256, 0) == 0    # P = 0


def test_backend_gate(hip, oracle_mod, monkeypatch):
    """FAK_KQ_INT8=1 sends the Backend mirror's Q4_K MatMul / BatchedMatMul through the int8
    route, as q4kSDOTEnabled does on the CPU; unset keeps the default route."""
    from fak_amd import backend as B
    out, in_, P = 64, 512, 5
    raw = synth.q4k_weights(out, in_, 77)
    X = synth.activations(P, in_, 78)
    monkeypatch.setenv("FAK_KQ_INT8", "1")
    be8 = B.RocmBackend()
    monkeypatch.delenv("FAK_KQ_INT8")
    be = B.RocmBackend()
    assert be8.kq_int8 and not be.kq_int8
    for b, want_int8 in ((be8, True), (be, False)):
        w = b.Upload(B.NewQ4K(b, [out, in_], raw))
        y = b.Read(b.MatMul(w, b.Upload(B.NewF32(b, [in_], X[0].copy()))))
        Y = b.Read(b.BatchedMatMul(w, b.Upload(B.NewF32(b, [P, in_], X)), P)).reshape(P, out)
        if want_int8:
            same_bits(y, oracle_mod.q4k_matrows_int8(raw, out, in_, X[0]))
            same_bits(Y, oracle_mod.q4k_gemm_int8(raw, out, in_, X, P))
        else:
            assert rel_err(y, oracle_mod.q4k_matrows(raw, out, in_, X[0])) <= 1e-3
        b.Free(w)
