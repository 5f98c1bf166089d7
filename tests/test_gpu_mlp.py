"""The fused decode MLP (fhip_q4k_mlp_f32 / fhip_q4k_mlp_q6down_f32) against the oracle's
denseSwiGLU chain (gate/up Q4_K GEMV -> silu(g) * u -> down GEMV, internal/model/moe.go:111-136)
on the same seeded weights and activations: max|dY|/RMS(Y) <= 1e-3, the GEMV bound, for Q4_K and
Q6_K down projections, 1..4 tokens, the 7B FFN shape and small / ragged tile counts."""
import numpy as np
import pytest

from fak_amd import fakhip, synth
from tests import q6k_cases as qc
from tests.gpu_util import Dev, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3


def weights(H, I, seed, q6):
    gate = synth.q4k_weights(I, H, seed)
    up = synth.q4k_weights(I, H, seed + 1)
    if q6:
        rng = np.random.default_rng(seed + 2)
        down = qc.pin_d(rng.integers(0, 256, H * (I // 256) * 210, dtype=np.uint8), 0x1000)
    else:
        down = synth.q4k_weights(H, I, seed + 2)
    return gate, up, down


def dev_mlp(gate, up, down, H, I, X, P, q6):
    lib = fakhip.load()
    wg = fakhip.alloc_call("fhip_q4k_upload", gate.ctypes.data, I, H)
    wu = fakhip.alloc_call("fhip_q4k_upload", up.ctypes.data, I, H)
    wd = fakhip.alloc_call("fhip_q6k_upload" if q6 else "fhip_q4k_upload", down.ctypes.data, H, I)
    try:
        with Dev.from_host(np.ascontiguousarray(X, np.float32)) as dx, Dev(P * H * 4) as dy:
            fn = "fhip_q4k_mlp_q6down_f32" if q6 else "fhip_q4k_mlp_f32"
            fakhip.call(fn, wg, wu, wd, dx.ptr, dy.ptr, H, I, P)
            return dy.to_host(np.float32).reshape(P, H)
    finally:
        for w in (wg, wu, wd):
            lib.fhip_free(w)


@pytest.mark.parametrize("q6", [False, True], ids=["q4down", "q6down"])
@pytest.mark.parametrize("H,I,P", [(3584, 18944, 1), (3584, 18944, 2), (3584, 18944, 3),
                                   (3584, 18944, 4), (512, 1024, 1), (512, 1024, 2),
                                   (256, 768, 3), (1024, 2816, 4), (768, 256, 1)])
def test_mlp_matches_oracle(hip, oracle_mod, H, I, P, q6):
    """At the 7B shape with 2..4 tokens the down projection's own scratch (K-range partials of
    the Q6_K kernel, global activation operands of the Q4_K one) is large: it must not land on
    the intermediate the down GEMV is reading."""
    print(f"[mlp] H={H} I={I} P={P} q6={q6}", flush=True)
    gate, up, down = weights(H, I, 10 * H + I + P, q6)
    X = synth.activations(P, H, 5 + P)
    Y = dev_mlp(gate, up, down, H, I, X, P, q6)
    ref = oracle_mod.q4k_mlp(gate, up, down, H, I, X, P, down_q6=q6, workers=8)
    assert np.all(np.isfinite(Y))
    assert rel_err(Y, ref) <= TOL, rel_err(Y, ref)


def test_mlp_repeat_is_deterministic(hip):
    H, I, P = 512, 1024, 1
    gate, up, down = weights(H, I, 77, False)
    X = synth.activations(P, H, 1)
    a = dev_mlp(gate, up, down, H, I, X, P, False)
    b = dev_mlp(gate, up, down, H, I, X, P, False)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_mlp_argument_errors(hip):
    lib = fakhip.load()
    H, I = 512, 1024
    gate, up, down = weights(H, I, 3, False)
    wg = fakhip.alloc_call("fhip_q4k_upload", gate.ctypes.data, I, H)
    wu = fakhip.alloc_call("fhip_q4k_upload", up.ctypes.data, I, H)
    wd = fakhip.alloc_call("fhip_q4k_upload", down.ctypes.data, H, I)
    try:
        with Dev(8 * H * 4) as dx, Dev(8 * H * 4) as dy:
            f = lib.fhip_q4k_mlp_f32
            assert f(wg, wu, wd, dx.ptr, dy.ptr, H, I, 0) == fakhip.OK
            for args in [(H, I, 5), (H, I, -1), (H + 1, I, 1), (H, I - 128, 1), (0, I, 1)]:
                assert f(wg, wu, wd, dx.ptr, dy.ptr, *args) == fakhip.EINVAL, args
            assert f(None, wu, wd, dx.ptr, dy.ptr, H, I, 1) == fakhip.EINVAL
            assert f(wg, wu, wd, dx.ptr + 4, dy.ptr, H, I, 1) == fakhip.EINVAL
            assert lib.fhip_q4k_mlp_q6down_f32(wg, wu, None, dx.ptr, dy.ptr, H, I, 1) == \
                fakhip.EINVAL
            assert "null" in fakhip.last_error()
    finally:
        for w in (wg, wu, wd):
            lib.fhip_free(w)
