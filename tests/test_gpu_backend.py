"""The compute.Backend mirror on the device: the reference's CUDA witness tests restated for the
ROCm backend (internal/compute/cuda_quant_test.go:278-330) with their exact inputs (lcg seeds
0x4b4b / 0x4b4c, out=320, in=256, P=8, non-IEEE f32ToF16Bits authoring), the argmax-exact gate
on the dominant row (dominantRow / alignActToRow, :48-84) and the recorded cosine floor
cudaQ4KCosineMin = 0.995 (internal/compute/cuda.go:127-129) — plus this backend's own tighter
max|d|/RMS bound.
"""
import numpy as np
import pytest

from fak_amd import backend as B
from fak_amd import synth
from tests import fixtures as fx
from tests.gpu_util import cosine, rel_err

pytestmark = pytest.mark.gpu

Q4K_COSINE_MIN = 0.995   # cudaQ4KCosineMin
Q8_COSINE_MIN = 0.999    # cudaQ8CosineMin


@pytest.fixture(scope="module")
def be(hip):
    b = B.register_rocm()
    assert b is not None
    return b


def test_registry_and_caps(be):
    b, ok = B.Lookup("rocm")
    assert ok and b is be
    assert be.Class() == B.CorrectnessClass.Approx
    assert not B.RequireReference(be)
    caps = be.Caps()
    assert caps.UploadDtype and caps.DeviceMemory
    assert be.Tier() == "gfx950"


def test_async_outputs_ready_after_fence(be):
    """cudaBuf.Ready (internal/compute/cuda.go:286-300): Caps.Async is advertised, so a matmul
    output is not Ready() until a host fence (Read) bumps the fence generation past the one it
    was enqueued in; one fence materializes every output enqueued before it; uploads are ready
    on return."""
    assert be.Caps().Async
    g = fx.LCG(0x4B4B)
    out, in_ = 320, 256
    wq = be.Upload(B.NewQ4K(be, [out, in_], fx.rand_q4k_bytes(g, out, in_)), B.Dtype.Q4_K)
    xd = be.Upload(B.NewF32(be, [in_], np.linspace(-1, 1, in_, dtype=np.float32)))
    assert wq.buf.Ready() and xd.buf.Ready()
    y1, y2 = be.MatMul(wq, xd), be.MatMul(wq, xd)
    assert not y1.buf.Ready() and not y2.buf.Ready()
    r2 = be.Read(y2)
    assert y1.buf.Ready() and y2.buf.Ready()
    y3 = be.MatMul(wq, xd)
    assert not y3.buf.Ready()
    r3 = be.Read(y3)
    assert y3.buf.Ready()
    assert np.array_equal(r2.view(np.uint32), r3.view(np.uint32))
    for t in (y1, y2, y3, xd):
        be.Free(t)


def test_q4k_matmul_witness(be, oracle_mod):
    """TestCUDAQ4KMatMulApproxMatchesRef on this backend."""
    print("[case] backend Q4_K MatMul witness", flush=True)
    g = fx.LCG(0x4B4B)
    out, in_ = 320, 256
    raw = fx.rand_q4k_bytes(g, out, in_)
    w = oracle_mod.q4k_dequant(raw, out, in_)
    target = int(np.argmax((w.astype(np.float64) ** 2).sum(axis=1)))
    x = w[target].copy()
    y_ref = oracle_mod.q4k_matrows(raw, out, in_, x)
    wq = be.Upload(B.NewQ4K(be, [out, in_], raw), B.Dtype.Q4_K)
    assert wq.Dtype == B.Dtype.Q4_K
    xd = be.Upload(B.NewF32(be, [in_], x))
    y = be.Read(be.MatMul(wq, xd))
    assert y.shape == (out,)
    assert int(np.argmax(y)) == int(np.argmax(y_ref)) == target
    others = np.arange(out) != target
    c = cosine(y[others], y_ref[others])
    print(f"    cosine={c:.9f} max|d|/RMS={rel_err(y, y_ref):.3e}", flush=True)
    assert c >= Q4K_COSINE_MIN
    assert rel_err(y, y_ref) <= 1e-3
    # the upload cache returns the same resident weight for the same host buffer (cuda.go:690-704)
    assert be.Upload(B.NewQ4K(be, [out, in_], raw), B.Dtype.Q4_K) is wq
    be.Free(wq)


def test_q4k_batched_matmul_witness(be, oracle_mod):
    """TestCUDAQ4KBatchedMatMulApproxMatchesRef on this backend (P=8 -> the small-M path)."""
    print("[case] backend Q4_K BatchedMatMul witness", flush=True)
    g = fx.LCG(0x4B4C)
    out, in_, P = 320, 256, 8
    raw = fx.rand_q4k_bytes(g, out, in_)
    X = fx.rscale(g, P * in_, 1.0)
    Y_ref = oracle_mod.q4k_gemm(raw, out, in_, X, P)
    wq = be.Upload(B.NewQ4K(be, [out, in_], raw), B.Dtype.Q4_K)
    Y = be.Read(be.BatchedMatMul(wq, be.Upload(B.NewF32(be, [P, in_], X)), P)).reshape(P, out)
    assert cosine(Y, Y_ref) >= Q4K_COSINE_MIN
    assert rel_err(Y, Y_ref) <= 1e-3
    be.Free(wq)


def test_q8_0_gguf_matmul(be, oracle_mod):
    """A raw GGUF Q8_0 weight through the backend: f32-activation semantics of
    kQuantMatRowsRange, argmax-exact on the dominant row, cosine >= cudaQ8CosineMin."""
    print("[case] backend Q8_0 MatMul", flush=True)
    out, in_ = 320, 256
    raw = synth.q8_0_weights(out, in_, seed=485)
    w = oracle_mod.q8_0_dequant(raw, out, in_)
    target = int(np.argmax((w.astype(np.float64) ** 2).sum(axis=1)))
    x = w[target].copy()
    y_ref = oracle_mod.q8_0_matrows(raw, out, in_, x)
    wq = be.Upload(B.NewQ8_0GGUF(be, [out, in_], raw), B.Dtype.Q8_0)
    y = be.Read(be.MatMul(wq, be.Upload(B.NewF32(be, [in_], x))))
    assert int(np.argmax(y)) == target
    assert cosine(y, y_ref) >= Q8_COSINE_MIN
    assert rel_err(y, y_ref) <= 1e-3
    be.Free(wq)


def test_shape_errors_raise(be):
    """The reference panics on a wrong-shaped activation / payload; this backend raises."""
    raw = synth.q4k_weights(16, 256, seed=1)
    with pytest.raises(ValueError):
        be.Upload(B.NewQ4K(be, [16, 256], raw[:-1]), B.Dtype.Q4_K)
    wq = be.Upload(B.NewQ4K(be, [16, 256], raw), B.Dtype.Q4_K)
    with pytest.raises(ValueError):
        be.MatMul(wq, be.Upload(B.NewF32(be, [255], np.zeros(255, np.float32))))
    with pytest.raises(NotImplementedError):
        be.RMSNorm(None, None, 1e-6)
    be.Free(wq)


def test_upload_cache_never_stale(be, oracle_mod):
    """A host tensor that is gone (its memory free for reuse by the next one) never hits the
    upload cache: every round's weight is its own."""
    out, in_ = 16, 256
    x = synth.activations(1, in_, 3)[0]
    xd = be.Upload(B.NewF32(be, [in_], x), B.Dtype.F32)
    kept = []
    for r in range(4):
        raw = synth.q4k_weights(out, in_, 100 + r)
        w = be.Upload(B.NewQ4K(be, [out, in_], raw.copy()), B.Dtype.Q4_K)  # host tensor dies
        y = be.Read(be.MatMul(w, xd))
        ref = oracle_mod.q4k_matrows(raw, out, in_, x)
        assert rel_err(y, ref) <= 1e-3, r
        kept.append(w)
    for w in kept:
        be.Free(w)
    be.Free(xd)
