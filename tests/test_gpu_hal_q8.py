"""The HAL Q8 lane on the device (fhip_q8_quantize_f32 / fhip_q8_matmul_f32): int8 codes +
f32 block scales with the activation quantized on the device. The contract is bit-identity with
the CPU reference — quantizeVecQ8 (internal/compute/cpuref.go:505-527), MatMul = qdot8scalar
(:532-548) and BatchedMatMul = qgemm8cell with 16 lanes (:553-577) — checked against the oracle's
restatement of exactly those functions. Then the reference's own CUDA witness tests
(TestCUDAQ8MatMulApproxMatchesRef / ...Batched..., internal/compute/cuda_quant_test.go:86-150:
lcg seeds 485 / 0x485b, out=320, in=256, P=8, argmax-exact on the dominant row, cosine >=
cudaQ8CosineMin = 0.999 vs the f32 matmul) through the Backend mirror.
"""
import numpy as np
import pytest

from fak_amd import backend as B
from fak_amd import fakhip
from tests import fixtures as fx
from tests.gpu_util import Dev, cosine

pytestmark = pytest.mark.gpu

Q8_COSINE_MIN = 0.999  # cudaQ8CosineMin


def dev_quantize(X: np.ndarray, rows: int, in_: int, block: int):
    with Dev.from_host(np.ascontiguousarray(X, np.float32)) as dx, Dev(rows * in_) as dq, \
            Dev(rows * (in_ // block) * 4) as ds:
        fakhip.call("fhip_q8_quantize_f32", dx.ptr, dq.ptr, ds.ptr, rows, in_, block)
        return dq.to_host(np.int8, rows * in_), ds.to_host(np.float32, rows * (in_ // block))


def dev_matmul(codes, scales, X, out, in_, P, block):
    with Dev.from_host(np.ascontiguousarray(codes, np.int8)) as dc, \
            Dev.from_host(np.ascontiguousarray(scales, np.float32)) as ds, \
            Dev.from_host(np.ascontiguousarray(X, np.float32)) as dx, Dev(P * out * 4) as dy:
        fakhip.call("fhip_q8_matmul_f32", dc.ptr, ds.ptr, dx.ptr, dy.ptr, out, in_, P, block)
        return dy.to_host(np.float32, P * out).reshape(P, out)


def edge_rows(in_: int, block: int, rng) -> np.ndarray:
    """Rows that exercise every branch of quantizeVecQ8 / q8round: all-zero blocks, values on
    exact half-steps (x*inv = k + 0.5 and k - 0.5, both signs), tiny, huge and negative-only
    blocks, and the block maximum at either end."""
    rows = []
    z = np.zeros(in_, np.float32)
    rows.append(z)
    r = z.copy()
    nb = in_ // block
    for b in range(nb):
        blk = np.arange(block, dtype=np.float32) - block / 2.0
        blk[-1] = 127.0                      # amax = 127 -> d = 1, inv = 1: x*inv = x exactly
        blk[: min(8, block - 1)] = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5],
                                            np.float32)[: min(8, block - 1)]
        r[b * block:(b + 1) * block] = blk
    rows.append(r)
    rows.append((rng.standard_normal(in_) * 1e-30).astype(np.float32))
    rows.append((rng.standard_normal(in_) * 1e30).astype(np.float32))
    rows.append(-np.abs(rng.standard_normal(in_)).astype(np.float32))
    v = rng.standard_normal(in_).astype(np.float32)
    v[0] = 40.0
    v[-1] = -41.0
    rows.append(v)
    return np.stack(rows)


@pytest.mark.parametrize("rows,in_,block", [(9, 512, 32), (40, 1024, 64), (7, 768, 256),
                                            (3, 96, 32)])
def test_quantize_bit_exact(hip, oracle_mod, rows, in_, block):
    print(f"[case] q8 quantize rows={rows} in={in_} block={block}", flush=True)
    rng = np.random.default_rng(rows * 1000 + in_)
    X = np.concatenate([rng.standard_normal((rows, in_)).astype(np.float32) * 0.3,
                        edge_rows(in_, block, rng)])
    n = X.shape[0]
    q, d = dev_quantize(X, n, in_, block)
    for r in range(n):
        qr, dr = oracle_mod.quantize_vec_q8(X[r], block)
        np.testing.assert_array_equal(q[r * in_:(r + 1) * in_], qr)
        np.testing.assert_array_equal(d[r * (in_ // block):(r + 1) * (in_ // block)].view(np.uint32),
                                      dr.view(np.uint32))


def rand_hal_weight(rng, out, in_, block):
    codes = rng.integers(-127, 128, size=out * in_, dtype=np.int8)
    scales = (np.abs(rng.standard_normal(out * (in_ // block))) * 0.01).astype(np.float32)
    return codes, scales


@pytest.mark.parametrize("out,in_,block", [(320, 256, 32), (1536, 576, 32), (64, 1024, 64),
                                           (17, 96, 32), (100, 512, 128)])
def test_matmul_decode_bit_exact(hip, oracle_mod, out, in_, block):
    """P = 1 follows qdot8scalar exactly."""
    print(f"[case] hal q8 matmul out={out} in={in_} block={block}", flush=True)
    rng = np.random.default_rng(out + in_)
    codes, scales = rand_hal_weight(rng, out, in_, block)
    x = rng.standard_normal(in_).astype(np.float32)
    y = dev_matmul(codes, scales, x, out, in_, 1, block)[0]
    ref = oracle_mod.hal_q8_matmul(codes, scales, x, out, in_, block)
    np.testing.assert_array_equal(y.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("out,in_,P,block", [(320, 256, 8, 32), (64, 1024, 2, 32),
                                             (33, 576, 17, 32), (48, 512, 5, 64)])
def test_matmul_batched_bit_exact(hip, oracle_mod, out, in_, P, block):
    """P > 1 follows qgemm8cell (16 lanes, pairwise tree) exactly, including its use of only
    the first 32 codes of a block longer than 32."""
    print(f"[case] hal q8 batched out={out} in={in_} P={P} block={block}", flush=True)
    rng = np.random.default_rng(out * P + in_)
    codes, scales = rand_hal_weight(rng, out, in_, block)
    X = rng.standard_normal((P, in_)).astype(np.float32)
    Y = dev_matmul(codes, scales, X, out, in_, P, block)
    ref = oracle_mod.hal_q8_batched_matmul(codes, scales, X, out, in_, P, block)
    np.testing.assert_array_equal(Y.view(np.uint32), ref.view(np.uint32))


def test_matmul_argument_errors(hip):
    with Dev(64) as a:
        lib = fakhip.load()
        assert lib.fhip_q8_matmul_f32(a.ptr, a.ptr, a.ptr, a.ptr, 4, 100, 1, 32) == -1  # in % block
        assert lib.fhip_q8_matmul_f32(a.ptr, a.ptr, a.ptr, a.ptr, 4, 64, 2, 16) == -1   # P > 1, block < 32
        assert lib.fhip_q8_matmul_f32(a.ptr, a.ptr, a.ptr, a.ptr, 4, 60, 1, 30) == -1   # block % 4
        assert lib.fhip_q8_quantize_f32(a.ptr, a.ptr, a.ptr, 1, 100, 32) == -1


@pytest.fixture(scope="module")
def be(hip):
    b = B.register_rocm()
    assert b is not None
    return b


def dominant_row(w: np.ndarray, out: int, in_: int) -> int:
    """dominantRow (cuda_quant_test.go:71-84): the row with the largest f32 sum of squares."""
    best, best_norm = 0, np.float32(-1)
    for o in range(out):
        n = np.float32(0)
        for v in w[o * in_:(o + 1) * in_]:
            n = np.float32(n + np.float32(v * v))
        if n > best_norm:
            best_norm, best = n, o
    return best


def test_backend_q8_matmul_witness(be, oracle_mod):
    """TestCUDAQ8MatMulApproxMatchesRef on this backend, plus bit-identity with the CPU
    reference's own Q8 lane on the same narrowed weight."""
    print("[case] backend HAL Q8 MatMul witness", flush=True)
    g = fx.LCG(485)
    out, in_ = 320, 256
    w = fx.rscale(g, out * in_, 0.2)
    target = dominant_row(w, out, in_)
    x = w[target * in_:(target + 1) * in_].copy()
    y_f32 = (w.reshape(out, in_).astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
    wq = be.Upload(B.NewF32(be, [out, in_], w), B.Dtype.Q8_0)
    assert wq.Dtype == B.Dtype.Q8_0
    y = be.Read(be.MatMul(wq, be.Upload(B.NewF32(be, [in_], x))))
    assert int(np.argmax(y_f32)) == int(np.argmax(y)) == target
    others = np.arange(out) != target
    c = cosine(y[others], y_f32[others])
    print(f"    cosine(non-target)={c:.8f}", flush=True)
    assert c >= Q8_COSINE_MIN
    codes, scales = [], []
    for o in range(out):
        q, d = oracle_mod.quantize_vec_q8(w[o * in_:(o + 1) * in_], 32)
        codes.append(q)
        scales.append(d)
    ref = oracle_mod.hal_q8_matmul(np.concatenate(codes), np.concatenate(scales), x, out, in_, 32)
    np.testing.assert_array_equal(y.view(np.uint32), ref.view(np.uint32))
    # the same host weight returns the cached resident weight
    assert be.Upload(B.NewF32(be, [out, in_], w), B.Dtype.Q8_0) is wq
    be.Free(wq)


def test_backend_q8_batched_matmul_witness(be, oracle_mod):
    """TestCUDAQ8BatchedMatMulApproxMatchesRef on this backend (NewQ8 host weight)."""
    print("[case] backend HAL Q8 BatchedMatMul witness", flush=True)
    g = fx.LCG(0x485B)
    out, in_, P = 320, 256, 8
    w = fx.rscale(g, out * in_, 0.2)
    X = fx.rscale(g, P * in_, 1.0)
    Y_f32 = (X.reshape(P, in_).astype(np.float64) @ w.reshape(out, in_).astype(np.float64).T)
    codes, scales = [], []
    for o in range(out):
        q, d = oracle_mod.quantize_vec_q8(w[o * in_:(o + 1) * in_], 32)
        codes.append(q)
        scales.append(d)
    codes, scales = np.concatenate(codes), np.concatenate(scales)
    wq = be.Upload(B.NewQ8(be, [out, in_], codes, scales, 32), B.Dtype.Q8_0)
    Y = be.Read(be.BatchedMatMul(wq, be.Upload(B.NewF32(be, [P, in_], X)), P)).reshape(P, out)
    c = cosine(Y, Y_f32)
    print(f"    cosine={c:.8f}", flush=True)
    assert c >= Q8_COSINE_MIN
    ref = oracle_mod.hal_q8_batched_matmul(codes, scales, X, out, in_, P, 32)
    np.testing.assert_array_equal(Y.view(np.uint32), ref.view(np.uint32))
    be.Free(wq)
