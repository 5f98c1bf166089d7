"""Small helpers for GPU tests: numpy <-> device buffers through the fakhip C ABI only."""
from __future__ import annotations

import contextlib

import numpy as np

from fak_amd import fakhip


@contextlib.contextmanager
def knobs(monkeypatch, **env):
    """Set FAK_HIP_* launch-shape overrides for the block. The library reads them once in
    fhip_init, so the block re-initialises on entry and again on exit."""
    for k, v in env.items():
        monkeypatch.setenv(k, str(v))
    fakhip.init()
    try:
        yield
    finally:
        for k in env:
            monkeypatch.delenv(k, raising=False)
        fakhip.init()


def rel_err_rows(got: np.ndarray, ref: np.ndarray) -> float:
    """The reference metric per token row (max over rows), so a row of tiny activations is judged
    against its own scale rather than hidden under a row of huge ones."""
    got = np.atleast_2d(got)
    ref = np.atleast_2d(ref)
    return max(rel_err(g, r) for g, r in zip(got, ref))


def spread_rows(n: int, per_block: int = 2, block: int = 128) -> np.ndarray:
    """Row indices for a sampled check of an n-row output that touch every block of `block` rows
    (the GEMM's row tile; each 16-row tile of the GEMV lies in one): `per_block` rows per block
    at offsets that differ from block to block (so every lane position is exercised over the
    blocks), plus the first and last row."""
    rows = {0, n - 1}
    for b in range(0, n, block):
        size = min(block, n - b)
        for j in range(per_block):
            rows.add(b + (37 * (b // block) + 61 * j + 5 * j * j) % size)
    return np.array(sorted(rows))


def scaled_activations(P: int, K: int, seed: int, pattern: str) -> np.ndarray:
    """N(0,1) activations reshaped to stress the activation scaling of every route:
    'big' rows x 1e5 (beyond f16), 'tiny' rows x 1e-20 (below f16), 'wee' rows x 1e-35 (block
    maxima below 2^-113, where 2^8 / e overflows f32), 'mixed' rows whose 32-value blocks
    alternate x 1e4 / x 1e-20, 'outlier' rows with one value of 7e4 (>= 65504), and 'all'
    cycling through big, tiny, mixed and outlier by row."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((P, K)).astype(np.float32)
    kinds = ["big", "tiny", "mixed", "outlier"] if pattern == "all" else [pattern]
    for t in range(P):
        k = kinds[t % len(kinds)]
        if k == "big":
            X[t] *= np.float32(1e5)
        elif k == "tiny":
            X[t] *= np.float32(1e-20)
        elif k == "wee":
            X[t] *= np.float32(1e-35)
        elif k == "mixed":
            f = np.where((np.arange(K) // 32) % 2 == 0, 1e4, 1e-20).astype(np.float32)
            X[t] *= f
        elif k == "outlier":
            X[t, (7 * t + 5) % K] = np.float32(7e4)
    return X


class Dev:
    """A device allocation from the fakhip pool, freed on close."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = fakhip.alloc_call("fhip_malloc", max(self.nbytes, 16))

    @classmethod
    def from_host(cls, a: np.ndarray) -> "Dev":
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes)
        if a.nbytes:
            fakhip.call("fhip_h2d", d.ptr, a.ctypes.data, a.nbytes)
        return d

    def to_host(self, dtype, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(n, dtype)
        if out.nbytes:
            fakhip.call("fhip_d2h", out.ctypes.data, self.ptr, out.nbytes)
        return out

    def close(self):
        if self.ptr:
            fakhip.load().fhip_free(self.ptr)
            self.ptr = 0

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """The reference's metric: max|got - ref| / RMS(ref) (internal/model/quant_q4k_test.go:140-158)."""
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref * ref))
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / rms)


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def q4k_matmul(raw: np.ndarray, out: int, in_: int, X: np.ndarray, P: int) -> np.ndarray:
    """Upload raw Q4_K, run fhip_q4k_matmul_f32 on X[P, in], return Y[P, out]."""
    lib = fakhip.load()
    w = fakhip.alloc_call("fhip_q4k_upload", np.ascontiguousarray(raw).ctypes.data, out, in_)
    try:
        with Dev.from_host(np.ascontiguousarray(X, np.float32)) as dx, Dev(P * out * 4) as dy:
            fakhip.call("fhip_q4k_matmul_f32", w, dx.ptr, dy.ptr, out, in_, P)
            return dy.to_host(np.float32).reshape(P, out)
    finally:
        lib.fhip_free(w)


def q4k_matmul_int8(raw: np.ndarray, out: int, in_: int, X: np.ndarray, P: int) -> np.ndarray:
    """Upload raw Q4_K, run the int8 route fhip_q4k_matmul_int8_f32 on X[P, in]."""
    lib = fakhip.load()
    w = fakhip.alloc_call("fhip_q4k_upload", np.ascontiguousarray(raw).ctypes.data, out, in_)
    try:
        with Dev.from_host(np.ascontiguousarray(X, np.float32)) as dx, Dev(P * out * 4) as dy:
            fakhip.call("fhip_q4k_matmul_int8_f32", w, dx.ptr, dy.ptr, out, in_, P)
            return dy.to_host(np.float32).reshape(P, out)
    finally:
        lib.fhip_free(w)


def q8_0_matmul(raw: np.ndarray, out: int, in_: int, X: np.ndarray, P: int) -> np.ndarray:
    lib = fakhip.load()
    w = fakhip.alloc_call("fhip_q8_0_upload", np.ascontiguousarray(raw).ctypes.data, out, in_)
    try:
        with Dev.from_host(np.ascontiguousarray(X, np.float32)) as dx, Dev(P * out * 4) as dy:
            fakhip.call("fhip_q8_0_matmul_f32", w, dx.ptr, dy.ptr, out, in_, P)
            return dy.to_host(np.float32).reshape(P, out)
    finally:
        lib.fhip_free(w)


def q4k_matmul_group(raws, outs, in_: int, X: np.ndarray, P: int) -> list:
    """Upload each raw Q4_K member, run fhip_q4k_matmul_group_f32 on the shared X[P, in],
    return [Y_i[P, out_i]]."""
    import ctypes as C
    lib = fakhip.load()
    ws = [fakhip.alloc_call("fhip_q4k_upload", np.ascontiguousarray(r).ctypes.data, o, in_)
          for r, o in zip(raws, outs)]
    ys = [Dev(P * o * 4) for o in outs]
    try:
        with Dev.from_host(np.ascontiguousarray(X, np.float32)) as dx:
            n = len(outs)
            wp = (C.c_void_p * n)(*ws)
            yp = (C.c_void_p * n)(*[y.ptr for y in ys])
            op = (C.c_int * n)(*outs)
            fakhip.call("fhip_q4k_matmul_group_f32", C.addressof(wp), C.addressof(yp),
                        C.addressof(op), n, dx.ptr, in_, P)
            return [y.to_host(np.float32).reshape(P, o) for y, o in zip(ys, outs)]
    finally:
        for y in ys:
            y.close()
        for w in ws:
            lib.fhip_free(w)
