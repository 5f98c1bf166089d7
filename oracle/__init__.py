"""The oracle: ctypes access to the C restatement of fak's Go Q4_K / Q8_0 CPU path.

TEST INFRASTRUCTURE ONLY. Only tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg may import this package, and only to check results against (or as the
timed CPU baseline). The product (``fak_amd``) never loads it.

Each wrapper names the reference function it restates; the C file carries the file:line
citations.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import build as _build

_lib = None

_u8p = C.POINTER(C.c_uint8)
_i8p = C.POINTER(C.c_int8)
_f32p = C.POINTER(C.c_float)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_build.LIB):
            _build.build()
        L = C.CDLL(_build.LIB)
        L.fr_f16_bits_to_f32_bits.restype = C.c_uint32
        L.fr_f16_bits_to_f32_bits.argtypes = [C.c_uint16]
        L.fr_get_scale_min_k4.argtypes = [C.c_int, _u8p, _u8p, _u8p]
        L.fr_q4k_dequant_superblock.argtypes = [_f32p, _u8p]
        L.fr_q4k_dequant_row.argtypes = [_f32p, _u8p, C.c_int]
        L.fr_q4k_matrows_range.argtypes = [_u8p, C.c_int, C.c_int, _f32p, _f32p, C.c_int, C.c_int]
        L.fr_q4k_gemm_range.argtypes = [_u8p, C.c_int, C.c_int, _f32p, C.c_int, _f32p, C.c_int,
                                        C.c_int]
        L.fr_q8_0_dequant_block.argtypes = [_f32p, _u8p]
        L.fr_q8_0_matrows_range.argtypes = [_u8p, C.c_int, C.c_int, _f32p, _f32p, C.c_int,
                                            C.c_int]
        L.fr_q8round.restype = C.c_int8
        L.fr_q8round.argtypes = [C.c_float]
        L.fr_quantize_vec_q8.argtypes = [_f32p, C.c_int, C.c_int, _i8p, _f32p]
        L.fr_qdot8.restype = C.c_float
        L.fr_qdot8.argtypes = [_i8p, _f32p, _i8p, _f32p, C.c_int, C.c_int]
        L.fr_qgemm8cell.restype = C.c_float
        L.fr_qgemm8cell.argtypes = [_i8p, _f32p, _i8p, _f32p, C.c_int, C.c_int]
        L.fr_hal_q8_matmul.argtypes = [_i8p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        L.fr_hal_q8_batched_matmul.argtypes = [_i8p, _f32p, _f32p, _f32p, C.c_int, C.c_int,
                                               C.c_int, C.c_int]
        _i32p = C.POINTER(C.c_int32)
        L.fr_q4k_reduce_row.argtypes = [_u8p, C.c_int, _i8p, _i32p, _i32p]
        L.fr_q4k_combine_row.restype = C.c_float
        L.fr_q4k_combine_row.argtypes = [_u8p, C.c_int, _f32p, _i32p, _i32p]
        L.fr_q4k_matrows_int8.argtypes = [_u8p, C.c_int, C.c_int, _f32p, _f32p]
        L.fr_q6k_dequant_superblock.argtypes = [_f32p, _u8p]
        L.fr_q6k_matrows_range.argtypes = [_u8p, C.c_int, C.c_int, _f32p, _f32p, C.c_int,
                                           C.c_int]
        L.fr_silu.restype = C.c_float
        L.fr_silu.argtypes = [C.c_float]
        L.fr_swiglu.argtypes = [_f32p, _f32p, C.c_int]
        for name in ("fr_q4k_matrows_par", "fr_q8_0_matrows_par"):
            fn = getattr(L, name)
            fn.restype = C.c_int
            fn.argtypes = [_u8p, C.c_int, C.c_int, _f32p, _f32p, C.c_int]
        L.fr_q4k_gemm_par.restype = C.c_int
        L.fr_q4k_gemm_par.argtypes = [_u8p, C.c_int, C.c_int, _f32p, C.c_int, _f32p, C.c_int]
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data_as(t)


def f16_bits_to_f32_bits(h: int) -> int:
    """internal/model/quantbits.go:15-36"""
    return int(lib().fr_f16_bits_to_f32_bits(h))


def get_scale_min_k4(j: int, q: np.ndarray) -> tuple[int, int]:
    """internal/model/quantbits.go:42-47"""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s, m = C.c_uint8(), C.c_uint8()
    lib().fr_get_scale_min_k4(j, _p(q, _u8p), C.byref(s), C.byref(m))
    return s.value, m.value


def q4k_dequant(raw: np.ndarray, out: int, in_: int) -> np.ndarray:
    """Row-wise internal/model/quant_q4k.go:90-111 over a [out, in/256, 144] weight."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    nblk = in_ // 256
    assert raw.size == out * nblk * 144
    w = np.empty((out, in_), np.float32)
    L = lib()
    for o in range(out):
        L.fr_q4k_dequant_row(_p(w[o], _f32p), _p(raw[o * nblk * 144:], _u8p), nblk)
    return w


def q4k_matrows(raw: np.ndarray, out: int, in_: int, x: np.ndarray, workers: int = 1) -> np.ndarray:
    """q4kMatRowsInto f32 route, internal/model/quant_q4k.go:125-165."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert in_ % 256 == 0 and raw.size == out * (in_ // 256) * 144 and x.size == in_
    y = np.empty(out, np.float32)
    rc = lib().fr_q4k_matrows_par(_p(raw, _u8p), out, in_, _p(x, _f32p), _p(y, _f32p), workers)
    assert rc == 0
    return y


def q4k_gemm(raw: np.ndarray, out: int, in_: int, X: np.ndarray, P: int, workers: int = 1) -> np.ndarray:
    """q4kGemmInto f32 route, internal/model/quant_q4k.go:190-218,378-405. Returns Y[P, out]."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    X = np.ascontiguousarray(X, dtype=np.float32).reshape(-1)
    assert X.size == P * in_
    Y = np.empty((P, out), np.float32)
    rc = lib().fr_q4k_gemm_par(_p(raw, _u8p), out, in_, _p(X, _f32p), P, _p(Y, _f32p), workers)
    assert rc == 0
    return Y


def q8_0_dequant(raw: np.ndarray, out: int, in_: int) -> np.ndarray:
    """internal/model/quant_iquant.go:14-19 over a [out, in/32, 34] weight."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    nblk = in_ // 32
    assert raw.size == out * nblk * 34
    w = np.empty(out * in_, np.float32)
    L = lib()
    for b in range(out * nblk):
        L.fr_q8_0_dequant_block(_p(w[b * 32:], _f32p), _p(raw[b * 34:], _u8p))
    return w.reshape(out, in_)


def q8_0_matrows(raw: np.ndarray, out: int, in_: int, x: np.ndarray, workers: int = 1) -> np.ndarray:
    """kQuantMatRowsInto(kind Q8_0) f32 route, internal/model/quant_kquant.go:188-232."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert in_ % 32 == 0 and raw.size == out * (in_ // 32) * 34 and x.size == in_
    y = np.empty(out, np.float32)
    rc = lib().fr_q8_0_matrows_par(_p(raw, _u8p), out, in_, _p(x, _f32p), _p(y, _f32p), workers)
    assert rc == 0
    return y


def q8_0_gemm(raw: np.ndarray, out: int, in_: int, X: np.ndarray, P: int) -> np.ndarray:
    """P independent kQuantMatRows calls (the reference has no batched raw-Q8_0 GEMM)."""
    X = np.ascontiguousarray(X, dtype=np.float32).reshape(P, in_)
    return np.stack([q8_0_matrows(raw, out, in_, X[t]) for t in range(P)]) if P else \
        np.empty((0, out), np.float32)


def q8round(x: float) -> int:
    """internal/compute/cpuref.go:486-501"""
    return int(lib().fr_q8round(x))


def quantize_vec_q8(x: np.ndarray, block: int = 32) -> tuple[np.ndarray, np.ndarray]:
    """internal/compute/cpuref.go:505-527"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.size, np.int8)
    d = np.empty(x.size // block, np.float32)
    lib().fr_quantize_vec_q8(_p(x, _f32p), x.size, block, _p(q, _i8p), _p(d, _f32p))
    return q, d


def qdot8(qw, dw, qx, dx, block: int = 32) -> float:
    """internal/compute/cpuref.go:531-549"""
    qw = np.ascontiguousarray(qw, np.int8)
    qx = np.ascontiguousarray(qx, np.int8)
    dw = np.ascontiguousarray(dw, np.float32)
    dx = np.ascontiguousarray(dx, np.float32)
    return float(lib().fr_qdot8(_p(qw, _i8p), _p(dw, _f32p), _p(qx, _i8p), _p(dx, _f32p),
                                qw.size, block))


def qgemm8cell(qw, dw, qx, dx, block: int = 32) -> float:
    """internal/compute/cpuref.go:553-577"""
    qw = np.ascontiguousarray(qw, np.int8)
    qx = np.ascontiguousarray(qx, np.int8)
    dw = np.ascontiguousarray(dw, np.float32)
    dx = np.ascontiguousarray(dx, np.float32)
    return float(lib().fr_qgemm8cell(_p(qw, _i8p), _p(dw, _f32p), _p(qx, _i8p), _p(dx, _f32p),
                                     qw.size // block, block))


def hal_q8_matmul(codes, scales, x, out: int, in_: int, block: int = 32) -> np.ndarray:
    """cpuBackend.MatMul Q8_0 branch, internal/compute/cpuref.go:128-135"""
    codes = np.ascontiguousarray(codes, np.int8).reshape(-1)
    scales = np.ascontiguousarray(scales, np.float32).reshape(-1)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(out, np.float32)
    lib().fr_hal_q8_matmul(_p(codes, _i8p), _p(scales, _f32p), _p(x, _f32p), _p(y, _f32p), out,
                           in_, block)
    return y


def hal_q8_batched_matmul(codes, scales, X, out: int, in_: int, P: int, block: int = 32) -> np.ndarray:
    """cpuBackend.BatchedMatMul Q8_0 branch, internal/compute/cpuref.go:160-176"""
    codes = np.ascontiguousarray(codes, np.int8).reshape(-1)
    scales = np.ascontiguousarray(scales, np.float32).reshape(-1)
    X = np.ascontiguousarray(X, np.float32).reshape(-1)
    Y = np.empty((P, out), np.float32)
    lib().fr_hal_q8_batched_matmul(_p(codes, _i8p), _p(scales, _f32p), _p(X, _f32p),
                                   _p(Y, _f32p), out, in_, P, block)
    return Y


_i32p = C.POINTER(C.c_int32)


def q4k_reduce_row(row: np.ndarray, nblk: int, qx: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """q4kReduceRowScalar, internal/model/quant_q4k_int8.go:72-100. Returns (IS, SS) int32."""
    row = np.ascontiguousarray(row, np.uint8).reshape(-1)
    qx = np.ascontiguousarray(qx, np.int8).reshape(-1)
    assert row.size >= nblk * 144 and qx.size >= nblk * 256
    IS = np.empty(nblk * 8, np.int32)
    SS = np.empty(nblk * 8, np.int32)
    lib().fr_q4k_reduce_row(_p(row, _u8p), nblk, _p(qx, _i8p), _p(IS, _i32p), _p(SS, _i32p))
    return IS, SS


def q4k_combine_row(row: np.ndarray, nblk: int, dx: np.ndarray, IS: np.ndarray,
                    SS: np.ndarray) -> float:
    """q4kCombineRow, internal/model/quant_q4k_int8.go:110-130."""
    row = np.ascontiguousarray(row, np.uint8).reshape(-1)
    dx = np.ascontiguousarray(dx, np.float32)
    IS = np.ascontiguousarray(IS, np.int32)
    SS = np.ascontiguousarray(SS, np.int32)
    return float(lib().fr_q4k_combine_row(_p(row, _u8p), nblk, _p(dx, _f32p), _p(IS, _i32p),
                                          _p(SS, _i32p)))


def q4k_matrows_int8(raw: np.ndarray, out: int, in_: int, x: np.ndarray) -> np.ndarray:
    """q4kMatRowsInto with q4kSDOTEnabled (FAK_KQ_INT8): quantizeVecQ8 once, then
    q4kMatRowsRangeInt8, internal/model/quant_q4k.go:125-136 + quant_q4k_int8.go:135-142."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert in_ % 256 == 0 and raw.size == out * (in_ // 256) * 144 and x.size == in_
    y = np.empty(out, np.float32)
    lib().fr_q4k_matrows_int8(_p(raw, _u8p), out, in_, _p(x, _f32p), _p(y, _f32p))
    return y


def q4k_gemm_int8(raw: np.ndarray, out: int, in_: int, X: np.ndarray, P: int) -> np.ndarray:
    """q4kGemmInto with q4kSDOTEnabled on amd64 (no extract-once): every token quantized on its
    own and run through the int8 GEMV, internal/model/quant_q4k.go:190-218,359-372."""
    X = np.ascontiguousarray(X, dtype=np.float32).reshape(P, in_)
    return np.stack([q4k_matrows_int8(raw, out, in_, X[t]) for t in range(P)]) if P else \
        np.empty((0, out), np.float32)


def q6k_dequant(raw: np.ndarray, out: int, in_: int) -> np.ndarray:
    """Row-wise q6kDequantSuperBlock, internal/model/quant_kquant.go:139-163."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    nblk = in_ // 256
    assert raw.size == out * nblk * 210
    w = np.empty((out, in_), np.float32)
    L = lib()
    for b in range(out * nblk):
        L.fr_q6k_dequant_superblock(_p(w.reshape(-1)[b * 256:], _f32p), _p(raw[b * 210:], _u8p))
    return w


def q6k_matrows(raw: np.ndarray, out: int, in_: int, x: np.ndarray) -> np.ndarray:
    """kQuantMatRowsInto(kind Q6_K) f32 route, internal/model/quant_kquant.go:188-232."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert in_ % 256 == 0 and raw.size == out * (in_ // 256) * 210 and x.size == in_
    y = np.empty(out, np.float32)
    lib().fr_q6k_matrows_range(_p(raw, _u8p), out, in_, _p(x, _f32p), _p(y, _f32p), 0, out)
    return y


def q6k_gemm(raw: np.ndarray, out: int, in_: int, X: np.ndarray, P: int) -> np.ndarray:
    """P tokens through the Q6_K GEMV, Y[P, out]."""
    X = np.ascontiguousarray(X, dtype=np.float32).reshape(P, in_)
    return np.stack([q6k_matrows(raw, out, in_, X[t]) for t in range(P)]) if P else \
        np.empty((0, out), np.float32)


def silu(z: float) -> np.float32:
    """internal/model/forward.go:452."""
    return np.float32(lib().fr_silu(float(np.float32(z))))


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """silu(g) * u elementwise (denseSwiGLU, internal/model/moe.go:111-136)."""
    g = np.array(g, np.float32).reshape(-1)
    u = np.ascontiguousarray(u, np.float32).reshape(-1)
    assert g.size == u.size
    lib().fr_swiglu(_p(g, _f32p), _p(u, _f32p), g.size)
    return g


def q4k_mlp(gate: np.ndarray, up: np.ndarray, down: np.ndarray, hidden: int, inter: int,
            X: np.ndarray, P: int, down_q6: bool = False, workers: int = 1) -> np.ndarray:
    """The dense SwiGLU FFN of a decode step on resident quantized weights (denseSwiGLU,
    internal/model/moe.go:111-136): g = gate x, u = up x (Q4_K GEMV), g = silu(g) * u, then
    y = down g (Q4_K, or Q6_K for the q4_k_m down projection), per token. Returns Y[P, hidden]."""
    X = np.ascontiguousarray(X, np.float32).reshape(P, hidden)
    G = q4k_gemm(gate, inter, hidden, X, P, workers)
    U = q4k_gemm(up, inter, hidden, X, P, workers)
    H = np.stack([swiglu(G[t], U[t]) for t in range(P)])
    if down_q6:
        return q6k_gemm(down, hidden, inter, H, P)
    return q4k_gemm(down, hidden, inter, H, P, workers)
