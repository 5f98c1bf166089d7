"""The C ABI's guards, on the device: a matmul refuses a pointer that is not a tiled weight of
the format and shape it is asked for (raw GGUF bytes uploaded with fhip_malloc + fhip_h2d, the
upload path of the CUDA tenant, internal/compute/cuda.go:803-822, would otherwise give plausible
garbage), and work queued on two created streams, each with its own scratch, matches the
oracle."""
import ctypes as C

import numpy as np
import pytest

from fak_amd import fakhip, synth
from tests.gpu_util import Dev, rel_err

pytestmark = pytest.mark.gpu


def test_raw_bytes_pointer_is_refused(hip):
    lib = fakhip.load()
    out, in_ = 64, 512
    raw = synth.q4k_weights(out, in_, seed=1)
    with Dev.from_host(raw) as draw, Dev.from_host(synth.activations(1, in_, 2)) as dx, \
            Dev(out * 4) as dy:
        rc = lib.fhip_q4k_matmul_f32(draw.ptr, dx.ptr, dy.ptr, out, in_, 1)
        assert rc == fakhip.EINVAL
        assert "not a tiled Q4_K weight" in fakhip.last_error()
        # laid out by fhip_q4k_repack, the same bytes are accepted
        with Dev(lib.fhip_q4k_packed_bytes(out, in_)) as dp:
            fakhip.call("fhip_q4k_repack", dp.ptr, draw.ptr, out, in_)
            fakhip.call("fhip_q4k_matmul_f32", dp.ptr, dx.ptr, dy.ptr, out, in_, 1)
            # any other write into it drops the record
            fakhip.call("fhip_memset_async", dp.ptr, 0, 16)
            assert lib.fhip_q4k_matmul_f32(dp.ptr, dx.ptr, dy.ptr, out, in_, 1) == fakhip.EINVAL


def test_wrong_shape_and_format_are_refused(hip):
    lib = fakhip.load()
    out, in_ = 48, 1024
    raw = synth.q4k_weights(out, in_, 3)  # kept alive across the upload's host read
    w = fakhip.alloc_call("fhip_q4k_upload", raw.ctypes.data, out, in_)
    try:
        with Dev.from_host(synth.activations(2, 2048, 4)) as dx, Dev(2 * 2048 * 4) as dy:
            for o, i in [(out + 16, in_), (out, in_ + 256), (out - 1, in_)]:
                assert lib.fhip_q4k_matmul_f32(w, dx.ptr, dy.ptr, o, i, 1) == fakhip.EINVAL
                assert "holds a tiled Q4_K weight [48, 1024]" in fakhip.last_error()
            assert lib.fhip_q8_0_matmul_f32(w, dx.ptr, dy.ptr, out, in_, 1) == fakhip.EINVAL
            assert lib.fhip_q6k_matmul_f32(w, dx.ptr, dy.ptr, out, in_, 1) == fakhip.EINVAL
            assert lib.fhip_q4k_matmul_int8_f32(w, dx.ptr, dy.ptr, out + 16, in_, 1) == \
                fakhip.EINVAL
            fakhip.call("fhip_q4k_matmul_f32", w, dx.ptr, dy.ptr, out, in_, 2)
    finally:
        lib.fhip_free(w)
    # freed: the pointer no longer names a weight (even before the pool hands it out again)
    with Dev(16) as dx, Dev(16 * 4) as dy:
        assert lib.fhip_q4k_matmul_f32(w, dx.ptr, dy.ptr, out, in_, 1) == fakhip.EINVAL


def test_copy_of_a_weight_is_a_weight(hip, oracle_mod):
    lib = fakhip.load()
    out, in_ = 100, 768
    raw = synth.q4k_weights(out, in_, 5)
    w = fakhip.alloc_call("fhip_q4k_upload", raw.ctypes.data, out, in_)
    nbytes = lib.fhip_q4k_packed_bytes(out, in_)
    c = fakhip.alloc_call("fhip_malloc", nbytes)
    try:
        fakhip.call("fhip_d2d", c, w, nbytes)
        X = synth.activations(3, in_, 6)
        with Dev.from_host(X) as dx, Dev(3 * out * 4) as dy:
            fakhip.call("fhip_q4k_matmul_f32", c, dx.ptr, dy.ptr, out, in_, 3)
            Y = dy.to_host(np.float32).reshape(3, out)
        assert rel_err(Y, oracle_mod.q4k_gemm(raw, out, in_, X, 3)) <= 1e-3
        # a partial copy is not
        fakhip.call("fhip_d2d", c, w, nbytes - 16)
        with Dev(16 * in_) as dx, Dev(16 * out * 4) as dy:
            assert lib.fhip_q4k_matmul_f32(c, dx.ptr, dy.ptr, out, in_, 1) == fakhip.EINVAL
    finally:
        lib.fhip_free(c)
        lib.fhip_free(w)


def test_two_streams_concurrently(hip, oracle_mod):
    """Two created streams each run matmuls that use scratch (a K-split prefill GEMM, a 16-token
    GEMV with K-range partials) with no synchronization between them; each stream's scratch is
    its own, so both results match the oracle."""
    lib = fakhip.load()
    cases = [(3584, 4096, 128), (2048, 6144, 16)]
    streams = []
    bufs = []
    ws = []
    outs = []
    try:
        for i, (out, in_, P) in enumerate(cases):
            raw = synth.q4k_weights(out, in_, 40 + i)
            X = synth.activations(P, in_, 50 + i)
            w = fakhip.alloc_call("fhip_q4k_upload", raw.ctypes.data, out, in_)
            dx, dy = Dev.from_host(X), Dev(P * out * 4)
            s = C.c_void_p()
            fakhip.call("fhip_stream_create", C.byref(s))
            streams.append(s)
            ws.append(w)
            bufs += [dx, dy]
            outs.append((raw, X, dy))
        for rep in range(3):
            for (out, in_, P), s, w, (raw, X, dy), dx in zip(cases, streams, ws, outs, bufs[0::2]):
                fakhip.call("fhip_set_stream", s)
                fakhip.call("fhip_q4k_matmul_f32", w, dx.ptr, dy.ptr, out, in_, P)
        fakhip.call("fhip_set_stream", None)
        for s in streams:
            fakhip.call("fhip_stream_sync", s)
        for (out, in_, P), (raw, X, dy) in zip(cases, outs):
            Y = dy.to_host(np.float32).reshape(P, out)
            ref = oracle_mod.q4k_gemm(raw, out, in_, X, P, workers=16)
            assert rel_err(Y, ref) <= (1e-3 if P <= 16 else 1e-2)
    finally:
        fakhip.call("fhip_set_stream", None)
        for s in streams:
            fakhip.call("fhip_stream_destroy", s)
        for b in bufs:
            b.close()
        for w in ws:
            lib.fhip_free(w)
