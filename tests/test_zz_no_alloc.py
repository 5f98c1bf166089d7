"""fhip_q4k_matmul_noalloc_f32, the Q4_K matmul whose scratch is a static device array: it runs
the kernels of fhip_q4k_matmul_f32, so its output must be the same bits, call after call, with
the array keeping an earlier, larger call's contents; a call needing more scratch than the array
holds is refused before anything is launched."""
import numpy as np
import pytest

from fak_amd import fakhip, synth
from tests.gpu_util import Dev, rel_err

pytestmark = pytest.mark.gpu


def run(fn, w, X, out, in_, P):
    with Dev.from_host(np.ascontiguousarray(X, np.float32)) as dx, Dev(P * out * 4) as dy:
        fakhip.call(fn, w, dx.ptr, dy.ptr, out, in_, P)
        return dy.to_host(np.float32).reshape(P, out)


# (out, in, P): a K-split prefill GEMM (operands + token scales + partials: ~56 MB of scratch),
# then smaller calls: a 16-token GEMV with K-range partials, a 3-token GEMV with global
# activation operands, one decode token, a 24-token call (the 17..32-token route, K-range
# partials sized for its tokens), a 4-token call at in >= 24576 (which takes the 5..16-token
# kernel's route from three tokens) and a 1024-token GEMM on 256-row workgroups in 4 K ranges
# (~52 MB of scratch).
CALLS = [(3584, 18944, 512), (2048, 6144, 16), (3584, 18944, 3), (1024, 3584, 1),
         (18944, 3584, 24), (5120, 25600, 4), (3584, 4096, 1024)]


@pytest.mark.parametrize("first,second", [(0, 1), (1, 2), (2, 3), (0, 3), (0, 4), (4, 5),
                                          (5, 3), (6, 0), (6, 1)])
def test_noalloc_matches_allocating_entry(hip, oracle_mod, first, second):
    lib = fakhip.load()
    for idx in (first, second):
        out, in_, P = CALLS[idx]
        print(f"[noalloc] out={out} in={in_} P={P}", flush=True)
        raw = synth.q4k_weights(out, in_, seed=idx + 1)
        X = synth.activations(P, in_, seed=idx + 11)
        w = fakhip.alloc_call("fhip_q4k_upload", raw.ctypes.data, out, in_)
        try:
            a = run("fhip_q4k_matmul_noalloc_f32", w, X, out, in_, P)
            b = run("fhip_q4k_matmul_f32", w, X, out, in_, P)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
            rows = np.arange(min(out, 64))
            rb = (in_ // 256) * 144
            sub = np.concatenate([raw[o * rb:(o + 1) * rb] for o in rows])
            ref = oracle_mod.q4k_gemm(sub, len(rows), in_, X, P, workers=16)
            assert rel_err(a[:, rows], ref) <= (1e-3 if P <= 16 else 1e-2)
        finally:
            lib.fhip_free(w)


def test_noalloc_refuses_oversized_scratch(hip):
    lib = fakhip.load()
    out, in_, P = 3584, 18944, 2048  # f16 prefill operands alone: 77.6 MB > 64 MiB
    raw = synth.q4k_weights(out, in_, 3)  # kept alive across the upload's host read
    w = fakhip.alloc_call("fhip_q4k_upload", raw.ctypes.data, out, in_)
    try:
        with Dev(P * in_ * 4) as dx, Dev(P * out * 4) as dy:
            assert lib.fhip_q4k_matmul_noalloc_f32(w, dx.ptr, dy.ptr, out, in_, P) == fakhip.EINVAL
            assert "static region" in fakhip.last_error()
            raw_ptr = dx.ptr
            assert lib.fhip_q4k_matmul_noalloc_f32(raw_ptr, dx.ptr, dy.ptr, out, in_, 1) == \
                fakhip.EINVAL
    finally:
        lib.fhip_free(w)


def test_noalloc_refuses_wide_head_at_16_tokens(hip):
    """The 5..32-token routes keep K-range partial sums of about 4 * P * out bytes per 1,024
    values of in: at 16 tokens a [17408, 65536] weight needs 71.3 MB, beyond the 64 MiB array, so
    the call is refused before any launch (the weight is laid out from zero bytes on the device:
    no host data of that size is needed)."""
    lib = fakhip.load()
    out, in_, P = 17408, 65536, 16
    nbytes = out * (in_ // 256) * 144
    with Dev(nbytes) as raw:
        fakhip.call("fhip_memset_async", raw.ptr, 0, nbytes)
        fakhip.call("fhip_sync")
        w = fakhip.alloc_call("fhip_malloc", lib.fhip_q4k_packed_bytes(out, in_))
        try:
            fakhip.call("fhip_q4k_repack", w, raw.ptr, out, in_)
            with Dev(P * in_ * 4) as dx, Dev(P * out * 4) as dy:
                assert lib.fhip_q4k_matmul_noalloc_f32(w, dx.ptr, dy.ptr, out, in_, P) == \
                    fakhip.EINVAL
                assert "static region" in fakhip.last_error()
                # 4 tokens of the same weight need only a little scratch: accepted.
                fakhip.call("fhip_q4k_matmul_noalloc_f32", w, dx.ptr, dy.ptr, out, in_, 4)
                fakhip.call("fhip_sync")
        finally:
            lib.fhip_free(w)
