"""Single-shape matmul microbenchmark, in the style of fak's cmd/q8kernel: one weight shape, M
tokens, a number of repetitions, median-free plain timing with HIP events, and a one-line report.
Used as the target program for rocprofv3 runs (kernel trace, counters) on one shape.

    python -m fak_amd.q4kbench --n 18944 --k 3584 --m 1 --reps 20 [--q8 | --q6k | --int8]
    python -m fak_amd.q4kbench --n 3584 --k 18944 --floor records|read

Weights rotate over enough distinct device copies (> 256 MB) that the Infinity Cache cannot
serve them. --floor times a launch that only moves the Q4_K weight's bytes, with no arithmetic:
`records` in the one-token GEMV's own grid and record loads (fhip_probe_q4k_records), `read` as
a plain grid-stride read of the same bytes (fhip_probe_read).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json

from . import fakhip, synth


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--n", type=int, required=True, help="output rows")
    ap.add_argument("--k", type=int, required=True, help="reduction dim")
    ap.add_argument("--m", type=int, default=1, help="tokens")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--q8", action="store_true", help="Q8_0 weights instead of Q4_K")
    ap.add_argument("--q6k", action="store_true", help="Q6_K weights instead of Q4_K")
    ap.add_argument("--int8", action="store_true",
                    help="the int8 Q4_K route (fhip_q4k_matmul_int8_f32) instead of the f32 one")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--floor", choices=("records", "read"), default=None,
                    help="time a no-arithmetic pass over the Q4_K weight instead of the matmul")
    a = ap.parse_args()
    fakhip.init()
    lib = fakhip.load()
    if a.q6k:
        import numpy as np
        rng = np.random.default_rng(a.seed)
        raw = rng.integers(0, 256, size=a.n * (a.k // 256) * 210, dtype=np.uint8).reshape(-1, 210)
        raw[:, 208:210] = (np.abs(rng.standard_normal(raw.shape[0])) * 1e-3).astype(
            np.float16).view(np.uint8).reshape(-1, 2)
        raw = raw.reshape(-1)
        up, mm, nbytes = "fhip_q6k_upload", "fhip_q6k_matmul_f32", lib.fhip_q6k_packed_bytes(a.n, a.k)
        alg = lib.fhip_q6k_bytes(a.n, a.k)
    elif a.q8:
        raw = synth.q8_0_weights(a.n, a.k, a.seed)
        up, mm, nbytes = "fhip_q8_0_upload", "fhip_q8_0_matmul_f32", lib.fhip_q8_0_packed_bytes(a.n, a.k)
        alg = a.n * (a.k // 32) * 34
    else:
        raw = synth.q4k_weights(a.n, a.k, a.seed)
        up, mm, nbytes = "fhip_q4k_upload", "fhip_q4k_matmul_f32", lib.fhip_q4k_packed_bytes(a.n, a.k)
        if a.int8:
            mm = "fhip_q4k_matmul_int8_f32"
        alg = a.n * (a.k // 256) * 144
    p0 = fakhip.alloc_call(up, raw.ctypes.data, a.n, a.k)
    ptrs = [p0]
    for _ in range(max(1, (300 << 20) // nbytes)):
        p = fakhip.alloc_call("fhip_malloc", nbytes)
        fakhip.call("fhip_d2d", p, p0, nbytes)
        ptrs.append(p)
    X = synth.activations(a.m, a.k, a.seed + 1)
    dx = fakhip.alloc_call("fhip_malloc", X.nbytes)
    fakhip.call("fhip_h2d", dx, X.ctypes.data, X.nbytes)
    dy = fakhip.alloc_call("fhip_malloc", a.m * a.n * 4)
    e0, e1 = C.c_void_p(), C.c_void_p()
    fakhip.call("fhip_event_create", C.byref(e0))
    fakhip.call("fhip_event_create", C.byref(e1))
    if a.floor:
        if a.q8 or a.q6k:
            raise SystemExit("--floor measures a Q4_K weight")
        if a.floor == "records":
            words = lib.fhip_probe_q4k_records_sink_words(a.n, a.k)
            sink = fakhip.alloc_call("fhip_malloc", 4 * words)
            run = lambda p: fakhip.call("fhip_probe_q4k_records", p, a.n, a.k, sink)
        else:
            words = lib.fhip_probe_read_sink_words(nbytes)
            sink = fakhip.alloc_call("fhip_malloc", 4 * words)
            run = lambda p: fakhip.call("fhip_probe_read", p, nbytes, sink)
    else:
        sink = None
        run = lambda p: fakhip.call(mm, p, dx, dy, a.n, a.k, a.m)
    run(ptrs[0])
    fakhip.call("fhip_sync")
    fakhip.call("fhip_event_record", e0)
    for i in range(a.reps):
        run(ptrs[i % len(ptrs)])
    fakhip.call("fhip_event_record", e1)
    ms = C.c_float()
    fakhip.call("fhip_event_elapsed_ms", e0, e1, C.byref(ms))
    us = ms.value * 1e3 / a.reps
    # a floor moves the packed weight only; the matmul counts its activations and outputs too
    bytes_ = nbytes if a.floor else alg + 4 * a.m * (a.n + a.k)
    print(json.dumps({"n": a.n, "k": a.k, "m": a.m, "q8_0": a.q8, "q6_k": a.q6k,
                      "floor": a.floor, "int8": a.int8, "reps": a.reps,
                      "us_per_call": round(us, 3), "GBs": round(bytes_ / us / 1e3, 1),
                      "TFLOPs": round(2.0 * a.m * a.n * a.k / us / 1e6, 2),
                      "weight_copies": len(ptrs)}), flush=True)
    for p in ptrs + [dx, dy] + ([sink] if sink else []):
        lib.fhip_free(p)


if __name__ == "__main__":
    main()
