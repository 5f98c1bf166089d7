"""Graph capture (fhip_graph_begin/end/launch): a captured sequence of matmul calls replays to the
same bits as the same calls run eagerly, replay after replay, with new activation contents and
eager work on the stream between replays (the way a decode loop reuses one captured token)."""
import ctypes as C

import numpy as np
import pytest

from fak_amd import fakhip, synth
from tests.gpu_util import Dev

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(hip):
    print("[case] graph capture: q4k gemv/group/gemm (unsplit, K-split, tail split), hal q8, "
          "gguf q8_0", flush=True)
    lib = fakhip.load()
    st = C.c_void_p()
    fakhip.call("fhip_stream_create", C.byref(st))
    fakhip.call("fhip_set_stream", st)
    allocs, devs = [], []
    try:
        K = 1024
        r1 = synth.q4k_weights(1024, K, 11)  # host arrays stay alive across each upload
        w1 = fakhip.alloc_call("fhip_q4k_upload", r1.ctypes.data, 1024, K)
        rg = [synth.q4k_weights(n, K, 12 + i) for i, n in enumerate((1024, 256, 256))]
        wg = [fakhip.alloc_call("fhip_q4k_upload", r.ctypes.data, r.size // (K // 256 * 144), K)
              for r in rg]
        r8 = synth.q8_0_weights(512, K, 15)
        w8 = fakhip.alloc_call("fhip_q8_0_upload", r8.ctypes.data, 512, K)
        # Prefill GEMMs that split K: 8 tiles in 4 K ranges (a grid smaller than the GPU), and
        # 258 tiles of which the last partial round (2 tiles) is split; both end in the reduce.
        K4, NT = 4 * K, 33024
        rs = synth.q4k_weights(1024, K4, 16)
        ws = fakhip.alloc_call("fhip_q4k_upload", rs.ctypes.data, 1024, K4)
        rt = synth.q4k_weights(NT, K, 17)
        wt = fakhip.alloc_call("fhip_q4k_upload", rt.ctypes.data, NT, K)
        allocs += [w1, w8, ws, wt] + wg
        rng = np.random.default_rng(7)
        codes = Dev.from_host(rng.integers(-127, 128, 320 * K, dtype=np.int8))
        scales = Dev.from_host((np.abs(rng.standard_normal(320 * K // 32)) * 0.01).astype(np.float32))
        x1 = Dev(K * 4)
        x40 = Dev(40 * K * 4)
        x40b = Dev(40 * K4 * 4)
        devs += [codes, scales, x1, x40, x40b]
        outs = {name: (Dev(n * 4), Dev(n * 4)) for name, n in
                [("gemv", 1024), ("g0", 1024), ("g1", 256), ("g2", 256), ("gemm", 40 * 1024),
                 ("gemm_split", 40 * 1024), ("gemm_tail", 40 * NT),
                 ("q8", 320), ("q8b", 4 * 320), ("gguf", 512)]}
        for a, b in outs.values():
            devs += [a, b]
        outs_all = list(outs.keys())
        gy = (C.c_void_p * 3)()
        gw = (C.c_void_p * 3)(*wg)
        gn = (C.c_int * 3)(1024, 256, 256)

        def run(k):  # k = 0: the buffers the graph writes; 1: the eager check buffers
            fakhip.call("fhip_q4k_matmul_f32", w1, x1.ptr, outs["gemv"][k].ptr, 1024, K, 1)
            for i, nm in enumerate(("g0", "g1", "g2")):
                gy[i] = outs[nm][k].ptr
            fakhip.call("fhip_q4k_matmul_group_f32", C.addressof(gw), C.addressof(gy),
                        C.addressof(gn), 3, x1.ptr, K, 1)
            fakhip.call("fhip_q4k_matmul_f32", w1, x40.ptr, outs["gemm"][k].ptr, 1024, K, 40)
            fakhip.call("fhip_q4k_matmul_f32", ws, x40b.ptr, outs["gemm_split"][k].ptr, 1024, K4,
                        40)
            fakhip.call("fhip_q4k_matmul_f32", wt, x40.ptr, outs["gemm_tail"][k].ptr, NT, K, 40)
            fakhip.call("fhip_q8_matmul_f32", codes.ptr, scales.ptr, x1.ptr, outs["q8"][k].ptr, 320,
                        K, 1, 32)
            fakhip.call("fhip_q8_matmul_f32", codes.ptr, scales.ptr, x40.ptr, outs["q8b"][k].ptr,
                        320, K, 4, 32)
            fakhip.call("fhip_q8_0_matmul_f32", w8, x1.ptr, outs["gguf"][k].ptr, 512, K, 1)

        def set_x(seed):
            a1, a40 = synth.activations(1, K, seed), synth.activations(40, K, seed + 1)
            a40b = synth.activations(40, K4, seed + 2)
            fakhip.call("fhip_h2d", x1.ptr, a1.ctypes.data, K * 4)
            fakhip.call("fhip_h2d", x40.ptr, a40.ctypes.data, 40 * K * 4)
            fakhip.call("fhip_h2d", x40b.ptr, a40b.ctypes.data, 40 * K4 * 4)

        set_x(100)
        run(0)  # eager warm-up: sizes the workspace before capture
        fakhip.call("fhip_sync")
        fakhip.call("fhip_graph_begin")
        run(0)
        graph = C.c_void_p()
        fakhip.call("fhip_graph_end", C.byref(graph))
        try:
            for rep in range(3):
                set_x(200 + 10 * rep)
                run(1)                      # eager work on the stream between replays
                fakhip.call("fhip_graph_launch", graph)
                fakhip.call("fhip_stream_sync", st)
                for nm in outs_all:
                    a, b = outs[nm]
                    ga, eb = a.to_host(np.uint32), b.to_host(np.uint32)
                    assert np.array_equal(ga, eb), (rep, nm)
                print(f"    replay {rep}: all {len(outs_all)} outputs bit-identical", flush=True)
        finally:
            fakhip.call("fhip_graph_destroy", graph)
    finally:
        fakhip.call("fhip_set_stream", None)
        for d in devs:
            d.close()
        for p in allocs:
            lib.fhip_free(p)
        fakhip.call("fhip_stream_destroy", st)


def test_graph_begin_needs_a_created_stream(hip):
    fakhip.call("fhip_set_stream", None)
    assert fakhip.load().fhip_graph_begin() == -1


def test_graph_decode_ffn_replays(hip):
    """A decode step's FFN captured once: the fused MLP (Q4_K down and the q4_k_m Q6_K down, one
    and three tokens), Q6_K matmuls (GEMV and prefill GEMM) and 8-token verify matmuls (Q4_K and
    Q6_K: a main launch and an ordered reduce) replay to the bits of the same calls run eagerly,
    replay after replay, with new activations between replays."""
    print("[case] graph capture: fused MLP (q4/q6 down), q6k gemv/gemm, 8-token q4k/q6k", flush=True)
    from tests import q6k_cases as qc
    lib = fakhip.load()
    st = C.c_void_p()
    fakhip.call("fhip_stream_create", C.byref(st))
    fakhip.call("fhip_set_stream", st)
    allocs, devs = [], []
    try:
        H, I = 512, 2048  # K = 2048: the 8-token calls split K in two and reduce
        rng = np.random.default_rng(5)
        q6raw = qc.pin_d(rng.integers(0, 256, H * (I // 256) * 210, dtype=np.uint8), 0x1000)
        rgate, rup, rdown = (synth.q4k_weights(I, H, 31), synth.q4k_weights(I, H, 32),
                             synth.q4k_weights(H, I, 33))  # alive across the uploads
        g = fakhip.alloc_call("fhip_q4k_upload", rgate.ctypes.data, I, H)
        u = fakhip.alloc_call("fhip_q4k_upload", rup.ctypes.data, I, H)
        d4 = fakhip.alloc_call("fhip_q4k_upload", rdown.ctypes.data, H, I)
        d6 = fakhip.alloc_call("fhip_q6k_upload", q6raw.ctypes.data, H, I)
        allocs += [g, u, d4, d6]
        x3 = Dev(8 * H * 4)
        xi = Dev(20 * I * 4)
        devs += [x3, xi]
        names = [("mlp1", H), ("mlp3", 3 * H), ("mlp6", 3 * H), ("q6gemv", H), ("q6gemm", 20 * H),
                 ("q6v8", 8 * H), ("q4v8", 8 * H)]
        outs = {nm: (Dev(n * 4), Dev(n * 4)) for nm, n in names}
        for a, b in outs.values():
            devs += [a, b]

        def run(k):
            fakhip.call("fhip_q4k_mlp_f32", g, u, d4, x3.ptr, outs["mlp1"][k].ptr, H, I, 1)
            fakhip.call("fhip_q4k_mlp_f32", g, u, d4, x3.ptr, outs["mlp3"][k].ptr, H, I, 3)
            fakhip.call("fhip_q4k_mlp_q6down_f32", g, u, d6, x3.ptr, outs["mlp6"][k].ptr, H, I, 3)
            fakhip.call("fhip_q6k_matmul_f32", d6, xi.ptr, outs["q6gemv"][k].ptr, H, I, 1)
            fakhip.call("fhip_q6k_matmul_f32", d6, xi.ptr, outs["q6gemm"][k].ptr, H, I, 20)
            # verify widths: one main launch + the ordered reduce of the K-range partials
            fakhip.call("fhip_q6k_matmul_f32", d6, xi.ptr, outs["q6v8"][k].ptr, H, I, 8)
            fakhip.call("fhip_q4k_matmul_f32", d4, xi.ptr, outs["q4v8"][k].ptr, H, I, 8)

        def set_x(seed):
            a3, ai = synth.activations(8, H, seed), synth.activations(20, I, seed + 1)
            fakhip.call("fhip_h2d", x3.ptr, a3.ctypes.data, 8 * H * 4)
            fakhip.call("fhip_h2d", xi.ptr, ai.ctypes.data, 20 * I * 4)

        set_x(300)
        run(0)  # eager warm-up: sizes the workspace before capture
        fakhip.call("fhip_sync")
        fakhip.call("fhip_graph_begin")
        run(0)
        graph = C.c_void_p()
        fakhip.call("fhip_graph_end", C.byref(graph))
        try:
            for rep in range(3):
                set_x(400 + 10 * rep)
                run(1)
                fakhip.call("fhip_graph_launch", graph)
                fakhip.call("fhip_stream_sync", st)
                for nm, _ in names:
                    a, b = outs[nm]
                    assert np.array_equal(a.to_host(np.uint32), b.to_host(np.uint32)), (rep, nm)
                print(f"    replay {rep}: all {len(names)} outputs bit-identical", flush=True)
        finally:
            fakhip.call("fhip_graph_destroy", graph)
    finally:
        fakhip.call("fhip_set_stream", None)
        for d in devs:
            d.close()
        for p in allocs:
            lib.fhip_free(p)
        fakhip.call("fhip_stream_destroy", st)
