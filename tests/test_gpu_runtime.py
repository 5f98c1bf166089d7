"""The runtime's device memory over stream and graph lifetimes: every stream gets its own scratch
workspace, which must go back to the driver when the stream is destroyed (or, for a stream a
graph was captured on, once no graph is alive and the pool is trimmed), and a graph replays only
on the stream whose workspace its kernels use."""
import ctypes as C

import numpy as np
import pytest

from fak_amd import fakhip, synth
from tests.gpu_util import Dev

pytestmark = pytest.mark.gpu

MiB = 1 << 20
# A 16-token GEMV with K-range partials: the stream's workspace grows to >= 16 MiB on first use.
OUT, IN, P = 2048, 6144, 16


def free_bytes() -> int:
    lib = fakhip.load()
    lib.fhip_trim_pool(0)  # parked pool blocks back to the driver, so only live memory counts
    f, t = C.c_size_t(), C.c_size_t()
    fakhip.call("fhip_mem_info", C.byref(f), C.byref(t))
    return f.value


@pytest.fixture(scope="module")
def weight(hip):
    raw = synth.q4k_weights(OUT, IN, 91)
    w = fakhip.alloc_call("fhip_q4k_upload", raw.ctypes.data, OUT, IN)
    yield w
    fakhip.load().fhip_free(w)


def matmul_on(stream, w, dx, dy):
    fakhip.call("fhip_set_stream", stream)
    fakhip.call("fhip_q4k_matmul_f32", w, dx.ptr, dy.ptr, OUT, IN, P)


def test_stream_workspaces_are_freed(weight):
    """Create a stream, run a matmul that sizes its workspace, destroy it: 12 times over, device
    memory stays flat (each cycle used to keep >= 16 MiB for the life of the process)."""
    X = synth.activations(P, IN, 92)
    with Dev.from_host(X) as dx, Dev(P * OUT * 4) as dy:
        matmul_on(None, weight, dx, dy)
        fakhip.call("fhip_sync")
        before = free_bytes()
        for i in range(12):
            s = C.c_void_p()
            fakhip.call("fhip_stream_create", C.byref(s))
            try:
                matmul_on(s, weight, dx, dy)
                fakhip.call("fhip_stream_sync", s)
            finally:
                fakhip.call("fhip_set_stream", None)
                fakhip.call("fhip_stream_destroy", s)
        after = free_bytes()
        print(f"[runtime] free before {before / MiB:.0f} MiB, after 12 cycles {after / MiB:.0f} MiB",
              flush=True)
        assert after >= before - 8 * MiB


def test_captured_stream_workspace_freed_after_graph(weight):
    """A stream a graph was captured on keeps its workspace while the graph lives (the graph's
    kernels use it); once the graph and the stream are destroyed, fhip_trim_pool returns it. The
    graph replays only on its own stream: made current on another, launch is refused."""
    X = synth.activations(P, IN, 93)
    with Dev.from_host(X) as dx, Dev(P * OUT * 4) as dy, Dev(P * OUT * 4) as dy2:
        matmul_on(None, weight, dx, dy)
        fakhip.call("fhip_sync")
        want = dy.to_host(np.float32)
        before = free_bytes()
        s, other = C.c_void_p(), C.c_void_p()
        fakhip.call("fhip_stream_create", C.byref(s))
        fakhip.call("fhip_stream_create", C.byref(other))
        graph = C.c_void_p()
        try:
            matmul_on(s, weight, dx, dy2)  # sizes the workspace before capture
            fakhip.call("fhip_stream_sync", s)
            fakhip.call("fhip_graph_begin")
            fakhip.call("fhip_q4k_matmul_f32", weight, dx.ptr, dy2.ptr, OUT, IN, P)
            fakhip.call("fhip_graph_end", C.byref(graph))
            fakhip.call("fhip_set_stream", other)
            assert fakhip.load().fhip_graph_launch(graph) == fakhip.EINVAL
            assert "captured on" in fakhip.last_error()
            fakhip.call("fhip_set_stream", s)
            for _ in range(3):
                fakhip.call("fhip_graph_launch", graph)
                fakhip.call("fhip_stream_sync", s)
                assert np.array_equal(dy2.to_host(np.float32).view(np.uint32), want.view(np.uint32))
        finally:
            fakhip.call("fhip_set_stream", None)
            if graph:
                fakhip.call("fhip_graph_destroy", graph)
            fakhip.call("fhip_stream_destroy", s)
            fakhip.call("fhip_stream_destroy", other)
        after = free_bytes()
        print(f"[runtime] free before {before / MiB:.0f} MiB, after graph + stream "
              f"{after / MiB:.0f} MiB", flush=True)
        assert after >= before - 8 * MiB


def test_time_next_launch_stamps_one_dispatch(weight):
    """fhip_time_next_launch's events are stamped by the next one-token GEMV dispatch only: its
    duration is positive and below the launch-to-sync wall time of the same call, and a second
    call leaves the pair as it was."""
    import time
    lib = fakhip.load()
    X = synth.activations(1, IN, 94)
    ev = [C.c_void_p(), C.c_void_p()]
    for e in ev:
        fakhip.call("fhip_event_create", C.byref(e))
    try:
        with Dev.from_host(X) as dx, Dev(OUT * 4) as dy:
            fakhip.call("fhip_q4k_matmul_f32", weight, dx.ptr, dy.ptr, OUT, IN, 1)
            fakhip.call("fhip_sync")
            fakhip.call("fhip_time_next_launch", ev[0], ev[1])
            t0 = time.perf_counter()
            fakhip.call("fhip_q4k_matmul_f32", weight, dx.ptr, dy.ptr, OUT, IN, 1)
            fakhip.call("fhip_sync")
            wall_ms = 1e3 * (time.perf_counter() - t0)
            ms = C.c_float()
            fakhip.call("fhip_event_elapsed_ms", ev[0], ev[1], C.byref(ms))
            first = ms.value
            print(f"[runtime] dispatch {first * 1e3:.2f} us, wall {wall_ms * 1e3:.1f} us", flush=True)
            assert 0.0 < first < wall_ms
            fakhip.call("fhip_q4k_matmul_f32", weight, dx.ptr, dy.ptr, OUT, IN, 1)
            fakhip.call("fhip_sync")
            fakhip.call("fhip_event_elapsed_ms", ev[0], ev[1], C.byref(ms))
            assert ms.value == first
        assert lib.fhip_time_next_launch(None, ev[1]) == fakhip.EINVAL
    finally:
        for e in ev:
            fakhip.call("fhip_event_destroy", e)
