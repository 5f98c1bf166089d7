"""ctypes binding of the fakhip C ABI (include/fakhip.h).

This is the Python-side twin of the cgo block a Go host adds: one foreign
declaration per exported symbol, and a raise on any non-zero status. The library is loaded from
fak_amd/libfakhip.so; there is no fallback — if the library is missing the import fails with the
build command to run.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfakhip.so")

OK = 0
EINVAL = -1
ENODEV = -2
ENOMEM = -3


class FakHipError(RuntimeError):
    """A non-zero status from the C ABI (message from fhip_last_error)."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.code = code


_vp = C.c_void_p
_sz = C.c_size_t
_i = C.c_int

# name -> (restype, argtypes). Status-returning entries have restype c_int.
SIGNATURES = {
    "fhip_init": (_i, [C.c_char_p, _i, C.POINTER(_i), C.POINTER(_sz)]),
    "fhip_mem_info": (_i, [C.POINTER(_sz), C.POINTER(_sz)]),
    "fhip_last_error": (C.c_char_p, []),
    "fhip_malloc": (_vp, [_sz]),
    "fhip_free": (None, [_vp]),
    "fhip_trim_pool": (None, [_sz]),
    "fhip_h2d": (_i, [_vp, _vp, _sz]),
    "fhip_d2h": (_i, [_vp, _vp, _sz]),
    "fhip_d2d": (_i, [_vp, _vp, _sz]),
    "fhip_sync": (_i, []),
    "fhip_h2d_async": (_i, [_vp, _vp, _sz]),
    "fhip_d2h_async": (_i, [_vp, _vp, _sz]),
    "fhip_memset_async": (_i, [_vp, _i, _sz]),
    "fhip_stream_create": (_i, [C.POINTER(_vp)]),
    "fhip_stream_destroy": (_i, [_vp]),
    "fhip_set_stream": (_i, [_vp]),
    "fhip_stream_sync": (_i, [_vp]),
    "fhip_graph_begin": (_i, []),
    "fhip_graph_end": (_i, [C.POINTER(_vp)]),
    "fhip_graph_launch": (_i, [_vp]),
    "fhip_graph_destroy": (_i, [_vp]),
    "fhip_event_create": (_i, [C.POINTER(_vp)]),
    "fhip_event_destroy": (_i, [_vp]),
    "fhip_event_record": (_i, [_vp]),
    "fhip_time_next_launch": (_i, [_vp, _vp]),
    "fhip_event_elapsed_ms": (_i, [_vp, _vp, C.POINTER(C.c_float)]),
    "fhip_q4k_packed_bytes": (_sz, [_i, _i]),
    "fhip_probe_read_sink_words": (_sz, [_sz]),
    "fhip_probe_read": (_i, [_vp, _sz, _vp]),
    "fhip_probe_q4k_records_sink_words": (_sz, [_i, _i]),
    "fhip_probe_q4k_records": (_i, [_vp, _i, _i, _vp]),
    "fhip_q4k_repack": (_i, [_vp, _vp, _i, _i]),
    "fhip_q4k_unpack": (_i, [_vp, _vp, _i, _i]),
    "fhip_q4k_dequant_f32": (_i, [_vp, _vp, _i, _i]),
    "fhip_q4k_upload": (_vp, [_vp, _i, _i]),
    "fhip_q4k_matmul_f32": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "fhip_q8_0_packed_bytes": (_sz, [_i, _i]),
    "fhip_q8_0_repack": (_i, [_vp, _vp, _i, _i]),
    "fhip_q8_0_unpack": (_i, [_vp, _vp, _i, _i]),
    "fhip_q8_0_dequant_f32": (_i, [_vp, _vp, _i, _i]),
    "fhip_q8_0_upload": (_vp, [_vp, _i, _i]),
    "fhip_q8_0_matmul_f32": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "fhip_q4k_matmul_group_f32": (_i, [_vp, _vp, _vp, _i, _vp, _i, _i]),
    "fhip_q4k_matmul_int8_f32": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "fhip_q4k_matmul_noalloc_f32": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "fhip_q6k_bytes": (C.c_size_t, [_i, _i]),
    "fhip_q6k_packed_bytes": (C.c_size_t, [_i, _i]),
    "fhip_q6k_repack": (_i, [_vp, _vp, _i, _i]),
    "fhip_q6k_unpack": (_i, [_vp, _vp, _i, _i]),
    "fhip_q6k_upload": (_vp, [_vp, _i, _i]),
    "fhip_q6k_dequant_f32": (_i, [_vp, _vp, _i, _i]),
    "fhip_q6k_matmul_f32": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "fhip_q4k_mlp_f32": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i]),
    "fhip_q4k_mlp_q6down_f32": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i]),
    "fhip_q8_quantize_f32": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "fhip_q8_matmul_f32": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i]),
}

_lib = None


def load() -> C.CDLL:
    """Load libfakhip.so and declare every exported symbol (no device call is made)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m fak_amd.build` "
                              "(hipcc, gfx950)")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error() -> str:
    return (load().fhip_last_error() or b"").decode(errors="replace")


def check(fn: str, rc: int) -> None:
    if rc != OK:
        raise FakHipError(fn, rc, last_error())


def call(fn: str, *args) -> int:
    """Call a status-returning entry and raise FakHipError on a non-zero status."""
    rc = getattr(load(), fn)(*args)
    check(fn, rc)
    return rc


def alloc_call(fn: str, *args) -> int:
    """Call a pointer-returning entry (malloc/upload) and raise on NULL."""
    p = getattr(load(), fn)(*args)
    if not p:
        raise FakHipError(fn, ENOMEM, last_error())
    return p


def init() -> dict:
    name = C.create_string_buffer(256)
    arch = _i()
    total = _sz()
    call("fhip_init", name, 256, C.byref(arch), C.byref(total))
    return {"name": name.value.decode(errors="replace"), "arch": arch.value,
            "total_mem": total.value}
