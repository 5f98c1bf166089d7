"""The bandwidth-floor probes move every byte they claim to: the XOR of the sink words a probe
writes must equal the XOR of the 32-bit words it was given to read (the plain read: the whole
buffer; the record stream: the two 1 KB parts of every record, each read by one lane, while the
256-byte header is read by all four 16-lane groups of a wave and so cancels)."""

import numpy as np
import pytest

from fak_amd import fakhip, synth
from tests.gpu_util import Dev

pytestmark = pytest.mark.gpu

RECORD, HDR = 2304, 256


def xor_words(a: np.ndarray) -> int:
    return int(np.bitwise_xor.reduce(np.ascontiguousarray(a).view(np.uint32).ravel(), initial=0))


@pytest.mark.parametrize("nbytes", [16, 16 * 1000, 38_191_104, 16 * 4096 * 3 + 48])
def test_probe_read_folds_every_word(hip, nbytes):
    lib = fakhip.load()
    rng = np.random.default_rng(nbytes)
    data = rng.integers(0, 2**32, nbytes // 4, dtype=np.uint32)
    words = lib.fhip_probe_read_sink_words(nbytes)
    with Dev.from_host(data) as d, Dev(words * 4) as sink:
        fakhip.call("fhip_probe_read", d.ptr, nbytes, sink.ptr)
        fakhip.call("fhip_sync")
        assert xor_words(sink.to_host(np.uint32)) == xor_words(data)


@pytest.mark.parametrize("out,in_", [(18944, 3584), (3584, 18944), (40, 512)])
def test_probe_records_folds_every_part(hip, out, in_):
    lib = fakhip.load()
    raw = synth.q4k_weights(out, in_, 5)
    w = fakhip.alloc_call("fhip_q4k_upload", raw.ctypes.data, out, in_)
    try:
        nb = lib.fhip_q4k_packed_bytes(out, in_)
        packed = np.empty(nb, np.uint8)
        fakhip.call("fhip_d2h", packed.ctypes.data, w, nb)
        recs = packed.reshape(-1, RECORD)
        want = xor_words(recs[:, HDR:])
        words = lib.fhip_probe_q4k_records_sink_words(out, in_)
        assert words > 0
        with Dev(words * 4) as sink:
            fakhip.call("fhip_probe_q4k_records", w, out, in_, sink.ptr)
            fakhip.call("fhip_sync")
            assert xor_words(sink.to_host(np.uint32)) == want
    finally:
        lib.fhip_free(w)
