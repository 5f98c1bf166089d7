"""Device weight upload: the tiled layouts are lossless (repack -> unpack is the identity on the
GGUF bytes) and the device dequantizers are bit-identical to the oracle's q4kDequantSuperBlock /
q8_0DequantBlock (internal/model/quant_q4k.go:90-111, internal/model/quant_iquant.go:14-19).
"""
import numpy as np
import pytest

from fak_amd import fakhip, synth
from tests.gpu_util import Dev

pytestmark = pytest.mark.gpu


def _q4k_roundtrip(raw, out, in_):
    lib = fakhip.load()
    packed_bytes = lib.fhip_q4k_packed_bytes(out, in_)
    assert packed_bytes == -(-out // 16) * 16 * (in_ // 256) * 144
    with Dev.from_host(raw) as draw, Dev(packed_bytes) as dp, Dev(raw.nbytes) as dback, \
            Dev(out * in_ * 4) as dw:
        fakhip.call("fhip_q4k_repack", dp.ptr, draw.ptr, out, in_)
        fakhip.call("fhip_q4k_unpack", dback.ptr, dp.ptr, out, in_)
        fakhip.call("fhip_q4k_dequant_f32", dw.ptr, dp.ptr, out, in_)
        return dback.to_host(np.uint8), dw.to_host(np.float32).reshape(out, in_)


@pytest.mark.parametrize("out,in_", [(1, 256), (9, 512), (16, 256), (33, 768), (320, 256),
                                     (300, 3584)])
def test_q4k_repack_roundtrip_and_dequant(hip, oracle_mod, out, in_):
    print(f"[case] q4k layout out={out} in={in_}", flush=True)
    raw = synth.q4k_weights(out, in_, seed=out * 7 + in_)
    back, w = _q4k_roundtrip(raw, out, in_)
    np.testing.assert_array_equal(back, raw)
    ref = oracle_mod.q4k_dequant(raw, out, in_)
    np.testing.assert_array_equal(w.view(np.uint32), ref.view(np.uint32))


def test_q4k_dequant_every_f16_pattern(hip, oracle_mod):
    """65,536 super-blocks whose d walks every f16 bit pattern (dmin walks them in reverse):
    covers subnormals, infinities and NaNs. Finite results match bit for bit; non-finite ones
    match as non-finite (a NaN's quiet bit may differ between CPU and GPU multipliers)."""
    print("[case] q4k dequant all f16 patterns", flush=True)
    nb = 65536
    blk = np.zeros((nb, 144), np.uint8)
    pat = np.arange(nb, dtype=np.uint16)
    blk[:, 0:2] = pat.view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = pat[::-1].copy().view(np.uint8).reshape(nb, 2)
    blk[:, 4:16] = synth.pack_scale_min_k4(np.full((nb, 8), 1, np.uint8),
                                           np.full((nb, 8), 1, np.uint8))
    blk[:, 16:] = 0x21  # lo nibble 1, hi nibble 2
    raw = blk.reshape(-1)
    out, in_ = 256, 256 * 256
    back, w = _q4k_roundtrip(raw, out, in_)
    np.testing.assert_array_equal(back, raw)
    ref = oracle_mod.q4k_dequant(raw, out, in_)
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(w[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.array_equal(np.isnan(w), np.isnan(ref))
    assert np.array_equal(np.isinf(w), np.isinf(ref))
    assert fin.sum() > 0.9 * fin.size


@pytest.mark.parametrize("out,in_", [(1, 32), (9, 512), (17, 96), (1536, 576), (40, 1056)])
def test_q8_0_repack_roundtrip_and_dequant(hip, oracle_mod, out, in_):
    print(f"[case] q8_0 layout out={out} in={in_}", flush=True)
    lib = fakhip.load()
    raw = synth.q8_0_weights(out, in_, seed=out + in_)
    pb = lib.fhip_q8_0_packed_bytes(out, in_)
    with Dev.from_host(raw) as draw, Dev(pb) as dp, Dev(raw.nbytes) as dback, \
            Dev(out * in_ * 4) as dw:
        fakhip.call("fhip_q8_0_repack", dp.ptr, draw.ptr, out, in_)
        fakhip.call("fhip_q8_0_unpack", dback.ptr, dp.ptr, out, in_)
        fakhip.call("fhip_q8_0_dequant_f32", dw.ptr, dp.ptr, out, in_)
        np.testing.assert_array_equal(dback.to_host(np.uint8), raw)
        ref = oracle_mod.q8_0_dequant(raw, out, in_)
        np.testing.assert_array_equal(dw.to_host(np.float32).view(np.uint32),
                                      ref.reshape(-1).view(np.uint32))


def test_upload_entry_points(hip, oracle_mod):
    """fhip_q4k_upload / fhip_q8_0_upload (host bytes -> tiled device weight) agree with the
    explicit repack path."""
    print("[case] upload entry points", flush=True)
    lib = fakhip.load()
    out, in_ = 40, 512
    raw = synth.q4k_weights(out, in_, seed=5)
    w = fakhip.alloc_call("fhip_q4k_upload", raw.ctypes.data, out, in_)
    try:
        with Dev(raw.nbytes) as dback:
            fakhip.call("fhip_q4k_unpack", dback.ptr, w, out, in_)
            np.testing.assert_array_equal(dback.to_host(np.uint8), raw)
    finally:
        lib.fhip_free(w)
    raw8 = synth.q8_0_weights(out, in_, seed=6)
    w = fakhip.alloc_call("fhip_q8_0_upload", raw8.ctypes.data, out, in_)
    try:
        with Dev(raw8.nbytes) as dback:
            fakhip.call("fhip_q8_0_unpack", dback.ptr, w, out, in_)
            np.testing.assert_array_equal(dback.to_host(np.uint8), raw8)
    finally:
        lib.fhip_free(w)


def test_bad_arguments_are_rejected(hip):
    """Host-side argument checks return FHIP_EINVAL before any launch."""
    lib = fakhip.load()
    assert lib.fhip_q4k_repack(None, None, 16, 255) == fakhip.EINVAL
    assert lib.fhip_q4k_matmul_f32(None, None, None, 16, 512, 1) == fakhip.EINVAL
    assert lib.fhip_q4k_matmul_f32(None, None, None, 16, 500, 1) == fakhip.EINVAL
    assert lib.fhip_q8_0_matmul_f32(None, None, None, 16, 33, 1) == fakhip.EINVAL
    assert "multiple of 32" in fakhip.last_error()
    assert not lib.fhip_q4k_upload(None, 4, 256)
