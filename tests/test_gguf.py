"""The GGUF reader (fak_amd.gguf) against the reference's own reader tests
(internal/ggufload/gguf_test.go:26-152, 154-206, 992-1049, 1051-1064, 1221-1255): the same
byte streams, the same directory and alignment results, the same rejections, and the fixture
tensors' bytes decoding to the reference's expected values (through the oracle for Q8_0 / Q4_K /
Q6_K). The byte streams here are built field by field, independently of gguf.write, which is
then checked by round trip."""
import io
import struct

import numpy as np
import pytest

from fak_amd import gguf
from fak_amd.gguf import GGUFError, TensorType, ValueType


def s(x: str) -> bytes:
    e = x.encode()
    return struct.pack("<Q", len(e)) + e


def kv(key: str, typ: int, payload: bytes) -> bytes:
    return s(key) + struct.pack("<I", typ) + payload


def tinfo(name: str, dims, typ: int, off: int) -> bytes:
    return (s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            + struct.pack("<IQ", typ, off))


def header(tensors: int, kvs: int) -> bytes:
    return b"GGUF" + struct.pack("<IQQ", 3, tensors, kvs)


def directory_stream() -> bytes:
    """The stream of TestReadParsesMetadataTensorDirectoryAndConfig: 3 tensors, 14 KVs,
    general.alignment = 64."""
    u32 = lambda v: struct.pack("<I", v)
    u64 = lambda v: struct.pack("<Q", v)
    f32 = lambda v: struct.pack("<f", v)
    b = header(3, 14)
    b += kv("general.architecture", 8, s("qwen2"))
    b += kv("general.alignment", 4, u32(64))
    b += kv("qwen2.context_length", 10, u64(32768))
    b += kv("qwen2.embedding_length", 10, u64(32))
    b += kv("qwen2.block_count", 10, u64(2))
    b += kv("qwen2.feed_forward_length", 10, u64(64))
    b += kv("qwen2.rope.dimension_count", 10, u64(8))
    b += kv("qwen2.attention.head_count", 10, u64(4))
    b += kv("qwen2.attention.head_count_kv", 10, u64(2))
    b += kv("qwen2.attention.layer_norm_rms_epsilon", 6, f32(1e-5))
    b += kv("qwen2.rope.freq_base", 6, f32(1000000))
    b += kv("tokenizer.ggml.eos_token_id", 4, u32(2))
    b += kv("tokenizer.ggml.tokens", 9, u32(8) + u64(3) + s("<unk>") + s("hello") + s("world"))
    b += kv("tokenizer.ggml.token_type", 9, u32(5) + u64(3) + u32(1) * 3)
    b += tinfo("token_embd.weight", [32, 3], 0, 0)
    b += tinfo("output.weight", [32, 3], 12, 64)
    b += tinfo("blk.0.attn_q.bias", [32], 0, 128)
    return b


def test_read_parses_metadata_and_directory():
    b = directory_stream()
    f = gguf.read(io.BytesIO(b))
    assert f.Version == 3 and f.Alignment == 64
    assert f.TensorDataOffset % 64 == 0 and f.TensorDataOffset >= len(b)
    assert f.TensorDataOffset == (len(b) + 63) // 64 * 64
    assert len(f.Tensors) == 3
    t = f.Tensors[1]
    assert t.Name == "output.weight" and t.Type == TensorType.Q4_K
    assert t.FileOffset == f.TensorDataOffset + 64
    assert f.string_array("tokenizer.ggml.tokens") == ["<unk>", "hello", "world"]
    assert f.string_array("tokenizer.ggml.token_type") is None  # int items
    assert f.string("general.architecture") == "qwen2"
    assert f.uint64("qwen2.embedding_length") == 32
    assert f.Metadata["qwen2.attention.layer_norm_rms_epsilon"].Value == np.float32(1e-5)
    assert gguf.model_shape(f.Tensors[0]) == [3, 32]


def test_read_rejects_bad_alignment_and_bool():
    with pytest.raises(GGUFError, match="alignment"):
        gguf.read(io.BytesIO(header(0, 1) + kv("general.alignment", 4, struct.pack("<I", 7))))
    with pytest.raises(GGUFError, match="bool"):
        gguf.read(io.BytesIO(header(0, 1) + s("test.flag") + struct.pack("<I", 7) + b"\x02"))


@pytest.mark.parametrize("bad", [
    b"GGUX" + struct.pack("<IQQ", 3, 0, 0),            # magic
    b"GGUF" + struct.pack("<IQQ", 2, 0, 0),            # version
    header(0, 1) + kv("general.alignment", 4, struct.pack("<I", 0)),
    header(0, 1) + kv("general.alignment", 6, struct.pack("<f", 32.0)),  # not an integer
    header(0, 1) + kv("general.alignment", 5, struct.pack("<i", -32)),   # negative
    header(0, 1) + s("k") + struct.pack("<I", 13) + b"\0" * 8,           # unknown value type
    header(1, 0) + tinfo("t", [1, 1, 1, 1, 1], 0, 0),                    # 5 dims
    header(1, 0) + tinfo("t", [8], 0, 4),                                # misaligned offset
    header(0, 1) + struct.pack("<Q", (1 << 30) + 1),                     # oversize string
    header(1, 0)[:-3],                                                   # truncated
])
def test_read_rejects_malformed(bad):
    with pytest.raises(GGUFError):
        gguf.read(io.BytesIO(bad))


def test_signed_alignment_accepted():
    f = gguf.read(io.BytesIO(header(0, 1) + kv("general.alignment", 5, struct.pack("<i", 16))))
    assert f.Alignment == 16


def q4k_fixture():
    """q4KFixtureCodes + the tinyTensorGGUF header: d = 1, dmin = 0, every scale 1, min 0;
    codes of group g, lane l: low l % 16, high 15 - l % 16."""
    codes, want = bytearray(), np.zeros(256, np.float32)
    for g in range(0, 256, 64):
        for l in range(32):
            lo, hi = l % 16, 15 - l % 16
            codes.append(lo | hi << 4)
            want[g + l], want[g + 32 + l] = lo, hi
    blk = struct.pack("<HH", 0x3C00, 0) + bytes([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]) + bytes(codes)
    return blk, want


def q6k_fixture():
    """q6KFixtureBlock: code(i) = (7 i + 3) % 64, every scale 1, d = 1; weight i = code(i) - 32."""
    ql, qh = bytearray(128), bytearray(64)
    want = np.zeros(256, np.float32)
    code = lambda i: (i * 7 + 3) % 64
    for chunk in (0, 128):
        for l in range(32):
            c = [code(chunk + l + 32 * k) for k in range(4)]
            ql[chunk // 2 + l] = (c[0] & 15) | (c[2] & 15) << 4
            ql[chunk // 2 + 32 + l] = (c[1] & 15) | (c[3] & 15) << 4
            qh[chunk // 4 + l] = sum(((c[k] >> 4) & 3) << (2 * k) for k in range(4))
            for k in range(4):
                want[chunk + l + 32 * k] = c[k] - 32
    return bytes(ql) + bytes(qh) + bytes([1] * 16) + struct.pack("<H", 0x3C00), want


def tiny_tensor_stream() -> bytes:
    """tinyTensorGGUF's layout for the types this backend handles: the directory, 32-byte
    alignment, and each payload at its fixed data-relative offset."""
    q4, _ = q4k_fixture()
    q6, _ = q6k_fixture()
    q8 = struct.pack("<H", 0x3C00) + bytes((i - 16) & 0xFF for i in range(32))
    ents = [("f32.weight", [2], 0, 0, struct.pack("<ff", 1.25, -2.5)),
            ("f16.weight", [3], 1, 32, struct.pack("<HHH", 0x3C00, 0xC000, 0x3800)),
            ("bf16.weight", [2], 30, 64,
             struct.pack("<HH", struct.unpack("<I", struct.pack("<f", 3.5))[0] >> 16,
                         struct.unpack("<I", struct.pack("<f", -4.0))[0] >> 16)),
            ("q8.weight", [32], 8, 96, q8), ("q4k.weight", [256], 12, 160, q4),
            ("q6k.weight", [256], 14, 320, q6)]
    b = header(len(ents), 1) + kv("general.alignment", 4, struct.pack("<I", 32))
    for name, dims, typ, off, _ in ents:
        b += tinfo(name, dims, typ, off)
    b += b"\0" * (-len(b) % 32)
    start = len(b)
    data = bytearray()
    for _, _, _, off, payload in ents:
        data += b"\0" * (off - len(data))
        data += payload
    return bytes(b) + bytes(data), start


@pytest.fixture
def tiny_path(tmp_path):
    b, _ = tiny_tensor_stream()
    p = tmp_path / "tiny.gguf"
    p.write_bytes(b)
    return str(p)


def test_weight_source_fixture_tensors(tiny_path, oracle_mod):
    _, start = tiny_tensor_stream()
    with gguf.WeightSource(tiny_path) as ws:
        assert ws.file.TensorDataOffset == start
        np.testing.assert_array_equal(ws.tensor_f32("f32.weight"), [1.25, -2.5])
        np.testing.assert_array_equal(ws.tensor_f32("f16.weight"), [1, -2, 0.5])
        np.testing.assert_array_equal(ws.tensor_f32("bf16.weight"), [3.5, -4])
        raw = lambda n: np.frombuffer(ws.tensor_bytes(n), np.uint8).copy()
        assert len(raw("q8.weight")) == 34 and len(raw("q4k.weight")) == 144
        assert len(raw("q6k.weight")) == 210
        got = oracle_mod.q8_0_dequant(raw("q8.weight"), 1, 32).ravel()
        np.testing.assert_array_equal(got, np.arange(32, dtype=np.float32) - 16)
        _, want = q4k_fixture()
        np.testing.assert_array_equal(oracle_mod.q4k_dequant(raw("q4k.weight"), 1, 256).ravel(), want)
        _, want = q6k_fixture()
        np.testing.assert_array_equal(oracle_mod.q6k_dequant(raw("q6k.weight"), 1, 256).ravel(), want)
        assert ws.tensor("missing.weight") is None
        with pytest.raises(GGUFError, match="missing"):
            ws.tensor_bytes("missing.weight")
        with pytest.raises(GGUFError, match="device"):
            ws.tensor_f32("q4k.weight")


def test_tensor_bytes_overrun(tmp_path):
    b, _ = tiny_tensor_stream()
    p = tmp_path / "cut.gguf"
    p.write_bytes(b[:-10])  # the last tensor (q6k.weight) loses its tail
    with gguf.WeightSource(str(p)) as ws:
        assert len(ws.tensor_bytes("q4k.weight")) == 144
        with pytest.raises(GGUFError, match="overruns"):
            ws.tensor_bytes("q6k.weight")


@pytest.mark.parametrize("typ,elems,want", [
    (TensorType.F32, 7, 28), (TensorType.F16, 7, 14), (TensorType.BF16, 3, 6),
    (TensorType.Q8_0, 64, 68), (TensorType.Q4_0, 32, 18), (TensorType.Q4_1, 32, 20),
    (TensorType.Q5_0, 32, 22), (TensorType.Q5_1, 32, 24), (TensorType.Q2_K, 256, 84),
    (TensorType.Q3_K, 256, 110), (TensorType.Q4_K, 512, 288), (TensorType.Q5_K, 256, 176),
    (TensorType.Q6_K, 256, 210), (TensorType.MXFP4, 32, 17), (TensorType.IQ4_NL, 32, 18),
    (TensorType.IQ4_XS, 256, 136), (TensorType.IQ3_XXS, 256, 98),
])
def test_payload_bytes(typ, elems, want):
    assert gguf.tensor_payload_bytes(gguf.TensorInfo("t", [elems], int(typ), 0)) == want


def test_payload_bytes_rejects():
    with pytest.raises(GGUFError, match="multiple"):
        gguf.tensor_payload_bytes(gguf.TensorInfo("t", [100], int(TensorType.Q4_K), 0))
    with pytest.raises(GGUFError):
        gguf.tensor_payload_bytes(gguf.TensorInfo("t", [32], 99, 0))


def test_writer_round_trip(tmp_path, oracle_mod):
    rng = np.random.default_rng(5)
    q4 = rng.integers(0, 256, 2 * 144, dtype=np.uint8).tobytes()
    f32 = rng.standard_normal(5).astype(np.float32).tobytes()
    meta = [("general.architecture", ValueType.STRING, "llama"),
            ("x.count", ValueType.UINT64, 7), ("x.flag", ValueType.BOOL, True),
            ("x.neg", ValueType.INT8, -3), ("x.f64", ValueType.FLOAT64, 0.25),
            ("x.arr", ValueType.ARRAY, (ValueType.UINT16, [1, 2, 65535])),
            ("x.nested", ValueType.ARRAY, (ValueType.ARRAY, [(ValueType.STRING, ["a"])]))]
    tens = [("w.q4k", [256, 2], TensorType.Q4_K, q4), ("n.f32", [5], TensorType.F32, f32)]
    p = str(tmp_path / "rt.gguf")
    gguf.write(p, meta, tens, align=64)
    with gguf.WeightSource(p) as ws:
        f = ws.file
        assert f.Alignment == 64 and f.uint64("x.count") == 7
        assert f.Metadata["x.flag"].Value is True and f.Metadata["x.neg"].Value == -3
        assert f.uint64("x.neg") is None
        assert [v.Value for v in f.Metadata["x.arr"].Value] == [1, 2, 65535]
        assert f.Metadata["x.nested"].Value[0].Value[0].Value == "a"
        assert bytes(ws.tensor_bytes("w.q4k")) == q4
        assert bytes(ws.tensor_bytes("n.f32")) == f32
        assert gguf.model_shape(ws.tensor("w.q4k")) == [2, 256]
        assert all(t.FileOffset % 64 == 0 for t in f.Tensors)
