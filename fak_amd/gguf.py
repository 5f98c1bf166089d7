"""GGUF v3 reader and the direct-resident device loader for the matmul weights.

The reader restates fak's `ggufload.Read` (internal/ggufload/gguf_config.go:15-112; value and
string decoding internal/ggufload/gguf_dequant.go:845-968; alignment and payload sizes :14-128)
with the same checks and error conditions. The tensor data is memory-mapped, so a multi-GB file
is never read whole.

`load_resident` is the device half of the reference's direct-resident loader
(`QuantModelQ4KProfileOptions`, internal/ggufload/quant_q4k_loader.go:153-370): matmul weights
whose GGUF type has a device kernel (Q4_K, Q8_0, Q6_K) go to the device in their raw GGUF bytes
(`fhip_q4k_upload`, `fhip_q8_0_upload`, `fhip_q6k_upload`); the model shape is the reversed GGUF
dims (`modelShapeFromGGUFDims`, internal/ggufload/gguf_tensor_canonical.go:386-399).

`write` produces a GGUF v3 file from metadata and raw tensor payloads (test fixtures, tools).
"""
from __future__ import annotations

import dataclasses
import enum
import io
import mmap
import os
import struct
from typing import Any, BinaryIO, Optional

MAGIC = b"GGUF"
VERSION = 3
DEFAULT_ALIGN = 32
MAX_STRING_BYTES = 1 << 30
QK_K = 256


class ValueType(enum.IntEnum):
    """internal/ggufload/gguf.go:57-71."""
    UINT8 = 0
    INT8 = 1
    UINT16 = 2
    INT16 = 3
    UINT32 = 4
    INT32 = 5
    FLOAT32 = 6
    BOOL = 7
    STRING = 8
    ARRAY = 9
    UINT64 = 10
    INT64 = 11
    FLOAT64 = 12


class TensorType(enum.IntEnum):
    """internal/ggufload/gguf.go:78-96."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    IQ3_XXS = 18
    IQ4_NL = 20
    IQ4_XS = 23
    BF16 = 30
    MXFP4 = 39


# (elements per block, bytes per block): internal/ggufload/gguf.go:17-50
_BLOCK = {
    TensorType.F32: (1, 4), TensorType.F16: (1, 2), TensorType.BF16: (1, 2),
    TensorType.Q4_0: (32, 18), TensorType.Q4_1: (32, 20), TensorType.Q5_0: (32, 22),
    TensorType.Q5_1: (32, 24), TensorType.Q8_0: (32, 34), TensorType.Q2_K: (256, 84),
    TensorType.Q3_K: (256, 110), TensorType.Q4_K: (256, 144), TensorType.Q5_K: (256, 176),
    TensorType.Q6_K: (256, 210), TensorType.MXFP4: (32, 17), TensorType.IQ4_NL: (32, 18),
    TensorType.IQ4_XS: (256, 136), TensorType.IQ3_XXS: (256, 98),
}


class GGUFError(ValueError):
    pass


@dataclasses.dataclass
class Value:
    Type: ValueType
    Value: Any


@dataclasses.dataclass
class TensorInfo:
    Name: str
    Dims: list
    Type: int
    Offset: int
    FileOffset: int = 0


@dataclasses.dataclass
class File:
    Version: int
    Metadata: dict
    Tensors: list
    Alignment: int
    TensorDataOffset: int

    def string(self, key: str) -> Optional[str]:
        v = self.Metadata.get(key)
        return v.Value if v is not None and v.Type == ValueType.STRING else None

    def uint64(self, key: str) -> Optional[int]:
        v = self.Metadata.get(key)
        return _value_uint64(v) if v is not None else None

    def string_array(self, key: str) -> Optional[list]:
        """StringArray (internal/ggufload/gguf_meta.go): an array whose items are all strings."""
        v = self.Metadata.get(key)
        if v is None or v.Type != ValueType.ARRAY:
            return None
        if any(it.Type != ValueType.STRING for it in v.Value):
            return None
        return [it.Value for it in v.Value]


def _value_uint64(v: Value) -> Optional[int]:
    """valueUint64 (internal/ggufload/gguf_meta.go:148-): unsigned, or signed and >= 0."""
    if v.Type in (ValueType.UINT8, ValueType.UINT16, ValueType.UINT32, ValueType.UINT64):
        return int(v.Value)
    if v.Type in (ValueType.INT8, ValueType.INT16, ValueType.INT32, ValueType.INT64):
        return int(v.Value) if v.Value >= 0 else None
    return None


class _Reader:
    """countingReader: little-endian reads with a byte count."""

    def __init__(self, f: BinaryIO):
        self.f, self.n = f, 0

    def full(self, k: int) -> bytes:
        b = self.f.read(k)
        if len(b) != k:
            raise GGUFError("gguf: unexpected EOF")
        self.n += k
        return b

    def u32(self) -> int:
        return struct.unpack("<I", self.full(4))[0]

    def u64(self) -> int:
        return struct.unpack("<Q", self.full(8))[0]

    def str(self) -> str:
        n = self.u64()
        if n > MAX_STRING_BYTES:
            raise GGUFError(f"string too large: {n} bytes")
        return self.full(n).decode("utf-8", errors="surrogateescape")

    def value(self, typ: int) -> Value:
        if typ == ValueType.UINT8:
            return Value(ValueType.UINT8, self.full(1)[0])
        if typ == ValueType.INT8:
            return Value(ValueType.INT8, struct.unpack("<b", self.full(1))[0])
        if typ == ValueType.UINT16:
            return Value(ValueType.UINT16, struct.unpack("<H", self.full(2))[0])
        if typ == ValueType.INT16:
            return Value(ValueType.INT16, struct.unpack("<h", self.full(2))[0])
        if typ == ValueType.UINT32:
            return Value(ValueType.UINT32, self.u32())
        if typ == ValueType.INT32:
            return Value(ValueType.INT32, struct.unpack("<i", self.full(4))[0])
        if typ == ValueType.FLOAT32:
            return Value(ValueType.FLOAT32, struct.unpack("<f", self.full(4))[0])
        if typ == ValueType.BOOL:
            b = self.full(1)[0]
            if b > 1:
                raise GGUFError(f"invalid bool byte {b}")
            return Value(ValueType.BOOL, b == 1)
        if typ == ValueType.STRING:
            return Value(ValueType.STRING, self.str())
        if typ == ValueType.ARRAY:
            elem = self.u32()
            n = self.u64()
            return Value(ValueType.ARRAY, [self.value(elem) for _ in range(n)])
        if typ == ValueType.UINT64:
            return Value(ValueType.UINT64, self.u64())
        if typ == ValueType.INT64:
            return Value(ValueType.INT64, struct.unpack("<q", self.full(8))[0])
        if typ == ValueType.FLOAT64:
            return Value(ValueType.FLOAT64, struct.unpack("<d", self.full(8))[0])
        raise GGUFError(f"unsupported value type {typ}")


def alignment(meta: dict) -> int:
    """internal/ggufload/gguf_dequant.go:14-27."""
    align = DEFAULT_ALIGN
    if "general.alignment" in meta:
        got = _value_uint64(meta["general.alignment"])
        if got is None:
            raise GGUFError("gguf: general.alignment is not an unsigned integer")
        align = got
    if align == 0 or align % 8 != 0:
        raise GGUFError(f"gguf: invalid alignment {align}")
    return align


def align_offset(off: int, align: int) -> int:
    return off + (align - off % align) % align


def read(f: BinaryIO) -> File:
    """ggufload.Read: header, metadata, tensor directory, data offset."""
    r = _Reader(f)
    magic = r.full(4)
    if magic != MAGIC:
        raise GGUFError(f"gguf: bad magic {magic!r}")
    ver = r.u32()
    if ver != VERSION:
        raise GGUFError(f"gguf: unsupported version {ver}")
    tensor_count, kv_count = r.u64(), r.u64()
    meta = {}
    for i in range(kv_count):
        key = r.str()
        typ = r.u32()
        meta[key] = r.value(typ)
    tensors = []
    for i in range(tensor_count):
        name = r.str()
        nd = r.u32()
        if nd > 4:
            raise GGUFError(f"gguf: tensor {name} has {nd} dimensions")
        dims = [r.u64() for _ in range(nd)]
        typ = r.u32()
        off = r.u64()
        tensors.append(TensorInfo(name, dims, typ, off))
    align = alignment(meta)
    data = align_offset(r.n, align)
    for t in tensors:
        if t.Offset % align:
            raise GGUFError(f"gguf: tensor {t.Name} offset {t.Offset} is not {align}-byte aligned")
        t.FileOffset = data + t.Offset
    return File(ver, meta, tensors, align, data)


def tensor_elems(t: TensorInfo) -> int:
    n = 1
    for d in t.Dims:
        n *= int(d)
    return n


def tensor_payload_bytes(t: TensorInfo) -> int:
    """tensorPayloadBytes, internal/ggufload/gguf_dequant.go:44-128."""
    try:
        qk, bb = _BLOCK[TensorType(t.Type)]
    except (ValueError, KeyError):
        raise GGUFError(f"gguf: tensor {t.Name} type {t.Type} does not have a simple f32 payload")
    elems = tensor_elems(t)
    if elems % qk:
        raise GGUFError(f"gguf: tensor {t.Name} {TensorType(t.Type).name} element count {elems} "
                        f"is not a multiple of {qk}")
    return elems // qk * bb


def model_shape(t: TensorInfo) -> list:
    """modelShapeFromGGUFDims: the GGUF dims reversed ([in, out] -> [out, in])."""
    if not t.Dims:
        raise GGUFError(f"gguf: tensor {t.Name} has no dimensions")
    return [int(d) for d in reversed(t.Dims)]


class WeightSource:
    """A parsed file plus a memory map of its bytes (OpenWeights / TensorBytes,
    internal/ggufload/gguf_open.go:26-62, gguf_weightsource.go:81-119)."""

    def __init__(self, path: str):
        self._fh = open(path, "rb")
        self.file = read(self._fh)
        self.size = os.fstat(self._fh.fileno()).st_size
        self._mm = mmap.mmap(self._fh.fileno(), 0, access=mmap.ACCESS_READ) if self.size else None
        self._by_name = {t.Name: t for t in self.file.Tensors}

    def close(self) -> None:
        if self._mm is not None:
            self._mm.close()
            self._mm = None
        self._fh.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def tensor(self, name: str) -> Optional[TensorInfo]:
        return self._by_name.get(name)

    def tensor_bytes(self, name: str) -> memoryview:
        """The raw payload, bounds-checked against the file (a view into the map)."""
        info = self.tensor(name)
        if info is None:
            raise GGUFError(f"gguf: missing tensor {name}")
        n = tensor_payload_bytes(info)
        if info.FileOffset < 0 or info.FileOffset + n > self.size:
            raise GGUFError(f"gguf: tensor {name} overruns file")
        return memoryview(self._mm)[info.FileOffset:info.FileOffset + n]

    def tensor_f32(self, name: str):
        """Host f32 values of an F32 / F16 / BF16 tensor (norms, biases, embeddings that stay
        on the host). The quantized types are decoded on the device from their resident bytes
        (fhip_*_dequant_f32); asking for one here raises."""
        import numpy as np
        info = self.tensor(name)
        if info is None:
            raise GGUFError(f"gguf: missing tensor {name}")
        raw = np.frombuffer(self.tensor_bytes(name), np.uint8)
        if info.Type == TensorType.F32:
            return raw.view("<f4").astype(np.float32)
        if info.Type == TensorType.F16:
            return raw.view("<f2").astype(np.float32)
        if info.Type == TensorType.BF16:
            return (raw.view("<u2").astype(np.uint32) << 16).view(np.float32)
        raise GGUFError(f"gguf: tensor {name} type {info.Type} is decoded on the device")


# device uploads per GGUF type: (entry, block elements)
_UPLOAD = {TensorType.Q4_K: ("fhip_q4k_upload", 256), TensorType.Q8_0: ("fhip_q8_0_upload", 32),
           TensorType.Q6_K: ("fhip_q6k_upload", 256)}
# the matmul entry for each resident type
MATMUL = {TensorType.Q4_K: "fhip_q4k_matmul_f32", TensorType.Q8_0: "fhip_q8_0_matmul_f32",
          TensorType.Q6_K: "fhip_q6k_matmul_f32"}


@dataclasses.dataclass
class ResidentWeight:
    name: str
    type: TensorType
    shape: list  # [out, in]
    ptr: int     # device handle from the type's upload entry

    def matmul(self, dX: int, dY: int, P: int) -> None:
        from . import fakhip
        fakhip.call(MATMUL[self.type], self.ptr, dX, dY, self.shape[0], self.shape[1], P)

    def free(self) -> None:
        from . import fakhip
        if self.ptr:
            fakhip.load().fhip_free(self.ptr)
            self.ptr = 0


def load_resident(src: WeightSource, names=None) -> dict:
    """Upload every 2-D tensor (or those in `names`) whose type has a device kernel. Returns
    {name: ResidentWeight}; other tensors are left to the host."""
    import numpy as np

    from . import fakhip
    out = {}
    for info in src.file.Tensors:
        if names is not None and info.Name not in names:
            continue
        try:
            typ = TensorType(info.Type)
        except ValueError:
            continue
        if typ not in _UPLOAD or len(info.Dims) != 2:
            continue
        rows, cols = model_shape(info)
        entry, qk = _UPLOAD[typ]
        if cols % qk:
            raise GGUFError(f"gguf: tensor {info.Name} row length {cols} is not a multiple of {qk}")
        # the upload reads straight from the file mapping (no host copy of the payload)
        buf = np.frombuffer(src.tensor_bytes(info.Name), np.uint8)
        ptr = fakhip.alloc_call(entry, buf.ctypes.data, rows, cols)
        del buf
        out[info.Name] = ResidentWeight(info.Name, typ, [rows, cols], ptr)
    return out


def _w_str(b: io.BytesIO, s: str) -> None:
    e = s.encode("utf-8")
    b.write(struct.pack("<Q", len(e)))
    b.write(e)


def _w_value(b: io.BytesIO, typ: ValueType, v: Any) -> None:
    fmt = {ValueType.UINT8: "<B", ValueType.INT8: "<b", ValueType.UINT16: "<H",
           ValueType.INT16: "<h", ValueType.UINT32: "<I", ValueType.INT32: "<i",
           ValueType.FLOAT32: "<f", ValueType.UINT64: "<Q", ValueType.INT64: "<q",
           ValueType.FLOAT64: "<d"}
    if typ in fmt:
        b.write(struct.pack(fmt[typ], v))
    elif typ == ValueType.BOOL:
        b.write(bytes([1 if v else 0]))
    elif typ == ValueType.STRING:
        _w_str(b, v)
    elif typ == ValueType.ARRAY:
        elem, items = v
        b.write(struct.pack("<IQ", int(elem), len(items)))
        for it in items:
            _w_value(b, elem, it)
    else:
        raise GGUFError(f"unsupported value type {typ}")


def write(path: str, metadata: list, tensors: list, align: int = DEFAULT_ALIGN) -> None:
    """Write a GGUF v3 file. metadata: [(key, ValueType, value)] (an array value is
    (element ValueType, [items])); tensors: [(name, dims (GGUF order), TensorType, raw bytes)].
    A non-default `align` is recorded as general.alignment."""
    meta = list(metadata)
    if align != DEFAULT_ALIGN and not any(k == "general.alignment" for k, _, _ in meta):
        meta.append(("general.alignment", ValueType.UINT32, align))
    hdr = io.BytesIO()
    hdr.write(MAGIC)
    hdr.write(struct.pack("<IQQ", VERSION, len(tensors), len(meta)))
    for key, typ, v in meta:
        _w_str(hdr, key)
        hdr.write(struct.pack("<I", int(typ)))
        _w_value(hdr, typ, v)
    off = 0
    offsets = []
    for name, dims, typ, raw in tensors:
        offsets.append(off)
        _w_str(hdr, name)
        hdr.write(struct.pack("<I", len(dims)))
        for d in dims:
            hdr.write(struct.pack("<Q", int(d)))
        hdr.write(struct.pack("<IQ", int(typ), off))
        off = align_offset(off + len(raw), align)
    with open(path, "wb") as f:
        h = hdr.getvalue()
        f.write(h)
        f.write(b"\0" * (align_offset(len(h), align) - len(h)))
        for (name, dims, typ, raw), o in zip(tensors, offsets):
            f.write(bytes(raw))
            end = o + len(raw)
            f.write(b"\0" * (align_offset(end, align) - end))
