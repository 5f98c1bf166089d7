"""Host-side mirror of fak's compute HAL seam for the quantized matmul path.

The Go engine selects a device through ``compute.Backend`` (internal/compute/compute.go:318-347)
and a registry (``Register``/``Lookup``/``Pick``/``Default``, compute.go:464-519). The CUDA
tenant (internal/compute/cuda.go) implements Upload / Read / Free / MatMul / BatchedMatMul over
a flat C ABI. This module restates that contract for the ROCm backend over the fakhip C ABI, with
the same names, argument meaning and failure behaviour (a Go panic becomes a Python exception):

* ``Tensor`` carries Dtype, Layout, Shape, QuantSpec and an opaque buffer (compute.go:168-175).
* ``RocmBackend.Upload`` copies raw GGUF Q4_K bytes (``NewQ4K``, internal/compute/quant_q4k.go:
  37-44) or raw GGUF Q8_0 blocks resident in the tiled layout, caching by host buffer with an
  element-count guard (cuda.go:690-704, 803-822); F32 activations upload verbatim. HAL Q8 weights
  (``NewQ8``: int8 codes + f32 block scales, cpuref.go:53-56) upload as two device buffers, and
  ``Upload(f32 weight, Q8_0)`` narrows on the device with quantizeVecQ8 (cuda.go:714-750).
* ``MatMul(w, x)`` is y = x @ W^T (w [out,in], x [in] -> y [out]) and ``BatchedMatMul(w, X, P)``
  is the [P,in] -> [P,out] prefill GEMM, dispatched on ``w.Dtype`` (cuda.go:956-1035), each with
  the reference's shape post-condition. On a HAL Q8 weight they quantize the activation on the
  device and are bit-identical to cpuBackend.MatMul / BatchedMatMul (fhip_q8_matmul_f32).
* The backend class is Approx (harness-enforced, compute.go:212-217, 525).

Only the quantized weight path lives here; RMSNorm/RoPE/attention and the f32/f16 GEMMs are
outside this backend's scope and raise NotImplementedError.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import enum
import os
import weakref
from typing import Optional

import numpy as np

from . import fakhip


class Dtype(enum.IntEnum):
    """internal/compute/compute.go:53-64 (same order and values)."""
    F32 = 0
    F16 = 1
    BF16 = 2
    Q8_0 = 3
    I8 = 4
    I4 = 5
    FP8 = 6
    Q4_K = 7

    def __str__(self) -> str:  # compute.go:80-101
        return {0: "f32", 1: "f16", 2: "bf16", 3: "q8_0", 4: "i8", 5: "i4", 6: "fp8",
                7: "q4_k"}.get(int(self), "dtype?")


class Layout(enum.IntEnum):
    """internal/compute/compute.go:113-117."""
    RowMajor = 0
    ColMajor = 1
    Tiled = 2


class CorrectnessClass(enum.IntEnum):
    """internal/compute/compute.go:212-217."""
    Reference = 0
    Approx = 1


@dataclasses.dataclass
class QuantSpec:
    """internal/compute/compute.go:130-141."""
    Block: int = 0
    Axis: int = 0
    Bits: int = 0
    Symmetric: bool = False
    Scale: Optional[np.ndarray] = None


@dataclasses.dataclass
class Caps:
    """internal/compute/compute.go:234-256 (the fields this backend sets)."""
    Async: bool = False
    FusedAttn: bool = False
    FusedFFN: bool = False
    GraphCompile: bool = False
    UploadDtype: bool = False
    DeviceMemory: bool = False
    Collective: bool = False
    CapacityProbe: bool = False


class HostBuf:
    """A host-resident buffer (the reference's HostBuffer: F32() / I8() views)."""

    def __init__(self, f32: Optional[np.ndarray] = None, i8: Optional[np.ndarray] = None):
        self.f32 = f32
        self.i8 = i8

    def Ready(self) -> bool:
        return True


class DevBuf:
    """A device-resident buffer: pointer into the fakhip pool + byte length.

    An async op output (a matmul result) records the backend and the fence generation it was
    enqueued in, and is Ready() only once a host fence (Read) has bumped the generation past it
    (cudaBuf.Ready, internal/compute/cuda.go:286-300): the stream is FIFO, so one fence
    materializes every buffer enqueued before it. Synchronous buffers (uploads) have no backend
    and are ready on return."""

    def __init__(self, ptr: int, nbytes: int, be=None, born_gen: int = 0):
        self.ptr = ptr
        self.nbytes = nbytes
        self.be = be
        self.born_gen = born_gen

    def Ready(self) -> bool:
        if self.be is None:
            return True
        return self.be.fence_gen > self.born_gen


@dataclasses.dataclass
class Tensor:
    """internal/compute/compute.go:168-175."""
    Dtype: Dtype
    Layout: Layout
    Shape: list
    Quant: Optional[QuantSpec]
    buf: object
    be: object = None

    def Numel(self) -> int:
        n = 1
        for d in self.Shape:
            n *= d
        return n


def NewF32(be, shape, data) -> Tensor:
    """internal/compute/cpuref.go:47-49."""
    return Tensor(Dtype.F32, Layout.RowMajor, list(shape), None,
                  HostBuf(f32=np.ascontiguousarray(data, np.float32).reshape(-1)), be)


def NewQ4K(be, shape, raw) -> Tensor:
    """Raw GGUF Q4_K bytes as a host tensor (internal/compute/quant_q4k.go:37-44)."""
    raw = np.ascontiguousarray(raw, np.uint8).reshape(-1)
    return Tensor(Dtype.Q4_K, Layout.RowMajor, list(shape),
                  QuantSpec(Block=256, Axis=2, Bits=4, Symmetric=False), HostBuf(i8=raw), be)


class GGUFBlocks(HostBuf):
    """Host bytes holding raw GGUF blocks (not HAL int8 codes)."""


def NewQ8(be, shape, codes, scale, block: int = 32) -> Tensor:
    """A HAL Q8_0 weight: int8 codes [out*in] + f32 per-block scales [out*in/block]
    (internal/compute/cpuref.go:53-56)."""
    codes = np.ascontiguousarray(codes, np.int8).reshape(-1)
    scale = np.ascontiguousarray(scale, np.float32).reshape(-1)
    return Tensor(Dtype.Q8_0, Layout.RowMajor, list(shape),
                  QuantSpec(Block=block, Axis=2, Bits=8, Symmetric=True, Scale=scale),
                  HostBuf(i8=codes), be)


def NewQ8_0GGUF(be, shape, raw) -> Tensor:
    """Raw GGUF Q8_0 blocks (f16 d + 32 int8) as a host Q8_0 tensor. The scale is recorded per
    block as f32 (the exact widening of the stored f16), so the tensor carries the same values as
    the reference's resident kqw Q8_0 weight (internal/model/quant_kquant.go:237-248)."""
    raw = np.ascontiguousarray(raw, np.uint8).reshape(-1)
    out, in_ = shape
    blk = raw.reshape(out * (in_ // 32), 34)
    scale = blk[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
    return Tensor(Dtype.Q8_0, Layout.RowMajor, list(shape),
                  QuantSpec(Block=32, Axis=2, Bits=8, Symmetric=True, Scale=scale),
                  GGUFBlocks(i8=raw), be)


class DevQ8Buf:
    """A device HAL Q8 weight: codes and scales buffers from the fakhip pool."""

    def __init__(self, codes: int, scales: int, block: int):
        self.ptr = codes
        self.scales = scales
        self.block = block

    def Ready(self) -> bool:
        return True


Q8_DEVICE_BLOCK = 32  # q8DeviceBlock, internal/compute/cuda.go:210


class RocmBackend:
    """The ROCm (gfx950) Approx backend behind the compute.Backend seam."""

    def __init__(self, kq_int8: Optional[bool] = None):
        self.info = fakhip.init()
        # Host fences (Read) so far; async op outputs are ready once it passes their generation
        # (cudaBackend.fenceGen, internal/compute/cuda.go:327-331).
        self.fence_gen = 0
        # upload cache (cuda.go:680-704): (host address, weakref to the owning array, dtype,
        # resident tensor)
        self._upload_cache: list = []
        # The int8 Q4_K route is opt-in exactly as on the CPU: FAK_KQ_INT8 = 1 / on / true
        # (q4kInt8Default, internal/model/quant_amd64_q4k.go:54-61), resolved once here.
        if kq_int8 is None:
            kq_int8 = os.environ.get("FAK_KQ_INT8", "") in ("1", "on", "true")
        self.kq_int8 = bool(kq_int8)

    # ---- identity (compute.go:319-322) ----
    def Name(self) -> str:
        return "rocm"

    def Tier(self) -> str:
        return "gfx950"

    def Class(self) -> CorrectnessClass:
        return CorrectnessClass.Approx

    def Caps(self) -> Caps:
        return Caps(Async=True, UploadDtype=True, DeviceMemory=True, CapacityProbe=True)

    @staticmethod
    def _host_array(t: Tensor) -> np.ndarray:
        return t.buf.i8 if t.buf.i8 is not None else t.buf.f32

    @staticmethod
    def _owner(a: np.ndarray) -> np.ndarray:
        while isinstance(a.base, np.ndarray):
            a = a.base
        return a

    def _cached(self, t: Tensor, dtype: Dtype):
        """The reference shares one resident copy per host buffer address, dtype and element count
        (cuda.go:680-692) and accepts that a freed buffer's address can be reused; here a hit also
        needs the array that owns the memory to be alive, so a reused address never hits."""
        a = self._host_array(t)
        for ptr, owner, dt, res in self._upload_cache:
            if ptr == a.ctypes.data and owner() is self._owner(a) and dt == dtype and \
                    res.Numel() == t.Numel():
                return res
        return None

    def _remember(self, t: Tensor, dtype: Dtype, res: Tensor) -> None:
        a = self._host_array(t)
        self._upload_cache = [e for e in self._upload_cache if e[1]() is not None]
        self._upload_cache.append((a.ctypes.data, weakref.ref(self._owner(a)), dtype, res))

    # ---- residency ----
    def Upload(self, t: Tensor, as_: Dtype = Dtype.F32) -> Tensor:
        if not isinstance(t.buf, HostBuf):
            raise TypeError("compute: rocm Upload expects host data")
        if t.Dtype == Dtype.Q4_K:
            return self._upload_quant(t, "fhip_q4k_upload", 256, 144)
        if t.Dtype == Dtype.Q8_0 and isinstance(t.buf, GGUFBlocks):
            return self._upload_quant(t, "fhip_q8_0_upload", 32, 34)
        if t.Dtype == Dtype.Q8_0:
            return self._upload_hal_q8(t)
        if t.Dtype != Dtype.F32:
            raise TypeError(f"compute: rocm Upload supports F32 host data, raw Q4_K / Q8_0 "
                            f"blocks or HAL Q8 codes (got {t.Dtype})")
        if as_ == Dtype.Q8_0:
            return self._narrow_q8(t)
        f = t.buf.f32
        n = f.size * 4
        ptr = fakhip.alloc_call("fhip_malloc", max(n, 4))
        if n:
            fakhip.call("fhip_h2d", ptr, f.ctypes.data, n)
        return Tensor(Dtype.F32, Layout.RowMajor, list(t.Shape), None, DevBuf(ptr, n), self)

    def _upload_hal_q8(self, t: Tensor) -> Tensor:
        """A host HAL Q8 weight (codes + f32 scales) made resident as-is."""
        if len(t.Shape) != 2 or t.Quant is None or t.Quant.Scale is None:
            raise ValueError("compute: rocm Upload(Q8_0) expects a 2-D NewQ8 weight")
        out, in_ = t.Shape
        block = t.Quant.Block
        codes, scale = t.buf.i8, t.Quant.Scale
        if block <= 0 or in_ % block or codes.size != out * in_ or scale.size != out * (in_ // block):
            raise ValueError(f"compute: Q8_0 weight [{out},{in_}] block {block} has {codes.size} "
                             f"codes / {scale.size} scales")
        cached = self._cached(t, Dtype.Q8_0)
        if cached is not None:
            return cached
        cp = fakhip.alloc_call("fhip_malloc", max(codes.size, 4))
        sp = fakhip.alloc_call("fhip_malloc", max(scale.size * 4, 4))
        if codes.size:
            fakhip.call("fhip_h2d", cp, codes.ctypes.data, codes.size)
            fakhip.call("fhip_h2d", sp, scale.ctypes.data, scale.size * 4)
        res = Tensor(Dtype.Q8_0, Layout.RowMajor, [out, in_], t.Quant, DevQ8Buf(cp, sp, block),
                     self)
        self._remember(t, Dtype.Q8_0, res)
        return res

    def _narrow_q8(self, t: Tensor) -> Tensor:
        """Upload(f32 weight, Q8_0): quantizeVecQ8 per row with the device block (cuda.go:714-750),
        run on the device."""
        if len(t.Shape) != 2:
            raise ValueError("compute: rocm Upload(_, Q8_0) expects a 2-D [out,in] weight")
        out, in_ = t.Shape
        blk = Q8_DEVICE_BLOCK
        if in_ % blk:
            raise ValueError(f"compute: Q8_0 reduction dim {in_} not a multiple of {blk}")
        f = t.buf.f32
        if f.size != out * in_:
            raise ValueError(f"compute: f32 weight has {f.size} elements, want {out}x{in_}")
        cached = self._cached(t, Dtype.Q8_0)
        if cached is not None:
            return cached
        nblk = in_ // blk
        cp = fakhip.alloc_call("fhip_malloc", max(out * in_, 4))
        sp = fakhip.alloc_call("fhip_malloc", max(out * nblk * 4, 4))
        if f.size:
            tmp = fakhip.alloc_call("fhip_malloc", f.size * 4)
            try:
                fakhip.call("fhip_h2d", tmp, f.ctypes.data, f.size * 4)
                fakhip.call("fhip_q8_quantize_f32", tmp, cp, sp, out, in_, blk)
                fakhip.call("fhip_sync")
            finally:
                fakhip.load().fhip_free(tmp)
        res = Tensor(Dtype.Q8_0, Layout.RowMajor, [out, in_],
                     QuantSpec(Block=blk, Axis=2, Bits=8, Symmetric=True),
                     DevQ8Buf(cp, sp, blk), self)
        self._remember(t, Dtype.Q8_0, res)
        return res

    def _upload_quant(self, t: Tensor, fn: str, block: int, block_bytes: int) -> Tensor:
        if len(t.Shape) != 2:
            raise ValueError(f"compute: rocm Upload({t.Dtype}) expects a 2-D [out,in] weight")
        out, in_ = t.Shape
        raw = t.buf.i8
        if in_ % block:
            raise ValueError(f"compute: {t.Dtype} reduction dim {in_} not a multiple of {block}")
        want = out * (in_ // block) * block_bytes
        if raw.size != want:
            raise ValueError(f"compute: {t.Dtype} payload size {raw.size} != {want}")
        cached = self._cached(t, t.Dtype)
        if cached is not None:
            return cached
        ptr = fakhip.alloc_call(fn, raw.ctypes.data, out, in_)
        res = Tensor(t.Dtype, Layout.Tiled, [out, in_], t.Quant, DevBuf(ptr, want), self)
        self._remember(t, t.Dtype, res)
        return res

    def Host(self, t: Tensor):
        return None, False

    def Read(self, t: Tensor) -> np.ndarray:
        """Device -> host f32 (the host fence)."""
        if t.Dtype != Dtype.F32:
            raise TypeError("compute: rocm Read supports F32 tensors")
        out = np.empty(t.Numel(), np.float32)
        if out.size:
            fakhip.call("fhip_d2h", out.ctypes.data, t.buf.ptr, out.size * 4)
            # The copy drained the stream: everything enqueued before it is materialized
            # (cuda.go:896).
            self.fence_gen += 1
        return out

    def Free(self, t: Tensor) -> None:
        if isinstance(t.buf, (DevBuf, DevQ8Buf)) and t.buf.ptr:
            self._upload_cache = [e for e in self._upload_cache if e[3].buf is not t.buf]
            fakhip.load().fhip_free(t.buf.ptr)
            t.buf.ptr = 0
            if isinstance(t.buf, DevQ8Buf) and t.buf.scales:
                fakhip.load().fhip_free(t.buf.scales)
                t.buf.scales = 0

    # ---- the quantized matmul family ----
    def _dev_out(self, shape) -> Tensor:
        n = int(np.prod(shape)) * 4
        ptr = fakhip.alloc_call("fhip_malloc", max(n, 4))
        # An async output: not Ready() until the next host fence (cuda.go:583-596).
        return Tensor(Dtype.F32, Layout.RowMajor, list(shape), None,
                      DevBuf(ptr, n, be=self, born_gen=self.fence_gen), self)

    def _matmul(self, w: Tensor, X: Tensor, P: int, shape) -> Tensor:
        out, in_ = w.Shape
        if X.Dtype != Dtype.F32 or not isinstance(X.buf, DevBuf):
            raise TypeError("compute: rocm MatMul expects a device-resident F32 activation")
        if X.Numel() != P * in_:
            raise ValueError(f"compute: rocm MatMul activation has {X.Numel()} elements, want "
                             f"{P}x{in_}")
        y = self._dev_out(shape)
        if w.Dtype == Dtype.Q4_K:
            fn = "fhip_q4k_matmul_int8_f32" if self.kq_int8 else "fhip_q4k_matmul_f32"
            fakhip.call(fn, w.buf.ptr, X.buf.ptr, y.buf.ptr, out, in_, P)
        elif w.Dtype == Dtype.Q8_0 and isinstance(w.buf, DevQ8Buf):
            fakhip.call("fhip_q8_matmul_f32", w.buf.ptr, w.buf.scales, X.buf.ptr, y.buf.ptr, out,
                        in_, P, w.buf.block)
        elif w.Dtype == Dtype.Q8_0:
            fakhip.call("fhip_q8_0_matmul_f32", w.buf.ptr, X.buf.ptr, y.buf.ptr, out, in_, P)
        else:
            raise NotImplementedError(f"compute: rocm MatMul supports Q4_K / Q8_0 weights "
                                      f"(got {w.Dtype})")
        return y

    def MatMul(self, w: Tensor, x: Tensor) -> Tensor:
        out, in_ = w.Shape
        y = self._matmul(w, x, 1, [out])
        if y.Numel() != out:  # cuda.go:989-993
            raise RuntimeError(f"compute: rocm MatMul {w.Dtype} out={out} in={in_} produced "
                               f"{y.Numel()} rows")
        return y

    def BatchedMatMul(self, w: Tensor, X: Tensor, P: int) -> Tensor:
        out, in_ = w.Shape
        y = self._matmul(w, X, P, [P, out])
        if y.Numel() != P * out:  # cuda.go:1029-1033
            raise RuntimeError(f"compute: rocm BatchedMatMul {w.Dtype} out={out} in={in_} P={P} "
                               f"produced {y.Numel()} want {P * out}")
        return y

    # The rest of the Backend interface belongs to other kernels.
    def RMSNorm(self, *a):
        raise NotImplementedError("compute: rocm backend implements the quantized matmul only")

    RoPE = SwiGLU = AddInPlace = AddBias = Attention = Argmax = NewKV = RMSNorm


# ---- registry (internal/compute/compute.go:464-519) ----
_registry: list = []


def Register(b) -> None:
    for i, e in enumerate(_registry):
        if e.Name() == b.Name():
            _registry[i] = b
            return
    _registry.append(b)


def Registered() -> list:
    return [b.Name() for b in _registry]


def Lookup(name: str):
    for b in _registry:
        if b.Name() == name:
            return b, True
    return None, False


def Pick(name: str):
    if name:
        b, ok = Lookup(name)
        if ok:
            return b
    return Default()


def Default():
    for b in _registry:
        if b.Class() == CorrectnessClass.Reference:
            return b
    return _registry[0] if _registry else None


def RequireReference(b) -> bool:
    return b is not None and b.Class() == CorrectnessClass.Reference


def register_rocm() -> Optional[RocmBackend]:
    """The init() of cuda.go:212-232: register "rocm" when a gfx950 device is reachable."""
    try:
        be = RocmBackend()
    except fakhip.FakHipError:
        return None
    Register(be)
    return be
