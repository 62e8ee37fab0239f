"""eyebrowse-core / eyebrowse-gpu mirror over the C ABI: DType, EyebrowseError, Device,
Tensor, Recorder.

Names and meaning follow crates/eyebrowse-core/src/lib.rs (DType, EyebrowseError) and
crates/eyebrowse-gpu/src/{device,tensor,recorder}.rs. Kernel calls raise instead of
returning ``()``.
"""
from __future__ import annotations

import ctypes
import enum

import numpy as np

from ._lib import c_size, c_vp, lib


class DType(enum.IntEnum):
    """crates/eyebrowse-core/src/lib.rs:8-25; F8E4M3 (OCP FP8 E4M3 KV caches, one byte per
    element) has no counterpart in the reference."""
    F32 = 0
    F16 = 1
    U32 = 2
    I32 = 3
    F8E4M3 = 4

    def size(self) -> int:
        return int(lib().eb_dtype_size(int(self)))


class EyebrowseError(RuntimeError):
    """crates/eyebrowse-core/src/lib.rs:27-41; ``status`` is the eb_status code."""
    status = 6


class DeviceUnavailable(EyebrowseError):
    status = 1


class LoadError(EyebrowseError):
    status = 2


class UnsupportedConfig(EyebrowseError):
    status = 3


class ShapeMismatch(EyebrowseError):
    status = 4


class OutOfMemory(EyebrowseError):
    status = 5


_ERRORS = {c.status: c for c in (DeviceUnavailable, LoadError, UnsupportedConfig, ShapeMismatch,
                                 OutOfMemory, EyebrowseError)}


def check(status: int) -> None:
    """Raise the EyebrowseError subclass for a non-zero eb_status."""
    if status != 0:
        msg = lib().eb_last_error().decode()
        raise _ERRORS.get(status, EyebrowseError)(msg)


def _shape_arr(shape):
    shape = tuple(int(s) for s in shape)
    return (c_size * max(1, len(shape)))(*shape), len(shape)


class Device:
    """Device (crates/eyebrowse-gpu/src/device.rs:20-110): one HIP device, one stream,
    an exact-size buffer pool."""

    def __init__(self, handle: int):
        self._h = c_vp(handle)

    @classmethod
    def new(cls, ordinal: int = 0) -> "Device":
        out = c_vp()
        check(lib().eb_device_new(ordinal, ctypes.byref(out)))
        return cls(out.value)

    @property
    def handle(self):
        return self._h

    def synchronize(self) -> None:
        check(lib().eb_device_synchronize(self._h))

    @property
    def stream(self) -> int:
        return int(lib().eb_device_stream(self._h) or 0)

    @property
    def cu_count(self) -> int:
        return int(lib().eb_device_cu_count(self._h))

    def pooled(self, nbytes: int) -> int:
        """Free pooled buffers of exactly ``nbytes`` (device.rs:63-70)."""
        return int(lib().eb_device_pooled(self._h, nbytes))

    def begin_capture(self) -> None:
        """Start capturing the device stream into a HIP graph (no counterpart in the
        reference): kernels recorded until end_capture are captured, not run."""
        check(lib().eb_device_begin_capture(self._h))

    def end_capture(self, graph: "Graph | None" = None) -> "Graph":
        """End the capture: a new Graph, or `graph` updated in place."""
        h = c_vp(graph._h.value if graph is not None else None)
        check(lib().eb_device_end_capture(self._h, ctypes.byref(h)))
        if graph is not None:
            return graph
        return Graph(h.value, self)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib().eb_device_release(h)
            self._h = c_vp()


class Tensor:
    """Tensor (crates/eyebrowse-gpu/src/tensor.rs:34-157). Dropping it returns the buffer
    to the pool."""

    def __init__(self, handle: int, dev: Device):
        self._h = c_vp(handle)
        self.dev = dev

    @classmethod
    def empty(cls, dev: Device, shape, dtype: DType = DType.F32) -> "Tensor":
        arr, n = _shape_arr(shape)
        out = c_vp()
        check(lib().eb_tensor_empty(dev.handle, arr, n, int(dtype), ctypes.byref(out)))
        return cls(out.value, dev)

    @classmethod
    def from_f32(cls, dev: Device, shape, data) -> "Tensor":
        a = np.ascontiguousarray(np.asarray(data, dtype=np.float32)).ravel()
        arr, n = _shape_arr(shape)
        out = c_vp()
        check(lib().eb_tensor_from_f32(dev.handle, arr, n,
                                       a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), a.size,
                                       ctypes.byref(out)))
        return cls(out.value, dev)

    @classmethod
    def from_u32(cls, dev: Device, shape, data) -> "Tensor":
        a = np.ascontiguousarray(np.asarray(data, dtype=np.uint32)).ravel()
        arr, n = _shape_arr(shape)
        out = c_vp()
        check(lib().eb_tensor_from_u32(dev.handle, arr, n,
                                       a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), a.size,
                                       ctypes.byref(out)))
        return cls(out.value, dev)

    @classmethod
    def from_f16_packed(cls, dev: Device, logical_shape, data) -> "Tensor":
        """Tensor::from_f16_packed (crates/eyebrowse-gpu/src/tensor.rs:108-116): f32 data
        rounded to IEEE half (nearest even) and packed two per u32 word, low half first,
        odd tail zero-padded; a U32 tensor of ceil(n/2) words."""
        a = np.ascontiguousarray(np.asarray(data, dtype=np.float32)).ravel()
        assert a.size == int(np.prod(logical_shape)), "from_f16_packed: data len != shape numel"
        with np.errstate(over="ignore"):
            h = a.astype(np.float16).view(np.uint16)
        if h.size % 2:
            h = np.concatenate([h, np.zeros(1, np.uint16)])
        words = h[0::2].astype(np.uint32) | (h[1::2].astype(np.uint32) << 16)
        return cls.from_u32(dev, (words.size,), words)

    @property
    def handle(self):
        return self._h

    @property
    def shape(self) -> tuple:
        l = lib()
        return tuple(int(l.eb_tensor_dim(self._h, i)) for i in range(l.eb_tensor_ndim(self._h)))

    @property
    def dtype(self) -> DType:
        return DType(lib().eb_tensor_dtype(self._h))

    def numel(self) -> int:
        return int(lib().eb_tensor_numel(self._h))

    def byte_len(self) -> int:
        return int(lib().eb_tensor_nbytes(self._h))

    @property
    def data_ptr(self) -> int:
        return int(lib().eb_tensor_data(self._h) or 0)

    def to_f32(self) -> np.ndarray:
        out = np.empty(self.numel(), np.float32)
        check(lib().eb_tensor_to_f32(self._h, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                     out.size))
        return out

    def write(self, data) -> None:
        """Copy host data (same byte size as the tensor) into it, synchronously."""
        if isinstance(data, (bytes, bytearray)):
            buf = bytes(data)
        else:
            a = np.ascontiguousarray(data)
            if a.dtype == np.float64:
                a = a.astype(np.float32)
            buf = a.tobytes()
        check(lib().eb_tensor_write(self._h, buf, len(buf)))

    def read_bytes(self) -> bytes:
        buf = ctypes.create_string_buffer(self.byte_len())
        check(lib().eb_tensor_read_bytes(self._h, buf, self.byte_len()))
        return buf.raw

    def release(self) -> None:
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib().eb_tensor_release(h)
            self._h = c_vp()

    def __del__(self):
        self.release()


class Recorder:
    """Recorder (crates/eyebrowse-gpu/src/recorder.rs:10-35): kernels recorded through it
    run on the device stream in record order; ``submit`` reports launch errors.

    With ``deferred=True`` nothing recorded runs until ``submit`` (which waits for the
    work), and a recorder released without a submit discards its work, as the
    reference's; while it is open only it may record on the device."""

    def __init__(self, dev: Device, deferred: bool = False):
        out = c_vp()
        new = lib().eb_recorder_new_deferred if deferred else lib().eb_recorder_new
        check(new(dev.handle, ctypes.byref(out)))
        self._h = out
        self.dev = dev

    def release(self) -> None:
        """Drop the recorder without submitting."""
        h, self._h = self._h, c_vp()
        if h.value:
            lib().eb_recorder_release(h)

    def device(self) -> Device:
        return self.dev

    @property
    def handle(self):
        if not self._h.value:
            raise EyebrowseError("recorder already submitted")
        return self._h

    def submit(self) -> None:
        h, self._h = self._h, c_vp()
        check(lib().eb_recorder_submit(h))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib().eb_recorder_release(h)
            self._h = c_vp()


class Graph:
    """A captured step (Device.begin_capture / end_capture): one hipGraphLaunch replays
    every captured kernel on the device stream."""

    def __init__(self, handle: int, dev: Device):
        self._h = c_vp(handle)
        self.dev = dev

    def launch(self) -> None:
        check(lib().eb_graph_launch(self._h))

    def release(self) -> None:
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib().eb_graph_release(h)
            self._h = c_vp()

    def __del__(self):
        self.release()
