"""Python view of the RHI device (include/vdsl.h): devices, buffers, queues, graphs, events.

`Device(arch="hip")` stands in for `ti.init(arch=...)` (fractal.py:5); `Tensor` is a typed
device buffer, the storage behind a field (`ti.field`, fractal.py:8).  Buffers carry the
binding kinds of the `vernon.semantic` vocabulary (VernonToSpirv.cpp:43-56).
"""
from __future__ import annotations

import contextlib
import ctypes as C

import numpy as np

from . import _lib
from ._lib import call, lib

_NP_DTYPES = {_lib.F32: np.dtype(np.float32), _lib.BF16: np.dtype(np.uint16),
              _lib.I8: np.dtype(np.int8), _lib.I32: np.dtype(np.int32)}
DTYPE_NAMES = {"f32": _lib.F32, "bf16": _lib.BF16, "i8": _lib.I8, "i32": _lib.I32}


def dtype_code(dtype) -> int:
    if isinstance(dtype, int):
        return dtype
    return DTYPE_NAMES[dtype]


def np_dtype(dtype) -> np.dtype:
    """Host numpy dtype of a device dtype (bf16 is held as uint16 bit patterns)."""
    return _NP_DTYPES[dtype_code(dtype)]


def device_count() -> int:
    n = C.c_int(0)
    call("vdsl_device_count", _lib.DEVICE_HIP, C.byref(n))
    return n.value


class Device:
    def __init__(self, ordinal: int = 0, arch: str = "hip"):
        if arch != "hip":
            raise ValueError(f"arch={arch!r}: this library is the HIP device; the CPU executor is test-only")
        h = C.c_void_p()
        call("vdsl_device_open", _lib.DEVICE_HIP, ordinal, C.byref(h))
        self.handle = h
        self.ordinal = ordinal

    def info(self) -> dict:
        i = _lib.DeviceInfo()
        call("vdsl_device_get_info", self.handle, C.byref(i))
        return {"name": i.name.decode(), "arch": i.arch.decode(), "compute_units": i.compute_units,
                "clock_khz": i.clock_khz, "wavefront_size": i.wavefront_size,
                "lds_bytes_per_block": i.lds_bytes_per_block, "hbm_bytes": i.hbm_bytes}

    def close(self):
        if self.handle:
            call("vdsl_device_close", self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Buffer:
    def __init__(self, device: Device, nbytes: int, binding=_lib.BIND_STORAGE_BUFFER):
        if isinstance(binding, str):
            binding = _lib.SEMANTIC_TO_BINDING[binding]
        h = C.c_void_p()
        call("vdsl_buffer_alloc", device.handle, int(nbytes), int(binding), C.byref(h))
        self.handle = h
        self.device = device
        self.nbytes = int(nbytes)

    def free(self):
        if self.handle:
            call("vdsl_buffer_free", self.handle)
            self.handle = None

    def write(self, queue: "Queue", host: np.ndarray, offset: int = 0):
        host = np.ascontiguousarray(host)
        call("vdsl_buffer_write", queue.handle, self.handle, offset, host.ctypes.data_as(C.c_void_p), host.nbytes)

    def read_into(self, queue: "Queue", host: np.ndarray, offset: int = 0):
        assert host.flags.c_contiguous
        call("vdsl_buffer_read", queue.handle, self.handle, offset, host.ctypes.data_as(C.c_void_p), host.nbytes)
        return host

    def copy_from(self, queue: "Queue", src: "Buffer", nbytes: int | None = None, dst_offset: int = 0, src_offset: int = 0):
        """Device-to-device copy of nbytes (default: all of src) on the queue."""
        n = src.nbytes - src_offset if nbytes is None else nbytes
        call("vdsl_buffer_copy", queue.handle, self.handle, dst_offset, src.handle, src_offset, n)

    def fill_u32(self, queue: "Queue", pattern: int = 0, offset: int = 0, nbytes: int | None = None):
        n = self.nbytes - offset if nbytes is None else nbytes
        call("vdsl_buffer_fill_u32", queue.handle, self.handle, offset, n, pattern & 0xFFFFFFFF)

    def address(self) -> int:
        a = C.c_uint64()
        call("vdsl_buffer_device_address", self.handle, C.byref(a))
        return a.value

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Tensor:
    """A dense row-major device tensor: a Buffer plus shape and dtype."""

    def __init__(self, device: Device, shape, dtype="f32", binding=_lib.BIND_STORAGE_BUFFER):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype_code(dtype)
        self.numel = int(np.prod(self.shape)) if self.shape else 1
        self.buffer = Buffer(device, self.numel * np_dtype(self.dtype).itemsize, binding)
        self.device = device

    @property
    def handle(self):
        return self.buffer.handle

    @classmethod
    def from_numpy(cls, device: Device, queue: "Queue", host: np.ndarray, dtype=None, binding=_lib.BIND_STORAGE_BUFFER):
        if dtype is None:
            inv = {v: k for k, v in _NP_DTYPES.items()}
            dtype = inv[np.dtype(host.dtype)]
        if host.dtype != np_dtype(dtype):
            raise TypeError(f"host dtype {host.dtype} does not match device dtype {dtype}")
        t = cls(device, host.shape, dtype, binding)
        try:
            t.buffer.write(queue, host)
        except BaseException:
            t.free()
            raise
        return t

    def numpy(self, queue: "Queue") -> np.ndarray:
        out = np.empty(self.shape, dtype=np_dtype(self.dtype))
        return self.buffer.read_into(queue, out)

    def view(self, shape) -> "Tensor":
        """The same buffer as a tensor of another shape with the same element count (row-major
        data is unchanged); the view never frees the buffer, its owner does."""
        shape = tuple(int(s) for s in shape)
        if (int(np.prod(shape)) if shape else 1) != self.numel:
            raise ValueError(f"view: shape {shape} does not hold {self.numel} elements")
        v = object.__new__(Tensor)
        v.shape, v.dtype, v.numel, v.buffer, v.device = shape, self.dtype, self.numel, self.buffer, self.device
        v._view = True
        return v

    def free(self):
        if not getattr(self, "_view", False):
            self.buffer.free()


class Graph:
    def __init__(self, handle):
        self.handle = handle

    def launch(self, queue: "Queue"):
        call("vdsl_graph_launch", self.handle, queue.handle)

    def destroy(self):
        if self.handle:
            call("vdsl_graph_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Queue:
    def __init__(self, device: Device):
        h = C.c_void_p()
        call("vdsl_queue_create", device.handle, C.byref(h))
        self.handle = h
        self.device = device
        self.capturing = False  # between begin_graph() and end_graph()

    def sync(self):
        call("vdsl_queue_sync", self.handle)

    def begin_graph(self):
        call("vdsl_graph_begin", self.handle)
        self.capturing = True

    def end_graph(self) -> Graph:
        h = C.c_void_p()
        self.capturing = False
        call("vdsl_graph_end", self.handle, C.byref(h))
        return Graph(h)

    @contextlib.contextmanager
    def capture(self):
        """Record the ops issued inside the block into one hipGraph: `with q.capture() as rec: ...;
        g = rec.graph`."""
        class _Rec:
            graph = None
        rec = _Rec()
        self.begin_graph()
        try:
            yield rec
        except BaseException:
            try:
                self.end_graph().destroy()
            except Exception:
                pass
            raise
        rec.graph = self.end_graph()

    def destroy(self):
        if self.handle:
            call("vdsl_queue_destroy", self.handle)
            self.handle = None


class Event:
    def __init__(self, device: Device):
        h = C.c_void_p()
        call("vdsl_event_create", device.handle, C.byref(h))
        self.handle = h

    def record(self, queue: Queue):
        call("vdsl_event_record", self.handle, queue.handle)

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        call("vdsl_event_elapsed_ms", self.handle, end.handle, C.byref(ms))
        return ms.value

    def destroy(self):
        if self.handle:
            call("vdsl_event_destroy", self.handle)
            self.handle = None
