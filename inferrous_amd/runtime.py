"""Host runtime primitives over the C ABI.

Mirrors the cuda_core types the reference's host code uses
(crates/inferrous-qwen3/src/gpu.rs:8, src/conformance.rs:2): ``CudaContext``
(``new`` / ``new_stream`` / ``default_stream``), ``CudaStream``
(``synchronize``), ``DeviceBuffer`` (``from_host`` / ``zeroed`` /
``to_host_vec`` / ``copy_from_host``), ``PinnedHostBuffer`` and
``LaunchConfig`` with the ``cfg`` / ``rows`` helpers of src/gpu.rs:232-245.
Device memory, streams, events and graphs all come from the HIP library;
no torch types are involved.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import check, lib


@dataclass(frozen=True)
class LaunchConfig:
    """Accepted for signature parity with the reference; the HIP library
    chooses its own launch geometry, so the values are ignored."""
    grid_dim: tuple = (1, 1, 1)
    block_dim: tuple = (1, 1, 1)
    shared_mem_bytes: int = 0


def cfg(n: int) -> LaunchConfig:
    """src/gpu.rs:232-238."""
    return LaunchConfig(((n + 127) // 128, 1, 1), (128, 1, 1), 0)


def rows(n: int, threads: int) -> LaunchConfig:
    """src/gpu.rs:239-245."""
    return LaunchConfig((n, 1, 1), (threads, 1, 1), 0)


class CudaStream:
    def __init__(self, handle: int | None, owned: bool):
        self._h = handle
        self._owned = owned

    @property
    def handle(self) -> int | None:
        return self._h

    def synchronize(self) -> None:
        check(lib().w8a8_stream_synchronize(self._h), "stream synchronize")

    def __del__(self):
        if self._owned and self._h and _lib._lib is not None:
            lib().w8a8_stream_destroy(self._h)
            self._h = None


class CudaContext:
    """``CudaContext::new(device)`` followed by the module load
    (src/gpu.rs:248-250): fails unless the device is a gfx950."""

    def __init__(self, device: int = 0):
        check(lib().w8a8_init(device), f"init device {device}")
        self.device = device

    @staticmethod
    def new(device: int = 0) -> "CudaContext":
        return CudaContext(device)

    def new_stream(self) -> CudaStream:
        h = ctypes.c_void_p()
        check(lib().w8a8_stream_create(ctypes.byref(h)), "stream create")
        return CudaStream(h.value, owned=True)

    def default_stream(self) -> CudaStream:
        return CudaStream(None, owned=False)

    def info(self) -> tuple[int, str]:
        cu = ctypes.c_int()
        name = ctypes.create_string_buffer(64)
        check(lib().w8a8_device_info(ctypes.byref(cu), name, 64), "device info")
        return cu.value, name.value.decode()

    def clock_khz(self) -> int:
        """Peak engine clock reported by the driver (kHz)."""
        k = ctypes.c_int()
        check(lib().w8a8_device_clock_khz(ctypes.byref(k)), "device clock")
        return k.value


def device_count() -> int:
    c = ctypes.c_int()
    check(lib().w8a8_device_count(ctypes.byref(c)))
    return c.value


class DeviceBuffer:
    """Typed device allocation (``DeviceBuffer<T>``): a pointer, an element
    count and a numpy dtype.  Zero-filled on allocation."""

    def __init__(self, n: int, dtype):
        self.dtype = np.dtype(dtype)
        self.n = int(n)
        self.nbytes = self.n * self.dtype.itemsize
        p = ctypes.c_void_p()
        check(lib().w8a8_malloc(ctypes.byref(p), self.nbytes), f"malloc {self.nbytes} B")
        self._p = p.value
        self._base = None  # set for views

    @classmethod
    def zeroed(cls, stream: CudaStream | None, n: int, dtype=np.float32) -> "DeviceBuffer":
        return cls(n, dtype)

    @classmethod
    def from_host(cls, stream: CudaStream | None, array) -> "DeviceBuffer":
        a = np.ascontiguousarray(array)
        buf = cls(a.size, a.dtype)
        buf.copy_from_host(stream, a)
        return buf

    @classmethod
    def view_of(cls, base: "DeviceBuffer", offset_elems: int, n: int, dtype=None) -> "DeviceBuffer":
        """A non-owning window into ``base`` (same dtype unless given)."""
        v = cls.__new__(cls)
        v.dtype = np.dtype(dtype) if dtype is not None else base.dtype
        v.n = int(n)
        v.nbytes = v.n * v.dtype.itemsize
        v._p = base.ptr + offset_elems * base.dtype.itemsize
        v._base = base
        assert offset_elems * base.dtype.itemsize + v.nbytes <= base.nbytes
        return v

    @property
    def ptr(self) -> int:
        return self._p

    def __len__(self) -> int:
        return self.n

    def copy_from_host(self, stream: CudaStream | None, array) -> None:
        a = np.ascontiguousarray(array)
        if a.nbytes != self.nbytes:
            raise ValueError(f"host array has {a.nbytes} B, buffer {self.nbytes} B")
        h = stream.handle if stream else None
        check(lib().w8a8_memcpy_htod(self._p, a.ctypes.data, a.nbytes, h), "copy to device")
        check(lib().w8a8_stream_synchronize(h), "synchronize after copy")

    def to_host_vec(self, stream: CudaStream | None) -> np.ndarray:
        out = np.empty(self.n, self.dtype)
        h = stream.handle if stream else None
        check(lib().w8a8_memcpy_dtoh(out.ctypes.data, self._p, self.nbytes, h), "copy to host")
        check(lib().w8a8_stream_synchronize(h), "synchronize after copy")
        return out

    def fill_zero(self, stream: CudaStream | None) -> None:
        check(lib().w8a8_fill_zero(self._p, self.nbytes, stream.handle if stream else None))

    def free(self) -> None:
        if self._p and self._base is None and _lib._lib is not None:
            lib().w8a8_free(self._p)
        self._p = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class PinnedHostBuffer:
    """Page-locked host memory (src/gpu.rs:147-181) viewed as a numpy array."""

    def __init__(self, n: int, dtype):
        self.dtype = np.dtype(dtype)
        self.n = int(n)
        p = ctypes.c_void_p()
        check(lib().w8a8_host_malloc(ctypes.byref(p), max(1, self.n * self.dtype.itemsize)))
        self._p = p.value
        buf = (ctypes.c_byte * (self.n * self.dtype.itemsize)).from_address(self._p)
        self.array = np.frombuffer(buf, dtype=self.dtype, count=self.n)

    def __del__(self):
        if self._p and _lib._lib is not None:
            lib().w8a8_host_free(self._p)
            self._p = 0


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().w8a8_event_create(ctypes.byref(p)))
        self._p = p.value

    def record(self, stream: CudaStream | None) -> None:
        check(lib().w8a8_event_record(self._p, stream.handle if stream else None))

    def synchronize(self) -> None:
        check(lib().w8a8_event_synchronize(self._p))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().w8a8_event_elapsed_ms(ctypes.byref(ms), self._p, end._p))
        return ms.value

    def __del__(self):
        if self._p and _lib._lib is not None:
            lib().w8a8_event_destroy(self._p)
            self._p = 0


_CAPTURING: set = set()


def is_capturing(stream) -> bool:
    """True while a Graph context is capturing this stream (no allocation then)."""
    return stream is not None and stream.handle in _CAPTURING


class Graph:
    """Capture of everything queued on a (non-default) stream, then replay."""

    def __init__(self, stream: CudaStream):
        self.stream = stream
        self._p = None

    def __enter__(self):
        check(lib().w8a8_graph_capture_begin(self.stream.handle), "capture begin")
        _CAPTURING.add(self.stream.handle)
        return self

    def __exit__(self, exc_type, exc, tb):
        _CAPTURING.discard(self.stream.handle)
        p = ctypes.c_void_p()
        st = lib().w8a8_graph_capture_end(self.stream.handle, ctypes.byref(p))
        if exc_type is None:
            check(st, "capture end")
            self._p = p.value
        elif st == 0 and p.value:
            lib().w8a8_graph_destroy(p.value)   # capture abandoned by the exception
        return False

    def launch(self, stream: CudaStream | None = None) -> None:
        s = stream or self.stream
        check(lib().w8a8_graph_launch(self._p, s.handle if s else None), "graph launch")

    def __del__(self):
        if self._p and _lib._lib is not None:
            lib().w8a8_graph_destroy(self._p)
            self._p = None
