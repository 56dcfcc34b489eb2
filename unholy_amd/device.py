"""Device memory, streams and events through the library's C ABI (no torch: the library owns its HIP runtime)."""
from __future__ import annotations

import ctypes

import numpy as np

from ._lib import call


class DeviceBuffer:
    """A device allocation; `ptr` is the address passed to kernels."""

    def __init__(self, nbytes: int):
        p = ctypes.c_void_p()
        call("uh_malloc", ctypes.byref(p), max(int(nbytes), 1))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("upload larger than the buffer")
        call("uh_memcpy_h2d", self.ptr, a.ctypes.data, a.nbytes)

    def download(self, shape, dtype, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download past the end of the buffer")
        call("uh_memcpy_d2h", out.ctypes.data, self.ptr + offset, out.nbytes)
        return out

    def zero(self, stream=None) -> None:
        call("uh_memset", self.ptr, 0, self.nbytes, stream)

    def free(self) -> None:
        if self.ptr:
            call("uh_free", self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def __int__(self):
        return self.ptr


def ptr(x):
    """Device address of a DeviceBuffer / int / None."""
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)


def device_count() -> int:
    n = ctypes.c_int(0)
    try:
        call("uh_device_count", ctypes.byref(n))
    except Exception:
        return 0
    return n.value


def device_name() -> str:
    buf = ctypes.create_string_buffer(256)
    call("uh_device_name", buf, 256)
    return buf.value.decode()


def synchronize() -> None:
    call("uh_synchronize")


class Stream:
    def __init__(self):
        p = ctypes.c_void_p()
        call("uh_stream_create", ctypes.byref(p))
        self.handle = p.value

    def synchronize(self):
        call("uh_stream_synchronize", self.handle)


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        call("uh_event_create", ctypes.byref(p))
        self.handle = p.value

    def record(self, stream=None):
        call("uh_event_record", self.handle, None if stream is None else getattr(stream, "handle", stream))

    def synchronize(self):
        call("uh_event_synchronize", self.handle)

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0)
        call("uh_event_elapsed_ms", ctypes.byref(ms), self.handle, end.handle)
        return ms.value


class Graph:
    """The work `fn()` enqueues on `stream` (a created Stream), captured once as a HIP graph and replayed by launch()."""

    def __init__(self, stream: "Stream", fn):
        self.stream = stream
        call("uh_graph_capture_begin", stream.handle)
        p = ctypes.c_void_p()
        try:
            fn()
        finally:
            call("uh_graph_capture_end", stream.handle, ctypes.byref(p))
        self.handle = p.value

    def launch(self) -> None:
        call("uh_graph_launch", self.handle, self.stream.handle)

    def __del__(self):
        if getattr(self, "handle", None):
            try:
                call("uh_graph_destroy", self.handle)
            except Exception:
                pass


def fill_random_bytes(buf, n: int, seed: int, lo: int = 0, hi: int = 255, stream=None) -> None:
    call("uh_fill_random_bytes", ptr(buf), int(n), int(seed) & (2**64 - 1), lo, hi, stream)


def pointer_table(ptrs) -> DeviceBuffer:
    """A device array of device pointers (0 for a missing entry)."""
    arr = np.array([0 if p is None else ptr(p) for p in ptrs], np.uint64)
    return DeviceBuffer.from_array(arr)
