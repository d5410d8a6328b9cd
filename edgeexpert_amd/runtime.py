"""Device memory, streams, events and graphs over libtfq's runtime exports.

DeviceBuffer stands in for the reference's MTLBuffer: a hipMalloc'd region
with synchronous upload/download from numpy arrays. Nothing here computes.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, lib


class DeviceBuffer:
    """One hipMalloc allocation. `ptr(offset)` returns a device address."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().tfq_rt_malloc(C.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self._ptr = p.value

    @classmethod
    def from_array(cls, arr: np.ndarray, pad_to: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        buf = cls(max(a.nbytes, pad_to))
        if a.nbytes:
            check(lib().tfq_rt_memcpy_htod(buf._ptr, a.ctypes.data, a.nbytes), "upload")
        return buf

    def ptr(self, offset: int = 0) -> int:
        return self._ptr + int(offset)

    @property
    def value(self) -> int:
        return self._ptr

    def upload(self, arr: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(arr)
        assert offset + a.nbytes <= self.nbytes, "upload out of range"
        if a.nbytes:
            check(lib().tfq_rt_memcpy_htod(self._ptr + offset, a.ctypes.data, a.nbytes), "upload")

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype)
        assert offset + out.nbytes <= self.nbytes, "download out of range"
        if out.nbytes:
            check(lib().tfq_rt_memcpy_dtoh(out.ctypes.data, self._ptr + offset, out.nbytes),
                  "download")
        return out

    def fill(self, byte: int = 0):
        check(lib().tfq_rt_memset(self._ptr, byte, self.nbytes), "memset")

    def free(self):
        if self._ptr:
            lib().tfq_rt_free(self._ptr)
            self._ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = C.c_void_p()
        check(lib().tfq_rt_stream_create(C.byref(s)), "stream create")
        self.handle = s.value

    def sync(self):
        check(lib().tfq_rt_stream_sync(self.handle), "stream sync")

    def __del__(self):
        try:
            if self.handle:
                lib().tfq_rt_stream_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class Event:
    def __init__(self):
        e = C.c_void_p()
        check(lib().tfq_rt_event_create(C.byref(e)), "event create")
        self.handle = e.value

    def record(self, stream: Stream | None):
        check(lib().tfq_rt_event_record(self.handle, stream.handle if stream else None), "record")

    def sync(self):
        check(lib().tfq_rt_event_sync(self.handle), "event sync")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(lib().tfq_rt_event_elapsed_ms(C.byref(ms), self.handle, end.handle), "elapsed")
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                lib().tfq_rt_event_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class Graph:
    """Executable HIP graph captured from work enqueued on `stream` by `fn()`."""

    def __init__(self, stream: Stream, fn):
        check(lib().tfq_rt_capture_begin(stream.handle), "capture begin")
        try:
            fn()
        finally:
            g = C.c_void_p()
            rc = lib().tfq_rt_capture_end(stream.handle, C.byref(g))
        check(rc, "capture end")
        self.handle = g.value

    def launch(self, stream: Stream):
        check(lib().tfq_rt_graph_launch(self.handle, stream.handle), "graph launch")

    def __del__(self):
        try:
            if self.handle:
                lib().tfq_rt_graph_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


def device_count() -> int:
    n = C.c_int(0)
    rc = lib().tfq_rt_device_count(C.byref(n))
    return n.value if rc == 0 else 0


def device_info() -> tuple[str, str]:
    name = C.create_string_buffer(256)
    arch = C.create_string_buffer(256)
    check(lib().tfq_rt_device_info(name, 256, arch, 256), "device info")
    return name.value.decode(), arch.value.decode()


def synchronize():
    check(lib().tfq_rt_device_sync(), "device sync")
