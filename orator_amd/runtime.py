"""Device plumbing over the C ABI: buffers, streams, events.

Mirrors the reference's gpu runtime surface (include/gpu/memory.h:26-168): a
DeviceBuffer owns device memory and frees it on close/garbage collection; streams and
events wrap hipStream_t / hipEvent_t handles.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import call, lib


def device_count() -> int:
    n = C.c_int(0)
    call("orator_device_count", C.byref(n))
    return n.value


def set_device(dev: int) -> None:
    call("orator_set_device", dev)


def device_name() -> str:
    buf = C.create_string_buffer(256)
    call("orator_device_name", buf, 256)
    return buf.value.decode()


def synchronize() -> None:
    call("orator_device_synchronize")


def workspace_stats() -> tuple[int, int]:
    """(blocks, bytes) of library workspace held now, after freeing retired blocks whose
    stream work has completed."""
    blocks, nbytes = C.c_size_t(0), C.c_size_t(0)
    call("orator_workspace_stats", C.byref(blocks), C.byref(nbytes))
    return blocks.value, nbytes.value


class DeviceBuffer:
    """`nbytes` of device memory.  `ptr` is the device address as an int."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        call("orator_malloc", C.byref(p), max(int(nbytes), 1))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        if offset + arr.nbytes > self.nbytes:
            raise ValueError("upload past the end of the buffer")
        if arr.nbytes:
            call("orator_memcpy_htod", self.ptr + offset, arr.ctypes.data, arr.nbytes)

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download past the end of the buffer")
        if out.nbytes:
            call("orator_memcpy_dtoh", out.ctypes.data, self.ptr + offset, out.nbytes)
        return out

    def zero(self, stream=None) -> None:
        call("orator_memset", self.ptr, 0, self.nbytes, _sh(stream))

    def close(self) -> None:
        if getattr(self, "ptr", None):
            lib().orator_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __int__(self) -> int:
        return self.ptr


class Stream:
    def __init__(self):
        h = C.c_void_p()
        call("orator_stream_create", C.byref(h))
        self.handle = h.value

    def synchronize(self) -> None:
        call("orator_stream_synchronize", self.handle)

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().orator_stream_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        h = C.c_void_p()
        call("orator_event_create", C.byref(h))
        self.handle = h.value

    def record(self, stream=None) -> None:
        call("orator_event_record", self.handle, _sh(stream))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0)
        call("orator_event_elapsed_ms", C.byref(ms), self.handle, end.handle)
        return ms.value

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().orator_event_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _sh(stream) -> int | None:
    """Stream handle for the C ABI: None/0 -> default stream."""
    if stream is None or stream == 0:
        return None
    return stream.handle if isinstance(stream, Stream) else int(stream)


def ptr(x) -> int | None:
    """Device address of a DeviceBuffer / int (None stays NULL)."""
    if x is None:
        return None
    return x.ptr if isinstance(x, DeviceBuffer) else int(x)
