"""Device memory, streams and events through the library's own HIP plumbing.

No PyTorch is involved: buffers are raw device allocations made by
libkvcache_amd.so, host data moves as numpy arrays.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._native import KVC_F16, KVC_F32, check, lib


def has_device() -> bool:
    n = C.c_int(0)
    try:
        check(lib().kvc_device_count(C.byref(n)))
    except Exception:
        return False
    return n.value > 0


def np_dtype(dtype: int):
    return np.float16 if dtype == KVC_F16 else np.float32


def kvc_dtype(a) -> int:
    dt = np.dtype(a)
    if dt == np.float16:
        return KVC_F16
    if dt == np.float32:
        return KVC_F32
    raise ValueError(f"unsupported dtype {dt}")


class DeviceBuffer:
    """An owning device allocation (freed on close / garbage collection)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().kvc_malloc(C.byref(p), max(self.nbytes, 1)))
        self._ptr = p.value

    @property
    def ptr(self) -> int:
        if self._ptr is None:
            raise ValueError("buffer already freed")
        return self._ptr

    @classmethod
    def from_numpy(cls, a: np.ndarray, stream=None) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            check(lib().kvc_memcpy_h2d(b.ptr, a.ctypes.data, a.nbytes, stream))
            check(lib().kvc_stream_synchronize(stream))
        return b

    def upload(self, a: np.ndarray, stream=None) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("array larger than buffer")
        check(lib().kvc_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes, stream))
        check(lib().kvc_stream_synchronize(stream))

    def to_numpy(self, dtype, shape, stream=None) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("requested view larger than buffer")
        if out.nbytes:
            check(lib().kvc_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes, stream))
        return out

    def zero(self, stream=None) -> None:
        check(lib().kvc_memset(self.ptr, 0, self.nbytes, stream))

    def close(self) -> None:
        if self._ptr is not None:
            lib().kvc_free(self._ptr)
            self._ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def fill_normal(buf: DeviceBuffer, n: int, dtype: int, seed: int, stddev: float = 1.0, stream=None) -> None:
    check(lib().kvc_fill_normal(buf.ptr, n, dtype, seed, stddev, stream))


def synchronize() -> None:
    check(lib().kvc_device_synchronize())


class Stream:
    def __init__(self):
        s = C.c_void_p()
        check(lib().kvc_stream_create(C.byref(s)))
        self.handle = s.value

    def synchronize(self) -> None:
        check(lib().kvc_stream_synchronize(self.handle))

    def close(self) -> None:
        if self.handle:
            lib().kvc_stream_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = C.c_void_p()
        check(lib().kvc_event_create(C.byref(e)))
        self.handle = e.value

    def record(self, stream=None) -> None:
        check(lib().kvc_event_record(self.handle, stream))

    def synchronize(self) -> None:
        check(lib().kvc_event_synchronize(self.handle))

    def wait_on(self, stream) -> None:
        """Work queued on `stream` after this call waits for the event (no host wait)."""
        check(lib().kvc_stream_wait_event(stream, self.handle))

    def elapsed_ms(self, later: "Event") -> float:
        ms = C.c_float()
        check(lib().kvc_event_elapsed_ms(C.byref(ms), self.handle, later.handle))
        return ms.value

    def close(self) -> None:
        if self.handle:
            lib().kvc_event_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
