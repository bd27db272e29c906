"""Device buffers and thin helpers over the extension interface.

DeviceArray owns HBM allocated through nerf_ext_malloc and moves numpy data in
and out with nerf_ext_memcpy; it is how tests and bench.py stage inputs on the
GPU without any other GPU framework in the process.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib as L


class DeviceArray:
    """A contiguous device allocation with a numpy shape and dtype."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self._ptr = C.c_void_p()
        L.call("nerf_ext_malloc", C.byref(self._ptr), max(self.nbytes, 1))

    @property
    def ptr(self) -> int:
        return int(self._ptr.value or 0)

    @classmethod
    def from_numpy(cls, arr: np.ndarray) -> "DeviceArray":
        arr = np.ascontiguousarray(arr)
        out = cls(arr.shape, arr.dtype)
        out.upload(arr)
        return out

    @classmethod
    def zeros(cls, shape, dtype=np.float32) -> "DeviceArray":
        out = cls(shape, dtype)
        out.fill_bytes(0)
        return out

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        if arr.nbytes != self.nbytes:
            raise ValueError(f"upload of {arr.nbytes} bytes into a {self.nbytes}-byte buffer")
        if self.nbytes:
            L.call("nerf_ext_memcpy", self.ptr, arr.ctypes.data, self.nbytes, L.NERF_EXT_H2D)

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            L.call("nerf_ext_memcpy", out.ctypes.data, self.ptr, self.nbytes, L.NERF_EXT_D2H)
        return out

    def fill_bytes(self, value: int) -> None:
        if self.nbytes:
            L.call("nerf_ext_memset", self.ptr, int(value), self.nbytes)

    def free(self) -> None:
        if self._ptr.value:
            L.call("nerf_ext_free", self._ptr)
            self._ptr = C.c_void_p()

    def __del__(self):
        try:
            if self._ptr.value and L._lib is not None:
                L._lib.nerf_ext_free(self._ptr)
        except Exception:
            pass


def synchronize() -> None:
    L.call("nerf_ext_synchronize")


def device_info() -> L.NerfExtDeviceInfo:
    info = L.NerfExtDeviceInfo()
    L.call("nerf_ext_device_info", C.byref(info))
    return info


class Stream:
    def __init__(self):
        self._h = C.c_void_p()
        L.call("nerf_ext_stream_create", C.byref(self._h))

    @property
    def handle(self) -> int:
        return int(self._h.value or 0)

    def synchronize(self) -> None:
        L.call("nerf_ext_stream_synchronize", self._h)

    def __del__(self):
        try:
            if self._h.value and L._lib is not None:
                L._lib.nerf_ext_stream_destroy(self._h)
        except Exception:
            pass


class Event:
    def __init__(self):
        self._h = C.c_void_p()
        L.call("nerf_ext_event_create", C.byref(self._h))

    def record(self, stream: Stream | None = None) -> None:
        L.call("nerf_ext_event_record", self._h, stream.handle if stream else None)

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        L.call("nerf_ext_event_elapsed_ms", self._h, end._h, C.byref(ms))
        return float(ms.value)

    def __del__(self):
        try:
            if self._h.value and L._lib is not None:
                L._lib.nerf_ext_event_destroy(self._h)
        except Exception:
            pass
