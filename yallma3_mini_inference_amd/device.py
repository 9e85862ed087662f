"""Device buffers for the C ABI (yl_malloc / yl_memcpy_*), numpy in and out."""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, last_error, lib


def device_count() -> int:
    n = C.c_int(0)
    st = lib().yl_device_count(C.byref(n))
    return int(n.value) if st == 0 else 0


class DeviceBuffer:
    """An HBM allocation owned by Python; `ptr` is the raw device address."""

    def __init__(self, nbytes: int, dtype=np.uint8, shape=None):
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = shape if shape is not None else (self.nbytes // self.dtype.itemsize,)
        self.ptr = lib().yl_malloc(max(1, self.nbytes))
        if not self.ptr:
            raise MemoryError("yl_malloc failed: " + last_error())

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes, a.dtype, a.shape)
        if a.nbytes:
            check(lib().yl_memcpy_h2d(b.ptr, a.ctypes.data, a.nbytes))
        return b

    @classmethod
    def zeros(cls, shape, dtype) -> "DeviceBuffer":
        shape = tuple(shape) if hasattr(shape, "__len__") else (int(shape),)
        nbytes = int(np.prod(shape)) * np.dtype(dtype).itemsize
        b = cls(nbytes, dtype, shape)
        check(lib().yl_memset_d(b.ptr, 0, max(1, nbytes)))
        return b

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            check(lib().yl_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes))
        return out

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, self.dtype)
        assert a.nbytes <= self.nbytes
        check(lib().yl_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes))

    def free(self) -> None:
        if self.ptr:
            lib().yl_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
