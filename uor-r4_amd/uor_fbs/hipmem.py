"""Device arrays for the host side: hipMalloc'd buffers through the HIP runtime the library
itself links (libamdhip64.so.7), so that buffers, copies and launches share one runtime in the
process. Plain memory only: allocate, fill with zeros, copy in and out, free."""

from __future__ import annotations

import ctypes as C

import numpy as np

_rt = None
_H2D, _D2H = 1, 2


def runtime():
    global _rt
    if _rt is None:
        from . import hip
        hip.lib()  # the library first: its HIP runtime is the one to share
        rt = C.CDLL("libamdhip64.so.7")
        rt.hipGetErrorString.restype = C.c_char_p
        rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        rt.hipFree.argtypes = [C.c_void_p]
        rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        rt.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        rt.hipSetDevice.argtypes = [C.c_int]
        rt.hipGetDevice.argtypes = [C.POINTER(C.c_int)]
        _rt = rt
    return _rt


def _check(e: int, what: str):
    if e:
        raise RuntimeError(f"{what}: {runtime().hipGetErrorString(e).decode()}")


class _OnDevice:
    def __init__(self, device: int):
        self.device = device

    def __enter__(self):
        prev = C.c_int()
        _check(runtime().hipGetDevice(C.byref(prev)), "hipGetDevice")
        self.prev = prev.value
        _check(runtime().hipSetDevice(self.device), "hipSetDevice")

    def __exit__(self, *exc):
        runtime().hipSetDevice(self.prev)


class DeviceArray:
    """A C-contiguous array of `dtype` and `shape` in the memory of HIP device `device`."""

    def __init__(self, shape, dtype, device: int = 0):
        self.shape = tuple(int(x) for x in np.atleast_1d(shape))
        self.dtype = np.dtype(dtype)
        self.device = device
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self._p = C.c_void_p()
        with _OnDevice(device):
            _check(runtime().hipMalloc(C.byref(self._p), max(self.nbytes, 16)), "hipMalloc")
        self.zero()

    @property
    def ptr(self) -> C.c_void_p:
        return self._p

    def _at(self, index: int, row_bytes: int) -> C.c_void_p:
        """The address of row `index` of the first axis (checked against the allocation)."""
        index = int(index)
        if not 0 <= index < self.shape[0]:
            raise IndexError(f"row {index} outside the array's {self.shape[0]}")
        return C.c_void_p(self._p.value + index * row_bytes)

    def zero(self, rows=None):
        """Zeros over the whole array or over the given rows of its first axis (synchronous)."""
        row = self.nbytes // self.shape[0]
        with _OnDevice(self.device):
            if rows is None:
                _check(runtime().hipMemset(self._p, 0, self.nbytes), "hipMemset")
            else:
                for r in rows:
                    _check(runtime().hipMemset(self._at(r, row), 0, row), "hipMemset")

    def upload(self, a, row: int | None = None):
        """Copy a host array in (the whole array, or one row of the first axis)."""
        a = np.ascontiguousarray(a, dtype=self.dtype)
        nbytes = self.nbytes if row is None else self.nbytes // self.shape[0]
        if a.nbytes != nbytes:
            raise ValueError(f"{a.nbytes} bytes for a {nbytes}-byte destination")
        dst = self._p if row is None else self._at(row, nbytes)
        with _OnDevice(self.device):
            _check(runtime().hipMemcpy(dst, a.ctypes.data_as(C.c_void_p), nbytes, _H2D), "hipMemcpy")

    def download(self, row: int | None = None) -> np.ndarray:
        """Copy out (the whole array, or one row of the first axis); waits for the device."""
        shape = self.shape if row is None else self.shape[1:]
        out = np.empty(shape, self.dtype)
        src = self._p if row is None else self._at(row, self.nbytes // self.shape[0])
        with _OnDevice(self.device):
            _check(runtime().hipMemcpy(out.ctypes.data_as(C.c_void_p), src, out.nbytes, _D2H), "hipMemcpy")
        return out

    def free(self):
        if self._p.value:
            with _OnDevice(self.device):
                runtime().hipFree(self._p)
            self._p = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
