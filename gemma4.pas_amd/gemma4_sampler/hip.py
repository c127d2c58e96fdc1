"""Minimal ctypes binding of the HIP runtime: device memory, copies, streams,
events.  The sampler library links /opt/rocm's libamdhip64, so this module
loads that same runtime (torch's wheel bundles a different copy and is not
used here)."""
import ctypes
import os

import numpy as np

_HIP_PATHS = ("/opt/rocm/lib/libamdhip64.so.7", "/opt/rocm/lib/libamdhip64.so")

H2D, D2H, D2D = 1, 2, 3


class HipError(RuntimeError):
    pass


_lib = None


def lib():
    global _lib
    if _lib is None:
        err = None
        for p in _HIP_PATHS:
            if os.path.exists(p):
                try:
                    _lib = ctypes.CDLL(p)
                    break
                except OSError as e:  # pragma: no cover
                    err = e
        if _lib is None:
            raise HipError(f"cannot load the HIP runtime: {err}")
        _lib.hipGetErrorString.restype = ctypes.c_char_p
        _lib.hipGetErrorString.argtypes = [ctypes.c_int]
        _lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                             ctypes.c_void_p]
    return _lib


def check(rc, what="HIP call"):
    if rc != 0:
        raise HipError(f"{what} failed: {lib().hipGetErrorString(rc).decode()} ({rc})")


def device_count():
    n = ctypes.c_int(0)
    rc = lib().hipGetDeviceCount(ctypes.byref(n))
    return n.value if rc == 0 else 0


def synchronize():
    check(lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Buffer:
    """A device allocation of `nbytes` bytes."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = ctypes.c_void_p()
        check(lib().hipMalloc(ctypes.byref(self.ptr), ctypes.c_size_t(max(self.nbytes, 1))),
              f"hipMalloc({self.nbytes})")

    @property
    def addr(self):
        return self.ptr.value

    def offset(self, nbytes):
        return ctypes.c_void_p(self.ptr.value + int(nbytes))

    def upload(self, arr, offset=0):
        a = np.ascontiguousarray(arr)
        assert offset + a.nbytes <= self.nbytes
        check(lib().hipMemcpy(self.offset(offset), a.ctypes.data_as(ctypes.c_void_p),
                              ctypes.c_size_t(a.nbytes), H2D), "hipMemcpy H2D")
        return self

    def download(self, dtype, count=None, offset=0):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        check(lib().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), self.offset(offset),
                              ctypes.c_size_t(out.nbytes), D2H), "hipMemcpy D2H")
        return out

    def zero(self):
        check(lib().hipMemset(self.ptr, 0, ctypes.c_size_t(self.nbytes)), "hipMemset")
        return self

    def free(self):
        if self.ptr is not None and self.ptr.value:
            lib().hipFree(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    @classmethod
    def from_array(cls, arr):
        a = np.ascontiguousarray(arr)
        return cls(a.nbytes).upload(a)


class Stream:
    def __init__(self, nonblocking=False):
        """A HIP stream (default priority); nonblocking: hipStreamNonBlocking,
        no implicit ordering with the null stream."""
        self.handle = ctypes.c_void_p()
        if nonblocking:
            check(lib().hipStreamCreateWithFlags(ctypes.byref(self.handle), ctypes.c_uint(1)),
                  "hipStreamCreateWithFlags")
        else:
            check(lib().hipStreamCreate(ctypes.byref(self.handle)), "hipStreamCreate")

    def synchronize(self):
        check(lib().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def destroy(self):
        if self.handle is not None and self.handle.value:
            lib().hipStreamDestroy(self.handle)
        self.handle = None


class Event:
    def __init__(self):
        self.handle = ctypes.c_void_p()
        check(lib().hipEventCreate(ctypes.byref(self.handle)), "hipEventCreate")

    def record(self, stream=None):
        s = stream.handle if stream is not None else ctypes.c_void_p()
        check(lib().hipEventRecord(self.handle, s), "hipEventRecord")

    def synchronize(self):
        check(lib().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, later):
        ms = ctypes.c_float()
        check(lib().hipEventElapsedTime(ctypes.byref(ms), self.handle, later.handle),
              "hipEventElapsedTime")
        return ms.value

    def destroy(self):
        if self.handle is not None and self.handle.value:
            lib().hipEventDestroy(self.handle)
        self.handle = None
