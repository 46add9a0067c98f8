"""Device buffers through the HIP runtime libppocr_hip.so itself links
(ctypes), for callers of the ppocr_hip_* layer entry points that have no
device memory of their own. Using the library's runtime keeps one HIP
runtime per process."""

from __future__ import annotations

import ctypes as C

import numpy as np

_hip = None
H2D, D2H = 1, 2


def hip() -> C.CDLL:
    global _hip
    if _hip is None:
        from . import lib
        lib()  # loads libamdhip64 as the library's dependency
        h = C.CDLL("libamdhip64.so.7")
        h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        h.hipFree.argtypes = [C.c_void_p]
        h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        h.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        h.hipDeviceSynchronize.argtypes = []
        h.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        h.hipStreamDestroy.argtypes = [C.c_void_p]
        h.hipStreamSynchronize.argtypes = [C.c_void_p]
        h.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        h.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        h.hipEventSynchronize.argtypes = [C.c_void_p]
        h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        h.hipEventDestroy.argtypes = [C.c_void_p]
        _hip = h
    return _hip


def _ok(rc: int, what: str) -> None:
    if rc:
        raise RuntimeError(f"{what} failed with HIP error {rc}")


class DeviceArray:
    """`nbytes` of device memory, freed with the object."""

    def __init__(self, nbytes: int):
        self.nbytes = nbytes
        self.ptr = C.c_void_p()
        _ok(hip().hipMalloc(C.byref(self.ptr), max(nbytes, 4)), "hipMalloc")

    @classmethod
    def of(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes)
        d.upload(a)
        return d

    @property
    def addr(self) -> int:
        return self.ptr.value

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        _ok(hip().hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy")

    def download(self, count: int, dtype=np.float32) -> np.ndarray:
        out = np.empty(count, dtype)
        assert out.nbytes <= self.nbytes
        _ok(hip().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H), "hipMemcpy")
        return out

    def free(self) -> None:
        if self.ptr and self.ptr.value:
            hip().hipFree(self.ptr)
            self.ptr = C.c_void_p()

    __del__ = free


def synchronize() -> None:
    _ok(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Timer:
    """HIP events around work enqueued on `stream` (0 = the null stream)."""

    def __init__(self, stream: int = 0):
        self.stream = C.c_void_p(stream or None)
        self.a, self.b = C.c_void_p(), C.c_void_p()
        hip().hipEventCreate(C.byref(self.a))
        hip().hipEventCreate(C.byref(self.b))

    def start(self) -> None:
        hip().hipEventRecord(self.a, self.stream)

    def stop(self) -> float:
        hip().hipEventRecord(self.b, self.stream)
        _ok(hip().hipEventSynchronize(self.b), "hipEventSynchronize")
        ms = C.c_float()
        hip().hipEventElapsedTime(C.byref(ms), self.a, self.b)
        return ms.value

    def __del__(self):
        if self.a:
            hip().hipEventDestroy(self.a)
            hip().hipEventDestroy(self.b)
            self.a = self.b = None
