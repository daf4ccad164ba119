"""Minimal ctypes access to the HIP runtime that libredukt_gpu.so links.

The GPU tests and the benchmark need device buffers, copies and events on the
library's stream.  They use the very runtime instance the library uses (the
/opt/rocm libamdhip64), not a second copy such as the one bundled with PyTorch.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_CANDIDATES = ("libamdhip64.so.7", "/opt/rocm/lib/libamdhip64.so.7", "/opt/rocm/lib/libamdhip64.so")
_hip = None

H2D, D2H, D2D = 1, 2, 3


class HipError(RuntimeError):
    pass


def rt() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        err = None
        for name in _CANDIDATES:
            try:
                _hip = ctypes.CDLL(name)
                break
            except OSError as e:
                err = e
        if _hip is None:
            raise OSError(f"HIP runtime not found: {err}")
        h = _hip
        h.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        h.hipFree.argtypes = [ctypes.c_void_p]
        h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        h.hipMemset.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
        h.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
        h.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        h.hipEventDestroy.argtypes = [ctypes.c_void_p]
        h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        h.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
        h.hipGetDeviceCount.argtypes = [ctypes.POINTER(ctypes.c_int)]
        h.hipGetErrorString.argtypes = [ctypes.c_int]
        h.hipGetErrorString.restype = ctypes.c_char_p
        h.hipDeviceGetAttribute.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]
        h.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
    return _hip


def check(code: int, what: str) -> None:
    if code != 0:
        msg = rt().hipGetErrorString(code)
        raise HipError(f"{what}: {msg.decode() if msg else code}")


def device_count() -> int:
    n = ctypes.c_int(0)
    code = rt().hipGetDeviceCount(ctypes.byref(n))
    return n.value if code == 0 else 0


class DeviceBuffer:
    """A hipMalloc'd buffer freed on close()."""

    def __init__(self, nbytes: int):
        self.nbytes = nbytes
        p = ctypes.c_void_p()
        check(rt().hipMalloc(ctypes.byref(p), max(nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(rt().hipMemcpy(self.ptr + offset, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype)
        assert offset + out.nbytes <= self.nbytes
        check(rt().hipMemcpy(out.ctypes.data, self.ptr + offset, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def close(self) -> None:
        if self.ptr:
            rt().hipFree(self.ptr)
            self.ptr = None


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(rt().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.h = e.value

    def record(self, stream: int) -> None:
        check(rt().hipEventRecord(self.h, stream), "hipEventRecord")

    def synchronize(self) -> None:
        check(rt().hipEventSynchronize(self.h), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0)
        check(rt().hipEventElapsedTime(ctypes.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return ms.value

    def close(self) -> None:
        if self.h:
            rt().hipEventDestroy(self.h)
            self.h = None


def copy_d2d_async(dst: int, src: int, nbytes: int, stream: int) -> None:
    """Device-to-device copy on `stream` (hipMemcpyDeviceToDevice = 3)."""
    check(rt().hipMemcpyAsync(ctypes.c_void_p(dst), ctypes.c_void_p(src), nbytes, 3, ctypes.c_void_p(stream)),
          "hipMemcpyAsync")


def stream_sync(stream: int) -> None:
    check(rt().hipStreamSynchronize(stream), "hipStreamSynchronize")


def device_attribute(attr: int, device: int = 0) -> int:
    v = ctypes.c_int(0)
    check(rt().hipDeviceGetAttribute(ctypes.byref(v), attr, device), "hipDeviceGetAttribute")
    return v.value
