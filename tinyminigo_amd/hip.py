"""Device-memory plumbing through the HIP runtime that libtmg.so links.

Tests and benchmarks need raw device buffers for the kernel-level entry
point (tmg_gemv_bf16).  They must come from the same HIP runtime instance as
libtmg's own allocations: importing a second runtime into the process (for
example the one bundled with a PyTorch wheel) leaves one of the two without a
usable device.  This module binds libamdhip64 by the soname libtmg resolved.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib  # libtmg.so first, so the soname below is the one it loaded
from ._lib import finalizing, register

_hip = C.CDLL("libamdhip64.so.7")
_hip.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
_hip.hipFree.argtypes = [C.c_void_p]
_hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
_hip.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
_hip.hipDeviceSynchronize.argtypes = []
_hip.hipGetDeviceCount.argtypes = [C.POINTER(C.c_int)]
_hip.hipGetErrorString.restype = C.c_char_p
_hip.hipGetErrorString.argtypes = [C.c_int]
_hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
_hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
_hip.hipEventSynchronize.argtypes = [C.c_void_p]
_hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
_hip.hipEventDestroy.argtypes = [C.c_void_p]
_hip.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
_hip.hipStreamDestroy.argtypes = [C.c_void_p]
_hip.hipStreamSynchronize.argtypes = [C.c_void_p]
_hip.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
_hip.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
_hip.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]
_hip.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
_hip.hipGraphDestroy.argtypes = [C.c_void_p]
_hip.hipGraphExecDestroy.argtypes = [C.c_void_p]
_hip.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]

H2D, D2H, D2D = 1, 2, 3


def _ok(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: {_hip.hipGetErrorString(rc).decode()}")


def device_count() -> int:
    n = C.c_int(0)
    return n.value if _hip.hipGetDeviceCount(C.byref(n)) == 0 else 0


def synchronize() -> None:
    _ok(_hip.hipDeviceSynchronize(), "hipDeviceSynchronize")


class DeviceBuffer:
    """A hipMalloc'd buffer freed with the object."""

    def __init__(self, nbytes: int):
        self.nbytes = nbytes
        self.ptr = C.c_void_p()
        _ok(_hip.hipMalloc(C.byref(self.ptr), max(nbytes, 1)), "hipMalloc")
        register(self, 2)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        _ok(_hip.hipMemcpy(b.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return b

    @property
    def addr(self) -> int:
        return self.ptr.value

    def to_array(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype)
        _ok(_hip.hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def fill_byte(self, v: int) -> None:
        _ok(_hip.hipMemset(self.ptr, v, self.nbytes), "hipMemset")

    def close(self) -> None:
        if getattr(self, "ptr", None) is not None and self.ptr.value:
            _hip.hipFree(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        if not finalizing():
            self.close()


def copy_device(dst: "DeviceBuffer", src: "DeviceBuffer", nbytes: int) -> None:
    _ok(_hip.hipMemcpy(dst.ptr, src.ptr, nbytes, D2D), "hipMemcpy D2D")


class Stream:
    """A HIP stream (default priority) of the runtime libtmg uses."""

    def __init__(self):
        self.ptr = C.c_void_p()
        _ok(_hip.hipStreamCreate(C.byref(self.ptr)), "hipStreamCreate")
        register(self, 4)

    @property
    def addr(self) -> int:
        return self.ptr.value

    def synchronize(self) -> None:
        _ok(_hip.hipStreamSynchronize(self.ptr), "hipStreamSynchronize")

    def close(self) -> None:
        if getattr(self, "ptr", None) is not None and self.ptr.value:
            _hip.hipStreamSynchronize(self.ptr)
            _hip.hipStreamDestroy(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        if not finalizing():
            self.close()


class Graph:
    """The launches `enqueue(stream)` makes, captured once and replayed."""

    def __init__(self, stream: Stream, enqueue):
        self.stream = stream
        g = C.c_void_p()
        _ok(_hip.hipStreamBeginCapture(stream.ptr, 0), "hipStreamBeginCapture")
        try:
            enqueue(stream)
        finally:
            _ok(_hip.hipStreamEndCapture(stream.ptr, C.byref(g)), "hipStreamEndCapture")
        self.exec = C.c_void_p()
        rc = _hip.hipGraphInstantiate(C.byref(self.exec), g, None, None, 0)
        _hip.hipGraphDestroy(g)
        _ok(rc, "hipGraphInstantiate")
        register(self, 0)

    def launch(self) -> None:
        _ok(_hip.hipGraphLaunch(self.exec, self.stream.ptr), "hipGraphLaunch")

    def close(self) -> None:
        if getattr(self, "exec", None) is not None and self.exec.value:
            _hip.hipStreamSynchronize(self.stream.ptr)
            _hip.hipGraphExecDestroy(self.exec)
            self.exec = C.c_void_p()

    def __del__(self):
        if not finalizing():
            self.close()


class Timer:
    """HIP events around a region of one stream (the null stream by default)."""

    def __init__(self, stream: "Stream | None" = None):
        self.s = stream.ptr if stream is not None else None
        self.a, self.b = C.c_void_p(), C.c_void_p()
        _ok(_hip.hipEventCreate(C.byref(self.a)), "hipEventCreate")
        _ok(_hip.hipEventCreate(C.byref(self.b)), "hipEventCreate")
        register(self, 0)

    def start(self):
        _ok(_hip.hipEventRecord(self.a, self.s), "hipEventRecord")

    def stop(self) -> float:
        _ok(_hip.hipEventRecord(self.b, self.s), "hipEventRecord")
        _ok(_hip.hipEventSynchronize(self.b), "hipEventSynchronize")
        ms = C.c_float()
        _ok(_hip.hipEventElapsedTime(C.byref(ms), self.a, self.b), "hipEventElapsedTime")
        return ms.value

    def close(self) -> None:
        for e in (self.a, self.b):
            if e.value:
                _hip.hipEventDestroy(e)
                e.value = None

    def __del__(self):
        if not finalizing():
            self.close()
