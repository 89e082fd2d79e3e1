"""Minimal ctypes access to the HIP runtime: device buffers, pinned host
buffers, streams and events (used by bench.py and the device-pointer API)."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_hip = None

def rt() -> C.CDLL:
    global _hip
    if _hip is None:
        path = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib", "libamdhip64.so")
        _hip = C.CDLL(path)
        _hip.hipGetErrorString.restype = C.c_char_p
    return _hip

def check(err: int, what: str = "") -> None:
    if err != 0:
        raise RuntimeError(f"HIP error {err} ({rt().hipGetErrorString(err).decode()}) {what}")

H2D, D2H, D2D = 1, 2, 3

class DeviceBuffer:
    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = C.c_void_p()
        check(rt().hipMalloc(C.byref(self.ptr), C.c_size_t(max(self.nbytes, 1))), "hipMalloc")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        check(rt().hipMemcpy(b.ptr, a.ctypes.data_as(C.c_void_p), C.c_size_t(a.nbytes), H2D), "H2D")
        return b

    @property
    def addr(self) -> int:
        return int(self.ptr.value or 0)

    def free(self) -> None:
        if self.ptr:
            rt().hipFree(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

class PinnedBuffer:
    """Page-locked host memory allocated by hipHostMalloc, viewed as numpy."""

    def __init__(self, shape, dtype):
        self.dtype = np.dtype(dtype)
        self.shape = tuple(shape)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.ptr = C.c_void_p()
        check(rt().hipHostMalloc(C.byref(self.ptr), C.c_size_t(max(self.nbytes, 1)), C.c_uint(0)), "hipHostMalloc")
        buf = (C.c_char * max(self.nbytes, 1)).from_address(self.ptr.value)
        self.array = np.frombuffer(buf, dtype=self.dtype, count=int(np.prod(self.shape))).reshape(self.shape)

    def free(self) -> None:
        if self.ptr:
            rt().hipHostFree(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

class Stream:
    def __init__(self):
        self.h = C.c_void_p()
        check(rt().hipStreamCreate(C.byref(self.h)), "hipStreamCreate")

    def sync(self) -> None:
        check(rt().hipStreamSynchronize(self.h), "hipStreamSynchronize")

    def destroy(self) -> None:
        if self.h:
            rt().hipStreamDestroy(self.h)
            self.h = C.c_void_p()

class Event:
    def __init__(self):
        self.h = C.c_void_p()
        check(rt().hipEventCreate(C.byref(self.h)), "hipEventCreate")

    def record(self, stream: Stream) -> None:
        check(rt().hipEventRecord(self.h, stream.h), "hipEventRecord")

    def elapsed_ms(self, end: "Event") -> float:
        check(rt().hipEventSynchronize(end.h), "hipEventSynchronize")
        ms = C.c_float()
        check(rt().hipEventElapsedTime(C.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return float(ms.value)

def memcpy_d2h_async(dst: PinnedBuffer, src: DeviceBuffer, nbytes: int, stream: Stream) -> None:
    check(rt().hipMemcpyAsync(dst.ptr, src.ptr, C.c_size_t(nbytes), D2H, stream.h), "D2H")

def device_synchronize() -> None:
    check(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")
