"""Minimal ctypes binding of the HIP runtime: device memory, copies, streams
and events for the benchmark and the GPU tests.

It binds the same libamdhip64 that libkore_attn.so links (by soname, after
that library is loaded), so pointers and streams are shared with it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_hip = None


def lib() -> C.CDLL:
    global _hip
    if _hip is None:
        from . import _lib  # load libkore_attn.so first: it pins the runtime
        _lib.lib()
        try:
            h = C.CDLL("libamdhip64.so.7")
        except OSError:
            h = C.CDLL(os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib", "libamdhip64.so"))
        vp = C.c_void_p
        h.hipGetDeviceCount.argtypes = [C.POINTER(C.c_int)]
        h.hipMalloc.argtypes = [C.POINTER(vp), C.c_size_t]
        h.hipFree.argtypes = [vp]
        h.hipMemcpy.argtypes = [vp, vp, C.c_size_t, C.c_int]
        h.hipMemcpyAsync.argtypes = [vp, vp, C.c_size_t, C.c_int, vp]
        h.hipMemset.argtypes = [vp, C.c_int, C.c_size_t]
        h.hipDeviceSynchronize.argtypes = []
        h.hipStreamSynchronize.argtypes = [vp]
        h.hipEventCreate.argtypes = [C.POINTER(vp)]
        h.hipEventDestroy.argtypes = [vp]
        h.hipEventRecord.argtypes = [vp, vp]
        h.hipEventSynchronize.argtypes = [vp]
        h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), vp, vp]
        h.hipGetErrorString.argtypes = [C.c_int]
        h.hipGetErrorString.restype = C.c_char_p
        h.hipDeviceGetAttribute.argtypes = [C.POINTER(C.c_int), C.c_int, C.c_int]
        h.hipGetDevice.argtypes = [C.POINTER(C.c_int)]
        h.hipDeviceGetName.argtypes = [C.c_char_p, C.c_int, C.c_int]
        h.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
        _hip = h
    return _hip


class HipError(RuntimeError):
    pass


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().hipGetErrorString(rc).decode()
        raise HipError(f"{what}: {msg} ({rc})")


H2D, D2H, D2D = 1, 2, 3


def device_count() -> int:
    n = C.c_int(0)
    rc = lib().hipGetDeviceCount(C.byref(n))
    return n.value if rc == 0 else 0


def device_name(dev: int = 0) -> str:
    buf = C.create_string_buffer(256)
    check(lib().hipDeviceGetName(buf, 256, dev), "hipDeviceGetName")
    return buf.value.decode()


def synchronize() -> None:
    check(lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


def mem_info():
    free, total = C.c_size_t(0), C.c_size_t(0)
    check(lib().hipMemGetInfo(C.byref(free), C.byref(total)), "hipMemGetInfo")
    return free.value, total.value


class DeviceBuffer:
    """A hipMalloc'd float32 array."""

    def __init__(self, n: int):
        self.n = int(n)
        self.nbytes = max(4, self.n * 4)
        p = C.c_void_p()
        check(lib().hipMalloc(C.byref(p), self.nbytes), f"hipMalloc({self.nbytes})")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a, np.float32)
        b = cls(a.size)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, np.float32)
        assert a.size <= self.n
        check(lib().hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")

    def download(self, n: int | None = None, offset: int = 0) -> np.ndarray:
        """n floats (all from offset by default) starting `offset` floats in."""
        n = self.n - offset if n is None else n
        if offset < 0 or n < 0 or offset + n > self.n:
            raise ValueError("download range outside the buffer")
        out = np.empty(n, np.float32)
        check(lib().hipMemcpy(out.ctypes.data, self.ptr + 4 * offset, n * 4, D2H), "hipMemcpy D2H")
        return out

    def at(self, offset_floats: int) -> int:
        return self.ptr + 4 * int(offset_floats)

    def free(self) -> None:
        if self.ptr:
            lib().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = C.c_void_p()
        check(lib().hipEventCreate(C.byref(e)), "hipEventCreate")
        self.ev = e.value

    def record(self, stream=None) -> None:
        check(lib().hipEventRecord(self.ev, stream), "hipEventRecord")

    def synchronize(self) -> None:
        check(lib().hipEventSynchronize(self.ev), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0)
        check(lib().hipEventElapsedTime(C.byref(ms), self.ev, end.ev), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            if self.ev:
                lib().hipEventDestroy(self.ev)
        except Exception:
            pass
