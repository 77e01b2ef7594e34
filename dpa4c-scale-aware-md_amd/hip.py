"""Minimal ctypes binding of the HIP runtime: device buffers, copies, events and
synchronisation for the benchmark and the device-path tests (plumbing only;
the computation lives in libdpamd.so)."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HIP = None


def hip():
    global _HIP
    if _HIP is None:
        for name in ("libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
            try:
                _HIP = C.CDLL(name)
                break
            except OSError:
                continue
        if _HIP is None:
            raise RuntimeError("libamdhip64.so not found")
        P = C.c_void_p
        _HIP.hipMalloc.argtypes = [C.POINTER(P), C.c_size_t]
        _HIP.hipFree.argtypes = [P]
        _HIP.hipMemcpy.argtypes = [P, P, C.c_size_t, C.c_int]
        _HIP.hipMemset.argtypes = [P, C.c_int, C.c_size_t]
        _HIP.hipDeviceSynchronize.argtypes = []
        _HIP.hipSetDevice.argtypes = [C.c_int]
        _HIP.hipGetDeviceCount.argtypes = [C.POINTER(C.c_int)]
        _HIP.hipEventCreate.argtypes = [C.POINTER(P)]
        _HIP.hipEventRecord.argtypes = [P, P]
        _HIP.hipEventSynchronize.argtypes = [P]
        _HIP.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), P, P]
        _HIP.hipEventDestroy.argtypes = [P]
        _HIP.hipGetErrorString.argtypes = [C.c_int]
        _HIP.hipGetErrorString.restype = C.c_char_p
    return _HIP


def check(rc):
    if rc != 0:
        raise RuntimeError(f"HIP error {rc}: {hip().hipGetErrorString(rc).decode()}")


H2D, D2H, D2D = 1, 2, 3


def device_count() -> int:
    n = C.c_int(0)
    if hip().hipGetDeviceCount(C.byref(n)) != 0:
        return 0
    return n.value


def synchronize():
    check(hip().hipDeviceSynchronize())


def copy_d2d(dst: "DeviceArray", src: "DeviceArray", nbytes: int):
    check(hip().hipMemcpy(dst.ptr, src.ptr, nbytes, D2D))


class DeviceArray:
    """A device allocation holding a copy of a numpy array's bytes."""

    def __init__(self, host: np.ndarray | None = None, nbytes: int | None = None):
        self.nbytes = int(host.nbytes if host is not None else nbytes)
        p = C.c_void_p()
        check(hip().hipMalloc(C.byref(p), max(self.nbytes, 8)))
        self.ptr = p.value
        if host is not None:
            h = np.ascontiguousarray(host)
            check(hip().hipMemcpy(self.ptr, h.ctypes.data, self.nbytes, H2D))
        else:
            check(hip().hipMemset(self.ptr, 0, max(self.nbytes, 8)))

    def upload(self, host: np.ndarray):
        """Copy a host array of exactly this allocation's size into it."""
        h = np.ascontiguousarray(host)
        if h.nbytes != self.nbytes:
            raise ValueError(f"upload of {h.nbytes} bytes into a {self.nbytes}-byte buffer")
        check(hip().hipMemcpy(self.ptr, h.ctypes.data, self.nbytes, H2D))

    def to_host(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes == self.nbytes
        check(hip().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H))
        return out

    def free(self):
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = C.c_void_p()
        check(hip().hipEventCreate(C.byref(e)))
        self.e = e

    def record(self, stream=None):
        check(hip().hipEventRecord(self.e, stream))

    def elapsed_ms(self, later: "Event") -> float:
        check(hip().hipEventSynchronize(later.e))
        ms = C.c_float()
        check(hip().hipEventElapsedTime(C.byref(ms), self.e, later.e))
        return float(ms.value)


def visible() -> bool:
    return os.environ.get("HIP_VISIBLE_DEVICES", "0") != "" and device_count() > 0
