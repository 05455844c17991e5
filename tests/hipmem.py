"""Minimal HIP runtime access for tests (device buffers for the operator-level C ABI)."""
import ctypes as C

import numpy as np

_hip = None


def hip():
    global _hip
    if _hip is None:
        h = C.CDLL("libamdhip64.so")
        h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        h.hipFree.argtypes = [C.c_void_p]
        h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        h.hipDeviceSynchronize.argtypes = []
        h.hipGetDeviceCount.argtypes = [C.POINTER(C.c_int)]
        _hip = h
    return _hip


def device_count() -> int:
    n = C.c_int(0)
    try:
        if hip().hipGetDeviceCount(C.byref(n)) != 0:
            return 0
    except OSError:
        return 0
    return n.value


class DeviceArray:
    def __init__(self, host: np.ndarray):
        self.nbytes = host.nbytes
        self.p = C.c_void_p()
        assert hip().hipMalloc(C.byref(self.p), max(self.nbytes, 4)) == 0
        if self.nbytes:
            assert hip().hipMemcpy(self.p, host.ctypes.data, self.nbytes, 1) == 0  # H2D

    def to_host(self, like: np.ndarray) -> np.ndarray:
        out = np.empty_like(like)
        assert hip().hipMemcpy(out.ctypes.data, self.p, out.nbytes, 2) == 0  # D2H
        return out

    def free(self):
        if self.p:
            hip().hipFree(self.p)
            self.p = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
