"""Device buffers and events through the HIP runtime libditch_hip.so runs on.

Callers that hand device pointers to the C ABI (tests, bench.py) allocate them
here. Torch's wheel carries its own copy of the HIP runtime under the same
soname (libamdhip64.so.7) as the ROCm installation's; whichever copy is
loaded first in a process is the one libditch_hip.so binds to. The functions
below are therefore looked up through the library's own handle (dlsym
searches its dependencies), so buffers and events always live in the runtime
the library uses.
"""
import ctypes

import numpy as np

from . import load_library

_hip = None


def hip():
    """The HIP runtime functions libditch_hip.so resolves to."""
    global _hip
    if _hip is not None:
        return _hip
    lib = load_library()
    P, S = ctypes.c_void_p, ctypes.c_size_t
    proto = {
        "hipMalloc": [ctypes.POINTER(P), S],
        "hipFree": [P],
        "hipMemcpy": [P, P, S, ctypes.c_int],
        "hipMemcpyAsync": [P, P, S, ctypes.c_int, P],
        "hipMemset": [P, ctypes.c_int, S],
        "hipDeviceSynchronize": [],
        "hipStreamSynchronize": [P],
        "hipStreamCreateWithFlags": [ctypes.POINTER(P), ctypes.c_uint],
        "hipStreamDestroy": [P],
        "hipEventCreate": [ctypes.POINTER(P)],
        "hipEventDestroy": [P],
        "hipEventRecord": [P, P],
        "hipEventSynchronize": [P],
        "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), P, P],
        "hipGetErrorString": [ctypes.c_int],
        "hipSetDevice": [ctypes.c_int],
    }
    for n, args in proto.items():
        f = getattr(lib, n)
        f.argtypes = args
        f.restype = ctypes.c_char_p if n == "hipGetErrorString" else ctypes.c_int
    _hip = lib
    return lib


def check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what}: {hip().hipGetErrorString(rc).decode()}")


H2D, D2H, D2D = 1, 2, 3


class Buffer:
    """A device allocation (freed on close or garbage collection)."""

    def __init__(self, nbytes):
        self.nbytes = max(int(nbytes), 1)
        p = ctypes.c_void_p()
        check(hip().hipMalloc(ctypes.byref(p), self.nbytes), "hipMalloc")
        self.ptr = p

    @staticmethod
    def from_array(a):
        a = np.ascontiguousarray(a)
        b = Buffer(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(hip().hipMemcpy(self.ptr, a.ctypes.data_as(ctypes.c_void_p), a.nbytes, H2D), "hipMemcpy H2D")

    def download(self, dtype, shape):
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(hip().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), self.ptr, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def zero(self):
        check(hip().hipMemset(self.ptr, 0, self.nbytes), "hipMemset")

    def free(self):
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(hip().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.e = e

    def record(self, stream):
        check(hip().hipEventRecord(self.e, stream), "hipEventRecord")

    def synchronize(self):
        check(hip().hipEventSynchronize(self.e), "hipEventSynchronize")

    def elapsed_ms(self, end):
        ms = ctypes.c_float()
        check(hip().hipEventElapsedTime(ctypes.byref(ms), self.e, end.e), "hipEventElapsedTime")
        return ms.value


def synchronize():
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
