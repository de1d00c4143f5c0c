"""ditch_amd — MI355X (gfx950) device backend for ditch's operator seam.

The product is the C-ABI library `libditch_hip.so` built from csrc/ and
declared in include/ditch_hip.h. This package holds its sources, the build
script, and a thin ctypes binding (`ditch_amd.hip`) that Python callers use.
There is no CPU fallback: loading fails loudly when the library is missing.
"""
import ctypes
import os

from . import abi

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libditch_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "ditch_hip.h")

_lib = None


class LibraryMissing(RuntimeError):
    pass


def load_library():
    """Loads libditch_hip.so (built in-tree) and declares every prototype."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryMissing(
            f"{LIB_PATH} is not built; run `python -m ditch_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in abi.PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
