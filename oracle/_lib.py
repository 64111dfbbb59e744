"""CPU ORACLE -- TEST INFRASTRUCTURE ONLY.

ctypes loader for ``oracle/libcpuref.so`` (built from ``cpu_ref.c`` by
``oracle/Makefile``) and glibc's ``powf``, which the reference calls through
``std::pow(float, float)`` for the residual scale.
"""

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcpuref.so")

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run __graft_entry__.build())")
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.or_run.restype = ctypes.c_int
        _lib.or_run.argtypes = [
            ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        _lib.or_pack_planes.restype = None
        _lib.or_pack_planes.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                        ctypes.c_void_p]
    return _lib


_libm = ctypes.CDLL("libm.so.6")
_libm.powf.restype = ctypes.c_float
_libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]


def powf(x, y):
    return _libm.powf(float(x), float(y))
