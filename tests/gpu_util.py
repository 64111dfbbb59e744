"""Device buffers and streams for GPU tests, through the HIP runtime that
libmfhip.so itself links (ctypes; no torch import, which can take minutes on
a fresh box)."""

import ctypes

import numpy as np

from metalfish_amd import backend

H2D, D2H = 1, 2


class DeviceBuffers:
    """hipMalloc'd copies of numpy arrays, a caller-owned stream, freed on
    free()."""

    def __init__(self):
        backend.lib()  # loads libamdhip64 as a dependency
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self.hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                       ctypes.c_int]
        self.hip.hipFree.argtypes = [ctypes.c_void_p]
        self.hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
        self.hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
        self.hip.hipDeviceSynchronize.argtypes = []
        self.ptrs = []
        self.streams = []

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        assert self.hip.hipMalloc(ctypes.byref(p), max(int(nbytes), 4)) == 0
        self.ptrs.append(p.value)
        return p.value

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        p = self.alloc(arr.nbytes)
        if arr.nbytes:
            assert self.hip.hipMemcpy(p, arr.ctypes.data, arr.nbytes, H2D) == 0
        return p

    def write(self, ptr, arr):
        """Copies arr into an existing buffer (synchronous hipMemcpy)."""
        arr = np.ascontiguousarray(arr)
        assert self.hip.hipMemcpy(ptr, arr.ctypes.data, arr.nbytes, H2D) == 0

    def get(self, ptr, like):
        out = np.empty_like(like)
        assert self.hip.hipMemcpy(out.ctypes.data, ptr, out.nbytes, D2H) == 0
        return out

    def stream(self):
        """A new stream at the default priority."""
        s = ctypes.c_void_p()
        assert self.hip.hipStreamCreate(ctypes.byref(s)) == 0
        self.streams.append(s.value)
        return s.value

    def sync(self, stream=None):
        if stream is None:
            assert self.hip.hipDeviceSynchronize() == 0
        else:
            assert self.hip.hipStreamSynchronize(stream) == 0

    def free(self):
        self.sync()
        for p in self.ptrs:
            self.hip.hipFree(p)
        for s in self.streams:
            self.hip.hipStreamDestroy(s)
        self.ptrs = []
        self.streams = []
