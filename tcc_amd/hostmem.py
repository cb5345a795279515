"""Pinned, device-mapped host memory for zero-copy cold feature rows.

Allocated with hipHostMalloc(hipHostMallocMapped) (never hipHostRegister on
existing memory); the GPU reads it through the pointer from
hipHostGetDevicePointer, over PCIe, with ordinary global loads — the
single-GPU form of the reference's cpu_feature_cache_ptr
(spmm_cnic/src/core/spmm_kernel.cu:137-142).
"""
from __future__ import annotations

import ctypes

import numpy as np

_HIP_HOST_MALLOC_MAPPED = 0x2
_hip = None


def _lib():
    global _hip
    if _hip is None:
        h = ctypes.CDLL("libamdhip64.so")
        h.hipHostMalloc.restype = ctypes.c_int
        h.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
        h.hipHostFree.restype = ctypes.c_int
        h.hipHostFree.argtypes = [ctypes.c_void_p]
        h.hipHostGetDevicePointer.restype = ctypes.c_int
        h.hipHostGetDevicePointer.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_uint]
        _hip = h
    return _hip


class PinnedArray:
    """A numpy array in mapped pinned host memory, with its device pointer."""

    def __init__(self, shape, dtype=np.float32):
        dtype = np.dtype(dtype)
        n = int(np.prod(shape)) * dtype.itemsize
        self._ptr = ctypes.c_void_p()
        rc = _lib().hipHostMalloc(ctypes.byref(self._ptr), max(n, 1), _HIP_HOST_MALLOC_MAPPED)
        if rc != 0:
            raise MemoryError(f"hipHostMalloc({n}) failed ({rc})")
        buf = (ctypes.c_char * max(n, 1)).from_address(self._ptr.value)
        self.array = np.frombuffer(buf, dtype=dtype, count=int(np.prod(shape))).reshape(shape)
        dev = ctypes.c_void_p()
        rc = _lib().hipHostGetDevicePointer(ctypes.byref(dev), self._ptr, 0)
        if rc != 0:
            self.free()
            raise RuntimeError(f"hipHostGetDevicePointer failed ({rc})")
        self.device_ptr = dev.value

    def free(self) -> None:
        if self._ptr is not None and self._ptr.value:
            self.array = None
            _lib().hipHostFree(self._ptr)
            self._ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
