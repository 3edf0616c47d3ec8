"""Device buffers from the HIP runtime libironicl_hip.so itself links.

A process must hold one HIP runtime: PyTorch's wheel bundles its own
libamdhip64 / libhsa-runtime64 (an older ROCm), and two HSA runtimes cannot
both own the GPU. Buffers for the HBM-resident entry points
(irx_predictor_predict_device) therefore come from this module, never from
torch, in any process that loads the backend.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import hip

_rt = None
H2D, D2H, D2D = 1, 2, 3


def runtime() -> ctypes.CDLL:
    global _rt
    if _rt is None:
        hip.lib()  # loads libamdhip64.so.7 as the backend's dependency
        rt = ctypes.CDLL("libamdhip64.so.7")
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        rt.hipMalloc.argtypes = [ctypes.POINTER(vp), sz]
        rt.hipFree.argtypes = [vp]
        rt.hipMemcpy.argtypes = [vp, vp, sz, ctypes.c_int]
        rt.hipDeviceSynchronize.argtypes = []
        rt.hipSetDevice.argtypes = [ctypes.c_int]
        rt.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        rt.hipEventRecord.argtypes = [vp, vp]
        rt.hipEventSynchronize.argtypes = [vp]
        rt.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        rt.hipEventDestroy.argtypes = [vp]
        for fn in ("hipMalloc", "hipFree", "hipMemcpy", "hipDeviceSynchronize", "hipSetDevice", "hipEventCreate",
                   "hipEventRecord", "hipEventSynchronize", "hipEventElapsedTime", "hipEventDestroy"):
            getattr(rt, fn).restype = ctypes.c_int
        _rt = rt
    return _rt


def _ok(code: int, what: str) -> None:
    if code != 0:
        raise RuntimeError(f"{what} failed with HIP error {code}")


class DeviceArray:
    """A float32 buffer in HBM."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        _ok(runtime().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_host(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        _ok(runtime().hipMemcpy(d.ptr, a.ctypes.data, d.nbytes, H2D), "hipMemcpy H2D")
        return d

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        _ok(runtime().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    def free(self) -> None:
        if self.ptr:
            runtime().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize() -> None:
    _ok(runtime().hipDeviceSynchronize(), "hipDeviceSynchronize")
