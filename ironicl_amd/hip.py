"""ctypes bindings of libironicl_hip.so (include/ironicl_hip.h).

The library must have been built (``python ironicl_amd/build.py`` or
``__graft_entry__.build()``); loading fails loudly otherwise. There is no CPU
fallback here: a caller that wants the CPU path uses its own.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libironicl_hip.so")

OK, NO_DEVICE, OUT_OF_MEMORY, INVALID_ARGUMENT, DEVICE_ERROR, INTERRUPTED, DOES_NOT_FIT, NOT_FINITE, UNSUPPORTED = range(9)
STATUS_NAMES = ["OK", "NO_DEVICE", "OUT_OF_MEMORY", "INVALID_ARGUMENT", "DEVICE_ERROR", "INTERRUPTED",
                "DOES_NOT_FIT", "NOT_FINITE", "UNSUPPORTED"]
PRECISION_FP32 = 0
PRECISION_SPLIT = 1
PRECISION_HALF = 2
TASK_CLASSIFIER, TASK_REGRESSOR = 0, 1
STAGE_BUILD, STAGE_PREDICT = 0, 1

_F = ctypes.POINTER(ctypes.c_float)
_CF = ctypes.POINTER(ctypes.c_float)
_sz = ctypes.c_size_t
LOOKUP = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(_CF),
                          ctypes.POINTER(_sz))
PROGRESS = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_int, _sz, _sz)
ICL_SOURCE = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, _sz, ctypes.POINTER(_CF), ctypes.POINTER(_CF))


class Shape(ctypes.Structure):
    _fields_ = [("ensembles", _sz), ("features", _sz), ("rows", _sz), ("outputs", _sz)]


class BuildInputs(ctypes.Structure):
    _fields_ = [("shape", Shape), ("x", _CF), ("column_labels", _CF), ("icl_labels", _CF),
                ("inducing_queries", _CF * 3), ("base_scales", _CF * 12), ("rope_frequencies", _CF),
                ("cls_tokens", _CF), ("budget", _sz), ("progress", PROGRESS), ("progress_user", ctypes.c_void_p),
                ("targets", _CF)]


class BuildOutputs(ctypes.Structure):
    _fields_ = [("column_keys", _F * 3), ("column_values", _F * 3), ("icl_keys", _F * 12), ("icl_values", _F * 12)]


class ContextTensors(ctypes.Structure):
    _fields_ = [("shape", Shape), ("column_keys", _CF * 3), ("column_values", _CF * 3), ("icl", ICL_SOURCE),
                ("icl_user", ctypes.c_void_p), ("base_scales", _CF * 12), ("rope_frequencies", _CF),
                ("cls_tokens", _CF), ("budget", _sz)]


class KernelStats(ctypes.Structure):
    _fields_ = [("launches", ctypes.c_uint64), ("milliseconds", ctypes.c_double), ("flops", ctypes.c_double),
                ("bytes", ctypes.c_double), ("busy_milliseconds", ctypes.c_double)]


# Every entry point include/ironicl_hip.h declares, with its ctypes signature.
SIGNATURES = {
    "irx_last_error": (ctypes.c_char_p, []),
    "irx_abi_version": (ctypes.c_int, []),
    "irx_device_open": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]),
    "irx_device_close": (None, [ctypes.c_void_p]),
    "irx_device_free_memory": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(_sz)]),
    "irx_device_compute_units": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)]),
    "irx_weights_upload": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, LOOKUP, ctypes.c_void_p,
                                          ctypes.POINTER(ctypes.c_void_p)]),
    "irx_weights_retain": (None, [ctypes.c_void_p]),
    "irx_weights_release": (None, [ctypes.c_void_p]),
    "irx_weights_bytes": (_sz, [ctypes.c_void_p]),
    "irx_weights_budget": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint64, ctypes.POINTER(_sz)]),
    "irx_context_bytes": (_sz, [ctypes.c_int]),
    "irx_predict_workspace_bytes": (_sz, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, _sz]),
    "irx_build_fits": (ctypes.c_int, [_sz, ctypes.c_int, ctypes.POINTER(Shape)]),
    "irx_build": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(BuildInputs),
                                 ctypes.POINTER(BuildOutputs), ctypes.POINTER(ctypes.c_void_p)]),
    "irx_built_cache_free": (None, [ctypes.c_void_p]),
    "irx_predictor_new": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ContextTensors),
                                         ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]),
    "irx_predictor_free": (None, [ctypes.c_void_p]),
    "irx_predictor_streamed": (ctypes.c_int, [ctypes.c_void_p]),
    "irx_predictor_pass_rows": (_sz, [ctypes.c_void_p]),
    "irx_predictor_set_pass_rows": (ctypes.c_int, [ctypes.c_void_p, _sz]),
    "irx_predictor_set_streams": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "irx_predictor_set_graphs": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "irx_predictor_read_context": (ctypes.c_int, [ctypes.c_void_p, _sz, _sz, _sz, ctypes.c_void_p]),
    "irx_preprocess_fit": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, _sz, _sz,
                                          ctypes.c_void_p, _sz, ctypes.c_void_p, _sz, ctypes.c_double,
                                          ctypes.c_void_p]),
    "irx_preprocessor_new": (ctypes.c_int, [ctypes.c_void_p, _sz, ctypes.c_void_p, _sz, ctypes.c_void_p, _sz,
                                            ctypes.c_void_p, _sz, ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.POINTER(ctypes.c_void_p)]),
    "irx_preprocessor_free": (None, [ctypes.c_void_p]),
    "irx_test_power_fit": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, _sz, _sz, ctypes.c_void_p,
                                          ctypes.c_void_p]),
    "irx_preprocessor_transform": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, _sz, _sz,
                                                  ctypes.c_int, ctypes.c_void_p, ctypes.c_int]),
    "irx_predictor_predict": (ctypes.c_int, [ctypes.c_void_p, _CF, _sz, _F, ctypes.POINTER(ctypes.c_uint8),
                                             PROGRESS, ctypes.c_void_p]),
    "irx_predictor_predict_device": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, _sz, ctypes.c_void_p,
                                                    ctypes.POINTER(ctypes.c_uint8)]),
    "irx_profile_enable": (ctypes.c_int, [ctypes.c_uint]),
    "irx_profile_read": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(KernelStats)]),
    "irx_test_icl_attention": (ctypes.c_int, [ctypes.c_void_p, _CF, _CF, _CF, _sz, _sz, _sz, _F]),
    "irx_icl_attention_noalloc": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                 _sz, _sz, _sz, ctypes.c_void_p, ctypes.c_void_p]),
    "irx_test_icl_attention_precision": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _CF, _CF, _CF, _sz, _sz,
                                                        _sz, _F]),
    "irx_test_encode_icl8": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, _sz, _sz,
                                            ctypes.c_void_p]),
    "irx_test_products": (ctypes.c_int, [ctypes.c_void_p, _CF, _CF, _CF, _CF, _CF, _sz, _sz, _sz, _sz, _F, _F]),
    "irx_regression_summary": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, _sz, _sz, _sz, _CF, _sz,
                                              ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "irx_test_block_head": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _CF, _sz, _CF, _CF, _CF, _CF, _sz, _F]),
    "irx_test_block_tail": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _CF, _CF, _sz, _CF, _CF, _CF, _CF, _CF, _CF,
                                           _CF, _CF, _sz, _F]),
    "irx_test_column_block": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _CF, _sz, _sz, _CF, _CF, _CF, _CF, _CF,
                                             _CF, _CF, _CF, _CF, _CF, _CF, _CF, _CF, _CF, _sz, _F]),
    "irx_test_ln_linear": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _CF, _sz, _sz, _CF, _CF, _CF, _CF, _sz, _CF,
                                          _CF, _CF, _CF, _CF, _F]),
    "irx_test_layer_norm": (ctypes.c_int, [ctypes.c_void_p, _CF, _CF, _CF, _sz, _sz, _F]),
    "irx_test_gelu": (ctypes.c_int, [ctypes.c_void_p, _CF, _sz, _F]),
    "irx_test_copy": (ctypes.c_int, [ctypes.c_void_p, _sz]),
    "irx_test_small_attention": (ctypes.c_int, [ctypes.c_void_p, _CF, _CF, _CF, _sz, _sz, _sz, _F]),
    "irx_test_small_attention_rope": (ctypes.c_int, [ctypes.c_void_p, _CF, _CF, _CF, _CF, _CF, _sz, _sz, _sz, _F]),
    "irx_test_small_attention_tokens": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _CF, _CF, _CF, _CF, _CF, _sz,
                                                       _sz, _sz, _sz, _F, ctypes.c_int, _F]),
}

_lib = None


class HipError(RuntimeError):
    def __init__(self, status: int, message: str):
        name = STATUS_NAMES[status] if 0 <= status < len(STATUS_NAMES) else str(status)
        super().__init__(f"{name}: {message}")
        self.status = status


def lib() -> ctypes.CDLL:
    """The loaded backend. Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build the HIP backend first "
                               "(python ironicl_amd/build.py)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != OK:
        raise HipError(status, lib().irx_last_error().decode(errors="replace"))


def fptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_F)


def cache_ptr(a: np.ndarray | None):
    """A float* ABI field holding an FP32 or (FP16 cache tensors) FP16 array."""
    if a is None:
        return None
    assert a.dtype in (np.float32, np.float16) and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_F)


KERNEL_FAMILIES = ("gemm", "icl_attention", "icl_merge", "small_attention", "layer_norm", "glue")


def profile_enable(families=True) -> None:
    """Record the named kernel families (True: all; False or (): none)."""
    if families is True:
        mask = 0xFFFFFFFF
    elif not families:
        mask = 0
    else:
        mask = sum(1 << KERNEL_FAMILIES.index(f) for f in families)
    check(lib().irx_profile_enable(mask))


def profile_read(family: str) -> dict:
    s = KernelStats()
    check(lib().irx_profile_read(family.encode(), ctypes.byref(s)))
    return {"launches": int(s.launches), "milliseconds": s.milliseconds, "flops": s.flops, "bytes": s.bytes,
            "busy_milliseconds": s.busy_milliseconds}


class Device:
    """A ROCm device (Device::new, src/kernels/cuda/mod.rs:116-172)."""

    def __init__(self, ordinal: int = 0):
        h = ctypes.c_void_p()
        check(lib().irx_device_open(ordinal, ctypes.byref(h)))
        self.handle = h.value

    @classmethod
    def open(cls, ordinal: int = 0) -> "Device | None":
        try:
            return cls(ordinal)
        except HipError as e:
            if e.status == NO_DEVICE:
                return None
            raise

    def compute_units(self) -> int:
        n = ctypes.c_int()
        check(lib().irx_device_compute_units(self.handle, ctypes.byref(n)))
        return n.value

    def free_memory(self) -> int:
        n = _sz()
        check(lib().irx_device_free_memory(self.handle, ctypes.byref(n)))
        return n.value

    def close(self):
        if self.handle:
            lib().irx_device_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
