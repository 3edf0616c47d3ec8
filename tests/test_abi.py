"""The C ABI library (CPU-side checks, no GPU compute): it loads, exports
every entry point include/ironicl_hip.h declares, and answers host-only
queries as the header documents."""

import ctypes
import os
import re

import pytest

from conftest import ROOT
from ironicl_amd import hip

HEADER = os.path.join(ROOT, "include", "ironicl_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(irx_[a-z_0-9]+)\s*\(", text)
    return sorted(set(n for n in names if not n.endswith("_fn") and n not in ("irx_tensor_lookup", "irx_icl_source")))


def test_library_is_built():
    assert os.path.exists(hip.LIB_PATH), "run __graft_entry__.build() first"


def test_every_declared_entry_point_is_exported_and_bound():
    lib = hip.lib()
    names = declared_functions()
    assert len(names) >= 25
    for name in names:
        assert hasattr(lib, name), name
        assert name in hip.SIGNATURES, f"{name} has no ctypes signature"
    assert set(hip.SIGNATURES) == set(names)


def test_host_queries():
    lib = hip.lib()
    assert lib.irx_abi_version() == 1
    assert lib.irx_context_bytes(hip.PRECISION_FP32) == 4
    assert lib.irx_context_bytes(hip.PRECISION_SPLIT) == 2  # the FP16 ICL cache of optimize="auto"
    assert lib.irx_context_bytes(7) == 0
    small = hip.Shape(1, 5, 240, 10)
    assert lib.irx_build_fits(1 << 40, hip.PRECISION_FP32, ctypes.byref(small)) == 1
    assert lib.irx_build_fits(1 << 20, hip.PRECISION_FP32, ctypes.byref(small)) == 0
    tiny = hip.Shape(1, 5, 32, 10)  # fewer than 64 training rows build on the CPU
    assert lib.irx_build_fits(1 << 40, hip.PRECISION_FP32, ctypes.byref(tiny)) == 0
    huge = hip.Shape(8, 500, 200_000, 10)  # the 200k x 500 x 8 context fits 288 GB
    assert lib.irx_build_fits(280 << 30, hip.PRECISION_FP32, ctypes.byref(huge)) == 1
    assert lib.irx_build_fits(1 << 40, hip.PRECISION_SPLIT, ctypes.byref(small)) == 1
    assert lib.irx_build_fits(1 << 40, 7, ctypes.byref(small)) == 0


def test_disable_variable_means_no_device(monkeypatch):
    monkeypatch.setenv("IRONICL_NO_ROCM", "1")
    assert hip.Device.open(0) is None
    h = ctypes.c_void_p()
    assert hip.lib().irx_device_open(0, ctypes.byref(h)) == hip.NO_DEVICE
    assert b"IRONICL_NO_ROCM" in hip.lib().irx_last_error()


def test_null_arguments_are_errors_not_crashes():
    lib = hip.lib()
    assert lib.irx_device_open(0, None) == hip.INVALID_ARGUMENT
    assert lib.irx_weights_upload(None, 0, hip.LOOKUP(), None, None) == hip.INVALID_ARGUMENT
    assert lib.irx_build(None, 0, None, None, None) == hip.INVALID_ARGUMENT
    assert lib.irx_predictor_predict(None, None, 0, None, None, hip.PROGRESS(), None) == hip.INVALID_ARGUMENT
    lib.irx_predictor_free(None)
    lib.irx_weights_release(None)
    lib.irx_built_cache_free(None)


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(hip, "_lib", None)
    monkeypatch.setattr(hip, "LIB_PATH", "/nonexistent/libironicl_hip.so")
    with pytest.raises(RuntimeError, match="build the HIP backend"):
        hip.lib()
