"""CPU-side checks of the C ABI: librq.so loads, exports exactly what
include/rq.h declares, and its host-side validation answers without a GPU
(no compute call is made here)."""
import ctypes as C
import os
import re

import pytest

from raster_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "rq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rq_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in declared_symbols():
        assert hasattr(L, name), name


def test_version_and_status_strings():
    L = _lib.lib()
    assert L.rq_version() == 1
    assert L.rq_status_string(_lib.RQ_ERR_SHAPE) == b"bad shape"
    assert L.rq_status_string(999) == b"unknown status"


def test_invalid_handles_are_reported_not_dereferenced():
    L = _lib.lib()
    bogus = C.c_void_p(0x1234)
    assert L.rq_weight_destroy(None) == _lib.RQ_ERR_HANDLE
    assert L.rq_weight_destroy(bogus) == _lib.RQ_ERR_HANDLE
    assert L.rq_ctx_destroy(bogus) == _lib.RQ_ERR_HANDLE
    assert L.rq_qmatmul(bogus, bogus, None, 0, None, 0, 1, None) == _lib.RQ_ERR_HANDLE
    assert b"rq_ctx" in L.rq_last_error()
    assert L.rq_dequant(None, None, None, None) == _lib.RQ_ERR_HANDLE
    info = C.c_int()
    assert L.rq_weight_info(bogus, C.byref(info), None, None, None, None) == _lib.RQ_ERR_HANDLE
    assert L.rq_ctx_set_kernel_timing(bogus, 1) == _lib.RQ_ERR_HANDLE
    ms, n = C.c_double(), C.c_int64()
    assert L.rq_ctx_kernel_time(bogus, C.byref(ms), C.byref(n)) == _lib.RQ_ERR_HANDLE


def test_ctx_create_null_out():
    assert _lib.lib().rq_ctx_create(0, None) == _lib.RQ_ERR_NULL


@pytest.mark.skipif(os.environ.get("RQ_EXPECT_GPU") == "1", reason="GPU present")
def test_ctx_create_without_gpu_reports_device_error():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    h = C.c_void_p()
    assert _lib.lib().rq_ctx_create(0, C.byref(h)) == _lib.RQ_ERR_DEVICE
    assert not h.value


def test_nextpad_through_the_abi():
    # test/raster/quant/pack_test.clj:14-18, host-side only (no device work)
    L = _lib.lib()
    v = C.c_int64()
    got = []
    for i in (1, 256, 257, 640):
        assert L.rq_nextpad(i, C.byref(v)) == _lib.RQ_OK
        got.append(v.value)
    assert got == [256, 256, 512, 768]
    assert L.rq_nextpad(0, C.byref(v)) == _lib.RQ_ERR_SHAPE
    assert L.rq_nextpad(5, None) == _lib.RQ_ERR_NULL
