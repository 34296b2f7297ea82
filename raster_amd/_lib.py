"""ctypes binding of librq.so (include/rq.h).

This is the Python stand-in for the Panama FFM downcalls a JVM caller would
use: same symbols, same scalar/pointer arguments. There is no fallback: if the
library is missing or cannot load, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librq.so")

RQ_OK, RQ_ERR_SHAPE, RQ_ERR_DTYPE, RQ_ERR_NULL, RQ_ERR_OOM, RQ_ERR_HIP, RQ_ERR_HANDLE, RQ_ERR_DEVICE = range(8)
RQ_F32, RQ_BF16, RQ_F16 = 0, 1, 2
RQ_Q8_0, RQ_Q4_0, RQ_Q4_K, RQ_Q6_K = 0, 1, 2, 3

# every exported symbol of include/rq.h with (argtypes, restype)
_i, _i64, _p, _sz = C.c_int, C.c_int64, C.c_void_p, C.c_size_t
SIGNATURES = {
    "rq_version": ([], _i),
    "rq_status_string": ([_i], C.c_char_p),
    "rq_last_error": ([], C.c_char_p),
    "rq_ctx_create": ([_i, C.POINTER(_p)], _i),
    "rq_ctx_destroy": ([_p], _i),
    "rq_ctx_device_info": ([_p, C.POINTER(_i), C.POINTER(_i), C.POINTER(_i)], _i),
    "rq_ctx_set_kernel_timing": ([_p, _i], _i),
    "rq_ctx_kernel_time": ([_p, C.POINTER(C.c_double), C.POINTER(_i64)], _i),
    "rq_buf_alloc": ([_p, _sz, C.POINTER(_p)], _i),
    "rq_buf_free": ([_p, _p], _i),
    "rq_upload": ([_p, _p, _p, _sz, _p], _i),
    "rq_download": ([_p, _p, _p, _sz, _p], _i),
    "rq_stream_create": ([_p, C.POINTER(_p)], _i),
    "rq_stream_destroy": ([_p, _p], _i),
    "rq_sync": ([_p, _p], _i),
    "rq_weight_create_q8": ([_p, _p, _p, _i64, _i64, C.POINTER(_p)], _i),
    "rq_weight_create_q8_packed": ([_p, _p, _p, _i64, _i64, C.POINTER(_p)], _i),
    "rq_weight_create_q4": ([_p, _p, _p, _i, _i64, _i64, C.POINTER(_p)], _i),
    "rq_weight_create_x8": ([_p, _p, _p, _i, _i64, _i64, C.POINTER(_p)], _i),
    "rq_weight_create_q4k": ([_p, _p, _p, _p, _p, _p, _i64, _i64, C.POINTER(_p)], _i),
    "rq_weight_create_q6k": ([_p, _p, _p, _p, _i64, _i64, C.POINTER(_p)], _i),
    "rq_weight_destroy": ([_p], _i),
    "rq_weight_info": ([_p, C.POINTER(_i), C.POINTER(_i64), C.POINTER(_i64), C.POINTER(_i), C.POINTER(_sz)], _i),
    "rq_weight_device_ptrs": ([_p, C.POINTER(_p), C.POINTER(_p)], _i),
    "rq_qmatmul": ([_p, _p, _p, _i, _p, _i, _i64, _p], _i),
    "rq_qmatmul_fused": ([_p, _p, _p, _i, _p, _i, _i64, _p, _p], _i),
    "rq_qmatmul_noalloc": ([_p, _p, _p, _i, _p, _i, _i64, _p], _i),
    "rq_quantize_act_i8": ([_p, _p, _i64, _i64, _p, _p, _p, _p], _i),
    "rq_qmatmul_i8": ([_p, _p, _p, _p, _p, _p, _i, _i64, _p], _i),
    "rq_quantize_act_q8k": ([_p, _p, _i64, _i64, _i, _p, _p, _p, _p], _i),
    "rq_qmatmul_q8k": ([_p, _p, _p, _p, _p, _p, _i, _i64, _p], _i),
    "rq_i8gemv_dp4a": ([_p, _p, _p, _p, _i64, _i64, _p], _i),
    "rq_decode_attention": ([_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, C.c_double, C.c_double, _p, _p], _i),
    "rq_dequant": ([_p, _p, _p, _p], _i),
    "rq_qlinear_q8": ([_p, _p, _p, _p, _i64, _i64, _i64, _p], _i),
    "rq_qmatmul_dx": ([_p, _p, _p, _p, _i64, _p], _i),
    "rq_qlinear_q8_dx": ([_p, _p, _p, _p, _i64, _i64, _i64, _p], _i),
    "rq_nextpad": ([_i64, C.POINTER(_i64)], _i),
    "rq_q8_quantize": ([_p, _p, _i64, _i64, _p, _p, _p], _i),
    "rq_qlinear_i8": ([_p, _p, _p, _p, _i, _p, _i64, _i64], _i),
    "rq_q4k_of": ([_p, _p, _i64, _i64, _p, _p, _p, _p, _p, C.POINTER(_i64), _p], _i),
    "rq_quantize_weight_q6k": ([_p, _p, _i64, _i64, _p, _p, _p, _p], _i),
    "rq_stream_read": ([_p, _p, _sz, _i, _p, _p], _i),
    "rq_sgemm": ([_p, _p, _p, _p, _i64, _i64, _i64, C.c_float, C.c_float, _p], _i),
    "rq_sgemm_tn": ([_p, _p, _p, _p, _i64, _i64, _i64, C.c_float, C.c_float, _p], _i),
    "rq_sgemm_nt": ([_p, _p, _p, _p, _i64, _i64, _i64, C.c_float, C.c_float, _p], _i),
    "rq_linear": ([_p, _p, _p, _p, _p, _i64, _i64, _i64, _p], _i),
}


class FusedOps(C.Structure):
    """rq_fused_ops of include/rq.h."""

    _fields_ = [("norm_gain", _p), ("norm_eps", C.c_float), ("residual", _p), ("swiglu", _i), ("act_i8", _i)]


class RqError(RuntimeError):
    """A non-zero librq status (the ex-info of raster/gpu/ze_runtime.clj:281-291)."""

    def __init__(self, status: int, where: str, message: str):
        super().__init__(f"{where}: {message} (status {status})")
        self.status = status
        self.where = where


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m raster_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def check(status: int, where: str) -> None:
    if status != RQ_OK:
        msg = lib().rq_last_error()
        raise RqError(status, where, msg.decode() if msg else lib().rq_status_string(status).decode())


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
