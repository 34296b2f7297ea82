"""raster_amd — MI355X (gfx950) block-quantized matmul for Raster.

The product is librq.so (HIP kernels + the C ABI of include/rq.h); this package
holds its sources (csrc/), the build script and Python mirrors of Raster's
quantized-matmul call surface (quant.py) and of its dense f32 GEMM surface
(dense.py).
"""
from . import _lib, dense
from .quant import (RQ_BF16, RQ_F16, RQ_F32, RQ_Q4_0, RQ_Q8_0, Context, QWeight, RqError, context,
                    decode_attention, dequant_q8_dense, nextpad, q4k_of, q8_quantize, qlinear_i8, qlinear_i8_q8,
                    i8gemv_dp4a, qlinear_q8, qlinear_q8_dx, quantize_act_i8, quantize_act_q8k, quantize_weight_q6k)

__all__ = [
    "Context", "QWeight", "RqError", "context", "decode_attention", "quantize_act_i8", "quantize_act_q8k",
    "qlinear_q8", "qlinear_q8_dx", "dequant_q8_dense", "qlinear_i8", "qlinear_i8_q8", "nextpad", "q8_quantize",
    "q4k_of", "quantize_weight_q6k", "i8gemv_dp4a",
    "RQ_F32", "RQ_BF16", "RQ_F16", "RQ_Q8_0", "RQ_Q4_0",
]
