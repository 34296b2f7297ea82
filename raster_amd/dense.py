"""Host-side mirror of Raster's dense f32 GEMM surface over librq.

Names, argument order and result shapes follow the reference functions
(paths inside replikativ/raster); every array is a flat row-major f32 CUDA
tensor (torch is plumbing here: device memory and streams):

  dgemm(A, B, C, m, k, n, alpha, beta) -> C     dgemm!    raster/linalg/blas.clj:287-302
  dgemm_tn(A, B, C, m, k, n, alpha, beta) -> C  dgemm-tn! blas.clj:304-319 (A is [k*m])
  dgemm_nt(A, B, C, m, k, n, alpha, beta) -> C  dgemm-nt! blas.clj:321-337 (B is [n*k])
  matmul(A, B, m, k, n) -> C[m*n]               raster/dl/nn.clj:61-66
  matmul_(A, B, out, m, k, n) -> out            matmul!, nn.clj:69-73
  linear(x, W, b, batch, in_f, out_f) -> y      nn.clj:161-173
  linear_(x, W, b, y, batch, in_f, out_f) -> y  linear!, nn.clj:176-183

The dgemm arms write C in place and return it, as the reference's `!` ops
do. Every call goes through the C ABI (rq_sgemm, rq_sgemm_tn, rq_sgemm_nt,
rq_linear); there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C

from ._lib import call
from .quant import Context, _need, _stream_ptr, context

__all__ = ["dgemm", "dgemm_tn", "dgemm_nt", "matmul", "matmul_", "linear", "linear_"]


def _f32(t, n: int, what: str) -> None:
    import torch

    _need(t.is_cuda and t.is_contiguous() and t.dtype == torch.float32 and t.numel() >= n,
          f"{what} must be a contiguous f32 CUDA tensor of at least {n} elements")


def _gemm(entry: str, A, B, Cm, m: int, k: int, n: int, alpha: float, beta: float, ctx: Context | None, stream):
    import torch

    if m > 0 and n > 0 and k > 0:
        _f32(A, m * k, "A")
        _f32(B, k * n, "B")
        _f32(Cm, m * n, "C")
    ctx = ctx or context(Cm.device.index or 0)
    if stream is None:
        stream = torch.cuda.current_stream(Cm.device)
    call(entry, ctx.handle, C.c_void_p(A.data_ptr()), C.c_void_p(B.data_ptr()), C.c_void_p(Cm.data_ptr()), m, k, n,
         float(alpha), float(beta), _stream_ptr(stream))
    return Cm


def dgemm(A, B, Cm, m: int, k: int, n: int, alpha: float = 1.0, beta: float = 0.0, ctx: Context | None = None,
          stream=None):
    """C[m*n] = alpha A[m*k] B[k*n] + beta C (dgemm!, float arm)."""
    return _gemm("rq_sgemm", A, B, Cm, m, k, n, alpha, beta, ctx, stream)


def dgemm_tn(A, B, Cm, m: int, k: int, n: int, alpha: float = 1.0, beta: float = 0.0, ctx: Context | None = None,
             stream=None):
    """C[m*n] = alpha A^T B + beta C with A stored [k*m] (dgemm-tn!)."""
    return _gemm("rq_sgemm_tn", A, B, Cm, m, k, n, alpha, beta, ctx, stream)


def dgemm_nt(A, B, Cm, m: int, k: int, n: int, alpha: float = 1.0, beta: float = 0.0, ctx: Context | None = None,
             stream=None):
    """C[m*n] = alpha A B^T + beta C with B stored [n*k] (dgemm-nt!)."""
    return _gemm("rq_sgemm_nt", A, B, Cm, m, k, n, alpha, beta, ctx, stream)


def matmul(A, B, m: int, k: int, n: int, ctx: Context | None = None, stream=None):
    """C = A @ B, A [m*k], B [k*n] -> a new C [m*n] (nn/matmul)."""
    import torch

    out = torch.empty(max(m, 0) * max(n, 0), dtype=torch.float32, device=A.device)
    return matmul_(A, B, out, m, k, n, ctx, stream)


def matmul_(A, B, out, m: int, k: int, n: int, ctx: Context | None = None, stream=None):
    """matmul! into a pre-allocated out [m*n]."""
    return dgemm(A, B, out, m, k, n, 1.0, 0.0, ctx, stream)


def linear(x, W, b, batch: int, in_f: int, out_f: int, ctx: Context | None = None, stream=None):
    """y = x W^T + b, x [batch*in_f], W [out_f*in_f], b [out_f] -> a new y [batch*out_f] (nn/linear)."""
    import torch

    y = torch.empty(max(batch, 0) * max(out_f, 0), dtype=torch.float32, device=b.device)
    return linear_(x, W, b, y, batch, in_f, out_f, ctx, stream)


def linear_(x, W, b, y, batch: int, in_f: int, out_f: int, ctx: Context | None = None, stream=None):
    """linear! into a pre-allocated y [batch*out_f]: every row set to b, then y = x W^T + y."""
    import torch

    if batch > 0 and out_f > 0:
        _f32(b, out_f, "b")
        _f32(y, batch * out_f, "y")
        if in_f > 0:
            _f32(x, batch * in_f, "x")
            _f32(W, out_f * in_f, "W")
    ctx = ctx or context(y.device.index or 0)
    if stream is None:
        stream = torch.cuda.current_stream(y.device)
    ptr = lambda t: C.c_void_p(t.data_ptr()) if t is not None and t.numel() > 0 else None  # noqa: E731
    call("rq_linear", ctx.handle, ptr(x), ptr(W), ptr(b), ptr(y), batch, in_f, out_f, _stream_ptr(stream))
    return y
