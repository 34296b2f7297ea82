"""Host-side mirror of Raster's quantized-matmul call surface over librq.

Names, argument order and result shapes follow the reference functions
(paths inside replikativ/raster):

  qlinear_q8(x, codes, scales, m, in_, out) -> y[m*out]   raster/quant/train.clj:77-108
  qlinear_q8_dx(dy, codes, scales, m, in_, out) -> dx[m*in]  raster/quant/train.clj:110-137
  dequant_q8_dense(codes, scales, in_, out) -> W[out*in]  raster/quant/train.clj:60-71

plus the resident-weight object the GPU path needs (`QWeight`, the :constant
weights of raster/gpu/core.clj:889-940) and a per-device `Context`
(make-session, raster/gpu/core.clj:243-257). Every compute call goes through the
C ABI of include/rq.h; there is no CPU fallback. Device arrays are torch CUDA
tensors (plumbing only: memory and streams), host arrays are numpy.
"""
from __future__ import annotations

import ctypes as C
import threading

import numpy as np

from . import _lib
from ._lib import RQ_BF16, RQ_F16, RQ_F32, RQ_Q4_0, RQ_Q4_K, RQ_Q6_K, RQ_Q8_0, RqError, call, lib

__all__ = [
    "Context", "QWeight", "RqError", "context", "decode_attention", "quantize_act_i8", "quantize_act_q8k",
    "qlinear_q8", "qlinear_q8_dx", "dequant_q8_dense", "qlinear_i8", "qlinear_i8_q8", "nextpad", "q8_quantize",
    "q4k_of", "quantize_weight_q6k",
    "RQ_F32", "RQ_BF16", "RQ_F16", "RQ_Q8_0", "RQ_Q4_0",
]


def _np_ptr(a: np.ndarray):
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("host arrays must be C-contiguous")
    return a.ctypes.data_as(C.c_void_p)


class Context:
    """A librq context bound to one HIP device (raster/gpu/core.clj:243-293)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        call("rq_ctx_create", device, C.byref(h))
        self.handle = h
        self.device = device

    def device_info(self) -> dict:
        cu, ws, clk = C.c_int(), C.c_int(), C.c_int()
        call("rq_ctx_device_info", self.handle, C.byref(cu), C.byref(ws), C.byref(clk))
        return {"cu_count": cu.value, "wave_size": ws.value, "clock_khz": clk.value}

    def sync(self, stream=None) -> None:
        call("rq_sync", self.handle, _stream_ptr(stream))

    def set_kernel_timing(self, enable: bool) -> None:
        """Capture the dispatch timestamps of the main kernel of every matmul call."""
        call("rq_ctx_set_kernel_timing", self.handle, 1 if enable else 0)

    def kernel_time(self) -> tuple[float, int]:
        """(summed main-kernel milliseconds, launches) since the last read."""
        ms, n = C.c_double(), C.c_int64()
        call("rq_ctx_kernel_time", self.handle, C.byref(ms), C.byref(n))
        return ms.value, n.value

    def close(self) -> None:
        if self.handle:
            call("rq_ctx_destroy", self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


_ctx_lock = threading.Lock()
_contexts: dict[int, Context] = {}


def context(device: int = 0) -> Context:
    """Process-wide default context per device."""
    with _ctx_lock:
        c = _contexts.get(device)
        if c is None or c.handle is None:
            c = Context(device)
            _contexts[device] = c
        return c


def _stream_ptr(stream):
    if stream is None:
        return None
    if isinstance(stream, int):
        return C.c_void_p(stream)
    return C.c_void_p(stream.cuda_stream)  # torch.cuda.Stream


def _dtype_code(t) -> int:
    import torch

    if t.dtype == torch.float32:
        return RQ_F32
    if t.dtype == torch.bfloat16:
        return RQ_BF16
    raise TypeError(f"activations/outputs must be float32 or bfloat16, got {t.dtype}")


class QWeight:
    """A resident block-quantized weight [out x in] in HBM (one scale per 32 of `in`)."""

    def __init__(self, ctx: Context, handle: C.c_void_p):
        self.ctx = ctx
        self.handle = handle
        fmt, out, in_, sdt, nbytes = C.c_int(), C.c_int64(), C.c_int64(), C.c_int(), C.c_size_t()
        call("rq_weight_info", handle, C.byref(fmt), C.byref(out), C.byref(in_), C.byref(sdt), C.byref(nbytes))
        self.format, self.out, self.in_ = fmt.value, out.value, in_.value
        self.scale_dtype, self.device_bytes = sdt.value, nbytes.value

    # ---- constructors -------------------------------------------------------
    @classmethod
    def q8(cls, codes, scales, out: int, in_: int, ctx: Context | None = None) -> "QWeight":
        """From qlinear-q8's arrays: int8 codes[out*in], f32 scales[out*in/32]."""
        ctx = ctx or context()
        codes = np.ascontiguousarray(codes, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        _need(codes.size == out * in_ and scales.size == out * (in_ // 32), "array sizes do not match out x in")
        h = C.c_void_p()
        call("rq_weight_create_q8", ctx.handle, _np_ptr(codes), _np_ptr(scales), out, in_, C.byref(h))
        return cls(ctx, h)

    @classmethod
    def q8_packed(cls, wp, ws, out: int, in_: int, ctx: Context | None = None) -> "QWeight":
        """From quantize-one-q8's int32-packed words (raster/quant/pack.clj:55-81)."""
        ctx = ctx or context()
        wp = np.ascontiguousarray(wp, np.int32)
        ws = np.ascontiguousarray(ws, np.float32)
        _need(wp.size == out * in_ // 4 and ws.size == out * (in_ // 32), "array sizes do not match out x in")
        h = C.c_void_p()
        call("rq_weight_create_q8_packed", ctx.handle, _np_ptr(wp), _np_ptr(ws), out, in_, C.byref(h))
        return cls(ctx, h)

    @classmethod
    def q4(cls, packed, scales, out: int, in_: int, ctx: Context | None = None) -> "QWeight":
        """Row-major Q4_0: packed u8[out*in/2]; scales f32 or fp16 (np.float16 / uint16 bits)."""
        ctx = ctx or context()
        packed = np.ascontiguousarray(packed, np.uint8)
        scales = np.asarray(scales)
        if scales.dtype in (np.float16, np.uint16):
            scales, sdt = np.ascontiguousarray(scales).view(np.uint16), RQ_F16
        else:
            scales, sdt = np.ascontiguousarray(scales, np.float32), RQ_F32
        _need(packed.size == out * in_ // 2 and scales.size == out * (in_ // 32), "array sizes do not match out x in")
        h = C.c_void_p()
        call("rq_weight_create_q4", ctx.handle, _np_ptr(packed), _np_ptr(scales), sdt, out, in_, C.byref(h))
        return cls(ctx, h)

    @classmethod
    def q4k(cls, wq, da, db, aq, bq, out: int, in_: int, ctx: Context | None = None) -> "QWeight":
        """Q4_K from quantize-weight-q4k's arrays (in % 256 == 0): wq u8[out*in/2],
        da / db f32[out*in/256], aq u8[out*in/32], bq i8[out*in/32]."""
        ctx = ctx or context()
        wq, aq = np.ascontiguousarray(wq, np.uint8), np.ascontiguousarray(aq, np.uint8)
        da, db = np.ascontiguousarray(da, np.float32), np.ascontiguousarray(db, np.float32)
        bq = np.ascontiguousarray(bq, np.int8)
        _need(wq.size == out * in_ // 2 and da.size == db.size == out * (in_ // 256)
              and aq.size == bq.size == out * (in_ // 32), "array sizes do not match out x in")
        h = C.c_void_p()
        call("rq_weight_create_q4k", ctx.handle, _np_ptr(wq), _np_ptr(da), _np_ptr(db), _np_ptr(aq), _np_ptr(bq),
             out, in_, C.byref(h))
        return cls(ctx, h)

    @classmethod
    def q6k(cls, wq, sc, ds, out: int, in_: int, ctx: Context | None = None) -> "QWeight":
        """Q6_K from quantize-weight-q6k's arrays: wq u8[out*in], sc i8[out*in/16], ds f32[out*in/256]."""
        ctx = ctx or context()
        wq, sc = np.ascontiguousarray(wq, np.uint8), np.ascontiguousarray(sc, np.int8)
        ds = np.ascontiguousarray(ds, np.float32)
        _need(wq.size == out * in_ and sc.size == out * (in_ // 16) and ds.size == out * (in_ // 256),
              "array sizes do not match out x in")
        h = C.c_void_p()
        call("rq_weight_create_q6k", ctx.handle, _np_ptr(wq), _np_ptr(sc), _np_ptr(ds), out, in_, C.byref(h))
        return cls(ctx, h)

    @classmethod
    def x8(cls, wqi, wsi, nibble: bool, out: int, in_: int, ctx: Context | None = None) -> "QWeight":
        """From the repack-stream x8 layout of raster/compiler/core/layout.clj:246-286."""
        ctx = ctx or context()
        wqi = np.ascontiguousarray(wqi).view(np.uint8)
        wsi = np.ascontiguousarray(wsi, np.float32)
        h = C.c_void_p()
        call("rq_weight_create_x8", ctx.handle, _np_ptr(wqi), _np_ptr(wsi), int(bool(nibble)), out, in_, C.byref(h))
        return cls(ctx, h)

    # ---- compute --------------------------------------------------------------
    def matmul(self, x, y=None, out_dtype=None, stream=None):
        """y[m, out] = x[m, in] . dequant(W)^T on the device (x: torch f32/bf16 CUDA tensor).
        K-quant weights (Q4_K, Q6_K) take f32 x, quantized to q8_K inside the
        call: the same bits as quantize_act_q8k + matmul_q8k."""
        import torch

        _need(x.is_cuda and x.is_contiguous(), "x must be a contiguous CUDA tensor")
        _need(x.numel() % self.in_ == 0, "x.numel() must be a multiple of in")
        m = x.numel() // self.in_
        if y is None:
            y = torch.empty((m, self.out), dtype=out_dtype or torch.float32, device=x.device)
        _need(y.is_cuda and y.is_contiguous() and y.numel() == m * self.out, "y must be a contiguous [m, out] CUDA tensor")
        if stream is None:
            stream = torch.cuda.current_stream(x.device)
        call("rq_qmatmul", self.ctx.handle, self.handle, C.c_void_p(x.data_ptr()), _dtype_code(x),
             C.c_void_p(y.data_ptr()), _dtype_code(y), m, _stream_ptr(stream))
        return y

    def matmul_fused(self, x, y=None, out_dtype=None, norm_gain=None, norm_eps: float = 0.0, residual=None,
                     swiglu: bool = False, act_i8: bool = False, stream=None):
        """rq_qmatmul_fused (m <= 16): the decode matmul with an optional
        RMSNorm of x's rows (norm_gain f32[in]) before it, and either a SwiGLU
        of row pairs (rows 2i / 2i+1 = gate / up; y is [m, out/2]) or a
        residual add (residual [m, out], y's dtype) after it. act_i8 quantizes
        the activations to Raster's int8 blocks in the kernel."""
        import torch

        _need(x.is_cuda and x.is_contiguous(), "x must be a contiguous CUDA tensor")
        _need(x.numel() % self.in_ == 0, "x.numel() must be a multiple of in")
        m = x.numel() // self.in_
        ny = self.out // 2 if swiglu else self.out
        if y is None:
            y = torch.empty((m, ny), dtype=out_dtype or torch.float32, device=x.device)
        _need(y.is_cuda and y.is_contiguous() and y.numel() == m * ny, "y must be a contiguous CUDA tensor of m rows")
        ops = _lib.FusedOps(None, float(norm_eps), None, 1 if swiglu else 0, 1 if act_i8 else 0)
        if norm_gain is not None:
            _need(norm_gain.is_cuda and norm_gain.dtype == torch.float32 and norm_gain.is_contiguous()
                  and norm_gain.numel() == self.in_, "norm_gain must be a contiguous f32 CUDA tensor of in elements")
            ops.norm_gain = norm_gain.data_ptr()
        if residual is not None:
            _need(residual.is_cuda and residual.is_contiguous() and residual.dtype == y.dtype
                  and residual.numel() == m * ny, "residual must match y")
            ops.residual = residual.data_ptr()
        if stream is None:
            stream = torch.cuda.current_stream(x.device)
        call("rq_qmatmul_fused", self.ctx.handle, self.handle, C.c_void_p(x.data_ptr()), _dtype_code(x),
             C.c_void_p(y.data_ptr()), _dtype_code(y), m, C.byref(ops), _stream_ptr(stream))
        return y

    def matmul_i8(self, xq, xs, xsum=None, y=None, out_dtype=None, stream=None):
        """rq_qmatmul_i8: y[m, out] from int8 activations (xq int8 [m, in],
        xs f32 [m, in/32], xsum int32 [m, in/32], needed for Q4_0), as
        produced by quantize_act_i8."""
        import torch

        _need(xq.is_cuda and xq.is_contiguous() and xq.dtype == torch.int8, "xq must be a contiguous int8 CUDA tensor")
        _need(xq.numel() % self.in_ == 0, "xq.numel() must be a multiple of in")
        m = xq.numel() // self.in_
        _need(xs.is_cuda and xs.is_contiguous() and xs.dtype == torch.float32 and xs.numel() == m * (self.in_ // 32),
              "xs must be a contiguous f32 CUDA tensor of m*in/32 elements")
        if xsum is not None:
            _need(xsum.is_cuda and xsum.is_contiguous() and xsum.dtype == torch.int32 and xsum.numel() == xs.numel(),
                  "xsum must be a contiguous int32 CUDA tensor like xs")
        if y is None:
            y = torch.empty((m, self.out), dtype=out_dtype or torch.float32, device=xq.device)
        _need(y.is_cuda and y.is_contiguous() and y.numel() == m * self.out, "y must be a contiguous [m, out] CUDA tensor")
        if stream is None:
            stream = torch.cuda.current_stream(xq.device)
        call("rq_qmatmul_i8", self.ctx.handle, self.handle, C.c_void_p(xq.data_ptr()), C.c_void_p(xs.data_ptr()),
             C.c_void_p(xsum.data_ptr() if xsum is not None else None), C.c_void_p(y.data_ptr()), _dtype_code(y), m,
             _stream_ptr(stream))
        return y

    def matmul_q8k(self, xq, xs, bsums, y=None, out_dtype=None, stream=None):
        """rq_qmatmul_q8k: y[m, out] for a K-quant weight from q8_K activations
        (xq int8 [m, in], xs f32 [m, in/256], bsums int32 [m, in/sub])."""
        import torch

        _need(self.format in (_lib.RQ_Q4_K, _lib.RQ_Q6_K), "matmul_q8k needs a Q4_K or Q6_K weight")
        sub = 32 if self.format == _lib.RQ_Q4_K else 16
        _need(xq.is_cuda and xq.is_contiguous() and xq.dtype == torch.int8 and xq.numel() % self.in_ == 0,
              "xq must be a contiguous int8 CUDA tensor of m*in elements")
        m = xq.numel() // self.in_
        _need(xs.is_cuda and xs.is_contiguous() and xs.dtype == torch.float32 and xs.numel() == m * (self.in_ // 256),
              "xs must be a contiguous f32 CUDA tensor of m*in/256 elements")
        _need(bsums.is_cuda and bsums.is_contiguous() and bsums.dtype == torch.int32
              and bsums.numel() == m * (self.in_ // sub), f"bsums must be int32 [m, in/{sub}]")
        if y is None:
            y = torch.empty((m, self.out), dtype=out_dtype or torch.float32, device=xq.device)
        _need(y.is_cuda and y.is_contiguous() and y.numel() == m * self.out, "y must be a contiguous [m, out] CUDA tensor")
        if stream is None:
            stream = torch.cuda.current_stream(xq.device)
        call("rq_qmatmul_q8k", self.ctx.handle, self.handle, C.c_void_p(xq.data_ptr()), C.c_void_p(xs.data_ptr()),
             C.c_void_p(bsums.data_ptr()), C.c_void_p(y.data_ptr()), _dtype_code(y), m, _stream_ptr(stream))
        return y

    def matmul_dx(self, dy, dx=None, stream=None):
        """rq_qmatmul_dx (qlinear-q8-dx): dx[m, in] = dy[m, out] . dequant(W), f32."""
        import torch

        _need(dy.is_cuda and dy.is_contiguous() and dy.dtype == torch.float32 and dy.numel() % self.out == 0,
              "dy must be a contiguous f32 CUDA tensor of m*out elements")
        m = dy.numel() // self.out
        if dx is None:
            dx = torch.empty((m, self.in_), dtype=torch.float32, device=dy.device)
        _need(dx.is_cuda and dx.is_contiguous() and dx.dtype == torch.float32 and dx.numel() == m * self.in_,
              "dx must be a contiguous f32 [m, in] CUDA tensor")
        if stream is None:
            stream = torch.cuda.current_stream(dy.device)
        call("rq_qmatmul_dx", self.ctx.handle, self.handle, C.c_void_p(dy.data_ptr()), C.c_void_p(dx.data_ptr()), m,
             _stream_ptr(stream))
        return dx

    def dequant(self, stream=None):
        """Dequantized f32 W[out, in] computed on the device."""
        import torch

        w = torch.empty((self.out, self.in_), dtype=torch.float32, device=f"cuda:{self.ctx.device}")
        if stream is None:
            stream = torch.cuda.current_stream(w.device)
        call("rq_dequant", self.ctx.handle, self.handle, C.c_void_p(w.data_ptr()), _stream_ptr(stream))
        return w

    def device_ptrs(self):
        q, s = C.c_void_p(), C.c_void_p()
        call("rq_weight_device_ptrs", self.handle, C.byref(q), C.byref(s))
        return q.value, s.value

    def destroy(self) -> None:
        if self.handle:
            call("rq_weight_destroy", self.handle)
            self.handle = None


def quantize_act_i8(ctx: Context, x, in_: int, out=None, stream=None):
    """rq_quantize_act_i8 (quantize-act-i8): x f32 [m*in] on the device ->
    (xq int8 [m, in], xs f32 [m, in/32], xsum int32 [m, in/32]), written into
    `out` when given."""
    import torch

    _need(x.is_cuda and x.is_contiguous() and x.dtype == torch.float32, "x must be a contiguous f32 CUDA tensor")
    _need(in_ % 32 == 0 and x.numel() % in_ == 0, "x.numel() must be a multiple of in, in a multiple of 32")
    m = x.numel() // in_
    if out is None:
        xq = torch.empty((m, in_), dtype=torch.int8, device=x.device)
        xs = torch.empty((m, in_ // 32), dtype=torch.float32, device=x.device)
        xsum = torch.empty((m, in_ // 32), dtype=torch.int32, device=x.device)
    else:
        xq, xs, xsum = out
        _need(xq.numel() == m * in_ and xs.numel() == m * (in_ // 32) and xsum.numel() == xs.numel()
              and xq.dtype == torch.int8 and xs.dtype == torch.float32 and xsum.dtype == torch.int32
              and all(t.is_cuda and t.is_contiguous() for t in (xq, xs, xsum)), "out tensors do not match x")
    if stream is None:
        stream = torch.cuda.current_stream(x.device)
    call("rq_quantize_act_i8", ctx.handle, C.c_void_p(x.data_ptr()), m, in_, C.c_void_p(xq.data_ptr()),
         C.c_void_p(xs.data_ptr()), C.c_void_p(xsum.data_ptr()), _stream_ptr(stream))
    return xq, xs, xsum


def quantize_act_q8k(ctx: Context, x, in_: int, sub: int, out=None, stream=None):
    """rq_quantize_act_q8k (quantize-act-q8k): x f32 [m*in] on the device ->
    (xq int8 [m, in], xs f32 [m, in/256], bsums int32 [m, in/sub]); sub 32 for
    Q4_K, 16 for Q6_K."""
    import torch

    _need(x.is_cuda and x.is_contiguous() and x.dtype == torch.float32, "x must be a contiguous f32 CUDA tensor")
    _need(in_ % 256 == 0 and x.numel() % in_ == 0 and sub in (16, 32), "in % 256 == 0, sub 16 or 32")
    m = x.numel() // in_
    if out is None:
        out = (torch.empty((m, in_), dtype=torch.int8, device=x.device),
               torch.empty((m, in_ // 256), dtype=torch.float32, device=x.device),
               torch.empty((m, in_ // sub), dtype=torch.int32, device=x.device))
    xq, xs, bsums = out
    if stream is None:
        stream = torch.cuda.current_stream(x.device)
    call("rq_quantize_act_q8k", ctx.handle, C.c_void_p(x.data_ptr()), m, in_, sub, C.c_void_p(xq.data_ptr()),
         C.c_void_p(xs.data_ptr()), C.c_void_p(bsums.data_ptr()), _stream_ptr(stream))
    return xq, xs, bsums


def i8gemv_dp4a(ctx: Context, wp, xp, kw: int, out: int, y=None, stream=None):
    """rq_i8gemv_dp4a (i8gemv-dp4a!, raster/quant/kernels_k.clj:141-150):
    y[o] = (float) sum_w dp4a(wp[o*kw + w], xp[w]); wp int32 [out*kw], xp int32
    [kw] CUDA tensors (four little-endian int8 lanes per word) -> y f32 [out]."""
    import torch

    _need(wp.is_cuda and xp.is_cuda and wp.dtype == torch.int32 and xp.dtype == torch.int32,
          "wp and xp must be int32 CUDA tensors")
    _need(wp.is_contiguous() and xp.is_contiguous() and wp.numel() == out * kw and xp.numel() == kw,
          "wp must hold out*kw words and xp kw words, contiguous")
    if y is None:
        y = torch.empty(out, dtype=torch.float32, device=wp.device)
    if stream is None:
        stream = torch.cuda.current_stream(wp.device)
    call("rq_i8gemv_dp4a", ctx.handle, C.c_void_p(wp.data_ptr()), C.c_void_p(xp.data_ptr()),
         C.c_void_p(y.data_ptr()), kw, out, _stream_ptr(stream))
    return y


def decode_attention(ctx: Context, q, k, v, kcache, vcache, pos: int, n_q: int, n_kv: int, head_dim: int,
                     theta: float, scale: float, out=None, stream=None):
    """rq_decode_attention: RoPE of q [n_q*head_dim] and k [n_kv*head_dim] at
    `pos`, append of the rotated k and of v to row pos of kcache / vcache
    ([rows, n_kv*head_dim] f32), and single-query attention over rows 0..pos.
    Returns out [n_q*head_dim] f32."""
    import torch

    kvd = n_kv * head_dim
    for t, n in ((q, n_q * head_dim), (k, kvd), (v, kvd)):
        _need(t.is_cuda and t.is_contiguous() and t.dtype == torch.float32 and t.numel() == n,
              "q, k, v must be contiguous f32 CUDA tensors of n_q*head_dim / n_kv*head_dim elements")
    for t in (kcache, vcache):
        _need(t.is_cuda and t.is_contiguous() and t.dtype == torch.float32 and t.numel() >= (pos + 1) * kvd,
              "kcache / vcache must be contiguous f32 CUDA tensors of at least pos+1 rows")
    if out is None:
        out = torch.empty(n_q * head_dim, dtype=torch.float32, device=q.device)
    _need(out.is_cuda and out.is_contiguous() and out.dtype == torch.float32 and out.numel() == n_q * head_dim,
          "out must be a contiguous f32 CUDA tensor of n_q*head_dim elements")
    if stream is None:
        stream = torch.cuda.current_stream(q.device)
    ptr = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
    call("rq_decode_attention", ctx.handle, ptr(q), ptr(k), ptr(v), ptr(kcache), ptr(vcache), pos, n_q, n_kv,
         head_dim, float(theta), float(scale), ptr(out), _stream_ptr(stream))
    return out


def nextpad(in_: int) -> int:
    """raster.quant.pack/nextpad: `in` rounded up to a multiple of 256 (rq_nextpad)."""
    v = C.c_int64()
    call("rq_nextpad", int(in_), C.byref(v))
    return v.value


def q8_quantize(ctx: Context, W, out: int, in_: int, stream=None):
    """raster.quant.train/q8-quantize on the device (rq_q8_quantize): W f32
    [out*in] CUDA tensor -> (codes int8 [out, in], scales f32 [out, in/32])."""
    import torch

    _need(W.is_cuda and W.is_contiguous() and W.dtype == torch.float32 and W.numel() == out * in_,
          "W must be a contiguous f32 CUDA tensor of out*in elements")
    codes = torch.empty((out, in_), dtype=torch.int8, device=W.device)
    scales = torch.empty((out, in_ // 32), dtype=torch.float32, device=W.device)
    if stream is None:
        stream = torch.cuda.current_stream(W.device)
    call("rq_q8_quantize", ctx.handle, C.c_void_p(W.data_ptr()), out, in_, C.c_void_p(codes.data_ptr()),
         C.c_void_p(scales.data_ptr()), _stream_ptr(stream))
    return codes, scales


def q4k_of(ctx: Context, W, out: int, in_: int, stream=None):
    """raster.quant.pack/q4k-of on the device (rq_q4k_of): W f32 [out*in] CUDA
    tensor, rows zero-padded to inp = nextpad(in) -> dict(wq, da, db, aq, bq,
    in=inp, out=out) of CUDA tensors, the arrays QWeight.q4k takes."""
    import torch

    _need(W.is_cuda and W.is_contiguous() and W.dtype == torch.float32 and W.numel() == out * in_,
          "W must be a contiguous f32 CUDA tensor of out*in elements")
    inp = nextpad(in_)
    n = out * inp
    dev = W.device
    wq = torch.empty(n // 2, dtype=torch.uint8, device=dev)
    da, db = torch.empty(n // 256, device=dev), torch.empty(n // 256, device=dev)
    aq, bq = torch.empty(n // 32, dtype=torch.uint8, device=dev), torch.empty(n // 32, dtype=torch.int8, device=dev)
    got = C.c_int64()
    if stream is None:
        stream = torch.cuda.current_stream(dev)
    ptr = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
    call("rq_q4k_of", ctx.handle, ptr(W), out, in_, ptr(wq), ptr(da), ptr(db), ptr(aq), ptr(bq), C.byref(got),
         _stream_ptr(stream))
    return {"wq": wq, "da": da, "db": db, "aq": aq, "bq": bq, "in": got.value, "out": out}


def quantize_weight_q6k(ctx: Context, W, out: int, in_: int, stream=None):
    """quantize-weight-q6k on the device (rq_quantize_weight_q6k), in % 256 == 0:
    W f32 [out*in] CUDA tensor -> (wq u8 [out*in], sc i8 [out*in/16], ds f32 [out*in/256])."""
    import torch

    _need(W.is_cuda and W.is_contiguous() and W.dtype == torch.float32 and W.numel() == out * in_,
          "W must be a contiguous f32 CUDA tensor of out*in elements")
    dev = W.device
    wq = torch.empty(out * in_, dtype=torch.uint8, device=dev)
    sc = torch.empty(out * in_ // 16, dtype=torch.int8, device=dev)
    ds = torch.empty(out * in_ // 256, dtype=torch.float32, device=dev)
    if stream is None:
        stream = torch.cuda.current_stream(dev)
    call("rq_quantize_weight_q6k", ctx.handle, C.c_void_p(W.data_ptr()), out, in_, C.c_void_p(wq.data_ptr()),
         C.c_void_p(sc.data_ptr()), C.c_void_p(ds.data_ptr()), _stream_ptr(stream))
    return wq, sc, ds


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


# ---- Raster-named host-array entry points -------------------------------------

def qlinear_q8(x, codes, scales, m: int, in_: int, out: int, ctx: Context | None = None) -> np.ndarray:
    """raster.quant.train/qlinear-q8: y[m*out] = x[m*in] . dequant(codes, scales)^T, on the GPU."""
    ctx = ctx or context()
    x = np.ascontiguousarray(x, np.float32)
    codes = np.ascontiguousarray(codes, np.int8)
    scales = np.ascontiguousarray(scales, np.float32)
    if in_ % 32 != 0:
        raise AssertionError(f"in={in_} not a multiple of 32")
    _need(x.size == m * in_ and codes.size == out * in_ and scales.size == out * (in_ // 32), "array sizes")
    y = np.empty(m * out, np.float32)
    call("rq_qlinear_q8", ctx.handle, _np_ptr(x), _np_ptr(codes), _np_ptr(scales), m, in_, out, _np_ptr(y))
    return y


def qlinear_q8_dx(dy, codes, scales, m: int, in_: int, out: int, ctx: Context | None = None) -> np.ndarray:
    """raster.quant.train/qlinear-q8-dx: dx[m*in] = dy[m*out] . dequant(codes, scales), on the GPU."""
    ctx = ctx or context()
    dy = np.ascontiguousarray(dy, np.float32)
    codes, scales = np.ascontiguousarray(codes, np.int8), np.ascontiguousarray(scales, np.float32)
    _need(dy.size == m * out and codes.size == out * in_ and scales.size == out * (in_ // 32),
          "array sizes do not match m, in, out")
    dx = np.empty(m * in_, np.float32)
    call("rq_qlinear_q8_dx", ctx.handle, _np_ptr(dy), _np_ptr(codes), _np_ptr(scales), m, in_, out, _np_ptr(dx))
    return dx


def dequant_q8_dense(codes, scales, in_: int, out: int, ctx: Context | None = None) -> np.ndarray:
    """raster.quant.train/dequant-q8-dense, decoded on the GPU: f32 W[out*in]."""
    w = QWeight.q8(codes, scales, out, in_, ctx)
    try:
        import torch

        return w.dequant().cpu().numpy().ravel()
    finally:
        w.destroy()


def qlinear_i8(x, wqi, wsi, y, in_: int, out: int, ctx: Context | None = None, nibble: bool = True) -> np.ndarray:
    """raster.quant.op/qlinear-i8! (x wqi wsi y in out): y[out] = the int8
    linear of x[in] over an x8 repack-stream weight, y overwritten and returned.
    nibble=False is qlinear-i8-q8! (the zero-point-128 Q8 layout)."""
    ctx = ctx or context()
    x = np.ascontiguousarray(x, np.float32)
    wqi = np.ascontiguousarray(wqi).view(np.uint8)
    wsi = np.ascontiguousarray(wsi, np.float32)
    _need(isinstance(y, np.ndarray) and y.dtype == np.float32 and y.flags["C_CONTIGUOUS"] and y.size == out,
          "y must be a contiguous float32 array of out elements")
    _need(x.size == in_ and wsi.size == (out // 8) * (in_ // 32) * 8
          and wqi.size == (out // 8) * (in_ // 32) * (128 if nibble else 256), "array sizes do not match in, out")
    call("rq_qlinear_i8", ctx.handle, _np_ptr(x), _np_ptr(wqi), _np_ptr(wsi), 1 if nibble else 0, _np_ptr(y), in_, out)
    return y


def qlinear_i8_q8(x, wqi, wsi, y, in_: int, out: int, ctx: Context | None = None) -> np.ndarray:
    """raster.quant.op/qlinear-i8-q8!: qlinear_i8 over the Q8 x8 layout."""
    return qlinear_i8(x, wqi, wsi, y, in_, out, ctx, nibble=False)
