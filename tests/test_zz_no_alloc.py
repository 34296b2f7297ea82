"""rq_qmatmul_noalloc, the rq_qmatmul variant that allocates nothing, against
rq_qmatmul itself through the C ABI: bit-identical outputs on every kernel
route that uses scratch (K-slice partial sums of the decode kernels, the packed
activations of the bf16 GEMMs, both for the small-m GEMM, a K-quant weight's
q8_K activations) and on routes that
use none, two calls in a row with the second one smaller, and a call that needs
more than the fixed scratch is refused with RQ_ERR_SHAPE. The seeded shapes
of the GPU sweep (every dispatch route) give the same bits through both
entries, or RQ_ERR_SHAPE where a call needs more than the fixed scratch.
"""
import ctypes as C

import numpy as np
import pytest
from sweep_shapes import SHAPES, WIDE_SHAPES

from raster_amd import _lib
from raster_amd import workloads as wl

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[gpu] {msg}", flush=True)


@pytest.fixture(scope="module")
def torch():
    import torch as t

    if not t.cuda.is_available():
        pytest.skip("no GPU")
    return t


@pytest.fixture(scope="module")
def ctx(torch):
    import raster_amd

    c = raster_amd.Context(0)
    yield c
    c.close()


def weight(raster_amd, ctx, fmt, out, in_, seed):
    if fmt in ("q4k", "q6k"):
        rng = np.random.default_rng(seed)
        W = (rng.standard_normal(out * in_) * 0.05).astype(np.float32)
        from oracle import oracle as orc

        arrs = orc.quantize_weight_q4k(W) if fmt == "q4k" else orc.quantize_weight_q6k(W)
        make = raster_amd.QWeight.q4k if fmt == "q4k" else raster_amd.QWeight.q6k
        return make(*arrs, out, in_, ctx)
    if fmt == "q8":
        codes, scales = wl.q8_weights(out, in_, seed=seed)
        return raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    packed, sc16 = wl.q4_weights(out, in_, seed=seed)
    return raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)


def both(torch, ctx, w, m, xdt, ydt, seed):
    """(rq_qmatmul y, rq_qmatmul_noalloc y) for the same seeded x."""
    x = torch.from_numpy(wl.activations(m, w.in_, seed=seed)).cuda().reshape(m, w.in_)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    ytype = torch.bfloat16 if ydt == "bf16" else torch.float32
    y_ref = torch.full((m, w.out), float("nan"), dtype=ytype, device="cuda")
    y_na = torch.full((m, w.out), float("nan"), dtype=ytype, device="cuda")
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    xc, yc = (_lib.RQ_BF16 if xdt == "bf16" else _lib.RQ_F32), (_lib.RQ_BF16 if ydt == "bf16" else _lib.RQ_F32)
    _lib.call("rq_qmatmul", ctx.handle, w.handle, C.c_void_p(x.data_ptr()), xc, C.c_void_p(y_ref.data_ptr()), yc, m, s)
    _lib.call("rq_qmatmul_noalloc", ctx.handle, w.handle, C.c_void_p(x.data_ptr()), xc, C.c_void_p(y_na.data_ptr()),
              yc, m, s)
    torch.cuda.synchronize()
    return y_ref.float().cpu().numpy(), y_na.float().cpu().numpy()


# (format, out, in, [m of the first call, m of the second, smaller call], x dtype, y dtype)
CASES = [
    ("q8", 4096, 4096, [1, 1], "f32", "f32"),            # int8-level decode, no scratch
    ("q4", 14336, 4096, [1, 1], "f32", "f32"),           # v_dot4 GEMV, no scratch
    ("q8", 48, 8192, [16, 9], "f32", "f32"),             # MFMA decode with K-slices
    ("q4", 14336, 4096, [16, 6], "f32", "f32"),          # MFMA decode, Q4_0, K-slices
    ("q8", 4160, 8192, [12, 3], "f32", "f32"),           # int8-level decode with K-split (above 32 Mi)
    ("q4", 8192, 8192, [64, 32], "bf16", "bf16"),        # small-m GEMM: packed x + K-slices
    ("q8", 28672, 8192, [32, 17], "bf16", "bf16"),       # small-m GEMM, Q8_0: packed x + K-slices
    ("q8", 11008, 4096, [512, 128], "bf16", "bf16"),     # prefill GEMM: packed x (role-split kernel, then 128-row tiles)
    ("q8", 11008, 4096, [1024, 512], "bf16", "bf16"),    # 256 x 192 one-wave GEMM, then the role-split kernel
    ("q8", 1000, 1024, [300, 17], "f32", "f32"),         # exact-f32 GEMM, no scratch
    ("q4k", 4096, 4096, [8, 1], "f32", "f32"),           # K-quant: q8_K activations in scratch
    ("q6k", 1024, 2048, [40, 3], "f32", "bf16"),         # K-quant, m above the decode range
]


@pytest.mark.parametrize("fmt,out,in_,ms,xdt,ydt", CASES)
def test_noalloc_equals_qmatmul(torch, ctx, fmt, out, in_, ms, xdt, ydt):
    import raster_amd

    w = weight(raster_amd, ctx, fmt, out, in_, seed=out + in_)
    try:
        for i, m in enumerate(ms):
            note(f"noalloc {fmt} {out}x{in_} m={m} x={xdt} y={ydt}")
            y_ref, y_na = both(torch, ctx, w, m, xdt, ydt, seed=100 * i + m)
            assert np.all(np.isfinite(y_ref))
            assert np.array_equal(y_ref.view(np.uint32), y_na.view(np.uint32)), (fmt, m)
    finally:
        w.destroy()


def test_noalloc_rejects_calls_beyond_its_scratch(torch, ctx):
    import raster_amd

    # bf16 x of 4096 x 8192: the packed activations alone are 64 MiB
    m, out, in_ = 4096, 64, 8192
    w = weight(raster_amd, ctx, "q8", out, in_, seed=3)
    try:
        x = torch.zeros((m, in_), dtype=torch.bfloat16, device="cuda")
        y = torch.zeros((m, out), dtype=torch.bfloat16, device="cuda")
        st = _lib.lib().rq_qmatmul_noalloc(ctx.handle, w.handle, C.c_void_p(x.data_ptr()), _lib.RQ_BF16,
                                           C.c_void_p(y.data_ptr()), _lib.RQ_BF16, m, None)
        assert st == _lib.RQ_ERR_SHAPE
        assert b"fixed scratch" in _lib.lib().rq_last_error()
        # and the same call through rq_qmatmul still works
        w.matmul(x, y)
        torch.cuda.synchronize()
    finally:
        w.destroy()


# the wide prefill shapes need at most 14 MB of packed activations: all within the fixed scratch
NA_SHAPES = SHAPES + WIDE_SHAPES


@pytest.mark.parametrize("i,m,in_,out,fmt,xdt,ydt", NA_SHAPES, ids=[f"s{s[0]}" for s in NA_SHAPES])
def test_noalloc_sweep(torch, ctx, i, m, in_, out, fmt, xdt, ydt):
    import raster_amd

    if fmt == "q8":
        codes, scales = wl.q8_weights(out, in_, seed=3000 + i)
        w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    else:
        packed, sc16 = wl.q4_weights(out, in_, seed=3000 + i)
        w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
    try:
        note(f"noalloc sweep {i}: {fmt} m={m} in={in_} out={out} x={xdt} y={ydt}")
        x = torch.from_numpy(wl.activations(m, in_, seed=4000 + i)).cuda().reshape(m, in_)
        if xdt == "bf16":
            x = x.to(torch.bfloat16)
        ytype = torch.bfloat16 if ydt == "bf16" else torch.float32
        y_ref = torch.full((m, out), float("nan"), dtype=ytype, device="cuda")
        y_na = torch.full((m, out), float("nan"), dtype=ytype, device="cuda")
        s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        xc, yc = (_lib.RQ_BF16 if xdt == "bf16" else _lib.RQ_F32), (_lib.RQ_BF16 if ydt == "bf16" else _lib.RQ_F32)
        _lib.call("rq_qmatmul", ctx.handle, w.handle, C.c_void_p(x.data_ptr()), xc, C.c_void_p(y_ref.data_ptr()), yc,
                  m, s)
        st = _lib.lib().rq_qmatmul_noalloc(ctx.handle, w.handle, C.c_void_p(x.data_ptr()), xc,
                                           C.c_void_p(y_na.data_ptr()), yc, m, s)
        torch.cuda.synchronize()
        assert st in (_lib.RQ_OK, _lib.RQ_ERR_SHAPE)
        if st == _lib.RQ_OK:
            a, b = y_ref.float().cpu().numpy(), y_na.float().cpu().numpy()
            assert np.all(np.isfinite(a))
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    finally:
        w.destroy()
