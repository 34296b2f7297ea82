"""A seeded sweep of rq_qmatmul shapes across every dispatch route, against the C oracle.

The launch plans pick kernels by m (decode kernels up to 16 rows, the small-m
weight-stream GEMM to 64, the per-wave-weights GEMM to 128, the tile cost model
above), by format, activation dtype and weight size, and cut K into slices
by LDS fit and grid fill. The dedicated tests pin each route at chosen edges;
this sweep draws 48 shapes from a fixed seed over every m band (in a multiple
of 32, out anything), both formats, f32 and bf16 x, f32 and bf16 y, and 12
wide prefill shapes (m 129-1100, out 6000-30000, bf16 x) for the 32x32x16
GEMMs the tile cost model takes there, and holds
each to the oracle (qlinear-q8's loop, raster/quant/train.clj:77-108, over the
Q8_0 or Q4_0 dequant) on a subset of output rows: normwise max|y - ref| /
max|ref| < 1e-3 for f32 x and y, < 1e-2 with bf16 x or y. Each call is
repeated and must agree bit for bit (every split adds its slices in a fixed
order). tests/test_zz_no_alloc.py runs the same shapes through
rq_qmatmul_noalloc.
"""
import numpy as np
import pytest
from sweep_shapes import SHAPES, WIDE_SHAPES

from raster_amd import workloads as wl

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3
TOL_BF16 = 1e-2


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


@pytest.mark.parametrize("i,m,in_,out,fmt,xdt,ydt", SHAPES + WIDE_SHAPES,
                         ids=[f"s{s[0]}" for s in SHAPES + WIDE_SHAPES])
def test_sweep(torch, ctx, orc, i, m, in_, out, fmt, xdt, ydt):
    import raster_amd

    note(f"sweep {i}: {fmt} m={m} in={in_} out={out} x={xdt} y={ydt}")
    x = wl.activations(m, in_, seed=1000 + i, dtype=xdt)
    if fmt == "q8":
        codes, scales = wl.q8_weights(out, in_, seed=2000 + i)
        w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    else:
        packed, sc16 = wl.q4_weights(out, in_, seed=2000 + i)
        w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
    try:
        xt = torch.from_numpy(x).cuda().reshape(m, in_)
        if xdt == "bf16":
            xt = xt.to(torch.bfloat16)
        ytype = torch.bfloat16 if ydt == "bf16" else torch.float32
        y1 = w.matmul(xt, out_dtype=ytype)
        y2 = w.matmul(xt, out_dtype=ytype)
        torch.cuda.synchronize()
        a, b = y1.float().cpu().numpy(), y2.float().cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        rows = np.unique(np.concatenate([[0, out - 1], np.linspace(0, out - 1, min(out, 200)).astype(np.int64)]))
        if fmt == "q8":
            ref = orc.qlinear_q8(x, codes.reshape(out, in_)[rows].ravel(),
                                 scales.reshape(out, in_ // 32)[rows].ravel(), m, in_, len(rows))
        else:
            ref = orc.qlinear_q4(x, packed.reshape(out, in_ // 2)[rows].ravel(),
                                 sc16.reshape(out, in_ // 32)[rows].ravel(), m, in_, len(rows))
        tol = TOL_F32 if xdt == "f32" and ydt == "f32" else TOL_BF16
        assert np.all(np.isfinite(a))
        assert orc.normwise_relerr(a[:, rows], ref.reshape(m, len(rows))) < tol
    finally:
        w.destroy()
