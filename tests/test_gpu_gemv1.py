"""GPU parity of the m = 1 Q4_0 decode GEMV (plain rq_qmatmul, f32 or bf16
activations; v_dot4_i32_i8 on the 16-bit block fixed point of the int8-level
decode kernel) against the C oracle.

Bars: normwise < 1e-3 against the oracle's qlinear-q4 on the same
activations (bf16 inputs are exact values), and per output the fixed-point
bound of the decomposition: each activation is within 2^(e-16) of its
representation, e the exponent of its block's maximum (raised by one where
max * 2^(15-e) > 32639), so |y - exact| <= sum_b 2^(e_b - 16) sum_k |W[o, k]|
plus f32 accumulation slack. Shapes cover every tail of the 4-block loads
(5, 13, 129 blocks), the 16-wave plan (K = 28672) and the C3 shape.
"""
import numpy as np
import pytest

from raster_amd import workloads as wl

pytestmark = pytest.mark.gpu

TOL = 1e-3


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


def fixed_point_bound(x, wdense):
    """x [in], wdense [rows, in] (float64): per-row bound of the decomposition."""
    in_ = x.size
    xb = np.abs(np.asarray(x, np.float64).reshape(in_ // 32, 32))
    amax = xb.max(axis=1)
    _, e = np.frexp(amax)
    e = np.where(amax > 0, e, 0)
    e = np.where(np.ldexp(amax, 15 - e) > 32639.0, e + 1, e)
    step = np.ldexp(1.0, e - 16)
    wabs = np.abs(wdense).reshape(wdense.shape[0], in_ // 32, 32).sum(axis=2)
    mag = np.abs(wdense) @ np.abs(np.asarray(x, np.float64))
    return wabs @ step + 1e-6 * mag + 1e-30


def run(torch, w, x, xdt, ydt):
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda().reshape(1, -1)
    if xdt == "bf16":
        t = t.to(torch.bfloat16)
    y = w.matmul(t, out_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32)
    torch.cuda.synchronize()
    return y.float().cpu().numpy().ravel()


def weight(raster_amd, ctx, orc, out, in_, scale_kind, seed):
    packed, sc16 = wl.q4_weights(out, in_, seed=seed)
    scales = sc16.view(np.float16) if scale_kind == "f16" else orc.f16_bits_to_f32(sc16)
    return raster_amd.QWeight.q4(packed, scales, out, in_, ctx), packed, sc16


@pytest.mark.parametrize("in_,out", [(128, 16), (160, 33), (416, 520), (4128, 100), (2048, 5632), (28672, 64),
                                     (4096, 14336)])
@pytest.mark.parametrize("scale_kind", ["f16", "f32"])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_gemv1_q4(torch, ctx, orc, in_, out, scale_kind, xdt):
    import raster_amd

    x = wl.activations(1, in_, seed=in_ + out, dtype=xdt)
    note(f"gemv1 q4 {scale_kind} x={xdt} {out}x{in_}")
    w, packed, sc16 = weight(raster_amd, ctx, orc, out, in_, scale_kind, seed=out)
    y = run(torch, w, x, xdt, "f32")
    yb = run(torch, w, x, xdt, "bf16")
    w.destroy()
    assert np.array_equal(orc.f32_to_bf16_bits(y), orc.f32_to_bf16_bits(yb))
    rows = np.unique(np.linspace(0, out - 1, min(out, 512)).astype(np.int64))
    pk = packed.reshape(out, in_ // 2)[rows].ravel()
    ss = sc16.reshape(out, in_ // 32)[rows].ravel()
    ref = orc.qlinear_q4(x, pk, ss, 1, in_, len(rows))
    assert orc.normwise_relerr(y[rows], ref) < TOL
    dense = orc.dequant_q4(pk, ss, in_, len(rows)).reshape(len(rows), in_).astype(np.float64)
    exact = dense @ x.astype(np.float64)
    assert np.all(np.abs(y[rows] - exact) <= fixed_point_bound(x, dense))


def test_gemv1_special_activations(torch, ctx, orc):
    # 1e30 next to 1e-30 in one block, a zero block, tiny values: inside the
    # bound; an inf or a NaN anywhere makes every output non-finite
    import raster_amd

    in_, out = 512, 48
    w, packed, sc16 = weight(raster_amd, ctx, orc, out, in_, "f16", seed=9)
    dense = orc.dequant_q4(packed, sc16, in_, out).reshape(out, in_).astype(np.float64)
    x = wl.activations(1, in_, seed=10).copy()
    x[0], x[1] = 1e30, 1e-30
    x[64:96] = 0.0
    x[200:232] *= 1e-35
    note("gemv1 special activations")
    y = run(torch, w, x, "f32", "f32")
    assert np.all(np.abs(y - dense @ x.astype(np.float64)) <= fixed_point_bound(x, dense))
    for bad in (np.inf, np.nan):
        xb = x.copy()
        xb[300] = bad
        assert not np.any(np.isfinite(run(torch, w, xb, "f32", "f32")))
    w.destroy()


def test_gemv1_matches_int8_level_kernel(torch, ctx):
    # a fused call (zero residual) runs the int8-level kernel on the same
    # decomposition: the two differ only in the order of the f32 block sums
    import raster_amd

    in_, out = 4096, 2048
    packed, sc16 = wl.q4_weights(out, in_, seed=3)
    w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
    x = torch.from_numpy(wl.activations(1, in_, seed=4)).cuda().reshape(1, in_)
    a = w.matmul(x)
    b = w.matmul_fused(x, residual=torch.zeros((1, out), device="cuda"))
    torch.cuda.synchronize()
    w.destroy()
    d = (a - b).abs().max().item() / b.abs().max().item()
    assert d < 1e-5, d
