"""GPU parity of the MFMA decode kernel (plain rq_qmatmul, 8 < m <= 16, f32 or
bf16 activations) against the C oracle.

The kernel splits each f32 activation into bf16 hi + lo (|x - hi - lo| <=
2^-17 |x|), feeds the codes to the MFMA exactly with an offset (Q4 nibble n as
128 + n, Q8 code c as c + 128) and removes OFF * sum(hi + lo) per block before
the block scale. Besides the normwise bar of the workload (< 1e-3 f32 x, < 1e-2
bf16), every output is held to the error bound that construction gives:
2^-16 sum |x W| (the split), 2^-126 sum |W| (a bf16 part below the normal
range), and 2^-18 sum |x| (|W| + OFF |s|) for the f32 sums of the offset codes
and the subtraction. A wrong offset, a lost lo part or a mismatched k order
exceeds it by orders of magnitude.
"""
import numpy as np
import pytest

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


def make(raster_amd, ctx, orc, fmt, out, in_, seed):
    """Weight handle, dense f32 weights [out, in], per-element |scale| and OFF."""
    if fmt == "q8":
        codes, scales = wl.q8_weights(out, in_, seed=seed)
        w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
        dense = orc.dequant_q8_dense(codes, scales, in_, out).reshape(out, in_)
        s = np.repeat(np.abs(scales.reshape(out, in_ // 32)), 32, axis=1)
        return w, dense, s, 128.0
    packed, sc16 = wl.q4_weights(out, in_, seed=seed)
    if fmt == "q4":
        w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
    else:
        w = raster_amd.QWeight.q4(packed, orc.f16_bits_to_f32(sc16), out, in_, ctx)
    dense = orc.dequant_q4(packed, sc16, in_, out).reshape(out, in_)
    s = np.repeat(np.abs(orc.f16_bits_to_f32(sc16).reshape(out, in_ // 32)), 32, axis=1)
    return w, dense, s, 136.0


def mf_bound(x, dense, s, off):
    xa = np.abs(np.asarray(x, np.float64))
    wa = np.abs(np.asarray(dense, np.float64))
    return (2.0 ** -16 * (xa @ wa.T) + 2.0 ** -126 * wa.sum(axis=1)[None, :]
            + 2.0 ** -18 * (xa @ (wa + off * np.asarray(s, np.float64)).T) + 1e-37)


def run(torch, w, x, xdt, ydt):
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    if xdt == "bf16":
        t = t.to(torch.bfloat16)
    y = w.matmul(t, out_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


@pytest.mark.parametrize("m,in_,out", [(9, 4096, 520), (12, 416, 33), (16, 14336, 48), (16, 4096, 2048),
                                       (13, 32, 16), (10, 8192, 100)])
@pytest.mark.parametrize("fmt", ["q8", "q4", "q4f32"])
def test_mf_f32(torch, ctx, orc, m, in_, out, fmt):
    import raster_amd

    x = wl.activations(m, in_, seed=m * 31 + in_).reshape(m, in_)
    note(f"mf {fmt} f32 m={m} {out}x{in_}")
    w, dense, s, off = make(raster_amd, ctx, orc, fmt, out, in_, seed=out + in_)
    y = run(torch, w, x, "f32", "f32")
    y2 = run(torch, w, x, "f32", "f32")
    yb = run(torch, w, x, "f32", "bf16")
    w.destroy()
    assert np.array_equal(y, y2), "the K-slices are added in a fixed order"
    assert np.array_equal(orc.f32_to_bf16_bits(y), orc.f32_to_bf16_bits(yb))
    rows = np.unique(np.linspace(0, out - 1, min(out, 256)).astype(np.int64))
    ref = (x.astype(np.float64) @ dense[rows].astype(np.float64).T)
    assert orc.normwise_relerr(y[:, rows], ref) < TOL_F32
    assert np.all(np.abs(y[:, rows] - ref) <= mf_bound(x, dense[rows], s[rows], off))


@pytest.mark.parametrize("m,in_,out", [(11, 2048, 6144), (16, 96, 40), (9, 20480, 24)])
@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_mf_bf16(torch, ctx, orc, m, in_, out, fmt):
    # bf16 activations are exact in the MFMA: only the f32 sums remain
    import raster_amd

    x = wl.activations(m, in_, seed=m + 7 * in_, dtype="bf16").reshape(m, in_)
    note(f"mf {fmt} bf16 m={m} {out}x{in_}")
    w, dense, s, off = make(raster_amd, ctx, orc, fmt, out, in_, seed=in_ + 3)
    y = run(torch, w, x, "bf16", "f32")
    w.destroy()
    ref = x.astype(np.float64) @ dense.astype(np.float64).T
    assert orc.normwise_relerr(y, ref) < TOL_BF16
    assert np.all(np.abs(y - ref) <= mf_bound(x, dense, s, off))
    # the oracle's own qlinear on the same (bf16-exact) activations
    if fmt == "q8":
        codes, scales = wl.q8_weights(out, in_, seed=in_ + 3)
        ro = orc.qlinear_q8(x.ravel(), codes, scales, m, in_, out).reshape(m, out)
    else:
        packed, sc16 = wl.q4_weights(out, in_, seed=in_ + 3)
        ro = orc.qlinear_q4(x.ravel(), packed, sc16, m, in_, out).reshape(m, out)
    assert orc.normwise_relerr(y, ro) < TOL_F32


@pytest.mark.parametrize("m,in_,out", [(5, 4096, 520), (6, 416, 33), (8, 14336, 48), (7, 8192, 100)])
@pytest.mark.parametrize("fmt", ["q4", "q4f32"])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_mf_q4_small_m(torch, ctx, orc, m, in_, out, fmt, xdt):
    # Q4_0 plain calls with 4 < m <= 8 take the MFMA decode kernel as well
    import raster_amd

    x = wl.activations(m, in_, seed=m * 17 + in_, dtype=xdt).reshape(m, in_)
    note(f"mf {fmt} {xdt} m={m} {out}x{in_}")
    w, dense, s, off = make(raster_amd, ctx, orc, fmt, out, in_, seed=out + 2 * in_)
    y = run(torch, w, x, xdt, "f32")
    y2 = run(torch, w, x, xdt, "f32")
    w.destroy()
    assert np.array_equal(y, y2), "the K-slices are added in a fixed order"
    rows = np.unique(np.linspace(0, out - 1, min(out, 256)).astype(np.int64))
    ref = x.astype(np.float64) @ dense[rows].astype(np.float64).T
    assert orc.normwise_relerr(y[:, rows], ref) < (TOL_F32 if xdt == "f32" else TOL_BF16)
    assert np.all(np.abs(y[:, rows] - ref) <= mf_bound(x, dense[rows], s[rows], off))


def test_mf_special_activations(torch, ctx, orc):
    # one block holding 1e30 and 1e-30, a zero row, an inf row, a NaN row and
    # a row near the bottom of the normal range: finite rows stay inside the
    # bound, the zero row is zero, non-finite rows are non-finite
    import raster_amd

    m, in_, out = 12, 256, 40
    x = wl.activations(m, in_, seed=12).reshape(m, in_).copy()
    x[1, 0], x[1, 1] = 1e30, 1e-30
    x[2] = 0.0
    x[3, 70] = np.inf
    x[4, 5] = np.nan
    x[5] *= 1e-35
    x[6, 200] = -np.inf
    note("mf special activations")
    w, dense, s, off = make(raster_amd, ctx, orc, "q8", out, in_, seed=5)
    y = run(torch, w, x, "f32", "f32")
    w.destroy()
    fin = [0, 1, 2, 5, 7, 8, 9, 10, 11]
    ref = x[fin].astype(np.float64) @ dense.astype(np.float64).T
    assert np.all(np.abs(y[fin] - ref) <= mf_bound(x[fin], dense, s, off))
    assert np.all(y[2] == 0.0)
    for r in (3, 4, 6):
        assert not np.any(np.isfinite(y[r]))


def test_mf_matches_fused_path_closely(torch, ctx, orc):
    # a fused call (RMSNorm with unit gains and eps 0 of pre-normalised rows)
    # takes the int8 decode kernel; both stay within their bounds of the same
    # exact product, so they agree to the int8 kernel's bound
    import raster_amd

    m, in_, out = 12, 2048, 256
    x = wl.activations(m, in_, seed=3).reshape(m, in_)
    x = x / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True)).astype(np.float32)
    codes, scales = wl.q8_weights(out, in_, seed=4)
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    xt = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    a = w.matmul(xt)
    b = w.matmul_fused(xt, norm_gain=torch.ones(in_, device="cuda"), norm_eps=0.0)
    torch.cuda.synchronize()
    w.destroy()
    assert orc.normwise_relerr(a.cpu().numpy(), b.cpu().numpy().astype(np.float64)) < TOL_F32
