"""GPU parity of the backward-data matmul (rq_qmatmul_dx, rq_qlinear_q8_dx)
against the C oracle's qlinear-q8-dx (raster/quant/train.clj:110-137).

dx[m, i] = sum_o scale[o, i/32] * code[o, i] * dy[m, o]: per-term products
rounded to f32 on both sides, the GPU sums in f32 where Raster sums in double:
normwise max|dx - ref| / max|ref| < 2e-5. Q4_0 (Raster has no Q4 dx) is
checked against a float64 product with the bit-exact Q4_0 dequant. The
adjoint identity <dy, W x> = <dx, x> pins the transpose independently of the
oracle's dx.
"""
import numpy as np
import pytest

from raster_amd import workloads as wl

pytestmark = pytest.mark.gpu

TOL = 2e-5


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


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


@pytest.mark.parametrize("m,in_,out", [(1, 4096, 4096), (3, 96, 40), (5, 5632, 2048), (17, 2048, 33),
                                       (2, 256, 14336)])
def test_dx_q8(torch, ctx, orc, m, in_, out):
    import raster_amd

    codes, scales = wl.q8_weights(out, in_, seed=out)
    dy = wl.activations(m, out, seed=in_)
    note(f"dx q8 m={m} in={in_} out={out}")
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    dx = w.matmul_dx(dev(torch, dy).reshape(m, out))
    dx2 = w.matmul_dx(dev(torch, dy).reshape(m, out))
    torch.cuda.synchronize()
    w.destroy()
    assert torch.equal(dx, dx2), "the slice sums are added in a fixed order"
    ref = orc.qlinear_q8_dx(dy, codes, scales, m, in_, out).reshape(m, in_)
    assert orc.normwise_relerr(dx.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("scale_kind", ["f16", "f32"])
@pytest.mark.parametrize("m,in_,out", [(1, 4096, 14336), (4, 160, 48)])
def test_dx_q4(torch, ctx, orc, m, in_, out, scale_kind):
    import raster_amd

    packed, sc16 = wl.q4_weights(out, in_, seed=in_)
    dy = wl.activations(m, out, seed=out)
    if scale_kind == "f16":
        w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
    else:
        w = raster_amd.QWeight.q4(packed, orc.f16_bits_to_f32(sc16), out, in_, ctx)
    note(f"dx q4 {scale_kind} m={m} in={in_} out={out}")
    dx = w.matmul_dx(dev(torch, dy).reshape(m, out)).cpu().numpy()
    w.destroy()
    W = orc.dequant_q4(packed, sc16, in_, out).reshape(out, in_).astype(np.float64)
    ref = dy.reshape(m, out).astype(np.float64) @ W
    assert orc.normwise_relerr(dx, ref) < TOL


def test_dx_adjoint_identity(torch, ctx, orc):
    # <dy, W x> = <W^T dy, x>: the GPU dx against the oracle's forward
    import raster_amd

    m, in_, out = 3, 1024, 768
    codes, scales = wl.q8_weights(out, in_, seed=4)
    x = wl.activations(m, in_, seed=5)
    dy = wl.activations(m, out, seed=6)
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    dx = w.matmul_dx(dev(torch, dy).reshape(m, out)).cpu().numpy().astype(np.float64)
    w.destroy()
    y = orc.qlinear_q8(x, codes, scales, m, in_, out).astype(np.float64)
    lhs = float(np.dot(dy.astype(np.float64), y.ravel()))
    rhs = float(np.dot(dx.ravel(), x.astype(np.float64)))
    assert abs(lhs - rhs) <= 1e-5 * (np.abs(dy).sum() * np.abs(y).max() + 1e-9)


def test_qlinear_q8_dx_host_surface(torch, ctx, orc):
    import raster_amd

    m, in_, out = 2, 512, 96
    codes, scales = wl.q8_weights(out, in_, seed=7)
    dy = wl.activations(m, out, seed=8)
    dx = raster_amd.qlinear_q8_dx(dy, codes, scales, m, in_, out, ctx)
    ref = orc.qlinear_q8_dx(dy, codes, scales, m, in_, out)
    assert dx.shape == (m * in_,)
    assert orc.normwise_relerr(dx, ref) < TOL
