"""GPU parity of the backward-data matmul (rq_qmatmul_dx, rq_qlinear_q8_dx)
against the C oracle's qlinear-q8-dx (raster/quant/train.clj:110-137).

dx[m, i] = sum_o scale[o, i/32] * code[o, i] * dy[m, o]. Up to 32 dy rows an
f32 MFMA kernel takes w = scale * code (Raster's f32 product) as stored and
forms and sums the products w * dy in f32 (Raster: double); above 32 rows the
bf16 MFMA GEMM carries w and dy each as bf16 hi + lo (relative 2^-16) and adds
hi*hi + hi*lo + lo*hi in f32, so each product is within about 3 * 2^-16 of
the f32 one (about 4e-6 normwise measured). Both: normwise max|dx - ref| /
max|ref| < 2e-5. Q4_0
(Raster has no Q4 dx) is checked against a float64 product with the bit-exact
Q4_0 dequant. The adjoint identity <dy, W x> = <dx, x> pins the transpose
independently of the oracle's dx.
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
@pytest.mark.parametrize("m,in_,out", [(1, 4096, 14336), (4, 160, 48), (16, 4096, 14336), (25, 512, 96)])
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


# ---------------------------------- f32 MFMA (m <= 32) and bf16 MFMA GEMM (m > 32)
@pytest.mark.parametrize("m,in_,out", [(16, 256, 200), (32, 1056, 48), (31, 4096, 11008), (33, 256, 200),
                                       (100, 256, 200), (130, 1056, 48), (512, 1024, 2048), (48, 4096, 11008)])
def test_dx_mfma_q8(torch, ctx, orc, m, in_, out):
    # f32 MFMA: 16, 32 (two dy-row tiles), 31 (a partial second tile, the C2
    # layer's weight, slices); bf16 GEMM: 33 (the smallest m there), 100 /
    # 130 (a partial last row tile), (512, 1024, 2048) and (48, .., 11008)
    # (the reduction cut into slices); in 1056: 33 blocks, a partial last
    # column tile; out 200 / 48: a partial last 16-row group
    import raster_amd

    codes, scales = wl.q8_weights(out, in_, seed=out + 1)
    dy = wl.activations(m, out, seed=in_ + 2)
    note(f"dx mfma q8 m={m} in={in_} out={out}")
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    dx = w.matmul_dx(dev(torch, dy).reshape(m, out))
    dx2 = w.matmul_dx(dev(torch, dy).reshape(m, out))
    torch.cuda.synchronize()
    w.destroy()
    assert torch.equal(dx, dx2), "fixed order: slices and MFMA chains"
    ref = orc.qlinear_q8_dx(dy, codes, scales, m, in_, out).reshape(m, in_)
    assert orc.normwise_relerr(dx.cpu().numpy(), ref) < TOL


def test_dx_mfma_c2_layer_rows(torch, ctx, orc):
    # the backward of the C2 layer (m = 512 dy rows, in 4096, out 11008) on
    # the GPU; rows 0, 1, 255 and 511 against the oracle, every row by the
    # adjoint identity <dy_r, W x> = <dx_r, x> with one x (the oracle's m = 1
    # forward)
    import raster_amd

    m, in_, out = 512, 4096, 11008
    codes, scales = wl.q8_weights(out, in_, seed=21)
    dy = wl.activations(m, out, seed=22).reshape(m, out)
    note(f"dx mfma q8 C2 layer m={m} in={in_} out={out}")
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    dx = w.matmul_dx(dev(torch, dy)).cpu().numpy().astype(np.float64)
    w.destroy()
    rows = [0, 1, 255, 511]
    ref = orc.qlinear_q8_dx(dy[rows], codes, scales, len(rows), in_, out).reshape(len(rows), in_)
    assert orc.normwise_relerr(dx[rows], ref) < TOL
    x = wl.activations(1, in_, seed=23)
    y = orc.qlinear_q8(x, codes, scales, 1, in_, out).astype(np.float64)
    lhs = dy.astype(np.float64) @ y
    rhs = dx @ x.astype(np.float64)
    bound = 1e-5 * (np.abs(dy).sum(axis=1) * np.abs(y).max() + 1e-9)
    assert np.all(np.abs(lhs - rhs) <= bound)


@pytest.mark.parametrize("scale_kind", ["f16", "f32"])
def test_dx_mfma_q4(torch, ctx, orc, scale_kind):
    import raster_amd

    m, in_, out = 64, 512, 160
    packed, sc16 = wl.q4_weights(out, in_, seed=31)
    dy = wl.activations(m, out, seed=32)
    if scale_kind == "f16":
        w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
    else:
        w = raster_amd.QWeight.q4(packed, orc.f16_bits_to_f32(sc16), out, in_, ctx)
    note(f"dx mfma q4 {scale_kind} m={m} in={in_} out={out}")
    dx = w.matmul_dx(dev(torch, dy).reshape(m, out)).cpu().numpy()
    w.destroy()
    W = orc.dequant_q4(packed, sc16, in_, out).reshape(out, in_).astype(np.float64)
    ref = dy.reshape(m, out).astype(np.float64) @ W
    assert orc.normwise_relerr(dx, ref) < TOL


@pytest.mark.parametrize("m", [5, 20])
def test_dx_dy_4_byte_aligned(torch, ctx, orc, m):
    # dy only 4-byte aligned (the entry's requirement), out not a multiple of 4:
    # the f32 MFMA kernel reads dy one float at a time
    import raster_amd

    in_, out = 512, 201
    codes, scales = wl.q8_weights(out, in_, seed=51)
    dy = wl.activations(m, out, seed=52)
    buf = torch.empty(m * out + 1, dtype=torch.float32, device="cuda")
    buf[1:] = dev(torch, dy)
    dyv = buf[1:]
    assert dyv.data_ptr() % 16 == 4
    note(f"dx q8 m={m} in={in_} out={out}, dy at a 4-byte offset")
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    dx = w.matmul_dx(dyv).cpu().numpy()
    w.destroy()
    ref = orc.qlinear_q8_dx(dy, codes, scales, m, in_, out).reshape(m, in_)
    assert orc.normwise_relerr(dx, ref) < TOL
