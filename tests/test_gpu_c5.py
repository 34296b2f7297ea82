"""GPU parity at the 70B-MLP workload's own shape: K = 8192, N = 28672.

The launch plans depend on the shape (K-slice counts rounded to powers of two,
the small-m GEMM's slices, the 32 Mi-element limit under which Q8_0 takes the
MFMA decode kernel, the GEMM tile chosen by its cost model), so each route is
checked where it is timed:

  Q4_0 (fp16 scales)   m = 1 (v_dot4 GEMV), 6 and 16 (MFMA decode, 4 / 8 K-slices),
                       32 and 64 (small-m GEMM with K-slices), 256 and 300
                       (prefill GEMM: role-split 256 x 128 tiles, 300 with a
                       partial second row tile)
  Q8_0 (f32 scales)    m = 1 (int8-level decode), 12 and 16 (int8-level decode:
                       the weight is above the MFMA decode's 32 Mi elements),
                       32 (small-m GEMM with K-slices), 256 and 300 (prefill GEMM)

and the role-split 256 x 128 tiles with a partial last column tile (K = 4096,
N = 28656, m = 300).

bf16 activations as the workload defines them, plus f32 activations at the
decode sizes. Each output is checked against the C oracle (qlinear-q8's loop,
raster/quant/train.clj:77-108, over the Q4_0 or Q8_0 dequant) on a subset of
output rows that includes the first and last rows and every 16-row group
boundary case: normwise max|y - ref| / max|ref| < 1e-3 for f32 activations and
f32 outputs, < 1e-2 with bf16 activations or outputs. The int8-level decode
rows are also held to the fixed-point construction's per-output bound.
"""
import numpy as np
import pytest

from raster_amd import workloads as wl

pytestmark = pytest.mark.gpu

K, N = 8192, 28672
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


def rows_subset():
    # first / last rows, both rows of a 16-row group edge, and a spread
    edges = [0, 1, 15, 16, 17, 4095, 4096, 14335, 14336, N - 17, N - 16, N - 2, N - 1]
    return np.unique(np.concatenate([edges, np.linspace(0, N - 1, 131).astype(np.int64)]))


ROWS = rows_subset()


@pytest.fixture(scope="module")
def q4(torch, ctx):
    import raster_amd

    packed, sc16 = wl.q4_weights(N, K, seed=55)
    note(f"C5 q4 weight {N}x{K}")
    w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), N, K, ctx)
    sub = (packed.reshape(N, K // 2)[ROWS].ravel(), sc16.reshape(N, K // 32)[ROWS].ravel())
    yield w, sub
    w.destroy()


@pytest.fixture(scope="module")
def q8(torch, ctx):
    import raster_amd

    codes, scales = wl.q8_weights(N, K, seed=56)
    note(f"C5 q8 weight {N}x{K}")
    w = raster_amd.QWeight.q8(codes, scales, N, K, ctx)
    sub = (codes.reshape(N, K)[ROWS].ravel(), scales.reshape(N, K // 32)[ROWS].ravel())
    yield w, sub
    w.destroy()


def run(torch, w, x, m, xdt, ydt):
    xt = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda().reshape(m, K)
    if xdt == "bf16":
        xt = xt.to(torch.bfloat16)
    y = w.matmul(xt, out_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


@pytest.mark.parametrize("m,xdt", [(1, "bf16"), (1, "f32"), (6, "bf16"), (6, "f32"), (16, "bf16"), (16, "f32"),
                                   (32, "bf16"), (64, "bf16"), (256, "bf16"), (300, "bf16")])
def test_c5_q4(torch, orc, q4, m, xdt):
    w, (pk, sc) = q4
    x = wl.activations(m, K, seed=500 + m, dtype=xdt)
    note(f"C5 q4 m={m} x={xdt}")
    ydt = "bf16" if xdt == "bf16" else "f32"
    y = run(torch, w, x, m, xdt, ydt)
    y2 = run(torch, w, x, m, xdt, ydt)
    assert np.array_equal(y, y2), "repeated calls must agree bitwise"
    ref = orc.qlinear_q4(x, pk, sc, m, K, len(ROWS)).reshape(m, len(ROWS))
    assert orc.normwise_relerr(y[:, ROWS], ref) < (TOL_BF16 if ydt == "bf16" else TOL_F32)
    if xdt == "bf16":
        y32 = run(torch, w, x, m, xdt, "f32")
        assert orc.normwise_relerr(y32[:, ROWS], ref) < (TOL_F32 if m <= 16 else TOL_BF16)


@pytest.mark.parametrize("m,xdt", [(1, "bf16"), (1, "f32"), (12, "f32"), (16, "bf16"), (32, "bf16"), (256, "bf16"),
                                   (300, "bf16")])
def test_c5_q8(torch, orc, q8, m, xdt):
    w, (cs, ss) = q8
    x = wl.activations(m, K, seed=600 + m, dtype=xdt)
    note(f"C5 q8 m={m} x={xdt}")
    ydt = "bf16" if xdt == "bf16" else "f32"
    y = run(torch, w, x, m, xdt, ydt)
    ref = orc.qlinear_q8(x, cs, ss, m, K, len(ROWS)).reshape(m, len(ROWS))
    assert orc.normwise_relerr(y[:, ROWS], ref) < (TOL_BF16 if ydt == "bf16" else TOL_F32)
    if m <= 16 and xdt == "f32":
        # the int8-level decode kernel: per-output fixed-point bound
        from test_gpu_parity import decomposition_bound

        dense = orc.dequant_q8_dense(cs, ss, K, len(ROWS))
        bound = decomposition_bound(x.reshape(m, K), dense, m, K, len(ROWS))
        assert np.all(np.abs(y[:, ROWS] - ref) <= bound)


@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_kpair_128_partial_tiles(torch, ctx, orc, fmt):
    # m = 300, K = 4096, N = 28656: the tile cost model takes the role-split
    # kernel's 256 x 128 tiles (448 tiles, two rounds of the CUs, against 512
    # of 256 x 112); the second row tile holds 44 rows and the last column
    # tile 112 columns. Checked against the oracle on rows at both tile edges,
    # bf16 y against the RNE of f32 y, repeated calls bitwise.
    import raster_amd

    m, k2, n2 = 300, 4096, 28656
    edges = [0, 1, 127, 128, 255, 256, 14335, 14336, n2 - 113, n2 - 112, n2 - 17, n2 - 16, n2 - 1]
    rows = np.unique(np.concatenate([edges, np.linspace(0, n2 - 1, 97).astype(np.int64)]))
    note(f"role-split 256x128 partial tiles {fmt} m={m} {n2}x{k2}")
    if fmt == "q8":
        codes, scales = wl.q8_weights(n2, k2, seed=71)
        w = raster_amd.QWeight.q8(codes, scales, n2, k2, ctx)
        sub = (codes.reshape(n2, k2)[rows].ravel(), scales.reshape(n2, k2 // 32)[rows].ravel())
    else:
        packed, sc16 = wl.q4_weights(n2, k2, seed=72)
        w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), n2, k2, ctx)
        sub = (packed.reshape(n2, k2 // 2)[rows].ravel(), sc16.reshape(n2, k2 // 32)[rows].ravel())
    x = wl.activations(m, k2, seed=73, dtype="bf16")
    xt = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda().reshape(m, k2).to(torch.bfloat16)
    yb = w.matmul(xt, out_dtype=torch.bfloat16)
    yb2 = w.matmul(xt, out_dtype=torch.bfloat16)
    yf = w.matmul(xt, out_dtype=torch.float32)
    torch.cuda.synchronize()
    w.destroy()
    assert torch.equal(yb, yb2), "repeated calls must agree bitwise"
    assert torch.equal(yb, yf.to(torch.bfloat16)), "bf16 y must be the RNE of f32 y"
    y = yf.cpu().numpy()
    if fmt == "q8":
        ref = orc.qlinear_q8(x, sub[0], sub[1], m, k2, len(rows))
    else:
        ref = orc.qlinear_q4(x, sub[0], sub[1], m, k2, len(rows))
    assert orc.normwise_relerr(y[:, rows], ref.reshape(m, len(rows))) < TOL_BF16
