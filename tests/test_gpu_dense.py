"""GPU parity of the dense f32 GEMM surface (rq_sgemm / rq_sgemm_tn /
rq_sgemm_nt, the float arms of raster/linalg/blas.clj:287-337, and rq_linear,
raster/dl/nn.clj:161-183) against the C oracle (f64 sums, one f32 rounding).

The library sums its products in f32 in an order of its own, so each element
is held to the a priori bound of an f32 dot product of length k, whatever its
order: |c - c_ref| <= gamma (|alpha| sum_p |a_ip b_pj| + |beta c0_ij|) + u |c_ref|
with u = 2^-24 and gamma = (k + 2) u / (1 - (k + 2) u). The reference tests'
integer known answers are exact in f32 and checked exactly.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


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


def bound(A, B, C0, m, k, n, ta, tb, alpha, beta, ref):
    Am = np.abs(A.reshape(k, m).T if ta else A.reshape(m, k)).astype(np.float64)
    Bm = np.abs(B.reshape(n, k).T if tb else B.reshape(k, n)).astype(np.float64)
    g = (k + 2) * U / (1 - (k + 2) * U)
    return g * (abs(alpha) * (Am @ Bm) + abs(beta) * np.abs(C0.reshape(m, n))) + U * np.abs(ref.reshape(m, n))


def test_reference_known_answers(torch, ctx):
    # test/raster/linalg/blas_test.clj:11-77 (integers, exact in f32)
    from raster_amd import dense

    f = lambda v: dev(torch, np.array(v, np.float32))  # noqa: E731
    note("dense known answers")
    assert dense.dgemm(f([1, 0, 0, 1]), f([5, 6, 7, 8]), f([0] * 4), 2, 2, 2, 1.0, 0.0, ctx).tolist() == [5, 6, 7, 8]
    assert dense.dgemm(f([1, 2, 3, 4, 5, 6]), f([7, 8, 9, 10, 11, 12]), f([0] * 4), 2, 3, 2, 1.0, 0.0,
                       ctx).tolist() == [58, 64, 139, 154]
    assert dense.dgemm(f([1, 0, 0, 1]), f([5, 6, 7, 8]), f([10, 20, 30, 40]), 2, 2, 2, 2.0, 3.0,
                       ctx).tolist() == [40, 72, 104, 136]
    assert dense.dgemm_tn(f([1, 4, 2, 5, 3, 6]), f([7, 8, 9, 10, 11, 12]), f([0] * 4), 2, 3, 2, 1.0, 0.0,
                          ctx).tolist() == [58, 64, 139, 154]
    assert dense.dgemm_nt(f([1, 2, 3, 4, 5, 6]), f([7, 9, 11, 8, 10, 12]), f([0] * 4), 2, 3, 2, 1.0, 0.0,
                          ctx).tolist() == [58, 64, 139, 154]
    # test/raster/dl/nn_test.clj:42-61 and 93-117
    assert dense.matmul(f([1, 2, 3, 4, 5, 6]), f([7, 8, 9, 10, 11, 12]), 2, 3, 2, ctx).tolist() == [58, 64, 139, 154]
    y = dense.linear(f([1, 2, 3]), f([1, 0, 0, 0, 1, 0]), f([0.1, 0.2]), 1, 3, 2, ctx).cpu().numpy()
    assert list(y) == [np.float32(1) + np.float32(0.1), np.float32(2) + np.float32(0.2)]
    y = dense.linear(f([1, 2, 3, 4, 5, 6]), f([1, 0, 0, 0, 1, 0]), f([0, 0]), 2, 3, 2, ctx)
    assert y.tolist() == [1, 2, 4, 5]


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 13, 5), (64, 64, 64), (33, 4096, 47), (512, 4096, 1024),
                                   (3, 11008, 17)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True)])
def test_sgemm_vs_oracle(torch, ctx, orc, m, k, n, ta, tb):
    from raster_amd import dense

    rng = np.random.default_rng(m * 131 + k * 7 + n)
    A = rng.standard_normal(m * k).astype(np.float32)
    B = rng.standard_normal(k * n).astype(np.float32)
    C0 = rng.standard_normal(m * n).astype(np.float32)
    alpha, beta = (1.0, 0.0) if (m + n) % 2 else (0.5, -2.0)
    note(f"sgemm ta={ta} tb={tb} m={m} k={k} n={n} alpha={alpha} beta={beta}")
    fn = dense.dgemm_tn if ta else dense.dgemm_nt if tb else dense.dgemm
    Cg = fn(dev(torch, A), dev(torch, B), dev(torch, C0), m, k, n, alpha, beta, ctx)
    got = Cg.cpu().numpy()
    ref = orc.sgemm(ta, tb, A, B, C0, m, k, n, alpha, beta)
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64)).reshape(m, n)
    assert np.all(err <= bound(A, B, C0, m, k, n, ta, tb, alpha, beta, ref)), float(err.max())
    # f32 products, not a reduced-precision mode (xf32 or bf16 inputs would
    # put this near 1e-4 at these sizes; f32 sums land near 1e-7)
    rel = float(err.max() / max(np.abs(ref).max(), 1e-30))
    note(f"  normwise error {rel:.2e}")
    assert rel < 1e-5, rel
    # the library's atomics are off: a repeat is bitwise the same
    again = fn(dev(torch, A), dev(torch, B), dev(torch, C0), m, k, n, alpha, beta, ctx).cpu().numpy()
    assert np.array_equal(again.view(np.uint32), got.view(np.uint32))


@pytest.mark.parametrize("batch,in_f,out_f", [(1, 3, 2), (5, 96, 40), (64, 4096, 11008), (17, 2048, 33)])
def test_linear_vs_oracle(torch, ctx, orc, batch, in_f, out_f):
    from raster_amd import dense

    rng = np.random.default_rng(batch + in_f + out_f)
    x = rng.standard_normal(batch * in_f).astype(np.float32)
    W = (rng.standard_normal(out_f * in_f) * 0.05).astype(np.float32)
    b = rng.standard_normal(out_f).astype(np.float32)
    note(f"linear batch={batch} in={in_f} out={out_f}")
    y = dense.linear(dev(torch, x), dev(torch, W), dev(torch, b), batch, in_f, out_f, ctx).cpu().numpy()
    ref = orc.linear(x, W, b, batch, in_f, out_f)
    bias = np.tile(b, batch)
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64)).reshape(batch, out_f)
    assert np.all(err <= bound(x, W, bias, batch, in_f, out_f, False, True, 1.0, 1.0, ref)), float(err.max())
    rel = float(err.max() / max(np.abs(ref).max(), 1e-30))
    note(f"  normwise error {rel:.2e}")
    assert rel < 1e-5, rel


def test_degenerate_shapes(torch, ctx):
    # blas.clj:301,318,334: nothing unless m, n, k are all positive; linear
    # with in_f = 0 still writes the bias rows (nn.clj:170-171)
    from raster_amd import dense

    C0 = dev(torch, np.array([1, 2, 3, 4], np.float32))
    empty = torch.empty(0, dtype=torch.float32, device="cuda")
    for m, k, n in ((0, 2, 2), (2, 0, 2), (2, 2, 0)):
        assert dense.dgemm(empty, empty, C0, m, k, n, 1.0, 0.0, ctx).tolist() == [1, 2, 3, 4]
    y = dense.linear(empty, empty, dev(torch, np.array([3, 4], np.float32)), 2, 0, 2, ctx)
    assert y.tolist() == [3, 4, 3, 4]


def test_errors(torch, ctx):
    import ctypes as C

    from raster_amd import _lib

    L = _lib.lib()
    assert L.rq_sgemm(ctx.handle, None, None, None, 2, 2, 2, 1.0, 0.0, None) == _lib.RQ_ERR_NULL
    assert L.rq_linear(ctx.handle, None, None, None, None, 2, 2, 2, None) == _lib.RQ_ERR_NULL
    big = C.c_int64(1 << 31)
    p = C.c_void_p(1)
    assert L.rq_sgemm_nt(ctx.handle, p, p, p, big, 1, 1, 1.0, 0.0, None) == _lib.RQ_ERR_SHAPE
    assert L.rq_sgemm(C.c_void_p(0x1234), p, p, p, 1, 1, 1, 1.0, 0.0, None) == _lib.RQ_ERR_HANDLE
