"""GPU parity of rq_i8gemv_dp4a, the raw int8 GEMV core i8gemv-dp4a!
(raster/quant/kernels_k.clj:141-150): y[o] = (float) sum_w dp4a(wp[o*kw+w], xp[w]).

The reference checks it exactly against a scalar int8 dot on the device
(test/raster/quant/kernels_k_gpu_test.clj:139-155: out 16, in 256, kw 64);
here the same shape and larger ones are compared exactly with the oracle's
restatement (oracle rqo_i8gemv_dp4a, pinned on the CPU by the reference's
dp4a known answers in test_oracle.py) and with an int64 numpy dot of the
unpacked bytes: sums past 2^24 check the single rounding to f32, sums past
2^31 the 64-bit accumulation, odd kw the unaligned-row path, kw 0 a zero row.
"""
import numpy as np
import pytest

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


def numpy_ref(W, x, out, kw):
    # exact int64 dot of the unpacked lanes, then one rounding to f32
    return (W.reshape(out, 4 * kw).astype(np.int64) @ x.astype(np.int64)).astype(np.float32)


@pytest.mark.parametrize("out,kw,kind", [(16, 64, "rand"), (1000, 1024, "rand"), (37, 333, "rand"), (256, 4096, "rand"),
                                          (8, 65536, "extreme"), (64, 4099, "extreme"), (5, 0, "rand")])
def test_i8gemv_dp4a_exact(torch, ctx, orc, out, kw, kind):
    import raster_amd

    note(f"i8gemv_dp4a out={out} kw={kw} {kind}")
    rng = np.random.default_rng(out * 7 + kw)
    if kind == "rand":
        W = rng.integers(-128, 128, size=out * 4 * kw, dtype=np.int8)
        x = rng.integers(-128, 128, size=4 * kw, dtype=np.int8)
    else:
        # all -128 (largest products, sums past 2^31 at kw 65536), some rows +127
        W = np.full(out * 4 * kw, -128, np.int8)
        W[: 4 * kw] = 127
        x = np.full(4 * kw, -128, np.int8)
        x[::7] = 127
    wp, xp = W.view(np.int32).copy(), x.view(np.int32).copy()
    ref = numpy_ref(W, x, out, kw)
    orc_y = orc.i8gemv_dp4a(wp, xp, kw, out)
    assert np.array_equal(orc_y.view(np.uint32), ref.view(np.uint32))
    y = raster_amd.i8gemv_dp4a(ctx, torch.from_numpy(wp).cuda(), torch.from_numpy(xp).cuda(), kw, out)
    got = y.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), np.flatnonzero(got != ref)[:8]


def test_i8gemv_dp4a_rejects_bad_shapes(torch, ctx):
    import ctypes as C

    from raster_amd import _lib

    L = _lib.lib()
    buf = torch.zeros(64, dtype=torch.int32, device="cuda")
    p = C.c_void_p(buf.data_ptr())
    assert L.rq_i8gemv_dp4a(ctx.handle, p, p, p, -1, 4, None) == _lib.RQ_ERR_SHAPE
    assert L.rq_i8gemv_dp4a(ctx.handle, None, p, p, 4, 4, None) == _lib.RQ_ERR_NULL
    assert L.rq_i8gemv_dp4a(ctx.handle, p, p, C.c_void_p(buf.data_ptr() + 2), 4, 4, None) == _lib.RQ_ERR_SHAPE
    assert L.rq_i8gemv_dp4a(ctx.handle, p, p, p, (1 << 20) + 1, 1, None) == _lib.RQ_ERR_SHAPE
