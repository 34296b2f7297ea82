"""GPU parity of the weight encoders, the padded K-quant ingestion, the
qlinear-i8! op and the format registry.

  rq_q8_quantize          q8-quantize (raster/quant/train.clj:34-58): codes and scales bit-exact
  rq_q4k_of               q4k-of (raster/quant/pack.clj:45-53): rows zero-padded to nextpad(in),
                          quantize-weight-q4k (raster/compiler/backend/cpu/quant.clj:92-137): bit-exact
  rq_quantize_weight_q6k  quantize-weight-q6k (quant.clj:214-239): bit-exact
  q4k-of weight, in=640   K dot over the padded weight and zero-padded x, against the oracle's
                          qmatmul-q4k-composable! (raster/quant/kernels_k.clj:15-46): normwise < 2e-5
  rq_qlinear_i8           qlinear-i8! / qlinear-i8-q8! (raster/quant/op.clj:43-51,81-90) against the
                          oracle's quantize-act-i8 + qmatmul-q4-x8! / qmatmul-q8-x8!
                          (raster/quant/kernels.clj:216-247,308-333): normwise < 2e-5 (both sum f32
                          terms, in different orders)
  registry                QMatrix{:q4_K,:q6_K} . x equals the raw device path bit for bit and the
                          oracle within 2e-5 (test/raster/quant/core_test.clj:15-45); a user format
                          dispatches (core_test.clj:58-69)

The oracle's encoders are pinned on the CPU (test_oracle.py) by the
reference's own tests (pack_test.clj, quant_k_test.clj, train_test.clj).
"""
import numpy as np
import pytest

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
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bits_equal(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


def weights(out, in_, seed):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal(out * in_) * rng.uniform(0.01, 2.0, out * in_)).astype(np.float32)
    # special blocks: all zero, a single nonzero, ties at half steps, one huge value
    W[:32] = 0.0
    W[32:64] = 0.0
    W[40] = -3.5
    W[64:96] = np.linspace(-127, 127, 32).astype(np.float32) / 2.0
    W[96:128] *= 1e30
    return W


@pytest.mark.parametrize("out,in_", [(4096, 4096), (7, 96), (300, 1024)])
def test_q8_quantize_bit_exact(torch, ctx, orc, out, in_):
    import raster_amd

    W = weights(out, in_, out + in_)
    note(f"q8_quantize {out}x{in_}")
    codes, scales = raster_amd.q8_quantize(ctx, dev(torch, W), out, in_)
    torch.cuda.synchronize()
    rc, rs = orc.q8_quantize(W, out, in_)
    assert bits_equal(codes.cpu().numpy().ravel(), rc)
    assert bits_equal(scales.cpu().numpy().ravel(), rs)


@pytest.mark.parametrize("out,in_", [(3, 640), (2, 256), (5, 1), (4, 300), (1024, 4096), (16, 5632)])
def test_q4k_of_bit_exact(torch, ctx, orc, out, in_):
    import raster_amd

    W = weights(out, in_, 7 * out + in_) if in_ >= 128 else np.random.default_rng(1).standard_normal(
        out * in_).astype(np.float32)
    note(f"q4k_of {out}x{in_}")
    got = raster_amd.q4k_of(ctx, dev(torch, W), out, in_)
    torch.cuda.synchronize()
    *ref, inp = orc.q4k_of(W, out, in_)
    assert got["in"] == inp == orc.nextpad(in_)
    for k, r in zip(("wq", "da", "db", "aq", "bq"), ref):
        assert bits_equal(got[k].cpu().numpy(), r), k


@pytest.mark.parametrize("out,in_", [(4, 256), (300, 4096), (16, 5632)])
def test_quantize_weight_q6k_bit_exact(torch, ctx, orc, out, in_):
    import raster_amd

    W = weights(out, in_, 11 * out + in_)
    note(f"quantize_weight_q6k {out}x{in_}")
    wq, sc, ds = raster_amd.quantize_weight_q6k(ctx, dev(torch, W), out, in_)
    torch.cuda.synchronize()
    rwq, rsc, rds = orc.quantize_weight_q6k(W)
    assert bits_equal(wq.cpu().numpy(), rwq)
    assert bits_equal(sc.cpu().numpy(), rsc)
    assert bits_equal(ds.cpu().numpy(), rds)


def test_q4k_of_padded_weight_matmul(torch, ctx, orc):
    # pack_test.clj:61-69's shape (out 3, in 640 -> 768) and a larger one: the
    # q4k-of buffer set goes to rq_weight_create_q4k with in = nextpad(in);
    # x is zero-padded to the same width, as the reference's caller does
    import raster_amd

    for out, in_, m in ((3, 640, 1), (96, 1000, 3)):
        W = orc.jfill_uniform_centered(13, out * in_)
        wq, da, db, aq, bq, inp = orc.q4k_of(W, out, in_)
        x = np.zeros((m, inp), np.float32)
        x[:, :in_] = np.random.default_rng(in_).standard_normal((m, in_))
        note(f"q4k-of weight {out}x{in_} -> {inp}, m={m}")
        w = raster_amd.QWeight.q4k(wq, da, db, aq, bq, out, inp, ctx)
        xq = raster_amd.quantize_act_q8k(ctx, dev(torch, x.ravel()), inp, 32)
        y = w.matmul_q8k(*xq)
        torch.cuda.synchronize()
        w.destroy()
        rxq, rxs, rbs = orc.quantize_act_q8k(x.ravel(), m, inp, 32)
        assert bits_equal(xq[0].cpu().numpy().ravel(), rxq)
        ref = orc.qmatmul_q4k(rxq, rxs, rbs, wq, da, db, aq, bq, m, inp, out).reshape(m, out)
        assert orc.normwise_relerr(y.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("nibble", [True, False])
@pytest.mark.parametrize("out,in_", [(8, 64), (4096, 4096), (520, 1024)])
def test_qlinear_i8_against_x8_oracle(torch, ctx, orc, nibble, out, in_):
    import raster_amd

    rng = np.random.default_rng(out + in_ + nibble)
    W = rng.standard_normal(out * in_).astype(np.float32)
    x = rng.standard_normal(in_).astype(np.float32)
    wq, ws = orc.quantize_weight_q4(W) if nibble else orc.quantize_weight_q8u(W)
    wqi, wsi = orc.repack_x8(wq, ws, out, in_, nibble)
    note(f"qlinear_i8 nibble={nibble} {out}x{in_}")
    y = np.full(out, np.nan, np.float32)
    got = raster_amd.qlinear_i8(x, wqi, wsi, y, in_, out, ctx=ctx, nibble=nibble)
    assert got is y and np.all(np.isfinite(y))
    xq, xs, xsum = orc.quantize_act_i8(x, 1, in_)
    ref = orc.qmatmul_x8(xq, xs, xsum, wqi, wsi, in_, out, nibble)
    assert orc.normwise_relerr(y, ref) < TOL
    if not nibble:
        y8 = raster_amd.qlinear_i8_q8(x, wqi, wsi, np.empty(out, np.float32), in_, out, ctx=ctx)
        assert np.array_equal(y8, y)


def test_qlinear_i8_rejects_bad_shapes(torch, ctx):
    import raster_amd

    with pytest.raises(raster_amd.RqError) as e:
        raster_amd.quant.call("rq_qlinear_i8", ctx.handle, None, None, None, 1, None, 64, 12)
    assert e.value.status == raster_amd._lib.RQ_ERR_NULL
    x, y = np.zeros(64, np.float32), np.zeros(12, np.float32)
    wqi, wsi = np.zeros(256, np.uint8), np.zeros(16, np.float32)
    with pytest.raises(raster_amd.RqError) as e:
        raster_amd.quant.call("rq_qlinear_i8", ctx.handle, x.ctypes.data, wqi.ctypes.data, wsi.ctypes.data, 1,
                              y.ctypes.data, 64, 12)
    assert e.value.status == raster_amd._lib.RQ_ERR_SHAPE


@pytest.mark.parametrize("fmt,sub", [("q4_K", 32), ("q6_K", 16)])
def test_registry_kquant_plumbing(torch, ctx, orc, fmt, sub):
    # test/raster/quant/core_test.clj:15-45: QMatrix{fmt} . x equals the raw
    # path (here: the device encoder, resident weight and K-quant GEMV called
    # directly) bit for bit, and the oracle's composable path within 2e-5
    import raster_amd
    from raster_amd import registry as qm

    out, in_ = 8, 256
    W = orc.jfill_uniform_centered(1 if fmt == "q4_K" else 3, out * in_)
    x = orc.jfill_uniform_centered(2 if fmt == "q4_K" else 4, in_)
    note(f"registry {fmt}")
    q = qm.qmatrix(fmt, W, out, in_)
    y = qm.matmul(q, x)
    assert isinstance(y, np.ndarray) and y.shape == (out,)
    if fmt == "q4_K":
        arrs = orc.quantize_weight_q4k(W)
        w = raster_amd.QWeight.q4k(*arrs, out, in_, ctx)
    else:
        arrs = orc.quantize_weight_q6k(W)
        w = raster_amd.QWeight.q6k(*arrs, out, in_, ctx)
    xq = raster_amd.quantize_act_q8k(ctx, dev(torch, x), in_, sub)
    yraw = w.matmul_q8k(*xq).cpu().numpy().ravel()
    w.destroy()
    assert np.array_equal(y, yraw)
    rxq, rxs, rbs = orc.quantize_act_q8k(x, 1, in_, sub)
    f = orc.qmatmul_q4k if fmt == "q4_K" else orc.qmatmul_q6k
    ref = f(rxq, rxs, rbs, *arrs, 1, in_, out)
    assert orc.normwise_relerr(y, ref) < TOL
    qm.release(q)


def test_registry_dispatch_and_user_format(torch, ctx, orc):
    # core_test.clj:47-69: matmul dispatches on the format; a user format
    # registered at run time is dispatched to with no other change
    from raster_amd import registry as qm

    out, in_ = 8, 256
    W = orc.jfill_uniform_centered(5, out * in_)
    x = orc.jfill_uniform_centered(6, in_)
    q4, q6 = qm.qmatrix("q4_K", W, out, in_), qm.qmatrix("q6_K", W, out, in_)
    y4, y6 = qm.matmul(q4, x), qm.matmul(q6, x)
    assert y4.shape == y6.shape == (out,) and not np.array_equal(y4, y6)
    qm.release(q4)
    qm.release(q6)
    qm.register_quant("dense_f32", {"descriptor": {"name": "dense_f32"},
                                    "quantize": lambda W, r, c, d: {"w": np.asarray(W, np.float32).reshape(r, c)},
                                    "apply": lambda q, x: (q.arrays["w"].astype(np.float64) @ x).astype(np.float32)})
    assert "dense_f32" in qm.registered_formats()
    Wd, xd = orc.jfill_uniform_centered(7, 4 * 16), orc.jfill_uniform_centered(8, 16)
    yd = qm.matmul(qm.qmatrix("dense_f32", Wd, 4, 16), xd)
    assert np.allclose(yd, Wd.reshape(4, 16).astype(np.float64) @ xd, rtol=1e-6)
    with pytest.raises(KeyError):
        qm.qmatrix("no_such_format", W, out, in_)


def test_registry_q8_0_and_padded_q4_K(torch, ctx, orc):
    # the device q8_0 format (q8-quantize + qlinear-q8) and q4_K over a width
    # that q4k-of pads (640 -> 768), against the oracle
    from raster_amd import registry as qm

    rng = np.random.default_rng(77)
    out, in_ = 64, 640
    W = rng.standard_normal(out * in_).astype(np.float32)
    x = rng.standard_normal(in_).astype(np.float32)
    q = qm.qmatrix("q8_0", W, out, in_)
    y = qm.matmul(q, x)
    qm.release(q)
    codes, scales = orc.q8_quantize(W, out, in_)
    ref = orc.qlinear_q8(x, codes, scales, 1, in_, out)
    assert orc.normwise_relerr(y, ref) < 1e-3
    q = qm.qmatrix("q4_K", W, out, in_)
    assert q.arrays["in"] == 768
    y = qm.matmul(q, x)
    qm.release(q)
    wq, da, db, aq, bq, inp = orc.q4k_of(W, out, in_)
    xp = np.zeros(inp, np.float32)
    xp[:in_] = x
    rxq, rxs, rbs = orc.quantize_act_q8k(xp, 1, inp, 32)
    ref = orc.qmatmul_q4k(rxq, rxs, rbs, wq, da, db, aq, bq, 1, inp, out)
    assert orc.normwise_relerr(y, ref) < TOL
