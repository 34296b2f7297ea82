"""GPU parity of the K-quant path (Q4_K, Q6_K) against the C oracle.

  rq_quantize_act_q8k  quantize-act-q8k (raster/compiler/backend/cpu/quant.clj:158-176): bit-exact
  rq_dequant           dequant-q4k / dequant-q6k (quant.clj:139-156,241-252): bit-exact
  rq_qmatmul_q8k       qmatmul-q4k-dp4a! / qmatmul-q6k-dp4a! (raster/quant/kernels_k.clj:186-297):
                       exact integer sub-block dots, scale terms summed in f32 where Raster sums
                       in double: normwise max|y - ref| / max|ref| < 2e-5 (f32 y), 1e-2 (bf16 y)
  rq_qmatmul (K-quant, f32 x)  the two calls above in one (QMatrix apply, raster/quant/core.clj:55-75):
                       bit-identical to them, and through them to the oracle's bound

The oracle's restatements are pinned on the CPU (test_oracle.py) by the
reference's own K-quant tests (test/raster/quant/kernels_k_test.clj), the exact
dot = dequant . dequant identity and the encoders' invariants. Weights come from
the oracle's restatement of Raster's encoders.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 2e-5
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


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def encode(orc, fmt, out, in_, seed):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal(out * in_) * rng.uniform(0.02, 0.1)).astype(np.float32)
    return orc.quantize_weight_q4k(W) if fmt == "q4k" else orc.quantize_weight_q6k(W)


def make_weight(raster_amd, ctx, fmt, arrs, out, in_):
    return raster_amd.QWeight.q4k(*arrs, out, in_, ctx) if fmt == "q4k" else raster_amd.QWeight.q6k(*arrs, out, in_,
                                                                                                       ctx)


def oracle_y(orc, fmt, arrs, xq, xs, bs, m, in_, out, rows=None):
    if rows is not None:  # a subset of weight rows (whole rows of every array)
        if fmt == "q4k":
            wq, da, db, aq, bq = arrs
            arrs = (wq.reshape(out, -1)[rows].ravel(), da.reshape(out, -1)[rows].ravel(),
                    db.reshape(out, -1)[rows].ravel(), aq.reshape(out, -1)[rows].ravel(),
                    bq.reshape(out, -1)[rows].ravel())
        else:
            arrs = tuple(a.reshape(out, -1)[rows].ravel() for a in arrs)
        out = len(rows)
    f = orc.qmatmul_q4k if fmt == "q4k" else orc.qmatmul_q6k
    return f(xq, xs, bs, *arrs, m, in_, out).reshape(m, out)


@pytest.mark.parametrize("sub", [32, 16])
@pytest.mark.parametrize("m,in_", [(1, 256), (3, 4096), (5, 5632)])
def test_quantize_act_q8k_bit_exact(torch, ctx, orc, sub, m, in_):
    import raster_amd

    rng = np.random.default_rng(m + in_)
    x = rng.standard_normal(m * in_).astype(np.float32)
    x[:256] = 0.0
    x[256 * (m * in_ // 256 - 1):] *= 1e-30
    note(f"quantize-act-q8k sub={sub} m={m} in={in_}")
    xq, xs, bs = raster_amd.quantize_act_q8k(ctx, dev(torch, x), in_, sub)
    torch.cuda.synchronize()
    rq, rs, rb = orc.quantize_act_q8k(x, m, in_, sub)
    assert np.array_equal(xq.cpu().numpy().ravel(), rq)
    assert np.array_equal(xs.cpu().numpy().ravel().view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(bs.cpu().numpy().ravel(), rb)


@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
@pytest.mark.parametrize("out,in_", [(8, 256), (37, 1024), (256, 4096)])
def test_kquant_dequant_bit_exact(torch, ctx, orc, fmt, out, in_):
    import raster_amd

    arrs = encode(orc, fmt, out, in_, seed=out)
    note(f"dequant {fmt} {out}x{in_}")
    w = make_weight(raster_amd, ctx, fmt, arrs, out, in_)
    d = w.dequant()
    torch.cuda.synchronize()
    w.destroy()
    ref = orc.dequant_q4k(*arrs, out * in_) if fmt == "q4k" else orc.dequant_q6k(*arrs, out * in_)
    assert np.array_equal(d.cpu().numpy().ravel().view(np.uint32), ref.view(np.uint32))


def run_gemv(torch, ctx, orc, fmt, m, out, in_, seed, ydt="f32", rows_cap=None):
    import raster_amd

    sub = 32 if fmt == "q4k" else 16
    arrs = encode(orc, fmt, out, in_, seed=seed)
    x = np.random.default_rng(seed + 1).standard_normal(m * in_).astype(np.float32)
    w = make_weight(raster_amd, ctx, fmt, arrs, out, in_)
    xq, xs, bs = raster_amd.quantize_act_q8k(ctx, dev(torch, x), in_, sub)
    y = w.matmul_q8k(xq, xs, bs, out_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32)
    torch.cuda.synchronize()
    w.destroy()
    y = y.float().cpu().numpy()
    rows = None
    if rows_cap and out > rows_cap:
        rows = np.unique(np.concatenate([[0, out - 1], np.linspace(0, out - 1, rows_cap).astype(np.int64)]))
    ref = oracle_y(orc, fmt, arrs, xq.cpu().numpy().ravel(), xs.cpu().numpy().ravel(), bs.cpu().numpy().ravel(), m,
                   in_, out, rows)
    return (y if rows is None else y[:, rows]), ref


@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
@pytest.mark.parametrize("m,out,in_", [(1, 4096, 4096), (3, 37, 256), (4, 1000, 5632), (7, 16, 14336),
                                       (1, 14336, 4096), (4, 64, 32256)])
def test_kquant_gemv(torch, ctx, orc, fmt, m, out, in_):
    note(f"K-quant gemv {fmt} m={m} {out}x{in_}")
    y, ref = run_gemv(torch, ctx, orc, fmt, m, out, in_, seed=out + in_ + m, rows_cap=512)
    assert orc.normwise_relerr(y, ref) < TOL


@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
def test_kquant_gemv_bf16_out(torch, ctx, orc, fmt):
    y, ref = run_gemv(torch, ctx, orc, fmt, 2, 512, 2048, seed=9, ydt="bf16")
    assert orc.normwise_relerr(y, ref) < TOL_BF16


@pytest.mark.parametrize("fmt,wseed,xseed", [("q4k", 1, 2), ("q6k", 3, 4)])
def test_kquant_reference_test_on_gpu(torch, ctx, orc, fmt, wseed, xseed):
    # test/raster/quant/kernels_k_test.clj:31-61 with the GPU GEMV: out 8,
    # in 256, java.util.Random inputs, within 1e-2 of dequant-matmul per row
    import raster_amd

    out, in_ = 8, 256
    W = orc.jfill_uniform_centered(wseed, out * in_)
    x = orc.jfill_uniform_centered(xseed, in_)
    sub = 32 if fmt == "q4k" else 16
    arrs = orc.quantize_weight_q4k(W) if fmt == "q4k" else orc.quantize_weight_q6k(W)
    w = make_weight(raster_amd, ctx, fmt, arrs, out, in_)
    xq, xs, bs = raster_amd.quantize_act_q8k(ctx, dev(torch, x), in_, sub)
    y = w.matmul_q8k(xq, xs, bs).cpu().numpy().ravel()
    w.destroy()
    wdq = orc.dequant_q4k(*arrs, out * in_) if fmt == "q4k" else orc.dequant_q6k(*arrs, out * in_)
    xdq = (xs.cpu().numpy()[0, 0] * xq.cpu().numpy().ravel().astype(np.float32)).astype(np.float32)
    yref = (wdq.reshape(out, in_).astype(np.float64) @ xdq.astype(np.float64)).astype(np.float32)
    assert np.all(np.abs(y - yref) < 1e-2)


@pytest.mark.parametrize("fmt", ["q4k", "q6k"])
@pytest.mark.parametrize("m,out,in_,ydt", [(1, 4096, 4096, "f32"), (5, 1000, 5632, "f32"), (33, 256, 2048, "bf16"),
                                           (2, 14336, 4096, "bf16")])
def test_kquant_qmatmul_f32_x(torch, ctx, orc, fmt, m, out, in_, ydt):
    # rq_qmatmul with a K-quant weight and f32 x: the q8_K quantizer and the
    # K-quant GEMV inside one call, bit for bit the two separate calls; the
    # allocation-free variant gives the same bits
    import ctypes as C

    import raster_amd
    from raster_amd import _lib

    note(f"K-quant rq_qmatmul {fmt} m={m} {out}x{in_} y={ydt}")
    sub = 32 if fmt == "q4k" else 16
    arrs = encode(orc, fmt, out, in_, seed=out + m)
    w = make_weight(raster_amd, ctx, fmt, arrs, out, in_)
    ytype = torch.bfloat16 if ydt == "bf16" else torch.float32
    try:
        x = dev(torch, np.random.default_rng(m).standard_normal(m * in_).astype(np.float32)).reshape(m, in_)
        y1 = w.matmul(x, out_dtype=ytype)
        xq, xs, bs = raster_amd.quantize_act_q8k(ctx, x, in_, sub)
        y2 = w.matmul_q8k(xq, xs, bs, out_dtype=ytype)
        y3 = torch.full((m, out), float("nan"), dtype=ytype, device="cuda")
        yc = _lib.RQ_BF16 if ydt == "bf16" else _lib.RQ_F32
        _lib.call("rq_qmatmul_noalloc", ctx.handle, w.handle, C.c_void_p(x.data_ptr()), _lib.RQ_F32,
                  C.c_void_p(y3.data_ptr()), yc, m, C.c_void_p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        a, b, c = (t.float().cpu().numpy() for t in (y1, y2, y3))
        assert np.all(np.isfinite(a))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
        if ydt == "f32" and out <= 1000:  # and the oracle's bound, end to end
            ref = oracle_y(orc, fmt, arrs, xq.cpu().numpy().ravel(), xs.cpu().numpy().ravel(),
                           bs.cpu().numpy().ravel(), m, in_, out)
            assert orc.normwise_relerr(a, ref) < TOL
    finally:
        w.destroy()


def test_kquant_rejects(torch, ctx, orc):
    import ctypes as C

    import raster_amd
    from raster_amd import RqError
    from raster_amd import workloads as wl
    from raster_amd._lib import RQ_ERR_DTYPE, RQ_ERR_SHAPE, call

    arrs = encode(orc, "q4k", 16, 256, seed=1)
    w = raster_amd.QWeight.q4k(*arrs, 16, 256, ctx)
    with pytest.raises(RqError) as e:  # bf16 activations: the K-quants quantize f32 x to q8_K
        w.matmul(torch.zeros((1, 256), dtype=torch.bfloat16, device="cuda"))
    assert e.value.status == RQ_ERR_DTYPE
    with pytest.raises(RqError) as e:  # no fused decoder ops on the K-quant GEMV
        w.matmul_fused(torch.zeros((1, 256), device="cuda"), residual=torch.zeros((1, 16), device="cuda"))
    assert e.value.status == RQ_ERR_DTYPE
    with pytest.raises(RqError) as e:  # nor the int8 blocks of Q8_0 / Q4_0
        w.matmul_i8(torch.zeros(256, dtype=torch.int8, device="cuda"), torch.zeros(8, device="cuda"))
    assert e.value.status == RQ_ERR_DTYPE
    w.destroy()
    codes, scales = wl.q8_weights(16, 256, seed=1)
    w8 = raster_amd.QWeight.q8(codes, scales, 16, 256, ctx)
    xq, xs, bs = raster_amd.quantize_act_q8k(ctx, torch.zeros(256, device="cuda"), 256, 32)
    y = torch.empty(16, device="cuda")
    with pytest.raises(RqError) as e:  # a Q8_0 weight has no K dot
        call("rq_qmatmul_q8k", ctx.handle, w8.handle, C.c_void_p(xq.data_ptr()), C.c_void_p(xs.data_ptr()),
             C.c_void_p(bs.data_ptr()), C.c_void_p(y.data_ptr()), 0, 1, None)
    assert e.value.status == RQ_ERR_DTYPE
    w8.destroy()
    # in = 192: not whole super-blocks
    z8, zf = np.zeros(4 * 192, np.uint8), np.zeros(4, np.float32)
    h = C.c_void_p()
    with pytest.raises(RqError) as e:
        call("rq_weight_create_q4k", ctx.handle, z8.ctypes.data_as(C.c_void_p), zf.ctypes.data_as(C.c_void_p),
             zf.ctypes.data_as(C.c_void_p), z8.ctypes.data_as(C.c_void_p), z8.ctypes.data_as(C.c_void_p), 4, 192,
             C.byref(h))
    assert e.value.status == RQ_ERR_SHAPE
    # Q6_K codes are 6-bit (the device packs them): a byte above 63 is refused
    wq6, sc6, ds6 = encode(orc, "q6k", 4, 256, seed=2)
    wq6 = wq6.copy()
    wq6[5] = 64
    with pytest.raises(RqError) as e:
        raster_amd.QWeight.q6k(wq6, sc6, ds6, 4, 256, ctx)
    assert e.value.status == RQ_ERR_SHAPE
    # in = 32512: four Q6_K activation rows no longer fit the GEMV's LDS
    z8, zs, zf = np.zeros(4 * 32512, np.uint8), np.zeros(4 * 32512 // 16, np.int8), np.zeros(4 * 127, np.float32)
    with pytest.raises(RqError) as e:
        call("rq_weight_create_q6k", ctx.handle, z8.ctypes.data_as(C.c_void_p), zs.ctypes.data_as(C.c_void_p),
             zf.ctypes.data_as(C.c_void_p), 4, 32512, C.byref(h))
    assert e.value.status == RQ_ERR_SHAPE
