"""GPU parity of the int8-activation path against the C oracle.

rq_quantize_act_i8 restates quantize-act-i8
(raster/compiler/backend/cpu/quant.clj:282-305,399-415): bit-exact codes,
scales and sums (the oracle's restatement is pinned by test_oracle.py against
the quantizer's invariants and Java's rounding).

rq_qmatmul_i8 restates qmatmul-i8-gemm! (raster/quant/kernels_k.clj:357-370)
for Q8_0 weights and the int-activation Q4_0 numerics of
qmatmul-q4-composable (raster/quant/kernels.clj:140-184). The block dots are
exact integers on both sides; the GPU adds the block terms in f32 where Raster
adds in double, so the bar is normwise max|y - ref| / max|ref| < 2e-5 (f32 y)
and 1e-2 (bf16 y).

The fused decode option act_i8 quantizes in the kernel with the quantizer's
own math: without a norm it must equal quantizer + int8 matmul bit for bit.
"""
import numpy as np
import pytest

from raster_amd import workloads as wl

pytestmark = pytest.mark.gpu

TOL_I8 = 2e-5
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


def special_activations(m, in_, seed):
    """N(0, 1) rows with a zero block, exact ties, tiny and huge blocks."""
    x = wl.activations(m, in_, seed=seed).reshape(m, in_)
    x[0, :32] = 0.0
    if in_ >= 64:
        # max 127 -> d = 1, id = 1: x.5 values are exact ties
        x[0, 32:64] = np.array([127.0, -127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5] * 4, np.float32)
    if in_ >= 96:
        x[0, 64:96] *= 1e-30
    if m > 1 and in_ >= 64:
        x[1, 32:64] *= 1e30
    return np.ascontiguousarray(x.ravel())


def gpu_quantize(torch, ctx, x, m, in_):
    import raster_amd

    xq, xs, xsum = raster_amd.quantize_act_i8(ctx, dev(torch, x), in_)
    torch.cuda.synchronize()
    return xq, xs, xsum


@pytest.mark.parametrize("m,in_", [(1, 4096), (7, 96), (3, 32), (64, 8192), (1, 20480)])
def test_quantize_act_i8_bit_exact(torch, ctx, orc, m, in_):
    x = special_activations(m, in_, seed=m + in_)
    note(f"quantize-act-i8 m={m} in={in_}")
    xq, xs, xsum = gpu_quantize(torch, ctx, x, m, in_)
    rq, rs, rsum = orc.quantize_act_i8(x, m, in_)
    assert np.array_equal(xq.cpu().numpy().ravel(), rq)
    assert np.array_equal(xs.cpu().numpy().ravel().view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(xsum.cpu().numpy().ravel(), rsum)


def test_quantize_act_i8_infinite_block(torch, ctx, orc):
    # an infinite element: d = inf, id = 0, every code 0 (x * 0 is NaN or 0,
    # Math/round gives 0 for both); the other blocks are unaffected
    x = wl.activations(2, 64, seed=3)
    x[5] = np.inf
    xq, xs, xsum = gpu_quantize(torch, ctx, x, 2, 64)
    rq, rs, rsum = orc.quantize_act_i8(x, 2, 64)
    assert np.array_equal(xq.cpu().numpy().ravel(), rq)
    assert np.array_equal(xs.cpu().numpy().ravel().view(np.uint32), rs.view(np.uint32))
    assert np.isinf(rs[0]) and np.all(rq[:32] == 0)


def ref_q8(orc, xq, xs, codes, scales, m, in_, out):
    # qmatmul-i8-gemm!: activations and codes as little-endian int32 words
    return orc.qmatmul_i8_gemm(np.ascontiguousarray(xq).view(np.int32), xs, np.ascontiguousarray(codes).view(np.int32),
                               scales, in_, out, m).reshape(m, out)


def ref_q4(orc, xq, xs, xsum, packed, ws32, m, in_, out):
    nb = in_ // 32
    rows = [orc.qmatmul_q4_composable(xq[t * in_:(t + 1) * in_], xs[t * nb:(t + 1) * nb],
                                      xsum[t * nb:(t + 1) * nb], packed, ws32, in_, out) for t in range(m)]
    return np.stack(rows)


def make(raster_amd, ctx, orc, fmt, out, in_, seed):
    """(QWeight, reference y from (xq, xs, xsum, m))."""
    if fmt == "q8":
        codes, scales = wl.q8_weights(out, in_, seed=seed)
        w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
        return w, lambda xq, xs, xsum, m: ref_q8(orc, xq, xs, codes, scales, m, in_, out)
    packed, sc16 = wl.q4_weights(out, in_, seed=seed)
    if fmt == "q4f32":
        ws32 = orc.f16_bits_to_f32(sc16)
        w = raster_amd.QWeight.q4(packed, ws32, out, in_, ctx)
    else:
        ws32 = orc.f16_bits_to_f32(sc16)
        w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
    return w, lambda xq, xs, xsum, m: ref_q4(orc, xq, xs, xsum, packed, ws32, m, in_, out)


def run_i8(torch, ctx, orc, fmt, m, in_, out, seed, ydt="f32"):
    import raster_amd

    x = special_activations(m, in_, seed=seed)
    w, ref = make(raster_amd, ctx, orc, fmt, out, in_, seed=out + in_)
    xq, xs, xsum = gpu_quantize(torch, ctx, x, m, in_)
    y = w.matmul_i8(xq, xs, xsum, out_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32)
    torch.cuda.synchronize()
    y = y.float().cpu().numpy()
    w.destroy()
    r = ref(xq.cpu().numpy().ravel(), xs.cpu().numpy().ravel(), xsum.cpu().numpy().ravel(), m)
    return y, r


@pytest.mark.parametrize("m,in_,out", [(1, 4096, 4096), (3, 96, 40), (16, 4096, 64), (2, 20480, 32), (5, 160, 33),
                                       (1, 160, 33), (1, 14336, 64), (1, 416, 520)])
@pytest.mark.parametrize("fmt", ["q8", "q4", "q4f32"])
def test_qmatmul_i8_decode(torch, ctx, orc, m, in_, out, fmt):
    note(f"qmatmul-i8 decode {fmt} m={m} {out}x{in_}")
    y, r = run_i8(torch, ctx, orc, fmt, m, in_, out, seed=m * 7 + in_)
    assert orc.normwise_relerr(y, r) < TOL_I8


@pytest.mark.parametrize("m,in_,out", [(17, 256, 48), (64, 4096, 1000), (200, 1024, 40), (512, 4096, 512)])
@pytest.mark.parametrize("fmt", ["q8", "q4", "q4f32"])
def test_qmatmul_i8_gemm(torch, ctx, orc, m, in_, out, fmt):
    note(f"qmatmul-i8 gemm {fmt} m={m} {out}x{in_}")
    y, r = run_i8(torch, ctx, orc, fmt, m, in_, out, seed=m + in_)
    assert orc.normwise_relerr(y, r) < TOL_I8


@pytest.mark.parametrize("m", [1, 300])
def test_qmatmul_i8_bf16_out(torch, ctx, orc, m):
    y, r = run_i8(torch, ctx, orc, "q8", m, 2048, 256, seed=5, ydt="bf16")
    assert orc.normwise_relerr(y, r) < TOL_BF16


@pytest.mark.parametrize("m,in_,out", [(1, 2048, 2048), (4, 4096, 96), (2, 20480, 16), (1, 160, 33), (1, 14336, 48)])
@pytest.mark.parametrize("fmt", ["q8", "q4", "q4f32"])
def test_fused_act_i8_equals_two_step(torch, ctx, orc, m, in_, out, fmt):
    # quantizing inside the decode kernel gives the quantizer's codes, so the
    # fused call equals rq_quantize_act_i8 + rq_qmatmul_i8 bit for bit
    import raster_amd

    x = special_activations(m, in_, seed=in_ + m)
    w, ref = make(raster_amd, ctx, orc, fmt, out, in_, seed=out)
    xd = dev(torch, x).reshape(m, in_)
    y1 = w.matmul_fused(xd, act_i8=True)
    xq, xs, xsum = raster_amd.quantize_act_i8(ctx, xd.reshape(-1), in_)
    y2 = w.matmul_i8(xq, xs, xsum)
    torch.cuda.synchronize()
    w.destroy()
    assert torch.equal(y1, y2)
    r = ref(xq.cpu().numpy().ravel(), xs.cpu().numpy().ravel(), xsum.cpu().numpy().ravel(), m)
    assert orc.normwise_relerr(y1.cpu().numpy(), r) < TOL_I8


@pytest.mark.parametrize("m,in_,out", [(1, 4096, 256), (3, 416, 40)])
def test_fused_act_i8_bf16_x(torch, ctx, orc, m, in_, out):
    # bf16 activations widen exactly to f32: the fused quantization of bf16 x
    # equals rq_quantize_act_i8 of the widened rows, then rq_qmatmul_i8
    import raster_amd

    x = special_activations(m, in_, seed=in_ - m)
    w, _ = make(raster_amd, ctx, orc, "q4", out, in_, seed=out + 1)
    xb = dev(torch, x).reshape(m, in_).to(torch.bfloat16)
    y1 = w.matmul_fused(xb, act_i8=True)
    xq, xs, xsum = raster_amd.quantize_act_i8(ctx, xb.float().reshape(-1), in_)
    y2 = w.matmul_i8(xq, xs, xsum)
    torch.cuda.synchronize()
    w.destroy()
    assert torch.equal(y1, y2)


def test_fused_norm_act_i8(torch, ctx, orc):
    # Raster's int chain: rms-norm, quantize-act-i8, qmatmul-q4-composable.
    # The kernel quantizes x * gain and applies 1/rms to the result, so codes
    # may differ from the reference chain's by rounding: compared at 1e-3
    import raster_amd

    m, in_, out, eps = 2, 2048, 512, 1e-5
    x = wl.activations(m, in_, seed=1)
    g = np.random.default_rng(2).uniform(0.5, 1.5, in_).astype(np.float32)
    w, ref = make(raster_amd, ctx, orc, "q4", out, in_, seed=3)
    y = w.matmul_fused(dev(torch, x).reshape(m, in_), norm_gain=dev(torch, g), norm_eps=eps, act_i8=True)
    torch.cuda.synchronize()
    w.destroy()
    xn = orc.rms_norm(x, g, m, in_, eps, 0.0)
    rq, rs, rsum = orc.quantize_act_i8(xn, m, in_)
    r = ref(rq, rs, rsum, m)
    assert orc.normwise_relerr(y.cpu().numpy(), r) < 1e-3


def test_qmatmul_i8_rejects(torch, ctx):
    import raster_amd
    from raster_amd import RqError
    from raster_amd._lib import RQ_ERR_NULL

    packed, sc16 = wl.q4_weights(32, 64, seed=1)
    w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), 32, 64, ctx)
    xq = torch.zeros((1, 64), dtype=torch.int8, device="cuda")
    xs = torch.ones((1, 2), device="cuda")
    with pytest.raises(RqError) as e:
        w.matmul_i8(xq, xs, None)  # Q4_0 needs the sums
    assert e.value.status == RQ_ERR_NULL
    w.destroy()
