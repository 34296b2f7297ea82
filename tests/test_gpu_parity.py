"""GPU parity: the gfx950 kernels behind librq against the C oracle.

Bars (from the workload definition):
  * dequantized weights: bit-exact (IEEE f32 of scale * code);
  * outputs: normwise max|y - ref| / max|ref| < 1e-3 for f32 activations and
    < 1e-2 for bf16 activations or bf16 outputs
    (normwise as in test/raster/dl/decoder_layer_gpu_test.clj:17 of the reference).
Full-size configurations are checked on a subset of output rows where the
scalar oracle would otherwise take minutes; the subset always includes the
first and last rows and a spread in between.
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


def rows_subset(n, count):
    if n <= count:
        return np.arange(n)
    idx = np.unique(np.concatenate([[0, n - 1], np.linspace(0, n - 1, count - 2).astype(np.int64)]))
    return idx


def dev(torch, a, dtype="f32"):
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    return t.to(torch.bfloat16) if dtype == "bf16" else t


def run(torch, w, x_np, m, xdt, ydt):
    import raster_amd

    x = dev(torch, x_np, xdt).reshape(m, w.in_)
    y = w.matmul(x, out_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


# ---------------------------------------------------------------- dequant tiles
@pytest.mark.parametrize("out,in_", [(4096, 4096), (37, 96)])
def test_dequant_q8_bit_exact(torch, ctx, orc, out, in_):
    import raster_amd

    codes, scales = wl.q8_weights(out, in_, seed=0)
    note(f"dequant q8 {out}x{in_}")
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    got = w.dequant().cpu().numpy().ravel()
    w.destroy()
    ref = orc.dequant_q8_dense(codes, scales, in_, out)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("scale_kind", ["f16", "f32"])
@pytest.mark.parametrize("out,in_", [(14336, 4096), (13, 64)])
def test_dequant_q4_bit_exact(torch, ctx, orc, out, in_, scale_kind):
    import raster_amd

    packed, sc16 = wl.q4_weights(out, in_, seed=0)
    scales = sc16 if scale_kind == "f16" else sc16.view(np.float16).astype(np.float32)
    note(f"dequant q4 {out}x{in_} {scale_kind}")
    w = raster_amd.QWeight.q4(packed, scales if scale_kind == "f32" else sc16.view(np.float16), out, in_, ctx)
    got = w.dequant().cpu().numpy().ravel()
    w.destroy()
    ref = orc.dequant_q4(packed, sc16 if scale_kind == "f16" else scales, in_, out)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_q8_extreme_codes(torch, ctx, orc):
    import raster_amd

    out, in_ = 8, 256
    codes = np.tile(np.array([-128, 127, 0, -1, 1, -127, 64, -64], np.int8), out * in_ // 8)
    scales = np.full(out * in_ // 32, 0.0173, np.float32)
    scales[3] = 0.0
    scales[5] = np.float32(3.4e38) / 128
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    got = w.dequant().cpu().numpy().ravel()
    w.destroy()
    ref = orc.dequant_q8_dense(codes, scales, in_, out)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


# ---------------------------------------------------------------- GEMV (m <= 16)
@pytest.mark.parametrize("m", [1, 2, 3, 5, 16])
def test_gemv_q8_f32(torch, ctx, orc, m):
    import raster_amd

    out, in_ = (4096, 4096) if m == 1 else (300, 1024)
    codes, scales = wl.q8_weights(out, in_, seed=m)
    x = wl.activations(m, in_, seed=10 + m)
    note(f"gemv q8 f32 m={m} {out}x{in_}")
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    y = run(torch, w, x, m, "f32", "f32")
    w.destroy()
    ref = orc.qlinear_q8(x, codes, scales, m, in_, out).reshape(m, out)
    assert orc.normwise_relerr(y, ref) < TOL_F32


@pytest.mark.parametrize("m", [1, 4, 16])
def test_gemv_q4_f16_scales_c3(torch, ctx, orc, m):
    import raster_amd

    out, in_ = 14336, 4096
    packed, sc16 = wl.q4_weights(out, in_, seed=3)
    x = wl.activations(m, in_, seed=30 + m)
    note(f"gemv q4 f32 m={m} {out}x{in_}")
    w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
    y = run(torch, w, x, m, "f32", "f32")
    w.destroy()
    rows = rows_subset(out, 1024 if m > 1 else out)
    pk = packed.reshape(out, in_ // 2)[rows].ravel()
    sc = sc16.reshape(out, in_ // 32)[rows].ravel()
    ref = orc.qlinear_q4(x, pk, sc, m, in_, len(rows)).reshape(m, len(rows))
    assert orc.normwise_relerr(y[:, rows], ref) < TOL_F32


@pytest.mark.parametrize("fmt", ["q8", "q4"])
@pytest.mark.parametrize("m", [1, 7])
def test_gemv_bf16_in_bf16_out(torch, ctx, orc, fmt, m):
    import raster_amd

    out, in_ = 520, 8192
    x = wl.activations(m, in_, seed=50 + m, dtype="bf16")
    note(f"gemv {fmt} bf16 m={m} {out}x{in_}")
    if fmt == "q8":
        codes, scales = wl.q8_weights(out, in_, seed=5)
        w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
        ref = orc.qlinear_q8(x, codes, scales, m, in_, out)
    else:
        packed, sc16 = wl.q4_weights(out, in_, seed=5)
        w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
        ref = orc.qlinear_q4(x, packed, sc16, m, in_, out)
    y = run(torch, w, x, m, "bf16", "bf16")
    y32 = run(torch, w, x, m, "bf16", "f32")
    w.destroy()
    ref = ref.reshape(m, out)
    assert orc.normwise_relerr(y, ref) < TOL_BF16
    assert orc.normwise_relerr(y32, ref) < TOL_F32
    # the bf16 output is the RNE rounding of the kernel's own f32 result
    assert np.array_equal(orc.f32_to_bf16_bits(y32), orc.f32_to_bf16_bits(y))


# ---------------------------------------------------------------- GEMM (m > 16)
def test_gemm_q8_bf16_c2(torch, ctx, orc):
    import raster_amd

    m, in_, out = 512, 4096, 11008
    codes, scales = wl.q8_weights(out, in_, seed=2)
    x = wl.activations(m, in_, seed=20, dtype="bf16")
    note(f"gemm q8 bf16 m={m} {out}x{in_}")
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    y = run(torch, w, x, m, "bf16", "bf16")
    w.destroy()
    rows = rows_subset(out, 192)
    cs = codes.reshape(out, in_)[rows].ravel()
    ss = scales.reshape(out, in_ // 32)[rows].ravel()
    ref = orc.qlinear_q8(x, cs, ss, m, in_, len(rows)).reshape(m, len(rows))
    assert orc.normwise_relerr(y[:, rows], ref) < TOL_BF16


@pytest.mark.parametrize("m,in_,out", [(17, 32, 8), (129, 96, 100), (300, 256, 130), (64, 1024, 257)])
@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_gemm_ragged_f32(torch, ctx, orc, m, in_, out, fmt):
    import raster_amd

    x = wl.activations(m, in_, seed=m + out)
    note(f"gemm {fmt} f32 m={m} {out}x{in_}")
    if fmt == "q8":
        codes, scales = wl.q8_weights(out, in_, seed=out)
        w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
        ref = orc.qlinear_q8(x, codes, scales, m, in_, out)
    else:
        packed, sc16 = wl.q4_weights(out, in_, seed=out)
        w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
        ref = orc.qlinear_q4(x, packed, sc16, m, in_, out)
    y = run(torch, w, x, m, "f32", "f32")
    w.destroy()
    assert orc.normwise_relerr(y, ref.reshape(m, out)) < TOL_F32


@pytest.mark.parametrize("m,in_,out", [(17, 32, 8), (100, 64, 100), (129, 96, 130), (300, 160, 257),
                                       (257, 224, 96), (64, 416, 200), (520, 1024, 190)])
@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_gemm_bf16_ragged(torch, ctx, orc, m, in_, out, fmt):
    # bf16 activations take the dequantize-to-LDS MFMA kernel: K-block counts
    # 1, 2, 3, 5, 7, 13 and 32 exercise every tail of its 6-step unrolled
    # pipeline; M and N are ragged against the 64/128/256 x 64/96/128 tiles.
    import raster_amd

    x = wl.activations(m, in_, seed=3 * m + out, dtype="bf16")
    note(f"gemm {fmt} bf16 m={m} {out}x{in_}")
    if fmt == "q8":
        codes, scales = wl.q8_weights(out, in_, seed=out + 1)
        w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
        ref = orc.qlinear_q8(x, codes, scales, m, in_, out)
    else:
        packed, sc16 = wl.q4_weights(out, in_, seed=out + 1)
        w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
        ref = orc.qlinear_q4(x, packed, sc16, m, in_, out)
    y32 = run(torch, w, x, m, "bf16", "f32")
    y16 = run(torch, w, x, m, "bf16", "bf16")
    w.destroy()
    ref = ref.reshape(m, out)
    assert orc.normwise_relerr(y32, ref) < TOL_BF16
    assert orc.normwise_relerr(y16, ref) < TOL_BF16
    assert np.array_equal(orc.f32_to_bf16_bits(y32), orc.f32_to_bf16_bits(y16))


@pytest.mark.parametrize("m,in_,out", [(500, 96, 12004), (300, 416, 12000), (512, 1024, 11008), (200, 96, 27999),
                                       (256, 416, 28000), (300, 32, 12004), (300, 64, 12004), (300, 288, 12004)])
@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_gemm_bf16_wide_tiles(torch, ctx, orc, m, in_, out, fmt):
    # wide N: the tile cost model picks an 8-wave tile, one workgroup per CU
    # (256 x 96 near m = 512, 256 x 112 near N = 28672 at m <= 256): the
    # role-split 32x32x16 kernel where K is a multiple of 64 (one macro step at
    # K = 64; rows of N = 12004 in bf16 are not whole 16-byte pieces, so its
    # direct stores run), else the 16x16x32 kernel whose wave pairs split K
    # into even and odd blocks; ragged M and N, 1, 2, 3, 9 (one full ring turn
    # and half a step) and 13 K-blocks
    import raster_amd

    x = wl.activations(m, in_, seed=m + in_, dtype="bf16")
    note(f"gemm wide {fmt} bf16 m={m} {out}x{in_}")
    rows = rows_subset(out, 384)
    if fmt == "q8":
        codes, scales = wl.q8_weights(out, in_, seed=out)
        w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
        cs = codes.reshape(out, in_)[rows].ravel()
        ss = scales.reshape(out, in_ // 32)[rows].ravel()
        ref = orc.qlinear_q8(x, cs, ss, m, in_, len(rows))
    else:
        packed, sc16 = wl.q4_weights(out, in_, seed=out)
        w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
        pk = packed.reshape(out, in_ // 2)[rows].ravel()
        ss = sc16.reshape(out, in_ // 32)[rows].ravel()
        ref = orc.qlinear_q4(x, pk, ss, m, in_, len(rows))
    y32 = run(torch, w, x, m, "bf16", "f32")
    y16 = run(torch, w, x, m, "bf16", "bf16")
    w.destroy()
    assert orc.normwise_relerr(y32[:, rows], ref.reshape(m, len(rows))) < TOL_BF16
    assert np.array_equal(orc.f32_to_bf16_bits(y32), orc.f32_to_bf16_bits(y16))


@pytest.mark.parametrize("m,in_,out", [(17, 4096, 520), (32, 8192, 256), (48, 2080, 100), (64, 8192, 96),
                                       (33, 256, 14336), (20, 96, 40)])
@pytest.mark.parametrize("scale_kind", ["f16", "f32"])
def test_gemm_small_m_q4_kslices(torch, ctx, orc, m, in_, out, scale_kind):
    # Q4_0 with bf16 activations and 16 < m <= 64 takes the small-m GEMM: K is
    # cut into up to 8 slices when the grid would be thin (narrow N, long K),
    # their partial sums added in slice order, so two calls agree bit for bit.
    import raster_amd

    x = wl.activations(m, in_, seed=7 * m + out, dtype="bf16")
    packed, sc16 = wl.q4_weights(out, in_, seed=in_ + out)
    note(f"gemm-sm q4 {scale_kind} m={m} {out}x{in_}")
    scales = sc16.view(np.float16) if scale_kind == "f16" else orc.f16_bits_to_f32(sc16)
    w = raster_amd.QWeight.q4(packed, scales, out, in_, ctx)
    y32 = run(torch, w, x, m, "bf16", "f32")
    y32b = run(torch, w, x, m, "bf16", "f32")
    y16 = run(torch, w, x, m, "bf16", "bf16")
    w.destroy()
    assert np.array_equal(y32, y32b)
    assert np.array_equal(orc.f32_to_bf16_bits(y32), orc.f32_to_bf16_bits(y16))
    rows = rows_subset(out, 256)
    pk = packed.reshape(out, in_ // 2)[rows].ravel()
    ss = sc16.reshape(out, in_ // 32)[rows].ravel()
    ref = orc.qlinear_q4(x, pk, ss, m, in_, len(rows)).reshape(m, len(rows))
    assert orc.normwise_relerr(y32[:, rows], ref) < TOL_BF16


@pytest.mark.parametrize("m,in_,out", [(17, 4096, 520), (32, 8192, 256), (48, 2080, 100), (64, 8192, 96),
                                       (64, 4096, 96), (33, 256, 14336), (20, 96, 40)])
def test_gemm_small_m_q8_kslices(torch, ctx, orc, m, in_, out):
    # Q8_0 with bf16 activations takes the small-m GEMM at 16 < m <= 48, and
    # to m = 64 from in = 8192 (m = 64 at in 4096 stays on the per-wave GEMM):
    # K-slices added in slice order, so two calls agree bit for bit
    import raster_amd

    x = wl.activations(m, in_, seed=5 * m + out, dtype="bf16")
    codes, scales = wl.q8_weights(out, in_, seed=in_ + out)
    note(f"gemm-sm q8 m={m} {out}x{in_}")
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    y32 = run(torch, w, x, m, "bf16", "f32")
    y32b = run(torch, w, x, m, "bf16", "f32")
    y16 = run(torch, w, x, m, "bf16", "bf16")
    w.destroy()
    assert np.array_equal(y32, y32b)
    assert np.array_equal(orc.f32_to_bf16_bits(y32), orc.f32_to_bf16_bits(y16))
    rows = rows_subset(out, 256)
    cs = codes.reshape(out, in_)[rows].ravel()
    ss = scales.reshape(out, in_ // 32)[rows].ravel()
    ref = orc.qlinear_q8(x, cs, ss, m, in_, len(rows)).reshape(m, len(rows))
    assert orc.normwise_relerr(y32[:, rows], ref) < TOL_BF16


# ---------------------------------------------------------------- decode kernel edges
@pytest.mark.parametrize("m,in_,out", [(1, 32, 16), (3, 96, 40), (16, 160, 33), (5, 4096, 48), (16, 4096, 64)])
@pytest.mark.parametrize("fmt", ["q8", "q4"])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_decode_shapes_and_error_bound(torch, ctx, orc, m, in_, out, fmt, xdt):
    # odd block counts (1, 3, 5 blocks: a half window at the end), ragged
    # output rows, every m-group size; error inside the derived bound
    import raster_amd

    x = wl.activations(m, in_, seed=11 * m + in_, dtype=xdt)
    note(f"decode {fmt} {xdt} m={m} {out}x{in_}")
    if fmt == "q8":
        codes, scales = wl.q8_weights(out, in_, seed=out + in_)
        w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
        ref = orc.qlinear_q8(x, codes, scales, m, in_, out)
        dense = orc.dequant_q8_dense(codes, scales, in_, out)
    else:
        packed, sc16 = wl.q4_weights(out, in_, seed=out + in_)
        w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
        ref = orc.qlinear_q4(x, packed, sc16, m, in_, out)
        dense = orc.dequant_q4(packed, sc16, in_, out)
    y = run(torch, w, x, m, xdt, "f32")
    w.destroy()
    ref = ref.reshape(m, out)
    assert orc.normwise_relerr(y, ref) < TOL_F32
    assert np.all(np.abs(y - ref) <= decomposition_bound(x, dense, m, in_, out))


def test_decode_special_activations(torch, ctx, orc):
    # per-block exponents: a block with 1e30 next to 1e-30, a zero row, an
    # inf row and a NaN row; finite rows stay inside the bound, the zero row
    # is exactly zero, and rows with a non-finite activation are non-finite
    # (the kernel writes NaN; Raster's f32 loop gives +-inf or NaN)
    import raster_amd

    m, in_, out = 6, 128, 24
    codes, scales = wl.q8_weights(out, in_, seed=5)
    x = wl.activations(m, in_, seed=6).reshape(m, in_)
    x[1, 0], x[1, 1] = 1e30, 1e-30
    x[1, 40:64] *= 1e-20
    x[2] = 0.0
    x[3, 70] = np.inf
    x[4, 5] = np.nan
    x[5] *= 1e-35                       # subnormal-range block maxima
    x = np.ascontiguousarray(x.ravel())
    note("decode special activations")
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    y = run(torch, w, x, m, "f32", "f32")
    w.destroy()
    ref = orc.qlinear_q8(x, codes, scales, m, in_, out).reshape(m, out)
    dense = orc.dequant_q8_dense(codes, scales, in_, out)
    fin = [0, 1, 2, 5]
    xf = x.reshape(m, in_)[fin].ravel()
    bound = decomposition_bound(xf, dense, len(fin), in_, out)
    assert np.all(np.abs(y[fin] - ref[fin]) <= bound)
    assert np.all(y[2] == 0.0)
    assert not np.any(np.isfinite(y[3])) and not np.any(np.isfinite(y[4]))
    assert not np.any(np.isfinite(ref[3])) and not np.any(np.isfinite(ref[4]))


@pytest.mark.parametrize("m,in_,out", [(2, 20480, 16), (12, 8192, 4160), (16, 8192, 48), (9, 4096, 4096),
                                       (16, 14336, 64)])
def test_decode_k_split(torch, ctx, orc, m, in_, out):
    # K cut into slices whose partial sums a second kernel adds in slice order.
    # m = 2 and m = 12 over a weight above 32 Mi elements (34 Mi at 4160 x 8192):
    # the int8-level decode kernel, its activations too long for one
    # workgroup's LDS. The m = 9 / 16 rows below 32 Mi elements: the MFMA
    # decode kernel, whose slices also spread a thin grid over the CUs.
    import raster_amd

    codes, scales = wl.q8_weights(out, in_, seed=8)
    x = wl.activations(m, in_, seed=9)
    note(f"decode k-split m={m} in={in_} out={out}")
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    y = run(torch, w, x, m, "f32", "f32")
    y2 = run(torch, w, x, m, "f32", "f32")
    yb = run(torch, w, x, m, "bf16", "bf16")
    w.destroy()
    assert np.array_equal(y, y2), "split sums must be deterministic"
    rows = rows_subset(out, 48)
    ref = orc.qlinear_q8(x, codes.reshape(out, in_)[rows].ravel(), scales.reshape(out, -1)[rows].ravel(),
                         m, in_, len(rows)).reshape(m, len(rows))
    assert orc.normwise_relerr(y[:, rows], ref) < TOL_F32
    dense = orc.dequant_q8_dense(codes.reshape(out, in_)[rows].ravel(), scales.reshape(out, -1)[rows].ravel(),
                                 in_, len(rows))
    bound = decomposition_bound(x.reshape(m, in_), dense, m, in_, len(rows))
    assert np.all(np.abs(y[:, rows] - ref) <= bound)
    refb = orc.qlinear_q8(wl.bf16_round(x), codes.reshape(out, in_)[rows].ravel(),
                          scales.reshape(out, -1)[rows].ravel(), m, in_, len(rows)).reshape(m, len(rows))
    assert orc.normwise_relerr(yb[:, rows], refb) < TOL_BF16


def test_decode_split_scratch_reuse_across_shapes(torch, ctx, orc):
    # one stream, split calls of growing and shrinking group counts: every call
    # must find its counters at zero (left there by the previous call)
    import raster_amd

    for out, in_, m in ((16, 4096, 1), (64, 8192, 3), (32, 2048, 4), (16, 4096, 1)):
        codes, scales = wl.q8_weights(out, in_, seed=out + in_)
        x = wl.activations(m, in_, seed=m)
        w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
        y = run(torch, w, x, m, "f32", "f32")
        w.destroy()
        ref = orc.qlinear_q8(x, codes, scales, m, in_, out).reshape(m, out)
        assert orc.normwise_relerr(y, ref) < TOL_F32, (out, in_, m)


def test_gemm_q4_bf16_m256(torch, ctx, orc):
    import raster_amd

    m, in_, out = 256, 8192, 1536
    packed, sc16 = wl.q4_weights(out, in_, seed=7)
    x = wl.activations(m, in_, seed=70, dtype="bf16")
    note(f"gemm q4 bf16 m={m} {out}x{in_}")
    w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
    y = run(torch, w, x, m, "bf16", "bf16")
    w.destroy()
    rows = rows_subset(out, 128)
    pk = packed.reshape(out, in_ // 2)[rows].ravel()
    sc = sc16.reshape(out, in_ // 32)[rows].ravel()
    ref = orc.qlinear_q4(x, pk, sc, m, in_, len(rows)).reshape(m, len(rows))
    assert orc.normwise_relerr(y[:, rows], ref) < TOL_BF16


def test_zero_scale_blocks_and_zero_rows(torch, ctx, orc):
    import raster_amd

    m, in_, out = 40, 128, 24
    codes, scales = wl.q8_weights(out, in_, seed=9)
    scales.reshape(out, -1)[5, :] = 0.0
    scales.reshape(out, -1)[:, 2] = 0.0
    x = wl.activations(m, in_, seed=90)
    x.reshape(m, in_)[3] = 0.0
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    for mm in (m, 4):
        note(f"zero-scale q8 m={mm}")
        y = run(torch, w, x[: mm * in_], mm, "f32", "f32")
        ref = orc.qlinear_q8(x[: mm * in_], codes, scales, mm, in_, out).reshape(mm, out)
        assert orc.normwise_relerr(y, ref) < TOL_F32
        assert np.all(y[:, 5] == 0.0)
        if mm > 3:
            assert np.all(y[3] == 0.0)
    w.destroy()


@pytest.mark.parametrize("m,in_,out,route", [(40, 128, 24, "small-m GEMM"), (100, 128, 40, "64 < m <= 128 GEMM"),
                                             (300, 128, 11008, "role-split 256 x 96"),
                                             (1024, 128, 11008, "one wave per SIMD, 256 x 192")])
@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_gemm_bf16_special_values(torch, ctx, orc, m, in_, out, route, fmt):
    # every bf16-activation GEMM route with a weight row whose scales are all
    # zero (output column 5), a zero scale block column, a zero activation
    # row (3), an inf (row 7) and a NaN (row 9) activation: finite rows match
    # the oracle, column 5 and row 3 are exactly zero, rows 7 and 9 are
    # non-finite in every column (inf times a zero weight is NaN)
    import raster_amd

    note(f"gemm bf16 special values {fmt} {route} m={m} {out}x{in_}")
    x = wl.activations(m, in_, seed=m + 3, dtype="bf16").reshape(m, in_)
    x[3] = 0.0
    x[7, 70] = np.inf
    x[9, 5] = np.nan
    x = np.ascontiguousarray(x.ravel())
    cols = np.union1d(rows_subset(out, 256), [5])
    if fmt == "q8":
        codes, scales = wl.q8_weights(out, in_, seed=out + 1)
        scales.reshape(out, -1)[5, :] = 0.0
        scales.reshape(out, -1)[:, 2] = 0.0
        w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
        ref = orc.qlinear_q8(x, codes.reshape(out, in_)[cols].ravel(),
                             scales.reshape(out, -1)[cols].ravel(), m, in_, len(cols))
    else:
        packed, sc16 = wl.q4_weights(out, in_, seed=out + 1)
        s = sc16.view(np.float16)
        s.reshape(out, -1)[5, :] = 0.0
        s.reshape(out, -1)[:, 2] = 0.0
        w = raster_amd.QWeight.q4(packed, s, out, in_, ctx)
        ref = orc.qlinear_q4(x, packed.reshape(out, -1)[cols].ravel(), s.view(np.uint16).reshape(out, -1)[cols].ravel(),
                             m, in_, len(cols))
    y = run(torch, w, x, m, "bf16", "f32")
    w.destroy()
    ref = ref.reshape(m, len(cols))
    fin = np.setdiff1d(np.arange(m), [7, 9])
    assert orc.normwise_relerr(y[fin][:, cols], ref[fin]) < TOL_BF16
    assert np.all(y[fin, 5] == 0.0)
    assert np.all(y[3] == 0.0)
    assert not np.any(np.isfinite(y[7])) and not np.any(np.isfinite(y[9]))


@pytest.mark.parametrize("m,in_,out", [(40, 128, 24), (100, 128, 40), (300, 128, 11008), (1024, 128, 11008)])
@pytest.mark.parametrize("ydt", ["f32", "bf16"])
def test_gemm_output_one_element_off_alignment(torch, ctx, orc, m, in_, out, ydt):
    # y may start at any element (only x must be 16-byte aligned): the bf16-x
    # GEMM routes (small-m, 64 < m <= 128, role-split, 256 x 192) then store
    # element by element instead of staging whole 16-byte row pieces, and
    # must give the aligned call's bits
    import raster_amd

    note(f"gemm misaligned y {ydt} m={m} {out}x{in_}")
    codes, scales = wl.q8_weights(out, in_, seed=out + 2)
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    x = dev(torch, wl.activations(m, in_, seed=m + 4, dtype="bf16"), "bf16").reshape(m, in_)
    dt = torch.bfloat16 if ydt == "bf16" else torch.float32
    ya = w.matmul(x, out_dtype=dt)
    buf = torch.full((m * out + 1,), 7.0, dtype=dt, device="cuda")
    yb = buf[1:].view(m, out)
    assert yb.data_ptr() % 16 != 0
    w.matmul(x, y=yb)
    torch.cuda.synchronize()
    w.destroy()
    assert torch.equal(ya, yb)
    assert buf[0].item() == 7.0


# ---------------------------------------------------------------- ingestion formats
@pytest.mark.parametrize("nibble", [True, False])
def test_x8_layout_ingestion(torch, ctx, orc, nibble):
    import raster_amd

    rng = np.random.default_rng(31)
    out, in_, m = 64, 512, 3
    wf = rng.uniform(-0.5, 0.5, out * in_).astype(np.float32)
    if nibble:
        wq, ws = orc.quantize_weight_q4(wf)
    else:
        wq, ws = orc.quantize_weight_q8u(wf)
    wqi, wsi = orc.repack_x8(wq, ws, out, in_, nibble)
    note(f"x8 ingest nibble={nibble}")
    w = raster_amd.QWeight.x8(wqi, wsi, nibble, out, in_, ctx)
    got = w.dequant().cpu().numpy().ravel()
    zp = 8 if nibble else 128
    ref = orc.dequant_weight(wq, ws, out * in_, zp, nibble)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    x = wl.activations(m, in_, seed=32)
    y = run(torch, w, x, m, "f32", "f32")
    w.destroy()
    dense = orc.dense_matmul_nt_f64(x, ref, m, in_, out).reshape(m, out)
    assert orc.normwise_relerr(y, dense) < TOL_F32


def test_q8_packed_ingestion(torch, ctx, orc):
    import raster_amd

    rng = np.random.default_rng(33)
    out, in_, m = 40, 256, 20
    W = rng.standard_normal(out * in_).astype(np.float32)
    wp, ws = orc.quantize_one_q8(W, in_, out)
    note("q8 packed ingest")
    w = raster_amd.QWeight.q8_packed(wp, ws, out, in_, ctx)
    x = wl.activations(m, in_, seed=34)
    y = run(torch, w, x, m, "f32", "f32")
    w.destroy()
    ref = orc.qlinear_q8(x, wp.view(np.int8), ws, m, in_, out).reshape(m, out)
    assert orc.normwise_relerr(y, ref) < TOL_F32


# ---------------------------------------------------------------- host surface + errors
def decomposition_bound(x, wdense, m, in_, out):
    """Per-output bound on |decode kernel - exact| for f32/bf16 activations:
    the kernel rounds each activation to a 16-bit block fixed point with
    |error| <= 2^(e-16) (e from frexp of the block max, raised by one where
    max * 2^(15-e) > 32639), so |dy[m,o]| <= sum_b 2^(e_mb-16) sum_k |W[o,k]|,
    plus f32 accumulation slack."""
    xb = np.abs(np.asarray(x, np.float64).reshape(m, in_ // 32, 32))
    amax = xb.max(axis=2)
    _, e = np.frexp(amax)
    e = np.where(amax > 0, e, 0)
    e = np.where(np.ldexp(amax, 15 - e) > 32639.0, e + 1, e)
    step = np.ldexp(1.0, e - 16)                                 # [m, nb]
    wabs = np.abs(np.asarray(wdense, np.float64).reshape(out, in_ // 32, 32)).sum(axis=2)  # [out, nb]
    bound = step @ wabs.T                                        # [m, out]
    mag = np.abs(np.asarray(x, np.float64).reshape(m, in_)) @ np.abs(np.asarray(wdense, np.float64).reshape(out, in_)).T
    return bound + 1e-6 * mag + 1e-30


def test_qlinear_q8_host_surface(torch, ctx, orc):
    # the shapes of test/raster/quant/train_test.clj:26-40
    import raster_amd

    out, in_, m = 4, 64, 2
    W = orc.jfill_gauss(1, 0.3, out * in_)
    X = orc.jfill_gauss(2, 0.3, m * in_)
    codes, scales = orc.q8_quantize(W, out, in_)
    note("qlinear_q8 host")
    y = raster_amd.qlinear_q8(X, codes, scales, m, in_, out, ctx=ctx)
    ref = orc.qlinear_q8(X, codes, scales, m, in_, out)
    assert orc.normwise_relerr(y, ref) < TOL_F32
    dense = orc.dequant_q8_dense(codes, scales, in_, out)
    bound = decomposition_bound(X, dense, m, in_, out)
    assert np.all(np.abs(y.reshape(m, out) - ref.reshape(m, out)) <= bound)
    Wd = raster_amd.dequant_q8_dense(codes, scales, in_, out, ctx=ctx)
    assert np.array_equal(Wd, orc.dequant_q8_dense(codes, scales, in_, out))
    with pytest.raises(AssertionError):
        raster_amd.qlinear_q8(np.zeros(30, np.float32), np.zeros(30, np.int8), np.zeros(1, np.float32), 1, 30, 1)


def test_error_statuses_on_gpu(torch, ctx):
    import ctypes as C

    import raster_amd
    from raster_amd import _lib

    L = _lib.lib()
    codes, scales = wl.q8_weights(8, 64, seed=1)
    w = raster_amd.QWeight.q8(codes, scales, 8, 64, ctx)
    x = torch.zeros((2, 64), device="cuda")
    y = torch.zeros((2, 8), device="cuda")
    xp, yp = C.c_void_p(x.data_ptr()), C.c_void_p(y.data_ptr())
    assert L.rq_qmatmul(ctx.handle, w.handle, xp, 7, yp, 0, 2, None) == _lib.RQ_ERR_DTYPE
    assert L.rq_qmatmul(ctx.handle, w.handle, xp, 0, yp, 0, -1, None) == _lib.RQ_ERR_SHAPE
    assert L.rq_qmatmul(ctx.handle, w.handle, None, 0, yp, 0, 2, None) == _lib.RQ_ERR_NULL
    assert L.rq_qmatmul(ctx.handle, w.handle, C.c_void_p(x.data_ptr() + 4), 0, yp, 0, 1, None) == _lib.RQ_ERR_SHAPE
    assert L.rq_qmatmul(ctx.handle, w.handle, xp, 0, yp, 0, 0, None) == _lib.RQ_OK
    h = C.c_void_p()
    assert L.rq_weight_create_q8(ctx.handle, codes.ctypes.data_as(C.c_void_p),
                                 scales.ctypes.data_as(C.c_void_p), 8, 60, C.byref(h)) == _lib.RQ_ERR_SHAPE
    assert b"multiple of 32" in L.rq_last_error()
    big = C.c_void_p()
    assert L.rq_buf_alloc(ctx.handle, 1 << 50, C.byref(big)) == _lib.RQ_ERR_OOM
    handle = w.handle
    w.destroy()
    assert L.rq_weight_destroy(handle) == _lib.RQ_ERR_HANDLE
    assert L.rq_qmatmul(ctx.handle, handle, xp, 0, yp, 0, 2, None) == _lib.RQ_ERR_HANDLE
    buf = C.c_void_p()
    assert L.rq_buf_alloc(ctx.handle, 1024, C.byref(buf)) == _lib.RQ_OK
    assert L.rq_buf_free(ctx.handle, buf) == _lib.RQ_OK
    assert L.rq_buf_free(ctx.handle, buf) == _lib.RQ_ERR_HANDLE


def test_kernel_timing_counts_main_kernels(torch, ctx):
    import raster_amd

    codes, scales = wl.q8_weights(256, 1024, seed=3)
    w = raster_amd.QWeight.q8(codes, scales, 256, 1024, ctx)
    x1 = torch.randn((1, 1024), device="cuda")
    x64 = torch.randn((64, 1024), device="cuda").to(torch.bfloat16)
    ctx.kernel_time()
    w.matmul(x1)  # timing off: not counted
    torch.cuda.synchronize()
    assert ctx.kernel_time() == (0.0, 0)
    ctx.set_kernel_timing(True)
    try:
        for _ in range(3):
            w.matmul(x1)  # decode kernel
        w.matmul(x64, out_dtype=torch.bfloat16)  # pack + GEMM: one timed kernel
        ms, n = ctx.kernel_time()
        assert n == 4 and 0.0 < ms < 1000.0
        assert ctx.kernel_time() == (0.0, 0)  # read clears
    finally:
        ctx.set_kernel_timing(False)
    w.matmul(x1)
    torch.cuda.synchronize()
    assert ctx.kernel_time() == (0.0, 0)
    w.destroy()
