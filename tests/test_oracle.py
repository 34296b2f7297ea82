"""Pins the C oracle (oracle/rq_oracle.c) before anything is compared against it.

Three kinds of checks, each chosen so a plausible slip in the restatement
(dropped zero-point, swapped nibble, wrong block index, C-style rounding) fails:
  * known answers and properties asserted by the reference's own tests
    (file:line cited per test, paths inside replikativ/raster);
  * closed forms computed independently here in numpy (IEEE f32 multiply,
    int64 dot products, f64 brute force);
  * JDK constants for java.util.Random and Math.round.
"""
import numpy as np
import pytest


# ---------------------------------------------------------------- JDK semantics
def test_java_random_known_values(orc):
    # JDK constants: new Random(42).nextInt() == -1170105035,
    # new Random(0).nextInt() == -1155484576, new Random(0).nextGaussian() == 0.8025330637390305
    b = orc.jfill_bytes(42, 4).view(np.int32)[0]
    assert b == -1170105035
    b0 = orc.jfill_bytes(0, 4).view(np.int32)[0]
    assert b0 == -1155484576
    g = orc.jfill_gauss(0, 1.0, 1)[0]
    assert g == np.float32(0.8025330637390305)
    u = orc.jfill_uniform_centered(0, 1)[0]
    assert u == np.float32(0.730967787376657 - 0.5)


def test_java_round_ties_toward_positive_infinity(orc):
    # raster/compiler/backend/intrinsics.clj:39-45: :round is Java floor(x+0.5)
    cases = {2.5: 3, -2.5: -2, -0.5: 0, 0.5: 1, 1.5: 2, -1.5: -1,
             0.49999999999999994: 0, -127.5: -127, 126.5: 127, float("nan"): 0}
    for x, want in cases.items():
        assert orc.java_round(x) == want, x


# ---------------------------------------------------------------- conversions
def test_f16_widening_is_exact_for_every_half(orc):
    h = np.arange(65536, dtype=np.uint16)
    ours = orc.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(ours[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(ours[np.isnan(ref)]))


def test_f16_narrowing_matches_ieee_rne(orc):
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.uniform(0.005, 0.05, 4000), rng.standard_normal(4000) * 1e-5,
                        rng.standard_normal(4000) * 1e4]).astype(np.float32)
    L = orc.lib()
    ours = np.array([L.rqo_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(ours, x.astype(np.float16).view(np.uint16))


def test_bf16_rne(orc):
    # RNE: exact ties go to even; compare with float64 nearest-even arithmetic
    rng = np.random.default_rng(3)
    x = rng.standard_normal(20000).astype(np.float32)
    ties = (np.arange(1, 200, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties, -ties])
    bits = orc.f32_to_bf16_bits(x)
    back = orc.bf16_bits_to_f32(bits).astype(np.float64)
    err = np.abs(back - x.astype(np.float64))
    # the nearest bf16 neighbours: truncation and truncation + 1 ulp
    u = x.view(np.uint32)
    lo = (u & 0xFFFF0000).view(np.float32).astype(np.float64)
    hi = ((u & 0xFFFF0000) + 0x10000).view(np.float32).astype(np.float64)
    best = np.minimum(np.abs(lo - x), np.abs(hi - x))
    assert np.all(err == best)
    tie_out = orc.f32_to_bf16_bits(ties)
    assert np.all(tie_out % 2 == 0)
    L = orc.lib()
    assert all(L.rqo_f32_to_bf16(float(v)) == b for v, b in zip(x[:500], bits[:500]))


# ---------------------------------------------------------------- int MAC seam
def test_dp4a_known_answers(orc):
    # test/raster/quant/kernels_k_gpu_test.clj:131-137
    assert orc.dp4a(0x01020304, 0x01010101, 0) == 10
    assert orc.dp4a(0x01000000, 0x05000000, 95) == 100
    assert orc.dp4a(0x000000FF, 0x00000002, 0) == -2


def test_dp4a_matches_bytewise_dot(orc):
    rng = np.random.default_rng(11)
    a = rng.integers(-2**31, 2**31, 200, dtype=np.int64)
    b = rng.integers(-2**31, 2**31, 200, dtype=np.int64)
    for x, y in zip(a, b):
        xa = np.array([x], np.int64).astype(np.int32).view(np.int8).astype(np.int64)
        ya = np.array([y], np.int64).astype(np.int32).view(np.int8).astype(np.int64)
        assert orc.dp4a(int(x), int(y), 7) == 7 + int(np.dot(xa, ya))


def test_wi8_dot_q4_nibble_order(orc):
    # lo nibble = element k, hi nibble = element k+16 (cpu/quant.clj:27-31, kernels.clj:33-46)
    rng = np.random.default_rng(2)
    q = rng.integers(0, 16, 32)
    x = rng.integers(-127, 128, 32).astype(np.int8)
    wq = (q[:16] | (q[16:] << 4)).astype(np.uint8)
    assert orc.wi8_dot_q4(wq, 0, x, 0) == int(np.dot(q, x.astype(np.int64)))


# ---------------------------------------------------------------- Q8_0 (train.clj)
def test_q8_codec_roundtrip(orc):
    # test/raster/quant/train_test.clj:18-24
    out, in_ = 4, 64
    W = orc.jfill_gauss(1, 0.3, out * in_)
    codes, scales = orc.q8_quantize(W, out, in_)
    Wr = orc.dequant_q8_dense(codes, scales, in_, out)
    assert np.max(np.abs(W - Wr)) < 0.01
    assert codes.min() >= -127 and codes.max() <= 127


def test_q8_quantize_requires_in_multiple_of_32(orc):
    with pytest.raises(AssertionError):
        orc.q8_quantize(np.zeros(30, np.float32), 1, 30)


def test_dequant_q8_is_one_ieee_f32_multiply(orc):
    rng = np.random.default_rng(0)
    out, in_ = 16, 256
    codes = rng.integers(-127, 128, out * in_).astype(np.int8)
    scales = rng.uniform(0.002, 0.02, out * in_ // 32).astype(np.float32)
    W = orc.dequant_q8_dense(codes, scales, in_, out)
    ref = np.repeat(scales.reshape(out, -1), 32, axis=1).ravel() * codes.astype(np.float32)
    assert ref.dtype == np.float32
    assert np.array_equal(W.view(np.uint32), ref.view(np.uint32))


def test_qlinear_forward_matches_dense(orc):
    # test/raster/quant/train_test.clj:26-40 (< 1e-5)
    out, in_, m = 4, 64, 2
    W = orc.jfill_gauss(1, 0.3, out * in_)
    X = orc.jfill_gauss(2, 0.3, m * in_)
    codes, scales = orc.q8_quantize(W, out, in_)
    Wd = orc.dequant_q8_dense(codes, scales, in_, out)
    y = orc.qlinear_q8(X, codes, scales, m, in_, out)
    ref = (X.reshape(m, in_).astype(np.float64) @ Wd.reshape(out, in_).astype(np.float64).T).ravel()
    assert np.max(np.abs(y - ref)) < 1e-5


@pytest.mark.parametrize("m,in_,out", [(1, 32, 1), (3, 96, 5), (4, 256, 16)])
def test_qlinear_q8_brute_force(orc, m, in_, out):
    rng = np.random.default_rng(m * 100 + out)
    codes = rng.integers(-127, 128, out * in_).astype(np.int8)
    scales = rng.uniform(0.002, 0.02, out * in_ // 32).astype(np.float32)
    x = rng.standard_normal(m * in_).astype(np.float32)
    y = orc.qlinear_q8(x, codes, scales, m, in_, out)
    # independent: exact per-element products in f64, summed in f64
    s = np.repeat(scales.reshape(out, -1), 32, axis=1).astype(np.float64)
    ref = x.reshape(m, in_).astype(np.float64) @ (s * codes.reshape(out, in_)).T
    assert np.max(np.abs(y - ref.ravel())) <= 1e-5 * max(1.0, np.max(np.abs(ref)))


def test_dx_pullback_matches_finite_differences(orc):
    # test/raster/quant/train_test.clj:52-68 (< 2e-3 at eps 1e-3)
    out, in_, m = 4, 64, 2
    W = orc.jfill_gauss(1, 0.3, out * in_)
    x = orc.jfill_gauss(2, 0.3, m * in_)
    tgt = orc.jfill_gauss(3, 0.3, m * out)
    codes, scales = orc.q8_quantize(W, out, in_)

    def loss(xv):
        y = orc.qlinear_q8(xv, codes, scales, m, in_, out).astype(np.float64)
        return float(np.sum(0.5 * (y - tgt) ** 2))

    y = orc.qlinear_q8(x, codes, scales, m, in_, out)
    gx = orc.qlinear_q8_dx((y - tgt).astype(np.float32), codes, scales, m, in_, out)
    eps = 1e-3
    for idx in [3, 17, 40, 63, 64, 100]:
        xp, xm = x.copy(), x.copy()
        xp[idx] += np.float32(eps)
        xm[idx] -= np.float32(eps)
        num = (loss(xp) - loss(xm)) / (2 * eps)
        assert abs(gx[idx] - num) < 2e-3


# ---------------------------------------------------------------- parametric encoder
def test_parametric_encode(orc):
    # test/raster/compiler/backend/cpu/quant_encode_test.clj:26-44
    n = 256
    w = orc.jfill_uniform_centered(42, n)
    wq4, ws4 = orc.quantize_weight_q4(w)
    wq8, ws8 = orc.quantize_weight_q8u(w)
    assert wq4.size == n // 2 and wq8.size == n
    e4 = np.max(np.abs(w - orc.dequant_weight(wq4, ws4, n, 8, True)))
    e8 = np.max(np.abs(w - orc.dequant_weight(wq8, ws8, n, 128, False)))
    assert e4 > 0
    assert e8 < 0.2 * e4


def _decode_unsigned(wq, ws, n, zp, nibble):
    """Independent numpy decode of the parametric format
    (raster/compiler/backend/cpu/quant.clj:27-39,60-67): per 32-block b, byte k of
    a nibble block holds element k in its low nibble and element k + 16 in its
    high nibble; W = d * (q - zp) with one f32 rounding of the exact product."""
    nb = n // 32
    if nibble:
        by = wq.reshape(nb, 16).astype(np.int64)
        q = np.concatenate([by & 0xF, by >> 4], axis=1)  # elements 0..15, then 16..31
    else:
        q = wq.reshape(nb, 32).astype(np.int64)
    return q, (ws.astype(np.float64)[:, None] * (q - zp)).astype(np.float32).ravel()


@pytest.mark.parametrize("bits,zp,nibble", [(4, 8, True), (8, 128, False)])
def test_parametric_encode_decode_pinned(orc, bits, zp, nibble):
    # Pins the encoder and the decoder with checks a swapped nibble order, a
    # dropped zero point or a wrong scale sign fails:
    #  * the decoder equals an independent decode bit for bit;
    #  * every element whose code is not clamped lies within |d|/2 of its
    #    reconstruction (round to nearest), clamped ones sit at the range end;
    #  * the block's extreme element (d = v / -zp, quant.clj:55-60) is code 0
    #    and reconstructs exactly.
    rng = np.random.default_rng(40 + bits)
    n = 32 * 96
    w = (rng.standard_normal(n) * rng.uniform(0.01, 4.0, n)).astype(np.float32)
    w[32:64] = 0.0  # an all-zero block: d = 0, every code = zp, W = 0
    wq, ws = orc.quantize_weight(w, bits, zp, nibble)
    q, dec = _decode_unsigned(wq, ws, n, zp, nibble)
    assert np.array_equal(orc.dequant_weight(wq, ws, n, zp, nibble).view(np.uint32), dec.view(np.uint32))
    d = ws.astype(np.float64)
    wb = w.reshape(-1, 32).astype(np.float64)
    qmax = (1 << bits) - 1
    inner = (q > 0) & (q < qmax)
    err = np.abs(dec.reshape(-1, 32).astype(np.float64) - wb)
    half = np.abs(d)[:, None] / 2 * (1 + 1e-6) + 1e-30
    assert np.all(err[inner] <= np.broadcast_to(half, err.shape)[inner])
    ext = np.argmax(np.abs(wb), axis=1)
    nz = d != 0
    assert np.all(q[np.arange(len(d)), ext][nz] == 0)
    assert np.array_equal(dec.reshape(-1, 32)[np.arange(len(d)), ext][nz], w.reshape(-1, 32)[np.arange(len(d)), ext][nz])
    assert np.all(q[1] == zp) and np.all(dec[32:64] == 0)
    # the nibble order itself: a block whose element k is k - 16 (k < 16) and
    # k - 15 (k >= 16) encodes to bytes whose low nibble is element k
    if nibble:
        blk = np.concatenate([np.arange(-16, 0), np.arange(1, 17)]).astype(np.float32)
        bq, bs = orc.quantize_weight(blk, 4, 8, True)
        assert bs[0] == np.float32(2.0)  # d = -16 / -8
        # Java Math/round: ties toward +infinity (-7.5 -> -7)
        assert np.array_equal(bq & 0xF, np.floor(blk[:16] / 2 + 0.5).astype(np.int64) + 8)
        assert np.array_equal(bq >> 4, np.minimum(np.floor(blk[16:] / 2 + 0.5).astype(np.int64) + 8, 15))


def test_q4_dequant_closed_form(orc):
    rng = np.random.default_rng(9)
    out, in_ = 8, 128
    q = rng.integers(0, 16, (out, in_))
    # pack: byte k of block b = q[b*32+k] | q[b*32+k+16] << 4
    qb = q.reshape(out, in_ // 32, 2, 16)
    wq = (qb[:, :, 0, :] | (qb[:, :, 1, :] << 4)).astype(np.uint8).ravel()
    sc16 = rng.uniform(0.005, 0.05, out * in_ // 32).astype(np.float16)
    W = orc.dequant_q4(wq, sc16.view(np.uint16), in_, out)
    ref = np.repeat(sc16.astype(np.float32).reshape(out, -1), 32, axis=1) * (q - 8).astype(np.float32)
    assert np.array_equal(W.view(np.uint32), ref.astype(np.float32).ravel().view(np.uint32))
    W32 = orc.dequant_q4(wq, sc16.astype(np.float32), in_, out)
    assert np.array_equal(W32, W)


def test_qlinear_q4_brute_force(orc):
    rng = np.random.default_rng(4)
    m, in_, out = 3, 128, 12
    wq = rng.integers(0, 256, out * in_ // 2).astype(np.uint8)
    sc16 = rng.uniform(0.005, 0.05, out * in_ // 32).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(m * in_).astype(np.float32)
    y = orc.qlinear_q4(x, wq, sc16, m, in_, out)
    W = orc.dequant_q4(wq, sc16, in_, out).reshape(out, in_).astype(np.float64)
    ref = x.reshape(m, in_).astype(np.float64) @ W.T
    assert np.max(np.abs(y - ref.ravel())) <= 1e-5 * np.max(np.abs(ref))


# ---------------------------------------------------------------- act quant / int GEMV
def test_quantize_act_i8_properties(orc):
    rng = np.random.default_rng(8)
    M, in_ = 3, 256
    x = rng.standard_normal(M * in_).astype(np.float32)
    x[:32] = 0.0  # an all-zero block: d = 0, id = 0, codes 0
    xq, xs, xsum = orc.quantize_act_i8(x, M, in_)
    blocks = x.reshape(-1, 32).astype(np.float64)
    d = np.max(np.abs(blocks), axis=1) / 127.0
    assert np.array_equal(xs, d.astype(np.float32))
    q = xq.reshape(-1, 32).astype(np.int64)
    assert np.array_equal(xsum, q.sum(axis=1))
    nz = d > 0
    recon = q[nz] * d[nz, None]
    assert np.all(np.abs(recon - blocks[nz]) <= d[nz, None] / 2 + 1e-12)
    assert np.all(q[0] == 0) and xs[0] == 0


def test_q4_composable_equals_independent_int_dot(orc):
    # kernels.clj:140-184 vs the scalar oracle of bench/raster/quant_faithfulness.clj:55-75
    rng = np.random.default_rng(12)
    in_, out = 256, 24
    w = rng.uniform(-0.5, 0.5, out * in_).astype(np.float32)
    x = rng.uniform(-0.5, 0.5, in_).astype(np.float32)
    wq, ws = orc.quantize_weight_q4(w)
    xq, xs, xsum = orc.quantize_act_i8(x, 1, in_)
    y = orc.qmatmul_q4_composable(xq, xs, xsum, wq, ws, in_, out)
    q = np.empty((out, in_), np.int64)
    wr = wq.reshape(out, in_ // 32, 16).astype(np.int64)
    q.reshape(out, in_ // 32, 32)[:, :, :16] = wr & 0xF
    q.reshape(out, in_ // 32, 32)[:, :, 16:] = wr >> 4
    dots = ((q - 8).reshape(out, -1, 32) * xq.reshape(-1, 32).astype(np.int64)).sum(axis=2)
    ref = (dots * (xs.astype(np.float64)[None, :] * ws.reshape(out, -1).astype(np.float64))).sum(axis=1)
    assert np.max(np.abs(y - ref)) <= 1e-6 * np.max(np.abs(ref))


@pytest.mark.parametrize("out,in_", [(16, 64), (1024, 640), (8, 32), (24, 128)])
def test_x8_tile_matches_single_column(orc, out, in_):
    # test/raster/quant/tile_test.clj:13-30 (exact int32 dots)
    half, nb = in_ // 2, in_ // 32
    wq = orc.jfill_bytes(out + in_, out * in_ // 2).view(np.uint8)
    ws = np.ones(out * nb, np.float32)
    xq = orc.jfill_bytes(7 * (out + in_), in_)
    wqi, _ = orc.repack_x8(wq, ws, out, in_, True)
    groups = range(out // 8) if out <= 64 else [0, 1, out // 8 - 1]
    for gi in groups:
        for b in range(nb):
            out8 = orc.wi8_dot_x8(wqi, gi * nb * 128 + b * 128, xq, b * 32, True)
            for L in range(8):
                col = gi * 8 + L
                assert out8[L] == orc.wi8_dot_q4(wq, col * half + b * 16, xq, b * 32)


def test_x8_q8_tile_and_fold_match_row_major(orc):
    rng = np.random.default_rng(21)
    in_, out = 256, 32
    w = rng.uniform(-0.5, 0.5, out * in_).astype(np.float32)
    x = rng.uniform(-0.5, 0.5, in_).astype(np.float32)
    wq, ws = orc.quantize_weight_q8u(w)  # unsigned, zero-point 128
    wqi, wsi = orc.repack_x8(wq, ws, out, in_, False)
    xq, xs, xsum = orc.quantize_act_i8(x, 1, in_)
    y8 = orc.qmatmul_x8(xq, xs, xsum, wqi, wsi, in_, out, False)
    codes = (wq.astype(np.int64) - 128).reshape(out, -1, 32)
    dots = (codes * xq.reshape(-1, 32).astype(np.int64)).sum(axis=2)
    ref = (dots * (xs.astype(np.float64)[None, :] * ws.reshape(out, -1))).sum(axis=1)
    assert np.max(np.abs(y8 - ref)) <= 1e-5 * np.max(np.abs(ref))


@pytest.mark.parametrize("in_,out", [(256, 64), (512, 128)])
def test_x8_vs_composable(orc, in_, out):
    # test/raster/quant/x8_simd_test.clj:24-33 (< 1e-3)
    rng = np.random.default_rng(in_)
    w = (rng.random(out * in_) - 0.5).astype(np.float32)
    x = (rng.random(in_) - 0.5).astype(np.float32)
    wq, ws = orc.quantize_weight_q4(w)
    wqi, wsi = orc.repack_x8(wq, ws, out, in_, True)
    xq, xs, xsum = orc.quantize_act_i8(x, 1, in_)
    y8 = orc.qmatmul_x8(xq, xs, xsum, wqi, wsi, in_, out, True)
    yc = orc.qmatmul_q4_composable(xq, xs, xsum, wq, ws, in_, out)
    assert np.max(np.abs(y8 - yc)) < 1e-3


# ---------------------------------------------------------------- signed q8_0 prefill
def test_quantize_one_q8_roundtrip(orc):
    # test/raster/quant/pack_test.clj:20-40
    out, in_ = 4, 64
    nb = in_ // 32
    W = orc.jfill_uniform_centered(7, out * in_)
    wp, ws = orc.quantize_one_q8(W, in_, out)
    assert wp.size == out * in_ // 4 and ws.size == out * nb
    q = wp.view(np.int8).astype(np.int64).reshape(out, in_)
    d = np.repeat(ws.reshape(out, nb).astype(np.float64), 32, axis=1)
    assert q.min() >= -127 and q.max() <= 127
    assert np.all(np.abs(q * d - W.reshape(out, in_)) < 0.5 * d + 1e-7)
    with pytest.raises(AssertionError):
        orc.quantize_one_q8(np.zeros(30, np.float32), 30, 1)


def test_quantize_one_q8_agrees_with_q8_quantize(orc):
    # both are per-32-block d = max|w|/127 with Java rounding; only the packing differs
    W = orc.jfill_gauss(5, 0.3, 8 * 128)
    wp, ws = orc.quantize_one_q8(W, 128, 8)
    codes, scales = orc.q8_quantize(W, 8, 128)
    assert np.array_equal(wp.view(np.int8), codes)
    assert np.array_equal(ws, scales)


def test_quant_act_rows_matches_blockwise_quantizer(orc):
    rng = np.random.default_rng(17)
    T, in_ = 5, 128
    x = rng.standard_normal(T * in_).astype(np.float32)
    xp, xs = orc.quant_act_i8_rows(x, in_, T)
    xq, xs2, _ = orc.quantize_act_i8(x, T, in_)
    assert np.array_equal(xs, xs2)
    assert np.array_equal(xp.view(np.int8), xq)


def test_qmatmul_i8_gemm_exact_int_dots(orc):
    rng = np.random.default_rng(19)
    T, in_, out = 3, 128, 10
    W = rng.standard_normal(out * in_).astype(np.float32)
    x = rng.standard_normal(T * in_).astype(np.float32)
    wp, ws = orc.quantize_one_q8(W, in_, out)
    xp, xs = orc.quant_act_i8_rows(x, in_, T)
    y = orc.qmatmul_i8_gemm(xp, xs, wp, ws, in_, out, T).reshape(T, out)
    wq = wp.view(np.int8).astype(np.int64).reshape(out, -1, 32)
    xq = xp.view(np.int8).astype(np.int64).reshape(T, -1, 32)
    dots = np.einsum("obk,tbk->tob", wq, xq)
    sc = ws.reshape(out, -1).astype(np.float64)[None] * xs.reshape(T, -1).astype(np.float64)[:, None]
    ref = (dots * sc).sum(axis=2)
    assert np.max(np.abs(y - ref)) <= 1e-6 * np.max(np.abs(ref))
    # the dp4a GEMV is the same int core without scales
    yi = orc.i8gemv_dp4a(wp, xp[: in_ // 4], in_ // 4, out)
    assert np.array_equal(yi, wq.reshape(out, in_) @ xq[0].reshape(in_).astype(np.float64))


def test_staged_equals_flat_with_power_of_two_scales(orc):
    # staged_contract_device_test.clj:1-20: with power-of-two scales the per-block
    # (staged) sum and the dequantized (flat) sum are the same exact number
    rng = np.random.default_rng(23)
    m, in_, out = 2, 128, 8
    codes = rng.integers(-127, 128, out * in_).astype(np.int8)
    scales = (2.0 ** rng.integers(-8, -2, out * in_ // 32)).astype(np.float32)
    x = (rng.integers(-64, 64, m * in_) / 64.0).astype(np.float32)
    y = orc.qlinear_q8(x, codes, scales, m, in_, out)
    Wd = orc.dequant_q8_dense(codes, scales, in_, out)
    flat = orc.dense_matmul_nt_f64(x, Wd, m, in_, out)
    assert np.array_equal(y.astype(np.float64), flat)


# ---------------------------------------------------------------- decoder-step glue
def test_rms_norm_closed_forms(orc):
    # [3, 4]: mean square 12.5, so out = x / sqrt(12.5); scaling x leaves the
    # output unchanged (eps 0); the weight (plus the gain offset) scales it
    out = orc.rms_norm(np.array([3, 4], np.float32), np.ones(2, np.float32), 1, 2, 0.0, 0.0)
    assert np.allclose(out, np.array([3, 4]) / np.sqrt(12.5), rtol=1e-7)
    rng = np.random.default_rng(1)
    x = rng.standard_normal(3 * 64).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 64).astype(np.float32)
    a = orc.rms_norm(x, w, 3, 64, 0.0, 0.0)
    b = orc.rms_norm(x * np.float32(8), w, 3, 64, 0.0, 0.0)
    assert np.array_equal(a, b)  # power-of-two scale: exact
    one = orc.rms_norm(x, np.zeros(64, np.float32), 3, 64, 0.0, 1.0)  # gain-offset form (weight 0 + 1)
    rms = np.sqrt(np.mean(one.reshape(3, 64).astype(np.float64) ** 2, axis=1))
    assert np.allclose(rms, 1.0, atol=1e-6)
    assert np.allclose(a, one * np.tile(w, 3), rtol=2e-7, atol=1e-7)


def test_rope_pos_known_answer_and_rotation(orc):
    # head_dim 4, theta 1e4: pair (0, 2) turns by pos * 1, pair (1, 3) by pos * 1e-2;
    # NeoX half split: element i pairs with i + head_dim/2
    out = orc.rope_pos(np.array([1, 0, 0, 0], np.float32), 1, 1, 4, 1e4, 1)
    assert np.allclose(out, [np.cos(1.0), 0, np.sin(1.0), 0], atol=1e-7)
    out = orc.rope_pos(np.array([0, 1, 0, 0], np.float32), 1, 1, 4, 1e4, 3)
    assert np.allclose(out, [0, np.cos(0.03), 0, np.sin(0.03)], atol=1e-7)
    rng = np.random.default_rng(2)
    x = rng.standard_normal(2 * 3 * 16).astype(np.float32)  # 2 positions x 3 heads x 16
    assert np.array_equal(orc.rope_pos(x, 2, 3, 16, 1e4, 0)[:48], x[:48])  # position 0 is the identity
    r = orc.rope_pos(x, 2, 3, 16, 1e4, 5).reshape(2, 3, 2, 8).astype(np.float64)
    xr = x.reshape(2, 3, 2, 8).astype(np.float64)
    assert np.allclose((r ** 2).sum(axis=2), (xr ** 2).sum(axis=2), rtol=1e-6)  # pairwise norms kept
    # rotating by 5 then by 7 equals rotating by 12 (second token: positions 6 and 13)
    twice = orc.rope_pos(orc.rope_pos(x, 2, 3, 16, 1e4, 5), 2, 3, 16, 1e4, 7)
    once = orc.rope_pos(x, 2, 3, 16, 1e4, 12)
    assert np.allclose(twice[:48], once[:48], atol=1e-5)


def test_gqa_decode_attention_closed_forms(orc):
    hd = 8
    rng = np.random.default_rng(3)
    q = rng.standard_normal(2 * hd).astype(np.float32)
    k1 = rng.standard_normal(hd).astype(np.float32)
    v1 = rng.standard_normal(hd).astype(np.float32)
    # one cached position: every query head returns that value row
    out = orc.gqa_decode_attention(q, k1, v1, 1, 2, 1, hd, 0.5)
    assert np.allclose(out, np.tile(v1, 2), atol=1e-7)
    # two positions with equal keys: the mean of the values
    k = np.tile(k1, 2)
    v = rng.standard_normal(2 * hd).astype(np.float32)
    out = orc.gqa_decode_attention(q[:hd], k, v, 2, 1, 1, hd, 0.5)
    assert np.allclose(out, v.reshape(2, hd).mean(axis=0), atol=1e-6)
    # two positions whose scores differ by t: weights sigmoid(t), 1 - sigmoid(t)
    ka = np.zeros(hd, np.float32)
    ka[0] = 1.0
    kb = np.zeros(hd, np.float32)
    qq = np.zeros(hd, np.float32)
    qq[0] = 2.0
    out = orc.gqa_decode_attention(qq, np.concatenate([ka, kb]), v, 2, 1, 1, hd, 0.25)
    t = 2.0 * 0.25
    wa = 1.0 / (1.0 + np.exp(-t))
    assert np.allclose(out, wa * v[:hd] + (1 - wa) * v[hd:], atol=1e-6)
    # grouped heads: query heads 0,1 read kv head 0, heads 2,3 kv head 1
    kk = rng.standard_normal(3 * 2 * hd).astype(np.float32)
    vv = rng.standard_normal(3 * 2 * hd).astype(np.float32)
    qs = rng.standard_normal(4 * hd).astype(np.float32)
    full = orc.gqa_decode_attention(qs, kk, vv, 3, 4, 2, hd, 0.3)
    sel = lambda a, h: a.reshape(3, 2, hd)[:, h, :].ravel()
    for hq in range(4):
        one = orc.gqa_decode_attention(qs[hq * hd:(hq + 1) * hd], sel(kk, hq // 2), sel(vv, hq // 2), 3, 1, 1, hd, 0.3)
        assert np.array_equal(full[hq * hd:(hq + 1) * hd], one)


def test_silu_mul_and_residual_add(orc):
    g = np.array([0.0, 1.0, -1.0, 30.0], np.float32)
    u = np.array([5.0, 2.0, 2.0, 1.0], np.float32)
    out = orc.silu_mul(g, u, 4)
    assert out[0] == 0.0
    assert np.isclose(out[1], 2.0 / (1.0 + np.exp(-1.0)), rtol=1e-7)
    assert np.isclose(out[1] - out[2], 2.0, rtol=1e-6)  # silu(x) - silu(-x) = x
    assert np.isclose(out[3], 30.0, rtol=1e-7)
    a = np.array([1.0, 1e8, -3.5], np.float32)
    b = np.array([2.0, 1.0, 3.5], np.float32)
    assert np.array_equal(orc.residual_add(a, b, 3), a + b)  # correctly rounded f32 sum


def test_decoder_layer_composes_the_glue(orc):
    # the layer equals its steps run one by one through the oracle's own pieces
    # (checks the wiring: which buffer feeds which op, cache position, residuals)
    d, nq, hd, ffn, clen = 64, 2, 32, 96, 4
    rng = np.random.default_rng(4)
    ws = []
    for out, in_ in ((nq * hd, d), (nq * hd, d), (nq * hd, d), (d, nq * hd), (ffn, d), (ffn, d), (d, ffn)):
        ws.append((rng.integers(-127, 128, out * in_).astype(np.int8),
                   rng.uniform(0.002, 0.02, out * (in_ // 32)).astype(np.float32)))
    x = rng.standard_normal(d).astype(np.float32)
    g1 = rng.uniform(0.5, 1.5, d).astype(np.float32)
    g2 = rng.uniform(0.5, 1.5, d).astype(np.float32)
    kc = rng.standard_normal(clen * nq * hd).astype(np.float32)
    vc = rng.standard_normal(clen * nq * hd).astype(np.float32)
    y, kc2, vc2 = orc.decoder_layer(x, ws, g1, g2, kc, vc, d, nq, nq, hd, ffn, clen, 1e-5, 1e4)
    xn = orc.rms_norm(x, g1, 1, d, 1e-5, 0.0)
    q = orc.qlinear_q8(xn, *ws[0], 1, d, nq * hd)
    k = orc.qlinear_q8(xn, *ws[1], 1, d, nq * hd)
    v = orc.qlinear_q8(xn, *ws[2], 1, d, nq * hd)
    pos = clen - 1
    kr = orc.rope_pos(k, 1, nq, hd, 1e4, pos)
    kref, vref = kc.copy(), vc.copy()
    kref[pos * nq * hd:] = kr
    vref[pos * nq * hd:] = v
    assert np.array_equal(kc2, kref) and np.array_equal(vc2, vref)
    at = orc.gqa_decode_attention(orc.rope_pos(q, 1, nq, hd, 1e4, pos), kref, vref, clen, nq, nq, hd, hd ** -0.5)
    x1 = orc.residual_add(x, orc.qlinear_q8(at, *ws[3], 1, nq * hd, d), d)
    x1n = orc.rms_norm(x1, g2, 1, d, 1e-5, 0.0)
    h = orc.silu_mul(orc.qlinear_q8(x1n, *ws[4], 1, d, ffn), orc.qlinear_q8(x1n, *ws[5], 1, d, ffn), ffn)
    want = orc.residual_add(x1, orc.qlinear_q8(h, *ws[6], 1, ffn, d), d)
    assert np.array_equal(y, want)


# ---------------------------------------------------------------- K-quants
def _ref_matmul_f64(wdq, xdq, out, in_):
    # ref-matmul of test/raster/quant/kernels_k_test.clj:24-29: double sums, one narrowing
    return (wdq.reshape(out, in_).astype(np.float64) @ xdq.astype(np.float64)).astype(np.float32)


@pytest.mark.parametrize("fmt,wseed,xseed", [("q4k", 1, 2), ("q6k", 3, 4)])
def test_kquant_reference_test_reproduction(orc, fmt, wseed, xseed):
    # test/raster/quant/kernels_k_test.clj:31-61: out 8, in 256, java.util.Random
    # inputs; the composable K dot matches dequant-matmul within 1e-2 per row
    out, in_ = 8, 256
    W = orc.jfill_uniform_centered(wseed, out * in_)
    x = orc.jfill_uniform_centered(xseed, in_)
    if fmt == "q4k":
        wq, da, db, aq, bq = orc.quantize_weight_q4k(W)
        xq, xs, bs = orc.quantize_act_q8k(x, 1, in_, 32)
        y = orc.qmatmul_q4k(xq, xs, bs, wq, da, db, aq, bq, 1, in_, out)
        wdq = orc.dequant_q4k(wq, da, db, aq, bq, out * in_)
    else:
        wq, sc, ds = orc.quantize_weight_q6k(W)
        xq, xs, bs = orc.quantize_act_q8k(x, 1, in_, 16)
        y = orc.qmatmul_q6k(xq, xs, bs, wq, sc, ds, 1, in_, out)
        wdq = orc.dequant_q6k(wq, sc, ds, out * in_)
    xdq = (xs[0] * xq.astype(np.float32)).astype(np.float32)  # (float (* dact xq))
    yref = _ref_matmul_f64(wdq, xdq, out, in_)
    assert np.all(np.abs(y - yref) < 1e-2)


def test_q4k_dot_equals_dequant_dot(orc):
    # the K dot is the dot of the exact dequantized weight ((da*aq) q + db*bq,
    # unrounded) with the exact dequantized activation; an independent
    # vectorized restatement in float64 must agree to rounding
    rng = np.random.default_rng(21)
    m, out, in_ = 3, 12, 1024
    W = rng.standard_normal(out * in_).astype(np.float32)
    x = rng.standard_normal(m * in_).astype(np.float32)
    wq, da, db, aq, bq = orc.quantize_weight_q4k(W)
    xq, xs, bs = orc.quantize_act_q8k(x, m, in_, 32)
    y = orc.qmatmul_q4k(xq, xs, bs, wq, da, db, aq, bq, m, in_, out).reshape(m, out)
    nib = wq.reshape(out, in_ // 32, 16).astype(np.float64)
    q = np.concatenate([nib % 16, nib // 16], axis=2)  # element k low, k + 16 high
    a1 = (da.astype(np.float64).repeat(8).reshape(out, -1) * aq.reshape(out, -1).astype(np.float64))
    b1 = (db.astype(np.float64).repeat(8).reshape(out, -1) * bq.reshape(out, -1).astype(np.float64))
    wexact = (a1[:, :, None] * q + b1[:, :, None]).reshape(out, in_)
    xexact = (xs.astype(np.float64).reshape(m, -1).repeat(256, axis=1) * xq.reshape(m, in_).astype(np.float64))
    ref = xexact @ wexact.T
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) < 1e-6


def test_q6k_dot_equals_dequant_dot(orc):
    rng = np.random.default_rng(22)
    m, out, in_ = 2, 10, 768
    W = rng.standard_normal(out * in_).astype(np.float32)
    x = rng.standard_normal(m * in_).astype(np.float32)
    wq, sc, ds = orc.quantize_weight_q6k(W)
    xq, xs, bs = orc.quantize_act_q8k(x, m, in_, 16)
    y = orc.qmatmul_q6k(xq, xs, bs, wq, sc, ds, m, in_, out).reshape(m, out)
    a1 = ds.astype(np.float64).repeat(16).reshape(out, -1) * sc.reshape(out, -1).astype(np.float64)
    wexact = (a1[:, :, None] * (wq.reshape(out, -1, 16).astype(np.float64) - 32.0)).reshape(out, in_)
    xexact = (xs.astype(np.float64).reshape(m, -1).repeat(256, axis=1) * xq.reshape(m, in_).astype(np.float64))
    ref = xexact @ wexact.T
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) < 1e-6


def test_kquant_encoders_ranges_and_round_trip(orc):
    rng = np.random.default_rng(23)
    W = (rng.standard_normal(4 * 512) * rng.uniform(0.01, 3.0, 4 * 512)).astype(np.float32)
    wq, da, db, aq, bq = orc.quantize_weight_q4k(W)
    assert aq.max() <= 63 and bq.min() >= -32 and bq.max() <= 31
    deq = orc.dequant_q4k(wq, da, db, aq, bq, W.size).astype(np.float64)
    q = np.concatenate([wq.reshape(-1, 16) % 16, wq.reshape(-1, 16) // 16], axis=1).ravel()
    a1 = (da.astype(np.float64).repeat(8) * aq.astype(np.float64)).repeat(32)
    inner = (q > 0) & (q < 15)  # unclamped codes: within half a step
    assert np.all(np.abs(deq - W)[inner] <= a1[inner] / 2 * (1 + 1e-6) + 1e-7)
    wq6, sc, ds = orc.quantize_weight_q6k(W)
    assert wq6.max() <= 63 and sc.min() >= 0
    deq6 = orc.dequant_q6k(wq6, sc, ds, W.size).astype(np.float64)
    a6 = (ds.astype(np.float64).repeat(16) * sc.astype(np.float64)).repeat(16)
    inner6 = (wq6 > 0) & (wq6 < 63)
    assert np.all(np.abs(deq6 - W)[inner6] <= a6[inner6] / 2 * (1 + 1e-6) + 1e-7)


@pytest.mark.parametrize("sub", [32, 16])
def test_quantize_act_q8k_properties(orc, sub):
    rng = np.random.default_rng(24)
    m, in_ = 2, 768
    x = rng.standard_normal(m * in_).astype(np.float32)
    x[:256] = 0.0  # an all-zero super-block
    xq, xs, bs = orc.quantize_act_q8k(x, m, in_, sub)
    sb = x.reshape(-1, 256).astype(np.float64)
    d = np.max(np.abs(sb), axis=1) / 127.0
    assert np.array_equal(xs, d.astype(np.float32))
    assert np.array_equal(bs, xq.reshape(-1, sub).astype(np.int64).sum(axis=1))
    q = xq.reshape(-1, 256).astype(np.float64)
    nz = d > 0
    assert np.all(np.abs(q[nz] * d[nz, None] - sb[nz]) <= d[nz, None] / 2 + 1e-12)
    assert np.all(xq[:256] == 0)


# ---------------------------------------------------------------- q4k-of ingestion
def test_nextpad_known_answers(orc):
    # test/raster/quant/pack_test.clj:14-18
    assert [orc.nextpad(i) for i in (1, 256, 257, 640)] == [256, 256, 512, 768]
    assert orc.nextpad(512) == 512 and orc.nextpad(513) == 768


def test_q4k_of_no_pad_matches_the_packer(orc):
    # test/raster/quant/pack_test.clj:42-60: in = 256 needs no padding, so q4k-of
    # is the CPU packer's output byte for byte
    out, in_ = 2, 256
    W = orc.jfill_uniform_centered(11, out * in_)
    wq, da, db, aq, bq, inp = orc.q4k_of(W, out, in_)
    ref = orc.quantize_weight_q4k(W)
    assert inp == in_
    for a, b in zip((wq, da, db, aq, bq), ref):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))


def test_q4k_of_pads_rows_with_zeros(orc):
    # test/raster/quant/pack_test.clj:61-69: in = 640 pads rows to 768 and the
    # padded packing equals packing the zero-padded W; and each row's first
    # super-blocks (all real columns) equal the unpadded row's own packing
    out, in_, inp = 3, 640, 768
    W = orc.jfill_uniform_centered(13, out * in_)
    wq, da, db, aq, bq, got = orc.q4k_of(W, out, in_)
    assert got == inp
    Wp = np.zeros((out, inp), np.float32)
    Wp[:, :in_] = W.reshape(out, in_)
    ref = orc.quantize_weight_q4k(Wp.ravel())
    for a, b in zip((wq, da, db, aq, bq), ref):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    for o in range(out):
        r = orc.quantize_weight_q4k(W.reshape(out, in_)[o, :512].copy())
        assert np.array_equal(da.reshape(out, 3)[o, :2], r[1])
        assert np.array_equal(wq.reshape(out, inp // 2)[o, :256], r[0])
    # the padded columns of a zero-padded activation contribute nothing
    x = np.zeros(inp, np.float32)
    x[:in_] = orc.jfill_uniform_centered(14, in_)
    xq, xs, bs = orc.quantize_act_q8k(x, 1, inp, 32)
    assert np.all(xq[in_:] == 0) and np.all(bs[in_ // 32:] == 0)


# ---------------------------------------------------------------- the timed CPU baseline
@pytest.mark.parametrize("nibble", [True, False])
def test_cpu_baseline_x8_matches_the_oracle(orc, nibble):
    # the B2 route bench.py times (oracle/cpu_baseline.c) computes the oracle's
    # quantize-act-i8 + qmatmul-q4-x8! / qmatmul-q8-x8! (f32 lanes summed in
    # another association, so to 1e-5), on 1 and 4 threads
    import ctypes as C

    L = orc.baseline_lib()
    ptr = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    rng = np.random.default_rng(90 + nibble)
    out, in_ = 64, 512
    W = rng.standard_normal(out * in_).astype(np.float32)
    x = rng.standard_normal(in_).astype(np.float32)
    wq, ws = orc.quantize_weight_q4(W) if nibble else orc.quantize_weight_q8u(W)
    wqi, wsi = orc.repack_x8(wq, ws, out, in_, nibble)
    rxq, rxs, rxsum = orc.quantize_act_i8(x, 1, in_)
    ref = orc.qmatmul_x8(rxq, rxs, rxsum, wqi, wsi, in_, out, nibble)
    for threads in (1, 4):
        xq, xs, xsum = np.empty(in_, np.int8), np.empty(in_ // 32, np.float32), np.empty(in_ // 32, np.int32)
        L.rqb_quantize_act_i8(ptr(x), 1, in_, ptr(xq), ptr(xs), ptr(xsum), threads)
        assert np.array_equal(xq, rxq) and np.array_equal(xs, rxs) and np.array_equal(xsum, rxsum)
        y = np.empty(out, np.float32)
        fn = L.rqb_qmatmul_q4_x8 if nibble else L.rqb_qmatmul_q8_x8
        fn(ptr(xq), ptr(xs), ptr(xsum), ptr(wqi), ptr(wsi), ptr(y), in_, out, threads)
        assert orc.normwise_relerr(y, ref) < 1e-5


def test_cpu_baseline_qlinear_matches_the_oracle(orc):
    import ctypes as C

    L = orc.baseline_lib()
    ptr = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    rng = np.random.default_rng(92)
    m, out, in_ = 3, 40, 256
    codes = rng.integers(-127, 128, out * in_, dtype=np.int8)
    scales = rng.uniform(0.002, 0.02, out * in_ // 32).astype(np.float32)
    x = rng.standard_normal(m * in_).astype(np.float32)
    y = np.empty(m * out, np.float32)
    L.rqb_qlinear_q8(ptr(x), ptr(codes), ptr(scales), m, in_, out, ptr(y), 4)
    assert orc.normwise_relerr(y, orc.qlinear_q8(x, codes, scales, m, in_, out)) < 1e-6


# ---------------------------------------------------------------- dense f32 GEMM (blas.clj float arms, nn/linear)
def test_sgemm_reference_known_answers(orc):
    # test/raster/linalg/blas_test.clj:11-77: dgemm! identity, basic, alpha-beta,
    # dgemm-tn!, dgemm-nt! (integers, exact in f32)
    f = lambda v: np.array(v, np.float32)  # noqa: E731
    assert list(orc.sgemm(False, False, f([1, 0, 0, 1]), f([5, 6, 7, 8]), f([0] * 4), 2, 2, 2, 1.0, 0.0)) == [5, 6, 7, 8]
    assert list(orc.sgemm(False, False, f([1, 2, 3, 4, 5, 6]), f([7, 8, 9, 10, 11, 12]), f([0] * 4), 2, 3, 2, 1.0,
                          0.0)) == [58, 64, 139, 154]
    assert list(orc.sgemm(False, False, f([1, 0, 0, 1]), f([5, 6, 7, 8]), f([10, 20, 30, 40]), 2, 2, 2, 2.0,
                          3.0)) == [40, 72, 104, 136]
    assert list(orc.sgemm(True, False, f([1, 4, 2, 5, 3, 6]), f([7, 8, 9, 10, 11, 12]), f([0] * 4), 2, 3, 2, 1.0,
                          0.0)) == [58, 64, 139, 154]
    assert list(orc.sgemm(False, True, f([1, 2, 3, 4, 5, 6]), f([7, 9, 11, 8, 10, 12]), f([0] * 4), 2, 3, 2, 1.0,
                          0.0)) == [58, 64, 139, 154]


def test_linear_reference_known_answers(orc):
    # test/raster/dl/nn_test.clj:93-117: y = x W^T + b
    y = orc.linear(np.array([1, 2, 3], np.float32), np.array([1, 0, 0, 0, 1, 0], np.float32),
                   np.array([0.1, 0.2], np.float32), 1, 3, 2)
    assert list(y) == [np.float32(1) + np.float32(0.1), np.float32(2) + np.float32(0.2)]
    y = orc.linear(np.arange(1, 7, dtype=np.float32), np.array([1, 0, 0, 0, 1, 0], np.float32),
                   np.zeros(2, np.float32), 2, 3, 2)
    assert list(y) == [1, 2, 4, 5]


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True)])
def test_sgemm_against_numpy_f64(orc, ta, tb):
    # an independent f64 product (numpy), rounded once: a transposed operand,
    # a wrong leading dimension or a dropped alpha / beta term shows up far
    # above the f32 rounding of the two
    rng = np.random.default_rng(7)
    m, k, n = 7, 13, 5
    A = rng.standard_normal(m * k).astype(np.float32)
    B = rng.standard_normal(k * n).astype(np.float32)
    C0 = rng.standard_normal(m * n).astype(np.float32)
    Am = A.reshape(k, m).T if ta else A.reshape(m, k)
    Bm = B.reshape(n, k).T if tb else B.reshape(k, n)
    want = (0.75 * (Am.astype(np.float64) @ Bm.astype(np.float64)) - 1.5 * C0.reshape(m, n)).astype(np.float32)
    got = orc.sgemm(ta, tb, A, B, C0, m, k, n, 0.75, -1.5).reshape(m, n)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)


def test_sgemm_and_linear_degenerate_shapes_do_nothing(orc):
    # blas.clj:301,318,334 skip the call unless m, n and k are all positive;
    # nn/linear still writes the bias rows when in_f is 0 (nn.clj:170-171)
    C0 = np.array([1, 2, 3, 4], np.float32)
    for m, k, n in ((0, 2, 2), (2, 0, 2), (2, 2, 0)):
        assert list(orc.sgemm(False, False, np.ones(4, np.float32), np.ones(4, np.float32), C0, m, k, n, 1.0,
                              0.0)) == [1, 2, 3, 4]
    y = orc.linear(np.zeros(0, np.float32), np.zeros(0, np.float32), np.array([3, 4], np.float32), 2, 0, 2)
    assert list(y) == [3, 4, 3, 4]
