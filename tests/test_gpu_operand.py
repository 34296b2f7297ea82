"""The weight operand each matmul kernel actually consumes, read back bit for
bit, and full outputs at C2 and C5 (M = 256) against an f64 product.

One-hot activations: row r of x is 1 at a single k_r and 0 elsewhere. Every
product with 1 and every sum with 0 is exact in f32 (also across the K-split
kernels' partial sums), so y[r, o] is exactly the operand the kernel used
for W[o, k_r]:
  * bf16 GEMMs (bf16 x, m > 16): RNE-to-bf16 of Raster's dequant,
    f32(scale * code) (raster/quant/train.clj:60-71; Q4_0 scale * (q - 8),
    raster/compiler/backend/cpu/quant.clj:27-31), widened back to f32;
  * exact-code kernels (f32 x: the f32 GEMM, the MFMA decode, the int8-level
    decode, the v_dot4 GEMV): the f32 dequant itself.
The expected values come from the oracle's bit-exact dequant (pinned on the
CPU in test_oracle.py). At the C2 and C5 shapes, and for the 256 x 192 kernel
at M = 1024, consecutive calls take consecutive k ranges, so every element of
the weight is compared; the decode kernels take spread k positions covering
every in-block offset.

Full outputs: seeded bf16 x at C2 (M 512, K 4096, N 11008, Q8) and C5
(M 256, K 8192, N 28672, Q8 and Q4), every column of y against the f64 product
of x with the oracle's f32 dequantized weight: max|y - ref| <= 1e-2 max|ref|
(bf16 activations, north_star's bar).
"""
import numpy as np
import pytest

from raster_amd import workloads as wl

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


def make(raster_amd, ctx, fmt, out, in_, seed):
    if fmt == "q8":
        codes, scales = wl.q8_weights(out, in_, seed=seed)
        return raster_amd.QWeight.q8(codes, scales, out, in_, ctx), (codes, scales)
    packed, sc16 = wl.q4_weights(out, in_, seed=seed)
    return raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx), (packed, sc16)


def dequant_cols(orc, fmt, arrs, out, in_, k0, k1):
    """The oracle's f32 dequant of columns [k0, k1) (whole 32-blocks), [out, k1 - k0]."""
    nb, w = in_ // 32, k1 - k0
    if fmt == "q8":
        codes, scales = arrs
        c = codes.reshape(out, in_)[:, k0:k1]
        s = scales.reshape(out, nb)[:, k0 // 32:k1 // 32]
        return orc.dequant_q8_dense(c, s, w, out).reshape(out, w)
    packed, sc16 = arrs
    p = packed.reshape(out, in_ // 2)[:, k0 // 2:k1 // 2]
    s = sc16.reshape(out, nb)[:, k0 // 32:k1 // 32]
    return orc.dequant_q4(p, s, w, out).reshape(out, w)


def dequant_at(orc, fmt, arrs, out, in_, ks):
    """The oracle's f32 dequant of the columns ks, [out, len(ks)] (via their blocks)."""
    cols = []
    for k in ks:
        b = k // 32
        d = dequant_cols(orc, fmt, arrs, out, in_, 32 * b, 32 * b + 32)
        cols.append(d[:, k - 32 * b])
    return np.stack(cols, axis=1)


def one_hot(torch, m, in_, ks, xdt):
    x = torch.zeros((m, in_), dtype=torch.float32)
    x[torch.arange(m), torch.as_tensor(ks)] = 1.0
    x = x.cuda()
    return x.to(torch.bfloat16) if xdt == "bf16" else x


# (format, out, in, m, kernel): bf16 x, every weight element read back
GEMM_CASES = [
    ("q8", 11008, 4096, 512, "C2: role-split 256 x 96"),
    ("q4", 11008, 4096, 512, "role-split 256 x 96, Q4_0"),
    ("q8", 28672, 8192, 256, "C5: role-split 256 x 128"),
    ("q4", 28672, 8192, 256, "C5: role-split 256 x 128, Q4_0"),
    ("q8", 11008, 4096, 1024, "one wave per SIMD, 256 x 192"),
    ("q4", 4096, 2048, 48, "weight-stream small-m GEMM"),
    ("q8", 2048, 2048, 100, "64 < m <= 128 GEMM"),
]


@pytest.mark.parametrize("fmt,out,in_,m,kernel", GEMM_CASES, ids=[c[4] for c in GEMM_CASES])
def test_bf16_gemm_operand_is_rne_of_dequant(torch, ctx, orc, fmt, out, in_, m, kernel):
    import raster_amd

    w, arrs = make(raster_amd, ctx, fmt, out, in_, seed=out + in_ + m)
    try:
        calls = 0
        for k0 in range(0, in_, m):
            k1 = min(k0 + m, in_)
            ks = list(range(k0, k1))
            ks += [ks[-1]] * (m - len(ks))  # rows past K repeat the last column
            note(f"operand {kernel} {fmt} k {k0}..{k1}")
            y = w.matmul(one_hot(torch, m, in_, ks, "bf16"), out_dtype=torch.float32).cpu().numpy()
            a0, a1 = k0 // 32 * 32, (k1 + 31) // 32 * 32
            d = dequant_cols(orc, fmt, arrs, out, in_, a0, a1)[:, [k - a0 for k in ks]]
            exp = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(d)).reshape(out, m).T
            bad = np.flatnonzero(y.view(np.uint32) != exp.view(np.uint32))
            assert bad.size == 0, (kernel, k0, bad[:5], y.ravel()[bad[:5]], exp.ravel()[bad[:5]])
            calls += 1
        assert calls * m >= in_
    finally:
        w.destroy()


# (format, out, in, m, x dtype, kernel): exact-code kernels, spread k positions
EXACT_CASES = [
    ("q8", 1000, 1024, 300, "f32 GEMM"),
    ("q8", 4096, 4096, 16, "MFMA decode Q8_0"),
    ("q4", 14336, 4096, 8, "MFMA decode Q4_0"),
    ("q8", 4096, 4096, 4, "int8-level decode"),
    ("q4", 4096, 4096, 3, "int8-level decode Q4_0"),
    ("q4", 14336, 4096, 1, "v_dot4 GEMV"),
]


@pytest.mark.parametrize("fmt,out,in_,m,kernel", EXACT_CASES, ids=[c[4] for c in EXACT_CASES])
def test_exact_code_kernels_use_the_f32_dequant(torch, ctx, orc, fmt, out, in_, m, kernel):
    import raster_amd

    w, arrs = make(raster_amd, ctx, fmt, out, in_, seed=7 * out + in_ + m)
    try:
        # 288 positions (>= every in-block offset several times) spread over K
        npos = max(288, m)
        pos = [(37 * i + i // 32) % in_ for i in range(npos)]
        for c0 in range(0, npos, m):
            ks = pos[c0:c0 + m]
            ks += [ks[-1]] * (m - len(ks))
            note(f"exact {kernel} {fmt} call {c0 // m}")
            y = w.matmul(one_hot(torch, m, in_, ks, "f32"), out_dtype=torch.float32).cpu().numpy()
            exp = dequant_at(orc, fmt, arrs, out, in_, ks).T
            bad = np.flatnonzero(y.view(np.uint32) != exp.view(np.uint32))
            assert bad.size == 0, (kernel, c0, bad[:5], y.ravel()[bad[:5]], exp.ravel()[bad[:5]])
    finally:
        w.destroy()


FULL_CASES = [("q8", 11008, 4096, 512, "C2"), ("q8", 28672, 8192, 256, "C5 Q8"), ("q4", 28672, 8192, 256, "C5 Q4")]


@pytest.mark.parametrize("fmt,out,in_,m,name", FULL_CASES, ids=[c[4] for c in FULL_CASES])
def test_full_output_against_f64_product(torch, ctx, orc, fmt, out, in_, m, name):
    import raster_amd

    w, arrs = make(raster_amd, ctx, fmt, out, in_, seed=11 + m)
    try:
        note(f"full output {name}")
        x = wl.activations(m, in_, seed=23 + m, dtype="bf16").reshape(m, in_)
        xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
        y = w.matmul(xt, out_dtype=torch.bfloat16).float().cpu().numpy()
        x64 = x.astype(np.float64)
        worst, top = 0.0, 0.0
        for o0 in range(0, out, 4096):
            o1 = min(o0 + 4096, out)
            if fmt == "q8":
                codes, scales = arrs
                W = orc.dequant_q8_dense(codes[o0 * in_:o1 * in_], scales[o0 * in_ // 32:o1 * in_ // 32], in_, o1 - o0)
            else:
                packed, sc16 = arrs
                W = orc.dequant_q4(packed[o0 * in_ // 2:o1 * in_ // 2], sc16[o0 * in_ // 32:o1 * in_ // 32], in_,
                                   o1 - o0)
            ref = x64 @ W.reshape(o1 - o0, in_).astype(np.float64).T
            worst = max(worst, float(np.abs(y[:, o0:o1] - ref).max()))
            top = max(top, float(np.abs(ref).max()))
        note(f"full output {name}: max|y - ref| / max|ref| = {worst / top:.2e}")
        assert np.all(np.isfinite(y))
        assert worst <= 1e-2 * top
    finally:
        w.destroy()
