"""GPU parity of the fused decode chain against the C oracle.

rq_qmatmul_fused: the decode matmul with the input RMSNorm
(raster/dl/nn.clj:497-516) before it and either the SwiGLU of a gate/up row
pair (nn.clj:200-203) or the residual add (nn.clj:217-219) after it. The
oracle composes its own restatements of those ops with qlinear-q8 / the Q4_0
matmul; gains are random (not 1.0) so a dropped or misplaced gain fails.

rq_decode_attention: rope-pos (raster/dl/attention.clj:197-214), kv-append!
(attention.clj:413-416) and gqa-decode-attention (attention.clj:248-287) in
one launch, against the oracle's three functions in sequence.

Bars: normwise max|y - ref| / max|ref| < 1e-3 for f32 activations and < 1e-2
for bf16 (as for the plain matmul); the appended cache rows < 1e-6 (RoPE only:
both sides rotate in double and round once); untouched cache rows bit-exact.
"""
import math

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


def dev(torch, a, dtype="f32"):
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    return t.to(torch.bfloat16) if dtype == "bf16" else t


def gains(n, seed):
    # signed gains away from 1.0: a dropped gain or an offset shows
    rng = np.random.default_rng(seed)
    return (rng.uniform(0.25, 2.0, n) * rng.choice([-1.0, 1.0], n)).astype(np.float32)


def make_weight(raster_amd, ctx, orc, fmt, out, in_, seed):
    """(QWeight, oracle matmul x -> y[m*out])."""
    if fmt == "q8":
        codes, scales = wl.q8_weights(out, in_, seed=seed)
        w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
        return w, lambda x, m: orc.qlinear_q8(x, codes, scales, m, in_, out)
    packed, sc16 = wl.q4_weights(out, in_, seed=seed)
    w = raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)
    return w, lambda x, m: orc.qlinear_q4(x, packed, sc16, m, in_, out)


def xin(x, xdt):
    """The activations the kernel sees (bf16 inputs are rounded first)."""
    return wl.bf16_round(x) if xdt == "bf16" else x


# ---------------------------------------------------------------- fused matmul
@pytest.mark.parametrize("m,in_,out", [(1, 2048, 6144), (3, 160, 40), (16, 4096, 64), (2, 20480, 32)])
@pytest.mark.parametrize("fmt", ["q8", "q4"])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_fused_norm(torch, ctx, orc, m, in_, out, fmt, xdt):
    # RMSNorm of every row over all of K, then the matmul; (2, 20480) runs the
    # K-split kernel (every slice's workgroup forms the row norms itself)
    import raster_amd

    eps = 1e-5
    x = wl.activations(m, in_, seed=m + in_, dtype=xdt)
    g = gains(in_, seed=in_)
    note(f"fused norm {fmt} {xdt} m={m} {out}x{in_}")
    w, ref_mm = make_weight(raster_amd, ctx, orc, fmt, out, in_, seed=out + 3)
    y = w.matmul_fused(dev(torch, x, xdt).reshape(m, in_), norm_gain=dev(torch, g), norm_eps=eps)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    w.destroy()
    ref = ref_mm(orc.rms_norm(xin(x, xdt), g, m, in_, eps, 0.0), m).reshape(m, out)
    assert orc.normwise_relerr(y, ref) < (TOL_F32 if xdt == "f32" else TOL_BF16)


@pytest.mark.parametrize("m,in_,out", [(1, 2048, 2048), (5, 96, 48), (16, 5632, 80), (2, 20480, 16)])
@pytest.mark.parametrize("ydt", ["f32", "bf16"])
def test_fused_residual(torch, ctx, orc, m, in_, out, ydt):
    import raster_amd

    x = wl.activations(m, in_, seed=7 * m + in_)
    r = wl.activations(m, out, seed=out) * 3.0
    note(f"fused residual {ydt} m={m} {out}x{in_}")
    w, ref_mm = make_weight(raster_amd, ctx, orc, "q8", out, in_, seed=out + in_)
    tdt = torch.bfloat16 if ydt == "bf16" else torch.float32
    res = dev(torch, r, ydt).reshape(m, out)
    y = w.matmul_fused(dev(torch, x).reshape(m, in_), out_dtype=tdt, residual=res)
    torch.cuda.synchronize()
    y = y.float().cpu().numpy()
    w.destroy()
    rr = xin(r, ydt)
    ref = orc.residual_add(ref_mm(x, m), rr, m * out).reshape(m, out)
    assert orc.normwise_relerr(y, ref) < (TOL_F32 if ydt == "f32" else TOL_BF16)


@pytest.mark.parametrize("m,in_,ffn", [(1, 2048, 5632), (4, 128, 24), (16, 4096, 40), (1, 20480, 8),
                                       (16, 5632, 24), (9, 14336, 40)])
@pytest.mark.parametrize("norm", [False, True], ids=["plain", "norm"])
def test_fused_swiglu(torch, ctx, orc, m, in_, ffn, norm):
    # gate row i and up row i stored as rows 2i / 2i+1; y[m, ffn] =
    # silu(gate) * up, optionally of the RMSNorm of x; (1, 20480), (16, 5632)
    # and (9, 14336) cut K into slices (the epilogue runs in the reduce kernel)
    import raster_amd

    eps = 1e-5
    cg, sg = wl.q8_weights(ffn, in_, seed=ffn + 1)
    cu, su = wl.q8_weights(ffn, in_, seed=ffn + 2)
    codes = np.stack([cg.reshape(ffn, in_), cu.reshape(ffn, in_)], axis=1).reshape(-1)
    scales = np.stack([sg.reshape(ffn, -1), su.reshape(ffn, -1)], axis=1).reshape(-1)
    x = wl.activations(m, in_, seed=m * in_)
    g = gains(in_, seed=ffn)
    note(f"fused swiglu norm={norm} m={m} ffn={ffn} in={in_}")
    w = raster_amd.QWeight.q8(np.ascontiguousarray(codes), np.ascontiguousarray(scales), 2 * ffn, in_, ctx)
    kw = dict(norm_gain=dev(torch, g), norm_eps=eps) if norm else {}
    y = w.matmul_fused(dev(torch, x).reshape(m, in_), swiglu=True, **kw)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    w.destroy()
    xn = orc.rms_norm(x, g, m, in_, eps, 0.0) if norm else x
    gate = orc.qlinear_q8(xn, cg, sg, m, in_, ffn)
    up = orc.qlinear_q8(xn, cu, su, m, in_, ffn)
    ref = orc.silu_mul(gate, up, m * ffn).reshape(m, ffn)
    assert y.shape == (m, ffn)
    assert orc.normwise_relerr(y, ref) < TOL_F32


def test_fused_matches_plain_without_ops(torch, ctx):
    # an empty rq_fused_ops is the plain matmul, bit for bit
    import raster_amd

    m, in_, out = 4, 4096, 256
    codes, scales = wl.q8_weights(out, in_, seed=1)
    w = raster_amd.QWeight.q8(codes, scales, out, in_, ctx)
    x = dev(torch, wl.activations(m, in_, seed=2)).reshape(m, in_)
    a = w.matmul(x)
    b = w.matmul_fused(x)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    w.destroy()


def test_fused_rejects_bad_options(torch, ctx):
    import raster_amd
    from raster_amd import RqError
    from raster_amd._lib import RQ_ERR_SHAPE

    codes, scales = wl.q8_weights(48, 64, seed=1)
    w = raster_amd.QWeight.q8(codes, scales, 48, 64, ctx)
    x17 = torch.zeros((17, 64), device="cuda")
    g = torch.ones(64, device="cuda")
    with pytest.raises(RqError) as e:
        w.matmul_fused(x17, norm_gain=g)  # m > 16: no decode kernel
    assert e.value.status == RQ_ERR_SHAPE
    x = torch.zeros((1, 64), device="cuda")
    with pytest.raises(RqError) as e:
        w.matmul_fused(x, y=torch.empty((1, 24), device="cuda"), swiglu=True,
                       residual=None, norm_gain=torch.ones(68, device="cuda")[1:65])  # misaligned gain
    assert e.value.status == RQ_ERR_SHAPE
    with pytest.raises(RqError) as e:
        w.matmul_fused(x, y=torch.empty((1, 24), device="cuda"), swiglu=True,
                       residual=torch.zeros((1, 24), device="cuda"))
    assert e.value.status == RQ_ERR_SHAPE
    w.destroy()
    codes, scales = wl.q8_weights(47, 64, seed=1)
    w = raster_amd.QWeight.q8(codes, scales, 47, 64, ctx)
    with pytest.raises(RqError) as e:
        w.matmul_fused(x, y=torch.empty((1, 23), device="cuda"), swiglu=True)  # odd row count
    assert e.value.status == RQ_ERR_SHAPE
    w.destroy()


# ---------------------------------------------------------------- decode attention
@pytest.mark.parametrize("n_q,n_kv,hd,pos", [
    (16, 16, 128, 128), (8, 2, 64, 9), (32, 8, 128, 1000), (4, 4, 64, 0), (4, 1, 256, 5), (2, 2, 320, 3),
    (8, 8, 128, 20000), (4, 2, 128, 63), (4, 2, 128, 64), (4, 2, 128, 65), (6, 3, 96, 200), (2, 1, 512, 70),
    (4, 4, 16, 300), (4, 2, 66, 7), (2, 1, 18, 300), (3, 3, 66, 30000), (2, 1, 512, 2000), (4, 2, 96, 4100),
    (32, 8, 128, 2048), (16, 2, 128, 3000), (8, 2, 64, 5000), (16, 4, 256, 2100), (8, 1, 16, 2500),
    (8, 2, 64, 200), (4, 1, 256, 100), (4, 4, 16, 129)])
def test_decode_attention(torch, ctx, orc, n_q, n_kv, hd, pos):
    # head_dim a multiple of 4 up to 512 runs the chunk kernel (chunks of 64
    # rows at hd 128: pos 63 / 64 / 65 end inside, at and past a chunk;
    # hd 96 / 320 leave lanes idle); a single range longer than two chunks of
    # 2 rows per lane takes 8 (4 at hd > 256) rows per lane: (16, 16, 128, 128),
    # (4, 2, 128, 65), (6, 3, 96, 200), (2, 1, 512, 70), (8, 2, 64, 200),
    # (4, 1, 256, 100), (4, 4, 16, 129); from 256 cached rows the rows split into
    # ranges per head, merged by a second kernel ((.., 1000), (.., 20000),
    # (4, 4, 16, 300), (2, 1, 512, 2000), (4, 2, 96, 4100): ragged last
    # range); 66 and 18 run the generic kernel ((3, 3, 66, 30000): scores
    # beyond 64 KB of LDS). (.., 0): only the new key. From 2048 rows, 4 or 8
    # query heads per KV head take the grouped-query kernel (a workgroup per KV
    # head and range): (32, 8, 128, 2048), (16, 2, 128, 3000), (8, 2, 64, 5000),
    # (16, 4, 256, 2100), (8, 1, 16, 2500)
    import raster_amd

    kvd = n_kv * hd
    theta = 1e4
    rng = np.random.default_rng(n_q * 1000 + pos)
    q = rng.standard_normal(n_q * hd, dtype=np.float32)
    k = rng.standard_normal(kvd, dtype=np.float32)
    v = rng.standard_normal(kvd, dtype=np.float32)
    kc = np.zeros((pos + 2, kvd), np.float32)
    vc = np.zeros((pos + 2, kvd), np.float32)
    kc[:pos] = rng.standard_normal((pos, kvd), dtype=np.float32)
    vc[:pos] = rng.standard_normal((pos, kvd), dtype=np.float32)
    kc[pos + 1] = 7.0  # rows past pos stay untouched
    vc[pos + 1] = -7.0
    scale = 1.0 / math.sqrt(hd)
    note(f"decode attention n_q={n_q} n_kv={n_kv} hd={hd} pos={pos}")
    dkc, dvc = dev(torch, kc), dev(torch, vc)
    out = raster_amd.decode_attention(ctx, dev(torch, q), dev(torch, k), dev(torch, v), dkc, dvc, pos, n_q, n_kv, hd,
                                      theta, scale)
    torch.cuda.synchronize()
    out, gkc, gvc = out.cpu().numpy(), dkc.cpu().numpy(), dvc.cpu().numpy()

    qr = orc.rope_pos(q, 1, n_q, hd, theta, pos)
    rkc, rvc = kc.copy(), vc.copy()
    rkc[pos] = orc.rope_pos(k, 1, n_kv, hd, theta, pos)
    rvc[pos] = v
    ref = orc.gqa_decode_attention(qr, rkc, rvc, pos + 1, n_q, n_kv, hd, scale)
    assert np.array_equal(gkc[:pos], kc[:pos]) and np.array_equal(gvc[:pos], vc[:pos])
    assert np.array_equal(gkc[pos + 1:], kc[pos + 1:]) and np.array_equal(gvc[pos + 1:], vc[pos + 1:])
    assert np.array_equal(gvc[pos], v)
    assert orc.normwise_relerr(gkc[pos], rkc[pos]) < 1e-6
    assert orc.normwise_relerr(out, ref) < TOL_F32


def test_decode_attention_rejects_bad_shapes(torch, ctx):
    import raster_amd
    from raster_amd import RqError
    from raster_amd._lib import RQ_ERR_SHAPE

    z = lambda n: torch.zeros(n, device="cuda")  # noqa: E731
    with pytest.raises(RqError) as e:  # n_q not a multiple of n_kv
        raster_amd.decode_attention(ctx, z(3 * 64), z(2 * 64), z(2 * 64), z(4 * 128), z(4 * 128), 1, 3, 2, 64, 1e4,
                                    0.125)
    assert e.value.status == RQ_ERR_SHAPE
    with pytest.raises(RqError) as e:  # generic kernel: cache too long for LDS
        n = 50000
        raster_amd.decode_attention(ctx, z(66), z(66), z(66), z((n + 1) * 66), z((n + 1) * 66), n, 1, 1, 66, 1e4,
                                    0.125)
    assert e.value.status == RQ_ERR_SHAPE


@pytest.mark.parametrize("n_q,n_kv,hd,pos", [(16, 16, 128, 512), (32, 8, 128, 1000), (4, 4, 16, 300),
                                             (64, 8, 128, 4096)])
def test_decode_attention_split_repeats_and_graph(torch, ctx, orc, n_q, n_kv, hd, pos):
    # shapes that split the cached rows over several workgroups per head: each
    # range writes its softmax record, decode_attention_merge_kernel merges the
    # ranges in range order, so repeated calls, and replays of a captured call
    # with eager work in between, give the first call's output bit for bit
    import raster_amd

    kvd = n_kv * hd
    rng = np.random.default_rng(7 + pos)
    q = rng.standard_normal(n_q * hd, dtype=np.float32)
    k = rng.standard_normal(kvd, dtype=np.float32)
    v = rng.standard_normal(kvd, dtype=np.float32)
    kc = np.zeros((pos + 1, kvd), np.float32)
    vc = np.zeros((pos + 1, kvd), np.float32)
    kc[:pos] = rng.standard_normal((pos, kvd), dtype=np.float32)
    vc[:pos] = rng.standard_normal((pos, kvd), dtype=np.float32)
    scale = 1.0 / math.sqrt(hd)
    note(f"decode attention split repeats n_q={n_q} n_kv={n_kv} hd={hd} pos={pos}")
    dq, dk, dv, dkc, dvc = dev(torch, q), dev(torch, k), dev(torch, v), dev(torch, kc), dev(torch, vc)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    outs = []
    with torch.cuda.stream(s):
        out = torch.empty(n_q * hd, device="cuda")
        for _ in range(3):
            raster_amd.decode_attention(ctx, dq, dk, dv, dkc, dvc, pos, n_q, n_kv, hd, 1e4, scale, out=out)
            s.synchronize()
            outs.append(out.cpu().numpy().copy())
    qr = orc.rope_pos(q, 1, n_q, hd, 1e4, pos)
    rkc, rvc = kc.copy(), vc.copy()
    rkc[pos] = orc.rope_pos(k, 1, n_kv, hd, 1e4, pos)
    rvc[pos] = v
    ref = orc.gqa_decode_attention(qr, rkc, rvc, pos + 1, n_q, n_kv, hd, scale)
    assert orc.normwise_relerr(outs[0], ref) < TOL_F32
    assert all(np.array_equal(outs[0], o) for o in outs[1:])
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        raster_amd.decode_attention(ctx, dq, dk, dv, dkc, dvc, pos, n_q, n_kv, hd, 1e4, scale, out=out)
    for _ in range(3):
        out.fill_(0.0)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), outs[0])
        _ = torch.ones(16, device="cuda").sum().item()  # eager work between replays
