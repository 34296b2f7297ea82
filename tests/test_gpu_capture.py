"""Graph capture and concurrency of the matmul entries, where the design relies
on them (per-stream scratch, the no-alloc entry's fixed scratch, split kernels
that merge partial sums with a second launch).

The reference's GPU tests ask the same of its kernels: two bindings of one
kernel do not clobber each other, a quantizer -> matmul chain runs in one
graph, replays are idempotent and each op reads its own buffers
(test/raster/quant/kernels_k_gpu_test.clj:212-310).

  * one graph holding a bf16 prefill GEMM, an rq_quantize_act_i8 ->
    rq_qmatmul_i8 chain, a K-quant rq_qmatmul and rq_qmatmul_noalloc calls
    on two weights, replayed three times with eager calls on the same stream
    (and the same scratch) in between: every replay equals the eager results
    bit for bit;
  * a graph captured before a larger call on its stream grew the scratch
    still replays correctly (a grown buffer is retired, not freed);
  * two streams, and two host threads with a stream each, running split and
    GEMM calls of different shapes at once on one context: each result equals
    its single-stream result bit for bit.
"""
import threading

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


def q8(raster_amd, ctx, out, in_, seed):
    codes, scales = wl.q8_weights(out, in_, seed=seed)
    return raster_amd.QWeight.q8(codes, scales, out, in_, ctx)


def q4(raster_amd, ctx, out, in_, seed):
    packed, sc16 = wl.q4_weights(out, in_, seed=seed)
    return raster_amd.QWeight.q4(packed, sc16.view(np.float16), out, in_, ctx)


def q4k(raster_amd, ctx, orc, out, in_, seed):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal(out * in_) * 0.05).astype(np.float32)
    return raster_amd.QWeight.q4k(*orc.quantize_weight_q4k(W), out, in_, ctx)


def act(torch, m, in_, seed, dtype):
    x = torch.from_numpy(wl.activations(m, in_, seed=seed)).cuda().reshape(m, in_)
    return x.to(torch.bfloat16) if dtype == "bf16" else x


def bits(t):
    return t.contiguous().view(torch_int_like(t)).cpu().numpy().copy()


def torch_int_like(t):
    import torch

    return {torch.float32: torch.int32, torch.bfloat16: torch.int16, torch.int8: torch.int8,
            torch.int32: torch.int32}[t.dtype]


def noalloc(ctx, w, x, y, stream):
    import ctypes as C

    from raster_amd import _lib

    xc = _lib.RQ_BF16 if x.dtype.itemsize == 2 else _lib.RQ_F32
    yc = _lib.RQ_BF16 if y.dtype.itemsize == 2 else _lib.RQ_F32
    _lib.call("rq_qmatmul_noalloc", ctx.handle, w.handle, C.c_void_p(x.data_ptr()), xc, C.c_void_p(y.data_ptr()), yc,
              x.numel() // w.in_, C.c_void_p(stream.cuda_stream))


def test_graph_of_mixed_calls_replays_bit_for_bit(torch, ctx, orc):
    import raster_amd

    note("graph: bf16 GEMM + int8 chain + K-quant + no-alloc on two weights")
    wa = q8(raster_amd, ctx, 11008, 4096, seed=1)      # prefill GEMM (role-split kernel)
    wb = q4(raster_amd, ctx, 4096, 4096, seed=2)       # int8 chain: quantize_act_i8 -> int8 GEMM
    wc = q4k(raster_amd, ctx, orc, 2048, 2048, seed=3)  # K-quant, f32 x quantized in the call
    wd = q8(raster_amd, ctx, 4160, 8192, seed=4)       # no-alloc: int8-level decode with K-split
    we = q4(raster_amd, ctx, 8192, 8192, seed=5)       # no-alloc: small-m GEMM with K-slices
    s = torch.cuda.Stream()
    try:
        xa = act(torch, 512, 4096, 11, "bf16")
        xb = act(torch, 64, 4096, 12, "f32")
        xc = act(torch, 4, 2048, 13, "f32")
        xd = act(torch, 12, 8192, 14, "f32")
        xe = act(torch, 64, 8192, 15, "bf16")
        ya = torch.empty((512, 11008), dtype=torch.bfloat16, device="cuda")
        qb = (torch.empty((64, 4096), dtype=torch.int8, device="cuda"),
              torch.empty((64, 128), dtype=torch.float32, device="cuda"),
              torch.empty((64, 128), dtype=torch.int32, device="cuda"))
        yb = torch.empty((64, 4096), dtype=torch.float32, device="cuda")
        yc = torch.empty((4, 2048), dtype=torch.float32, device="cuda")
        yd = torch.empty((12, 4160), dtype=torch.float32, device="cuda")
        ye = torch.empty((64, 8192), dtype=torch.bfloat16, device="cuda")
        outs = [ya, yb, yc, yd, ye]

        def calls():
            wa.matmul(xa, y=ya, stream=s)
            raster_amd.quantize_act_i8(ctx, xb, 4096, out=qb, stream=s)
            wb.matmul_i8(*qb, y=yb, stream=s)
            wc.matmul(xc, y=yc, stream=s)
            noalloc(ctx, wd, xd, yd, s)
            noalloc(ctx, we, xe, ye, s)

        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            calls()  # eager: allocates the stream's scratch
        s.synchronize()
        ref = [bits(o) for o in outs]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            calls()
        # eager calls between replays: same stream, same scratch, other inputs
        xa2, xe2 = act(torch, 512, 4096, 21, "bf16"), act(torch, 64, 8192, 22, "bf16")
        ya2, ye2 = torch.empty_like(ya), torch.empty_like(ye)
        for r in range(3):
            for o in outs:
                o.zero_()
            g.replay()
            torch.cuda.synchronize()
            for name, o, want in zip("abcde", outs, ref):
                assert np.array_equal(bits(o), want), (r, name)
            with torch.cuda.stream(s):
                wa.matmul(xa2, y=ya2, stream=s)
                noalloc(ctx, we, xe2, ye2, s)
            _ = torch.ones(16, device="cuda").sum().item()
            s.synchronize()
    finally:
        for w in (wa, wb, wc, wd, we):
            w.destroy()


def test_graph_survives_scratch_growth(torch, ctx):
    import raster_amd

    note("graph captured before the stream's scratch grew")
    w = q8(raster_amd, ctx, 4096, 4096, seed=6)
    s = torch.cuda.Stream()
    try:
        xs_ = act(torch, 200, 4096, 31, "bf16")
        ys = torch.empty((200, 4096), dtype=torch.bfloat16, device="cuda")
        xl = act(torch, 2048, 4096, 32, "bf16")
        yl = torch.empty((2048, 4096), dtype=torch.bfloat16, device="cuda")
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            w.matmul(xs_, y=ys, stream=s)
        s.synchronize()
        ref = bits(ys)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            w.matmul(xs_, y=ys, stream=s)
        with torch.cuda.stream(s):
            w.matmul(xl, y=yl, stream=s)  # needs a larger packed-activation buffer
        s.synchronize()
        ref_l = bits(yl)
        for _ in range(3):
            ys.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(bits(ys), ref)
            with torch.cuda.stream(s):
                w.matmul(xl, y=yl, stream=s)
            s.synchronize()
            assert np.array_equal(bits(yl), ref_l)
    finally:
        w.destroy()


def concurrent_cases(raster_amd, ctx, torch):
    """(weight, x, y dtype) of calls with scratch: K-split decode, MFMA decode
    with slices, small-m GEMM with slices, prefill GEMM."""
    return [
        (q8(raster_amd, ctx, 4160, 8192, seed=41), act(torch, 12, 8192, 51, "f32"), torch.float32),
        (q4(raster_amd, ctx, 14336, 4096, seed=42), act(torch, 16, 4096, 52, "f32"), torch.float32),
        (q8(raster_amd, ctx, 28672, 8192, seed=43), act(torch, 32, 8192, 53, "bf16"), torch.bfloat16),
        (q8(raster_amd, ctx, 11008, 4096, seed=44), act(torch, 512, 4096, 54, "bf16"), torch.bfloat16),
    ]


def test_two_streams_at_once(torch, ctx):
    import raster_amd

    note("two streams, split and GEMM calls interleaved")
    cases = concurrent_cases(raster_amd, ctx, torch)
    try:
        ref = []
        for w, x, ydt in cases:
            ref.append(bits(w.matmul(x, out_dtype=ydt)))
        torch.cuda.synchronize()
        s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
        for st in (s1, s2):
            st.wait_stream(torch.cuda.current_stream())
        ys = [torch.empty((x.shape[0], w.out), dtype=ydt, device="cuda") for w, x, ydt in cases]
        for rep in range(4):
            for o in ys:
                o.zero_()
            torch.cuda.synchronize()
            # stream 1: cases 0 and 2, stream 2: cases 1 and 3, submitted alternately
            for i in (0, 1, 2, 3):
                st = s1 if i % 2 == 0 else s2
                w, x, _ = cases[i]
                w.matmul(x, y=ys[i], stream=st)
            torch.cuda.synchronize()
            for i, (o, want) in enumerate(zip(ys, ref)):
                assert np.array_equal(bits(o), want), (rep, i)
    finally:
        for w, _, _ in cases:
            w.destroy()


def test_two_host_threads_at_once(torch, ctx):
    import raster_amd

    note("two host threads, a stream each, on one context")
    cases = concurrent_cases(raster_amd, ctx, torch)
    try:
        ref = [bits(w.matmul(x, out_dtype=ydt)) for w, x, ydt in cases]
        torch.cuda.synchronize()
        errors = []

        def worker(ids):
            try:
                st = torch.cuda.Stream()
                st.wait_stream(torch.cuda.current_stream())
                ys = {i: torch.empty((cases[i][1].shape[0], cases[i][0].out), dtype=cases[i][2], device="cuda")
                      for i in ids}
                for rep in range(6):
                    for i in ids:
                        w, x, _ = cases[i]
                        w.matmul(x, y=ys[i], stream=st)
                    st.synchronize()
                    for i in ids:
                        if not np.array_equal(bits(ys[i]), ref[i]):
                            errors.append((rep, i))
            except Exception as e:  # reported by the main thread
                errors.append(repr(e))

        t1 = threading.Thread(target=worker, args=((0, 3),))
        t2 = threading.Thread(target=worker, args=((1, 2),))
        t1.start()
        t2.start()
        t1.join(timeout=90)
        t2.join(timeout=90)
        assert not t1.is_alive() and not t2.is_alive()
        assert not errors, errors
    finally:
        for w, _, _ in cases:
            w.destroy()
