"""Benchmark of librq's block-quantized matmul on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--suite all|headline]

Headline (the JSON `value`): the Q8 prefill GEMM of the second workload
configuration (C2), M=512 K=4096 N=11008, bf16 activations, bf16 output, f32
accumulation, weights resident in HBM. A step is one rq_qmatmul call over that
batch (activation packing + GEMM); `value` is TFLOP/s (2*M*K*N flop per step),
timed with HIP events on the stream the kernels run on. Before the W warm-up
steps the step runs untimed for RAMP_S seconds so that the timed steps see the
GPU at its working clocks.

Beside it, on the same JSON line (default suite "all"; "headline" keeps C2,
the C1 GEMV and the CPU baseline):
  gemv          C1: the M=1 Q8 decode GEMV (K=N=4096, f32 in/out).
  configs       every other workload configuration, one line per shape:
                C3 (Q4, M = 1 / 4 / 16, K=4096 N=14336, f32) and C5 (Q4 and Q8,
                K=8192 N=28672, bf16, M = 1 / 32 / 256).
  decoder       C4: the two-layer decode step in one captured HIP graph.
  read_ceiling  a plain streaming read (rq_stream_read) of the C1, C3 and C5
                weight sizes, timed like the decode lines: the most any
                kernel reading that many bytes per launch reaches here.
  int8, kquant  the int8-activation path and the K-quant GEMV (next-step
                rows of the path), as before.
  dx            backward-data (qlinear-q8-dx) of the C2 layer's weight at
                m = 16 and 512 dy rows (the MFMA GEMM path).
  dense         Raster's dense f32 surface (nn/linear, dgemm!) through
                rq_linear / rq_sgemm: the C2 layer's shape in f32 and 4096^3,
                against the f32 MFMA peak (157.3 TFLOP/s).
  roofline      the C2 GEMM kernel against dense bf16 MFMA peak (below).
  roofline_gemv the C1 decode kernel against HBM peak (below).
  cpu_baseline  Raster's CPU routes restated in C (oracle/cpu_baseline.c),
                timed on this box's host cores: reported only (below).

HBM-bound lines are measured "cold": the call rotates through enough weight
copies (> 2x the 256 MB Infinity Cache per cycle) that every call reads its
weight from HBM. Each gives
  per_call_us   100 calls captured back to back in one HIP graph, median of 5
                replays: launch gaps included (what a caller sees);
  kernel_us     the kernels' own duration, from HIP events librq records at
                the dispatch's start and end (rq_ctx_set_kernel_timing) over
                the same rotation, 100 calls queued behind a GPU spin so they
                run back to back: no launch gaps. Queued (not captured)
                dispatches of some kernels run slower than the same kernels
                inside a graph; the graph's per_call_us, which holds the
                call's kernels plus their launch gaps, then bounds their time
                in a graph from above, and kernel_us is the smaller of the
                two (kernel_us_queued keeps the event figure, kernel_from
                says which one it is);
  frac_hbm      algorithmic bytes / kernel_us / 8 TB/s (the roofline figure),
  frac_hbm_per_call  the same over per_call_us,
  frac_read_ceiling  read_ceiling time for the same bytes / kernel_us.
MFMA-bound lines (M = 256, and the headline) give kernel_us and TFLOP/s.

roofline: `achieved` = 46,170,898,432 flop per launch over the GEMM kernel's
average duration, which librq captures in HIP events on the call's stream
during the timed steps (from the end of the activation-packing kernel to the
end of the GEMM that follows it). `traffic` is HBM bytes per launch from the
rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE summaries under profiles/.
`dense_bf16_library` times the vendor library's dense bf16 GEMM (torch.matmul,
hipBLASLt) at the same shape with an unquantized bf16 weight: what the
library reaches on this shape without any dequantization, for comparison.

cpu_baseline: `value` is the qlinear-q8 loop (B1: f32 products, f64
accumulation, the arithmetic of the GPU path's reference) on all usable host
cores (at most 16, the box's share) over a row sample of C2, in TFLOP/s.
`legs` times B1 and B2 (quantize-act-i8 + the x8 dpbusd GEMV, Raster's
production int8 route; Q8 and Q4_0 tiles) at 1 thread (Raster's default
RASTER_DECODE_THREADS) and at all cores, on the C1, C3, C2 and C5 (M = 1)
shapes, each leg about one second; `cpu_model` names the host CPU. The legs
re-read one weight buffer, so small shapes run from the host's last-level
cache (warm), unlike the GPU decode lines (cold).

Multi-GPU runs are not part of this build: --gpus above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "qmatmul GEMV GB/s (% of HBM peak) at M=1; GEMM TFLOPS (% MFMA) at M=512"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
INT8_PEAK_TOPS = 5000.0
FP32_PEAK_TFLOPS = 157.3  # dense f32 MFMA
RAMP_S = 0.2  # seconds of untimed headline steps that bring an idle GPU to its working clocks
MALL_BYTES = 256 << 20
PROFILES = os.path.join(ROOT, "profiles")
CALLS = 100  # launches per captured graph
SPIN_CYCLES = 20_000_000  # GPU spin ahead of event-timed calls (~8 ms at 2.4 GHz), longer than their host launches


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def act_bytes(xdt):
    # bytes per activation element; int8: the code, f32 scale and int32 sum per 32
    return {"f32": 4, "bf16": 2, "i8": 1.25}[xdt]


def q8_bytes(m, k, n, xb, yb):
    return int(n * k + n * (k // 32) * 4 + m * k * xb + m * n * yb)


def q4_bytes(m, k, n, xb, yb):
    return int(n * k // 2 + n * (k // 32) * 2 + m * k * xb + m * n * yb)


def copies_for_cold(nbytes):
    return max(1, -(-2 * MALL_BYTES // nbytes))


class Weights:
    """`copies` resident copies of one seeded weight (rotated per call)."""

    def __init__(self, ctx, fmt, k, n, copies, seed=0):
        import numpy as np

        import raster_amd
        from raster_amd import workloads as wl

        self.fmt, self.k, self.n = fmt, k, n
        if fmt == "q8":
            codes, scales = wl.q8_weights(n, k, seed=seed)
            self.ws = [raster_amd.QWeight.q8(codes, scales, n, k, ctx) for _ in range(copies)]
        else:
            packed, sc16 = wl.q4_weights(n, k, seed=seed)
            self.ws = [raster_amd.QWeight.q4(packed, sc16.view(np.float16), n, k, ctx) for _ in range(copies)]

    def bytes(self, m, xdt, ydt):
        f = q8_bytes if self.fmt == "q8" else q4_bytes
        return f(m, self.k, self.n, act_bytes(xdt), 4 if ydt == "f32" else 2)

    def destroy(self):
        for w in self.ws:
            w.destroy()
        self.ws = []


class Case:
    """One matmul shape over a Weights set: step() calls the next copy."""

    def __init__(self, torch, ctx, weights, m, xdt, ydt, seed=1):
        import raster_amd
        from raster_amd import workloads as wl

        self.torch, self.w, self.m = torch, weights, m
        self.bytes = weights.bytes(m, xdt, ydt)
        self.flops = 2.0 * m * weights.k * weights.n
        x = torch.from_numpy(wl.activations(m, weights.k, seed=seed, dtype="f32" if xdt == "i8" else xdt)).cuda()
        self.x = x.reshape(m, weights.k).to(torch.bfloat16) if xdt == "bf16" else x.reshape(m, weights.k)
        self.xi8 = raster_amd.quantize_act_i8(ctx, x, weights.k) if xdt == "i8" else None
        self.y = torch.empty((m, weights.n), dtype=torch.bfloat16 if ydt == "bf16" else torch.float32, device="cuda")
        self.i = 0

    def step(self):
        w = self.w.ws[self.i % len(self.w.ws)]
        self.i += 1
        if self.xi8 is not None:
            w.matmul_i8(*self.xi8, y=self.y)
        else:
            w.matmul(self.x, self.y)


def time_eager(torch, step, steps, warmup):
    """Event-timed back-to-back calls on the current stream; ms per call."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(steps):
        step()
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def time_graph(torch, step, calls=CALLS, reps=5):
    """`calls` launches captured in one HIP graph, replayed `reps` times after a
    warm replay; returns (median ms per call, coefficient of variation). The
    warm-up runs on the capture stream itself, so per-stream scratch exists
    before capture begins."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            step()
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(calls):
            step()
    g.replay()
    torch.cuda.synchronize()
    times = []
    st = torch.cuda.current_stream()
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        g.replay()
        e1.record(st)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / calls)
    del g
    med = statistics.median(times)
    cv = statistics.pstdev(times) / med if med > 0 else 0.0
    return med, cv


def time_kernels(torch, ctx, step, calls=CALLS, warmup=10):
    """Average duration (ms) of the kernels of `calls` calls, from the dispatch
    timestamps librq records (rq_ctx_set_kernel_timing). The calls are queued
    behind a GPU spin of a few milliseconds so that they run back to back, as
    in a graph, instead of each starting on an idle GPU after the host's
    launch gap."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ctx.kernel_time()
    ctx.set_kernel_timing(True)
    torch.cuda._sleep(SPIN_CYCLES)
    for _ in range(calls):
        step()
    torch.cuda.synchronize()
    total, n = ctx.kernel_time()
    ctx.set_kernel_timing(False)
    return total / max(n, 1)


class ReadCeiling:
    """rq_stream_read over rotating slices of one buffer larger than 2x the MALL."""

    def __init__(self, torch, ctx):
        import ctypes as C

        from raster_amd import _lib

        self.torch, self.ctx, self.C, self._lib = torch, ctx, C, _lib
        self.buf = torch.zeros(600 << 20, dtype=torch.uint8, device="cuda")
        self.sink = torch.empty(ctx.device_info()["cu_count"] * 16 * 256, dtype=torch.int32, device="cuda")
        self.cache = {}

    def step_fn(self, nbytes, wg):
        nb = (nbytes + 255) // 256 * 256
        slots = max(1, self.buf.numel() // nb)
        st = {"i": 0}

        def step():
            off = (st["i"] % slots) * nb
            st["i"] += 1
            self._lib.call("rq_stream_read", self.ctx.handle, self.C.c_void_p(self.buf.data_ptr() + off), nb, wg,
                           self.C.c_void_p(self.sink.data_ptr()),
                           self.C.c_void_p(self.torch.cuda.current_stream().cuda_stream))
        return step

    def us(self, nbytes):
        """Best per-launch time (graph, launch gaps included) and kernel time
        over 2 / 4 / 8 workgroups per CU."""
        if nbytes not in self.cache:
            best = None
            for wg in (2, 4, 8):
                ms, _ = time_graph(self.torch, self.step_fn(nbytes, wg))
                # the same rule as the matmul lines: the smaller of the queued
                # kernel time and the graph's per-call time
                kms = min(ms, time_kernels(self.torch, self.ctx, self.step_fn(nbytes, wg)))
                if best is None or kms < best[1]:
                    best = (ms, kms, wg)
            vms = self.vendor_ms(nbytes)
            cms = self.vendor_copy_ms(nbytes)
            self.cache[nbytes] = {"bytes": nbytes, "per_call_us": round(best[0] * 1e3, 3),
                                  "kernel_us": round(best[1] * 1e3, 3),
                                  "GBs": round(nbytes / best[1] / 1e6, 1),
                                  "frac_hbm": round(nbytes / best[1] / 1e6 / HBM_PEAK_GBS, 4),
                                  "wg_per_cu": best[2],
                                  "vendor_sum_per_call_us": round(vms * 1e3, 3),
                                  "vendor_sum_GBs_per_call": round(nbytes / vms / 1e6, 1),
                                  "vendor_copy_per_call_us": round(cms * 1e3, 3),
                                  "vendor_copy_read_GBs_per_call": round(nbytes / cms / 1e6, 1)}
        return self.cache[nbytes]

    def vendor_ms(self, nbytes):
        """torch.sum (PyTorch's own reduction kernel) over the same rotation of
        cold slices, f32 view: the vendor's read of those bytes, per call in a
        graph of CALLS launches (launch gaps included, like per_call_us)."""
        nb = (nbytes + 255) // 256 * 256
        slots = max(1, self.buf.numel() // nb)
        views = [self.buf[i * nb:(i + 1) * nb].view(self.torch.float32) for i in range(slots)]
        acc = self.torch.empty((), dtype=self.torch.float32, device="cuda")
        st = {"i": 0}

        def step():
            self.torch.sum(views[st["i"] % slots], dim=0, out=acc)
            st["i"] += 1
        ms, _ = time_graph(self.torch, step)
        return ms

    def vendor_copy_ms(self, nbytes):
        """Device-to-device copy (the runtime's copy of a tensor) of the same
        rotation of cold slices into one destination buffer, per call in a graph
        of CALLS launches: it reads the slice's bytes and writes as many."""
        nb = (nbytes + 255) // 256 * 256
        slots = max(1, self.buf.numel() // nb)
        views = [self.buf[i * nb:(i + 1) * nb] for i in range(slots)]
        dst = self.torch.empty(nb, dtype=self.torch.uint8, device="cuda")
        st = {"i": 0}

        def step():
            dst.copy_(views[st["i"] % slots])
            st["i"] += 1
        ms, _ = time_graph(self.torch, step)
        return ms


def path_numerics(fmt, m, k, n, xdt):
    """The kernel a plain rq_qmatmul call of this shape runs and how it
    carries the activations, as include/rq.h ("Kernel by call", "Numerics")
    states the dispatch."""
    fixed = ("16-bit block fixed point (per 32-block exponent e, X = rint(x 2^(15-e)), |x - X 2^(e-15)| <= "
             "2^(e-16)), exact integer dots, block scales in f32")
    if xdt == "i8":
        kern = "v_dot4_i32_i8 GEMV" if (m == 1 and fmt == "q4") else "int8-level decode kernel"
        return kern + ": int8 activation codes with f32 block scales (quantize-act-i8), exact integer dots"
    if m == 1 and fmt == "q4":
        return "v_dot4_i32_i8 GEMV: " + fixed
    if m <= 16 and ((fmt == "q4" and m >= 5) or (fmt == "q8" and m >= 9 and n * k <= (1 << 25))):
        split = "f32 x as two bf16 terms (|x - hi - lo| <= 2^-17 |x|)" if xdt == "f32" else "bf16 x as is"
        return "MFMA decode: exact codes on bf16 MFMA, " + split + ", block scales in f32"
    if m <= 16:
        return "int8-level decode kernel (int8 MFMA on the raw codes): " + fixed
    if xdt == "bf16":
        return "bf16 MFMA GEMM: weights dequantized to bf16 (exact f32 scale * code, one RNE rounding)"
    return "f32 GEMM: exact codes on bf16 MFMA, f32 x as two bf16 terms, block scales in f32"


def hbm_line(torch, ctx, name, weights_cold, weights_warm, m, xdt, ydt, ceiling=None):
    """Cold (rotating copies) and warm numbers for an HBM-bound shape."""
    w = weights_cold
    out = {"workload": name, "fmt": w.fmt, "m": m, "k": w.k, "n": w.n, "x": xdt, "y": ydt,
           "numerics": path_numerics(w.fmt, m, w.k, w.n, xdt)}
    warm = Case(torch, ctx, weights_warm, m, xdt, ydt)
    warm_ms, warm_cv = time_graph(torch, warm.step)
    cold = Case(torch, ctx, w, m, xdt, ydt)
    cold_ms, cold_cv = time_graph(torch, cold.step)
    kern_q = time_kernels(torch, ctx, cold.step)
    kern_ms = min(kern_q, cold_ms)
    b = cold.bytes
    out.update(copies=len(w.ws), bytes=b, flop=cold.flops,
               per_call_us=round(cold_ms * 1e3, 3), kernel_us=round(kern_ms * 1e3, 3),
               kernel_us_queued=round(kern_q * 1e3, 3), kernel_from="events" if kern_q <= cold_ms else "graph per call",
               GBs=round(b / kern_ms / 1e6, 1), frac_hbm=round(b / kern_ms / 1e6 / HBM_PEAK_GBS, 4),
               frac_hbm_per_call=round(b / cold_ms / 1e6 / HBM_PEAK_GBS, 4), cold_cv=round(cold_cv, 4),
               warm_per_call_us=round(warm_ms * 1e3, 3), warm_GBs=round(b / warm_ms / 1e6, 1),
               warm_cv=round(warm_cv, 4))
    if ceiling is not None:
        c = ceiling.us(b)
        out["read_ceiling_kernel_us"] = c["kernel_us"]
        out["frac_read_ceiling"] = round(c["kernel_us"] / 1e3 / kern_ms, 4)
    return out


def mfma_line(torch, ctx, name, weights, m, xdt, ydt, steps=CALLS, warmup=5, cold=None):
    """An MFMA-bound shape on one resident weight (warm: it stays in the MALL
    when it fits) and, given `cold` (a rotation past 2x the MALL), the same
    shape reading every call's weight from HBM."""
    c = Case(torch, ctx, weights, m, xdt, ydt)
    ms = time_eager(torch, c.step, steps, warmup)
    kms = time_kernels(torch, ctx, c.step, calls=steps)
    tf = c.flops / kms / 1e9
    out = {"workload": name, "fmt": weights.fmt, "m": m, "k": weights.k, "n": weights.n, "x": xdt, "y": ydt,
           "calls": steps, "per_call_us": round(ms * 1e3, 3), "kernel_us": round(kms * 1e3, 3), "TFLOPs": round(tf, 2),
           "frac_bf16_mfma": round(tf / BF16_PEAK_TFLOPS, 4), "TFLOPs_per_call": round(c.flops / ms / 1e9, 2)}
    if cold is not None:
        cc = Case(torch, ctx, cold, m, xdt, ydt)
        cms, cv = time_graph(torch, cc.step)
        ckms = time_kernels(torch, ctx, cc.step)
        out["cold"] = {"copies": len(cold.ws), "calls": CALLS, "per_call_us": round(cms * 1e3, 3),
                       "kernel_us": round(ckms * 1e3, 3), "TFLOPs": round(cc.flops / ckms / 1e9, 2),
                       "frac_bf16_mfma": round(cc.flops / ckms / 1e9 / BF16_PEAK_TFLOPS, 4), "cv": round(cv, 4)}
    return out


def config_lines(torch, ctx, ceiling):
    """C3 and C5 at every M the workload definition names."""
    lines = []
    # C3: Q4_0, K=4096, N=14336, f32 in / out
    one = Weights(ctx, "q4", 4096, 14336, 1, seed=3)
    cold = Weights(ctx, "q4", 4096, 14336, copies_for_cold(one.bytes(1, "f32", "f32")), seed=3)
    for m in (1, 4, 16):
        ln = hbm_line(torch, ctx, "C3 Q4 decode skinny", cold, one, m, "f32", "f32", ceiling)
        log(f"C3 m={m}: kernel {ln['kernel_us']} us ({ln['frac_hbm']:.3f} of HBM, "
            f"{ln['frac_read_ceiling']:.3f} of the read ceiling), per call {ln['per_call_us']} us")
        lines.append(ln)
    cold.destroy()
    one.destroy()
    # C5: K=8192, N=28672, bf16 in / out, Q4_0 (fp16 scales) and Q8_0
    for fmt in ("q4", "q8"):
        one = Weights(ctx, fmt, 8192, 28672, 1, seed=5)
        cold = Weights(ctx, fmt, 8192, 28672, copies_for_cold(one.bytes(1, "bf16", "bf16")), seed=5)
        for m in (1, 32):
            ln = hbm_line(torch, ctx, f"C5 70B MLP", cold, one, m, "bf16", "bf16", ceiling)
            log(f"C5 {fmt} m={m}: kernel {ln['kernel_us']} us ({ln['frac_hbm']:.3f} of HBM), "
                f"per call {ln['per_call_us']} us")
            lines.append(ln)
        ln = mfma_line(torch, ctx, "C5 70B MLP", one, 256, "bf16", "bf16", cold=cold)
        log(f"C5 {fmt} m=256: kernel {ln['kernel_us']} us, {ln['TFLOPs']} TFLOP/s ({ln['frac_bf16_mfma']:.3f}); "
            f"cold {ln['cold']['kernel_us']} us ({ln['cold']['frac_bf16_mfma']:.3f})")
        lines.append(ln)
        cold.destroy()
        one.destroy()
    return lines


class QuantCase:
    """rq_quantize_act_i8 over an m x k f32 activation block."""

    def __init__(self, torch, ctx, m, k):
        import raster_amd

        self.ctx, self.k, self.raster_amd = ctx, k, raster_amd
        self.x = torch.randn(m * k, device="cuda")
        self.out = (torch.empty((m, k), dtype=torch.int8, device="cuda"),
                    torch.empty((m, k // 32), dtype=torch.float32, device="cuda"),
                    torch.empty((m, k // 32), dtype=torch.int32, device="cuda"))
        self.bytes = m * k * (4 + 1) + m * (k // 32) * 8

    def step(self):
        self.raster_amd.quantize_act_i8(self.ctx, self.x, self.k, out=self.out)


def dense_library_line(torch, M=512, K=4096, N=11008, warmup=200, calls=500):
    """A reference point for the headline GEMM's MFMA fraction: the vendor
    library's dense bf16 GEMM (torch.matmul -> hipBLASLt) at the same shape,
    y = x @ W^T with W a dense bf16 [N, K] tensor (no quantization, no
    dequantization), timed back to back with events on torch's stream."""
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(M, K, device="cuda", dtype=torch.bfloat16, generator=g)
    w = torch.randn(N, K, device="cuda", dtype=torch.bfloat16, generator=g)
    for _ in range(warmup):
        torch.matmul(x, w.t())
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(calls):
        torch.matmul(x, w.t())
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / calls * 1e3
    tflops = 2.0 * M * K * N / us / 1e6
    return {"what": f"torch.matmul bf16 x[{M},{K}] @ W[{N},{K}]^T (hipBLASLt), dense bf16 weight",
            "us_per_call": round(us, 3), "tflops": round(tflops, 3),
            "frac": round(tflops / BF16_PEAK_TFLOPS, 4)}


def dense_lines(torch, ctx, warmup=20, calls=100):
    """Raster's dense f32 surface (nn/linear -> blas/dgemm-nt! float arm) on
    the device through rq_linear: y = x W^T + b at the C2 layer's shape in
    f32 (x [512, 4096], W [11008, 4096]), and rq_sgemm (dgemm!, C = A B) at
    4096^3, each timed back to back with events on torch's stream. The
    product is rocBLAS's f32 GEMM, so `frac` is against the f32 MFMA peak."""
    from raster_amd import dense

    g = torch.Generator(device="cuda").manual_seed(11)
    out = {}
    for name, (M, K, N) in (("linear_f32_C2_shape", (512, 4096, 11008)), ("sgemm_f32_4096", (4096, 4096, 4096))):
        a = torch.randn(M * K, device="cuda", generator=g)
        b = torch.randn(K * N, device="cuda", generator=g)
        bias = torch.randn(N, device="cuda", generator=g)
        y = torch.empty(M * N, device="cuda")
        if name.startswith("linear"):
            step = lambda: dense.linear_(a, b, bias, y, M, K, N, ctx)  # noqa: E731
        else:
            step = lambda: dense.dgemm(a, b, y, M, K, N, 1.0, 0.0, ctx)  # noqa: E731
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(calls):
            step()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / calls * 1e3
        tf = 2.0 * M * K * N / us / 1e6
        out[name] = {"m": M, "k": K, "n": N, "us_per_call": round(us, 3), "tflops": round(tf, 2),
                     "frac_fp32_mfma": round(tf / FP32_PEAK_TFLOPS, 4)}
        del a, b, bias, y
    return out


def dx_lines(torch, ctx, calls=20):
    """Backward-data (qlinear-q8-dx) of the C2 layer's weight (Q8_0, in 4096,
    out 11008) at m = 4, 16 and 512 dy rows. `kernel_us` spans every kernel of
    the call (librq's kernel timing). m <= 32 runs the f32 MFMA kernel on the
    weight as stored, read once per 16 dy rows: `frac_hbm` = weight bytes /
    time / 8 TB/s, `frac_f32_mfma` = the f32 MFMA work it issues (2 x 16 x
    ceil(m / 16) x in x out) / 157.3 TFLOP/s. m = 512 runs the bf16 MFMA GEMM,
    three bf16 MFMAs per product (hi/lo operand splits): `frac_mfma` = 3 x
    tflops / dense bf16 peak."""
    import raster_amd

    out_, in_ = 11008, 4096
    from raster_amd import workloads as wl

    codes, scales = wl.q8_weights(out_, in_, seed=41)
    w = raster_amd.QWeight.q8(codes, scales, out_, in_, ctx)
    wbytes = q8_bytes(0, in_, out_, 0, 0)
    lines = {}
    for m in (4, 16, 512):
        g = torch.Generator(device="cuda").manual_seed(m)
        dy = torch.randn(m, out_, device="cuda", dtype=torch.float32, generator=g)
        dx = torch.empty(m, in_, device="cuda", dtype=torch.float32)
        for _ in range(3):
            w.matmul_dx(dy, dx)
        torch.cuda.synchronize()
        ctx.kernel_time()
        ctx.set_kernel_timing(True)
        for _ in range(calls):
            w.matmul_dx(dy, dx)
        torch.cuda.synchronize()
        total, n = ctx.kernel_time()
        ctx.set_kernel_timing(False)
        us = total / max(n, 1) * 1e3
        tflops = 2.0 * m * in_ * out_ / us / 1e6
        ln = {"m": m, "in": in_, "out": out_, "kernel_us": round(us, 3), "tflops": round(tflops, 3)}
        if m <= 32:
            issued = 2.0 * 16 * -(-m // 16) * in_ * out_ / us / 1e6
            ln.update(kernel="rq::dx_fm_kernel (f32 MFMA, weight as stored)", weight_bytes=wbytes,
                      frac_hbm=round(wbytes / us / 1e3 / HBM_PEAK_GBS, 4),
                      frac_f32_mfma=round(issued / FP32_PEAK_TFLOPS, 4))
        else:
            ln.update(kernel="rq::dx_mf_kernel (bf16 MFMA GEMM, hi/lo splits)",
                      frac_mfma=round(3 * tflops / BF16_PEAK_TFLOPS, 4))
        lines[f"dx_q8_m{m}_4096x11008"] = ln
    w.destroy()
    return lines


def int8_lines(torch, ctx):
    """The int8-activation path: the on-device quantizer (HBM-bound), the
    int8-MFMA GEMM at the headline shape (its activations quantized once,
    outside the timed region) and the int8 decode kernel at M = 1."""
    qc = QuantCase(torch, ctx, 512, 4096)
    q_ms, _ = time_graph(torch, qc.step)
    lines = {"quantize_act_i8": {"m": 512, "k": 4096, "us": round(q_ms * 1e3, 3),
                                 "GBs": round(qc.bytes / q_ms / 1e6, 1)}}
    w = Weights(ctx, "q8", 4096, 11008, 1)
    c = Case(torch, ctx, w, 512, "i8", "bf16")
    kms = time_kernels(torch, ctx, c.step, calls=50)
    w.destroy()
    lines["gemm_i8_q8_C2_shape"] = {"m": 512, "k": 4096, "n": 11008, "y": "bf16", "kernel_us": round(kms * 1e3, 3),
                                    "TOPs": round(c.flops / kms / 1e9, 1),
                                    "frac_int8_mfma": round(c.flops / kms / 1e9 / INT8_PEAK_TOPS, 4)}
    for fmt, k, n in (("q8", 4096, 4096), ("q4", 4096, 14336)):
        one = Weights(ctx, fmt, k, n, 1)
        cold = Weights(ctx, fmt, k, n, copies_for_cold(one.bytes(1, "i8", "f32")))
        ln = hbm_line(torch, ctx, "int8 decode", cold, one, 1, "i8", "f32")
        cold.destroy()
        one.destroy()
        lines[f"decode_i8_{fmt}_m1_{n}x{k}"] = {kk: ln[kk] for kk in ("kernel_us", "frac_hbm", "per_call_us",
                                                                      "warm_per_call_us")}
    return lines


class KquantCase:
    """rq_qmatmul_q8k of a synthetic K-quant weight with q8_K activations
    quantized once; `copies` weights rotated."""

    def __init__(self, torch, ctx, fmt, m, k, n, copies=1, seed=0):
        import raster_amd
        from raster_amd import workloads as wl

        if fmt == "q4k":
            arrs = wl.q4k_weights(n, k, seed)
            self.weights = [raster_amd.QWeight.q4k(*arrs, n, k, ctx) for _ in range(copies)]
            self.bytes = n * k // 2 + n * (k // 256) * 8 + n * (k // 32) * 2
        else:
            arrs = wl.q6k_weights(n, k, seed)
            self.weights = [raster_amd.QWeight.q6k(*arrs, n, k, ctx) for _ in range(copies)]
            # the device packs the 6-bit codes, 12 bytes per 16 (Raster's layout: a byte each)
            self.bytes = n * k // 4 * 3 + n * (k // 256) * 4 + n * (k // 16)
            self.raster_bytes = n * k + n * (k // 256) * 4 + n * (k // 16)
        x = torch.randn(m * k, device="cuda")
        self.xq = raster_amd.quantize_act_q8k(ctx, x, k, 32 if fmt == "q4k" else 16)
        self.y = torch.empty((m, n), device="cuda")
        self.i = 0

    def step(self):
        w = self.weights[self.i % len(self.weights)]
        self.i += 1
        w.matmul_q8k(*self.xq, y=self.y)

    def destroy(self):
        for w in self.weights:
            w.destroy()
        self.weights = []


def kquant_lines(torch, ctx, m=1, k=4096, n=14336):
    """The K-quant GEMV at the Q4 decode shape: cold kernel time and GB/s of weight bytes."""
    lines = {}
    for fmt in ("q4k", "q6k"):
        one = KquantCase(torch, ctx, fmt, m, k, n)
        wb = one.bytes
        warm_ms, _ = time_graph(torch, one.step)
        one.destroy()
        c = KquantCase(torch, ctx, fmt, m, k, n, copies=copies_for_cold(wb))
        cold_ms, _ = time_graph(torch, c.step)
        kms = time_kernels(torch, ctx, c.step)
        c.destroy()
        lines[f"{fmt}_m{m}_{n}x{k}"] = {"weight_bytes": wb, **({"raster_layout_bytes": one.raster_bytes}
                                                              if hasattr(one, "raster_bytes") else {}),
                                          "kernel_us": round(kms * 1e3, 3),
                                          "frac_hbm": round(wb / kms / 1e6 / HBM_PEAK_GBS, 4),
                                          "per_call_us": round(cold_ms * 1e3, 3),
                                          "warm_per_call_us": round(warm_ms * 1e3, 3)}
    return lines


def decoder_step_us(torch, ctx, fused, sets=1, replays=200):
    """us per replay of the two-layer decode step captured in one HIP graph,
    and the linears' weight bytes per step. With sets > 1 the graph holds one
    step per weight set (distinct copies of both layers) and the time is per
    step, so consecutive steps read their weights from HBM, not the MALL."""
    from raster_amd import workloads as wl
    from raster_amd.decoder import DecoderLayer

    cfg = wl.DECODER
    layers, x = wl.decoder_weights(cfg, seed=0)
    stacks = [[DecoderLayer(ctx, L["weights"], L["gain1"], L["gain2"], cfg["d"], cfg["n_q"], cfg["n_kv"],
                            cfg["head_dim"], cfg["ffn"], cfg["eps"], cfg["theta"], fused=fused) for L in layers]
              for _ in range(sets)]
    kcs = [torch.from_numpy(L["kcache"]).cuda() for L in layers]
    vcs = [torch.from_numpy(L["vcache"]).cuda() for L in layers]
    xin = torch.from_numpy(x).cuda()
    pos = cfg["cached"]

    def step(dl):
        h = xin
        for layer, kc, vc in zip(dl, kcs, vcs):
            h = layer.step(h, kc, vc, pos)
        return h

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(stacks[0])
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for dl in stacks:
            step(dl)
    for _ in range(10):
        g.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    reps = max(1, replays // sets)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / (reps * sets) * 1e3
    wbytes = sum(layer.matmul_bytes() for layer in stacks[0])
    del g
    for dl in stacks:
        for layer in dl:
            layer.destroy()
    return us, wbytes


def decoder_line(torch, ctx):
    """The two-layer decode step (d 2048, 16 x 128 heads, SwiGLU 5632, Q8_0,
    128 cached positions, batch 1), captured in one HIP graph and replayed
    back to back: us per step (one token) and tokens/s, for the fused chain
    (norms, SwiGLU and residuals in the matmuls, one attention kernel) warm
    (one weight set, which fits the MALL) and cold (5 weight sets rotated,
    580 MB), and for the unfused chain (torch glue) warm."""
    us, wbytes = decoder_step_us(torch, ctx, fused=True)
    us_cold, _ = decoder_step_us(torch, ctx, fused=True, sets=5)
    us_unfused, _ = decoder_step_us(torch, ctx, fused=False)
    return {"workload": "C4 two-layer decode step, d 2048, 16x128 heads, SwiGLU 5632, Q8_0, 128 cached positions",
            "us_per_step": round(us_cold, 3), "tokens_per_s": round(1e6 / us_cold, 1), "weight_bytes": wbytes,
            "weight_GBs": round(wbytes / us_cold / 1e3, 1),
            "frac_hbm": round(wbytes / us_cold / 1e3 / HBM_PEAK_GBS, 4),
            "warm_us_per_step": round(us, 3), "warm_tokens_per_s": round(1e6 / us, 1),
            "unfused_warm_us_per_step": round(us_unfused, 3),
            "note": "us_per_step: 5 weight sets rotated in the graph (cold); warm: one set, MALL-resident; "
                    "fused: 5 librq launches per layer"}


COPY_ELEMS = 64 << 20  # f32 elements of the calibration copy: 256 MiB read + 256 MiB written


def traffic_run(torch, ctx, launches=5):
    """Kernels for the HBM-traffic counter passes, `launches` of each:
    torch.neg over COPY_ELEMS f32 (a plain elementwise copy reading and writing
    exactly 256 MiB, the calibration of the counters), the headline GEMM step
    (activation pack + GEMM kernel) and the C1 decode kernel on its cold weight
    rotation."""
    src = torch.randn(COPY_ELEMS, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(launches):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    w = Weights(ctx, "q8", 4096, 11008, 1)
    head = Case(torch, ctx, w, 512, "bf16", "bf16")
    for _ in range(launches):
        head.step()
    torch.cuda.synchronize()
    w.destroy()
    one = q8_bytes(1, 4096, 4096, 4, 4)
    dw = Weights(ctx, "q8", 4096, 4096, copies_for_cold(one))
    dec = Case(torch, ctx, dw, 1, "f32", "f32")
    for _ in range(len(dw.ws)):
        dec.step()
    torch.cuda.synchronize()
    dw.destroy()
    log(f"traffic run: {launches} x neg({COPY_ELEMS} f32), {launches} x C2 GEMM step, "
        f"{copies_for_cold(one)} x C1 decode (cold rotation)")


def read_traffic(kernel_tag):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary
    (profiles/<kernel_tag>_pmc.txt, line `traffic_bytes_per_launch: N`)."""
    path = os.path.join(PROFILES, f"{kernel_tag}_pmc.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def host_cores():
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return max(1, min(n, 16))


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed(fn, budget_s):
    """Calls fn() until about budget_s seconds have passed; (calls, seconds)."""
    n, dt = 0, 0.0
    while n == 0 or dt < budget_s:
        t0 = time.perf_counter()
        fn()
        dt += time.perf_counter() - t0
        n += 1
    return n, dt


def cpu_baseline(leg_s=1.0, head_s=10.0):
    """Raster's CPU routes (oracle/cpu_baseline.c) on this host; see the module
    docstring. B1 runs a row sample of each shape sized to the budget, B2 one
    activation row at a time as qlinear-i8! does (its M rows are M calls)."""
    import ctypes as C

    import numpy as np

    from oracle import oracle
    from raster_amd import workloads as wl

    L = oracle.baseline_lib()
    cores = host_cores()
    ptr = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731

    def b1(m, k, n, threads, budget):
        codes, scales = wl.q8_weights(n, k, seed=0)
        x = wl.activations(m, k, seed=1)
        y = np.empty(m * n, np.float32)
        t0 = time.perf_counter()
        L.rqb_qlinear_q8(ptr(x), ptr(codes), ptr(scales), 1, k, n, ptr(y), threads)
        t1 = time.perf_counter() - t0
        rows = int(max(1, min(m, budget / max(t1, 1e-6) / 2)))
        calls, dt = _timed(lambda: L.rqb_qlinear_q8(ptr(x), ptr(codes), ptr(scales), rows, k, n, ptr(y), threads),
                           budget)
        return calls * rows, dt

    def b2(fmt, m, k, n, threads, budget):
        rng = np.random.default_rng(0)
        nb = k // 32
        if fmt == "q8":
            wqi = rng.integers(0, 256, size=(n // 8) * nb * 256, dtype=np.uint8)
            fn = L.rqb_qmatmul_q8_x8
        else:
            wqi = rng.integers(0, 256, size=(n // 8) * nb * 128, dtype=np.uint8)
            fn = L.rqb_qmatmul_q4_x8
        wsi = rng.uniform(0.002, 0.02, (n // 8) * nb * 8).astype(np.float32)
        x = wl.activations(1, k, seed=1)
        xq, xs, xsum = np.empty(k, np.int8), np.empty(nb, np.float32), np.empty(nb, np.int32)
        y = np.empty(n, np.float32)

        def one():
            L.rqb_quantize_act_i8(ptr(x), 1, k, ptr(xq), ptr(xs), ptr(xsum), threads)
            fn(ptr(xq), ptr(xs), ptr(xsum), ptr(wqi), ptr(wsi), ptr(y), k, n, threads)
        one()
        return _timed(one, budget)

    def c4_step(route, threads, budget):
        """The two-layer C4 decode step on the host: per layer RMSNorm, the q / k
        / v GEMVs, RoPE, attention over the 128 cached rows, the o GEMV and
        residual, RMSNorm, gate / up, SwiGLU, down and residual. The glue is the
        oracle's C restatement of Raster's (nn.clj, attention.clj), one thread;
        the 14 GEMVs run B1 (qlinear-q8 loop) or B2 (quantize-act-i8 + x8
        dpbusd) on `threads`."""
        cfg = wl.DECODER
        d, nq, nkv, hd, ffn, cached = cfg["d"], cfg["n_q"], cfg["n_kv"], cfg["head_dim"], cfg["ffn"], cfg["cached"]
        shapes_ = [(d, nq * hd), (d, nkv * hd), (d, nkv * hd), (nq * hd, d), (d, ffn), (d, ffn), (ffn, d)]
        rng = np.random.default_rng(0)
        mats = []
        for k, n in shapes_:
            if route == "B1":
                codes, scales = wl.q8_weights(n, k, seed=k + n)
                mats.append((k, n, codes, scales))
            else:
                nb = k // 32
                wqi = rng.integers(0, 256, size=(n // 8) * nb * 256, dtype=np.uint8)
                wsi = rng.uniform(0.002, 0.02, (n // 8) * nb * 8).astype(np.float32)
                mats.append((k, n, wqi, wsi))
        kc = rng.standard_normal((cached + 1) * nkv * hd).astype(np.float32)
        vc = rng.standard_normal((cached + 1) * nkv * hd).astype(np.float32)
        gain = np.ones(d, np.float32)
        x0 = wl.activations(1, d, seed=1)
        bufs = {n: np.empty(n, np.float32) for _, n in shapes_}
        xq, xs, xsum = np.empty(ffn, np.int8), np.empty(ffn // 32, np.float32), np.empty(ffn // 32, np.int32)

        def gemv(i, v):
            k, n, a, b = mats[i]
            y = np.empty(n, np.float32)
            v = np.ascontiguousarray(v, np.float32)
            if route == "B1":
                L.rqb_qlinear_q8(ptr(v), ptr(a), ptr(b), 1, k, n, ptr(y), threads)
            else:
                L.rqb_quantize_act_i8(ptr(v), 1, k, ptr(xq), ptr(xs), ptr(xsum), threads)
                L.rqb_qmatmul_q8_x8(ptr(xq), ptr(xs), ptr(xsum), ptr(a), ptr(b), ptr(y), k, n, threads)
            return y

        def step():
            x = x0
            for _ in range(cfg["layers"]):
                h = oracle.rms_norm(x, gain, 1, d, cfg["eps"], 0.0)
                q = oracle.rope_pos(gemv(0, h), 1, nq, hd, cfg["theta"], cached)
                kc[cached * nkv * hd:] = oracle.rope_pos(gemv(1, h), 1, nkv, hd, cfg["theta"], cached)
                vc[cached * nkv * hd:] = gemv(2, h)
                att = oracle.gqa_decode_attention(q, kc, vc, cached + 1, nq, nkv, hd, 1.0 / hd ** 0.5)
                x1 = oracle.residual_add(x, gemv(3, att), d)
                h2 = oracle.rms_norm(x1, gain, 1, d, cfg["eps"], 0.0)
                f = oracle.silu_mul(gemv(4, h2), gemv(5, h2), ffn)
                x = oracle.residual_add(x1, gemv(6, f), d)
        _ = bufs
        step()
        return _timed(step, budget)

    legs = []
    # B2 takes one activation row per call (as qlinear-i8! does): an M-row leg is M calls
    shapes = [("C1", "q8", 1, 4096, 4096), ("C3", "q4", 1, 4096, 14336), ("C3", "q4", 4, 4096, 14336),
              ("C3", "q4", 16, 4096, 14336), ("C2", "q8", 512, 4096, 11008), ("C5", "q8", 1, 8192, 28672),
              ("C5", "q4", 1, 8192, 28672), ("C5", "q8", 32, 8192, 28672), ("C5", "q4", 32, 8192, 28672),
              ("C5", "q8", 256, 8192, 28672), ("C5", "q4", 256, 8192, 28672)]
    for route in ("B1", "B2"):
        for threads in (1, cores):
            steps_, dt = c4_step(route, threads, leg_s)
            legs.append({"config": "C4", "route": f"{route} two-layer decode step (14 GEMVs + glue)", "m": 1,
                         "threads": threads, "steps_timed": steps_, "seconds": round(dt, 3),
                         "us_per_step": round(dt / steps_ * 1e6, 2),
                         "tokens_per_s": round(steps_ / dt, 2)})
    for cfg, fmt, m, k, n in shapes:
        for threads in (1, cores):
            if fmt == "q8":
                rows, dt = b1(m, k, n, threads, leg_s)
                legs.append({"config": cfg, "route": "B1 qlinear-q8 loop", "fmt": "q8_0", "m": m, "k": k, "n": n,
                             "threads": threads, "rows_timed": rows, "seconds": round(dt, 3),
                             "us_per_row": round(dt / rows * 1e6, 2),
                             "GFLOPs": round(2.0 * rows * k * n / dt / 1e9, 2)})
            calls, dt = b2(fmt, m, k, n, threads, leg_s)
            wb = n * k + n * (k // 32) * 4 if fmt == "q8" else n * k // 2 + n * (k // 32) * 4
            legs.append({"config": cfg, "route": f"B2 quantize-act-i8 + x8 dpbusd GEMV ({fmt})", "m": m, "k": k,
                         "n": n, "threads": threads, "rows_timed": calls, "seconds": round(dt, 3),
                         "us_per_row": round(dt / calls * 1e6, 2), "us_per_call_of_m_rows": round(dt / calls * m * 1e6, 2),
                         "GFLOPs": round(2.0 * calls * k * n / dt / 1e9, 2),
                         "weight_GBs": round(wb * calls / dt / 1e9, 2)})
    # the headline value: B1 on all cores over a row sample of C2, ~head_s seconds
    M, K, N = 512, 4096, 11008
    rows, dt = b1(M, K, N, cores, head_s)
    L.rqb_pool_shutdown()
    flop = 2.0 * rows * K * N
    return {"value": round(flop / dt / 1e12, 6), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"B1 qlinear-q8 loop (f32 products, f64 accumulation) over {rows} activation rows of the C2 "
                      f"GEMM (K={K}, N={N}) in {dt:.2f} s on {cores} threads; TFLOP/s of that sample",
            "cpu_model": cpu_model(), "vnni": bool(L.rqb_have_vnni()),
            "note": ("every leg re-reads one weight buffer: up to tens of MB it stays in the host's last-level "
                     "cache, so weight_GBs is a warm rate and can exceed DRAM bandwidth; the GPU decode lines "
                     "rotate copies past the 256 MB MALL (cold)"),
            "legs": legs}


def headline(torch, ctx, args):
    """The C2 GEMM: ramp, W warm-up steps, K timed steps."""
    M, K, N = 512, 4096, 11008
    log(f"headline gemm q8 m={M} k={K} n={N} steps={args.steps} warmup={args.warmup}")
    w = Weights(ctx, "q8", K, N, 1)
    head = Case(torch, ctx, w, M, "bf16", "bf16")
    # An idle GPU ramps its clocks over the first milliseconds of work: before
    # the W counted warm-up steps the step runs untimed for RAMP_S seconds;
    # the timed region is unchanged.
    t_ramp = time.perf_counter()
    while time.perf_counter() - t_ramp < RAMP_S:
        for _ in range(20):
            head.step()
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        head.step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ctx.kernel_time()
    ctx.set_kernel_timing(True)
    e0.record(stream)
    for _ in range(args.steps):
        head.step()
    e1.record(stream)
    torch.cuda.synchronize()
    kern_total, kern_n = ctx.kernel_time()
    ctx.set_kernel_timing(False)
    ms = e0.elapsed_time(e1) / args.steps
    kern_ms = kern_total / max(kern_n, 1)
    w.destroy()
    cold = None
    if not args.only_gemm:
        cold = mfma_cold(torch, ctx, "q8", M, K, N)
    return head.flops, ms, kern_ms, kern_n, cold


def mfma_cold(torch, ctx, fmt, m, k, n, seed=0):
    """A GEMM shape over weight copies rotated past 2x the MALL (each call reads
    its weight from HBM): CALLS launches per captured graph (per call, launch
    gaps included) and the kernels' average duration over the same rotation."""
    one = q8_bytes(0, k, n, 0, 0) if fmt == "q8" else q4_bytes(0, k, n, 0, 0)
    ws = Weights(ctx, fmt, k, n, copies_for_cold(one), seed=seed)
    c = Case(torch, ctx, ws, m, "bf16", "bf16")
    per_ms, cv = time_graph(torch, c.step)
    kern_ms = time_kernels(torch, ctx, c.step)
    out = {"copies": len(ws.ws), "weight_bytes_per_copy": one, "calls": CALLS, "per_call_us": round(per_ms * 1e3, 3),
           "kernel_us": round(kern_ms * 1e3, 3), "TFLOPs": round(c.flops / kern_ms / 1e9, 2),
           "frac_bf16_mfma": round(c.flops / kern_ms / 1e9 / BF16_PEAK_TFLOPS, 4), "cv": round(cv, 4)}
    ws.destroy()
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--suite", choices=["headline", "all"], default="all")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only-gemm", action="store_true", help="time the headline GEMM only (for profiling)")
    ap.add_argument("--only-decode", action="store_true",
                    help="the decode shapes only (C1, C3, C5 at M = 1 and 32, the decoder step) for profiling")
    ap.add_argument("--counter-run", action="store_true",
                    help="a short run for rocprofv3 --pmc instruction / busy counters: the headline GEMM, then "
                         "the int8 GEMM at the same shape, 10 calls each")
    ap.add_argument("--traffic-run", action="store_true",
                    help="a short run for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes: a copy kernel of "
                         "known size (calibration), then the headline GEMM and the cold C1 decode kernel")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every box has one MI355X). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    import raster_amd

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (gfx950) GPU", file=sys.stderr)
        sys.exit(1)
    ctx = raster_amd.Context(0)
    info = ctx.device_info()
    clock_ghz = info["clock_khz"] / 1e6
    # dense bf16 MFMA: 4 SIMDs per CU, 1024 flop per clock per SIMD on CDNA4
    peak_props = info["cu_count"] * 4 * 1024 * clock_ghz / 1e3
    log(f"device: {torch.cuda.get_device_name(0)} cu={info['cu_count']} clock={clock_ghz:.3f} GHz")

    if args.traffic_run:
        traffic_run(torch, ctx)
        ctx.close()
        return

    if args.counter_run:
        w = Weights(ctx, "q8", 4096, 11008, 1)
        for xdt in ("bf16", "i8"):
            c = Case(torch, ctx, w, 512, xdt, "bf16")
            for _ in range(10):
                c.step()
            torch.cuda.synchronize()
            log(f"counter run: 10 x C2-shape GEMM, {xdt} activations")
        w.destroy()
        ctx.close()
        return

    if args.only_decode:
        ceiling = ReadCeiling(torch, ctx)
        one = Weights(ctx, "q8", 4096, 4096, 1)
        cold = Weights(ctx, "q8", 4096, 4096, copies_for_cold(one.bytes(1, "f32", "f32")))
        lines = [hbm_line(torch, ctx, "C1 Q8 decode GEMV", cold, one, 1, "f32", "f32", ceiling)]
        cold.destroy()
        one.destroy()
        lines += [ln for ln in config_lines(torch, ctx, ceiling) if ln["m"] <= 32]
        dec = decoder_line(torch, ctx)
        ctx.close()
        print(json.dumps({"decode": lines, "decoder": dec}), flush=True)
        return

    flops, ms, kern_ms, kern_n, head_cold = headline(torch, ctx, args)
    tflops, kern_tflops = flops / ms / 1e9, flops / kern_ms / 1e9
    log(f"headline: {ms * 1e3:.2f} us/call, {tflops:.1f} TFLOP/s; "
        f"GEMM kernel {kern_ms * 1e3:.2f} us avg over {kern_n} launches, {kern_tflops:.1f} TFLOP/s")
    result = {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded: int8 codes U{-127..127}, f32 scales U(0.002,0.02), x N(0,1) rounded to bf16)",
        "config": {"workload": "Q8 prefill GEMM, Llama-7B MLP up-projection: M=512 K=4096 N=11008, "
                               "bf16 activations, f32 accumulation, bf16 output",
                   "m": 512, "k": 4096, "n": 11008, "weights": "q8_0 resident in HBM"},
        "roofline": {"bound": "mfma", "achieved": round(kern_tflops, 3), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(kern_tflops / BF16_PEAK_TFLOPS, 4),
                     "traffic": read_traffic("gemm_rs_q8_C2"),
                     "peak_from_device_props": round(peak_props, 1),
                     "kernel": "rq::gemm_rs_kernel", "flop_per_launch": flops,
                     "kernel_avg_us": round(kern_ms * 1e3, 3), "kernel_launches": kern_n},
    }
    if head_cold is not None:
        result["roofline"]["cold"] = head_cold
        log(f"headline cold ({head_cold['copies']} weight copies): {head_cold['per_call_us']} us/call, kernel "
            f"{head_cold['kernel_us']} us ({head_cold['frac_bf16_mfma']:.3f} of peak)")

    if not args.only_gemm:
        result["roofline"]["dense_bf16_library"] = lib = dense_library_line(torch)
        log(f"dense bf16 library GEMM at the C2 shape: {lib['us_per_call']} us, {lib['tflops']} TFLOP/s")
        ceiling = ReadCeiling(torch, ctx)
        log("C1 gemv q8 m=1 k=4096 n=4096 (cold rotation + warm)")
        one = Weights(ctx, "q8", 4096, 4096, 1)
        cold = Weights(ctx, "q8", 4096, 4096, copies_for_cold(one.bytes(1, "f32", "f32")))
        gv = hbm_line(torch, ctx, "C1 Q8 decode GEMV", cold, one, 1, "f32", "f32", ceiling)
        cold.destroy()
        one.destroy()
        result["gemv"] = gv
        result["roofline_gemv"] = {"bound": "hbm", "achieved": gv["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                   "frac": gv["frac_hbm"], "traffic": read_traffic("skinny_q8_f32_C1"),
                                   "kernel": "rq::skinny_kernel", "bytes_per_launch": gv["bytes"],
                                   "kernel_avg_us": gv["kernel_us"], "per_call_us": gv["per_call_us"],
                                   "frac_per_call": gv["frac_hbm_per_call"],
                                   "read_ceiling_kernel_us": gv["read_ceiling_kernel_us"],
                                   "frac_read_ceiling": gv["frac_read_ceiling"], "numerics": gv["numerics"]}
        log(f"C1: kernel {gv['kernel_us']} us = {gv['GBs']} GB/s ({gv['frac_hbm']:.3f} of HBM, "
            f"{gv['frac_read_ceiling']:.3f} of the read ceiling); per call {gv['per_call_us']} us")

    if args.suite == "all" and not args.only_gemm:
        result["configs"] = config_lines(torch, ctx, ceiling)
        log("C4 two-layer decode step")
        result["decoder"] = dec = decoder_line(torch, ctx)
        log(f"C4: {dec['us_per_step']} us/step cold, {dec['warm_us_per_step']} warm, "
            f"{dec['unfused_warm_us_per_step']} unfused warm")
        result["read_ceiling"] = sorted(ceiling.cache.values(), key=lambda d: d["bytes"])
        log("int8-activation path")
        result["int8"] = int8_lines(torch, ctx)
        log("backward-data (dx) GEMM")
        result["dx"] = dx_lines(torch, ctx)
        log("K-quant GEMV")
        result["kquant"] = kquant_lines(torch, ctx)
        log("dense f32 GEMM (nn/linear, dgemm!)")
        result["dense"] = dense_lines(torch, ctx)
    elif not args.only_gemm:
        result["read_ceiling"] = sorted(ceiling.cache.values(), key=lambda d: d["bytes"])

    if not args.no_cpu and not args.only_gemm:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline()
        log(f"cpu baseline: {result['cpu_baseline']['value']} TFLOP/s on {result['cpu_baseline']['cores']} cores "
            f"({result['cpu_baseline']['cpu_model']})")
    else:
        result["cpu_baseline"] = None
    ctx.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
