"""numpy front-end for the C oracle (oracle/rq_oracle.c) and CPU baseline.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the thing
measured or shipped. Each wrapper names the reference function it restates
(paths inside replikativ/raster).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_BUILD = os.path.join(_HERE, "build")
_ORACLE_SO = os.path.join(_BUILD, "librq_oracle.so")
_BASELINE_SO = os.path.join(_BUILD, "librq_cpu_baseline.so")


def build(force: bool = False) -> None:
    """Compile the oracle and the CPU baseline with oracle/Makefile."""
    args = ["make", "-C", _HERE]
    if force:
        args.append("-B")
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)


def _load(path):
    if not os.path.exists(path):
        build()
    return C.CDLL(path)


_lib = None
_blib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load(_ORACLE_SO)
        _declare(_lib)
    return _lib


def baseline_lib():
    global _blib
    if _blib is None:
        _blib = _load(_BASELINE_SO)
        i64, i32, p = C.c_int64, C.c_int, C.c_void_p
        _blib.rqb_qlinear_q8.argtypes = [p, p, p, i64, i64, i64, p, i32]
        _blib.rqb_quantize_act_i8.argtypes = [p, i64, i64, p, p, p, i32]
        _blib.rqb_qmatmul_q8_x8.argtypes = [p, p, p, p, p, p, i64, i64, i32]
        _blib.rqb_qmatmul_q4_x8.argtypes = [p, p, p, p, p, p, i64, i64, i32]
        _blib.rqb_have_vnni.restype = C.c_int
        _blib.rqb_pool_shutdown.argtypes = []
    return _blib


def _declare(L):
    i64, i32, p, d = C.c_int64, C.c_int32, C.c_void_p, C.c_double
    sig = {
        "rqo_jfill_gauss": ([i64, d, p, i64], None),
        "rqo_jfill_uniform_centered": ([i64, p, i64], None),
        "rqo_jfill_bytes": ([i64, p, i64], None),
        "rqo_java_round": ([d], C.c_int64),
        "rqo_f16_to_f32": ([C.c_uint16], C.c_float),
        "rqo_f32_to_f16": ([C.c_float], C.c_uint16),
        "rqo_bf16_to_f32": ([C.c_uint16], C.c_float),
        "rqo_f32_to_bf16": ([C.c_float], C.c_uint16),
        "rqo_dp4a": ([i32, i32, i64], C.c_int64),
        "rqo_wi8_dot_q4": ([p, i64, p, i64], C.c_int64),
        "rqo_wi8_dot": ([p, i64, p, i64, i64], C.c_int64),
        "rqo_q8_quantize": ([p, i64, i64, p, p], C.c_int),
        "rqo_dequant_q8_dense": ([p, p, i64, i64, p], None),
        "rqo_qlinear_q8": ([p, p, p, i64, i64, i64, p], None),
        "rqo_rms_norm": ([p, p, p, i64, i64, d, d], None),
        "rqo_rope_pos": ([p, p, i64, i64, i64, d, i64], None),
        "rqo_gqa_decode_attention": ([p, p, p, i64, i64, i64, i64, d, p, p], None),
        "rqo_silu_mul": ([p, p, p, i64], None),
        "rqo_residual_add": ([p, p, p, i64], None),
        "rqo_kv_append": ([p, p, i64, i64], None),
        "rqo_decoder_layer": ([p, p, p, p, p, p, p, i64, i64, i64, i64, i64, i64, d, d, p], None),
        "rqo_qlinear_q8_dx": ([p, p, p, i64, i64, i64, p], None),
        "rqo_quantize_weight": ([p, i64, C.c_int, C.c_int, C.c_int, p, p], None),
        "rqo_dequant_weight": ([p, p, i64, C.c_int, C.c_int, p], None),
        "rqo_dequant_q4_f16": ([p, p, i64, i64, p], None),
        "rqo_dequant_q4_f32": ([p, p, i64, i64, p], None),
        "rqo_qlinear_q4": ([p, p, p, p, i64, i64, i64, p], None),
        "rqo_quantize_act_i8": ([p, i64, i64, p, p, p], None),
        "rqo_qmatmul_q4_composable": ([p, p, p, p, p, p, i64, i64, i64, i64], None),
        "rqo_repack_x8": ([p, p, i64, i64, C.c_int, p, p], C.c_int),
        "rqo_wi8_dot_q4_x8": ([p, i64, p, i64, p], None),
        "rqo_wi8_dot_q8_x8": ([p, i64, p, i64, p], None),
        "rqo_qmatmul_q4_x8": ([p, p, p, p, p, p, i64, i64, i64, i64], None),
        "rqo_qmatmul_q8_x8": ([p, p, p, p, p, p, i64, i64, i64, i64], None),
        "rqo_quantize_one_q8": ([p, i64, i64, p, p], C.c_int),
        "rqo_quant_act_i8_rows": ([p, p, p, i64, i64], None),
        "rqo_qmatmul_i8_gemm": ([p, p, p, p, p, i64, i64, i64], None),
        "rqo_i8gemv_dp4a": ([p, p, p, i64, i64], None),
        "rqo_dense_matmul_nt_f64": ([p, p, i64, i64, i64, p], None),
        "rqo_sgemm": ([C.c_int, C.c_int, i64, i64, i64, C.c_float, p, p, C.c_float, p], None),
        "rqo_linear": ([p, p, p, p, i64, i64, i64], None),
        "rqo_quantize_weight_q4k": ([p, i64, p, p, p, p, p], None),
        "rqo_nextpad": ([i64], C.c_int64),
        "rqo_q4k_of": ([p, i64, i64, p, p, p, p, p], C.c_int64),
        "rqo_dequant_q4k": ([p, p, p, p, p, i64, p], None),
        "rqo_quantize_weight_q6k": ([p, i64, p, p, p], None),
        "rqo_dequant_q6k": ([p, p, p, i64, p], None),
        "rqo_quantize_act_q8k": ([p, i64, i64, i64, p, p, p], None),
        "rqo_qmatmul_q4k": ([p, p, p, p, p, p, p, p, i64, i64, i64, p], None),
        "rqo_qmatmul_q6k": ([p, p, p, p, p, p, i64, i64, i64, p], None),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- Java RNG
def jfill_gauss(seed: int, mult: float, n: int) -> np.ndarray:
    """(float (* mult (.nextGaussian (java.util.Random. seed)))) x n."""
    out = np.empty(n, np.float32)
    lib().rqo_jfill_gauss(seed, mult, _ptr(out), n)
    return out


def jfill_uniform_centered(seed: int, n: int) -> np.ndarray:
    """(float (- (.nextDouble r) 0.5)) x n."""
    out = np.empty(n, np.float32)
    lib().rqo_jfill_uniform_centered(seed, _ptr(out), n)
    return out


def jfill_bytes(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.int8)
    lib().rqo_jfill_bytes(seed, _ptr(out), n)
    return out


def java_round(x: float) -> int:
    return lib().rqo_java_round(float(x))


# ---------------------------------------------------------------- conversions
def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.uint16).ravel()
    L = lib()
    return np.array([L.rqo_f16_to_f32(int(v)) for v in h], np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Vectorised RNE f32 -> bf16 bits (same rule as rqo_f32_to_bf16)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- int MAC seam
def dp4a(a: int, b: int, acc: int) -> int:
    def s32(v):
        v &= 0xFFFFFFFF
        return v - (1 << 32) if v >= (1 << 31) else v

    return lib().rqo_dp4a(s32(a), s32(b), acc)


def wi8_dot_q4(wq, woff, xq, xoff) -> int:
    wq, xq = _c(wq, np.uint8), _c(xq, np.int8)
    return lib().rqo_wi8_dot_q4(_ptr(wq), woff, _ptr(xq), xoff)


# ---------------------------------------------------------------- Q8_0
def q8_quantize(W, out: int, in_: int):
    """raster.quant.train/q8-quantize -> (codes int8[out*in], scales f32[out*in/32])."""
    W = _c(W, np.float32)
    codes = np.empty(out * in_, np.int8)
    scales = np.empty(out * (in_ // 32), np.float32)
    if lib().rqo_q8_quantize(_ptr(W), out, in_, _ptr(codes), _ptr(scales)) != 0:
        raise AssertionError(f"in={in_} not a multiple of 32")
    return codes, scales


def dequant_q8_dense(codes, scales, in_: int, out: int) -> np.ndarray:
    codes, scales = _c(codes, np.int8), _c(scales, np.float32)
    W = np.empty(out * in_, np.float32)
    lib().rqo_dequant_q8_dense(_ptr(codes), _ptr(scales), in_, out, _ptr(W))
    return W


def qlinear_q8(x, codes, scales, m: int, in_: int, out: int) -> np.ndarray:
    x, codes, scales = _c(x, np.float32), _c(codes, np.int8), _c(scales, np.float32)
    y = np.empty(m * out, np.float32)
    lib().rqo_qlinear_q8(_ptr(x), _ptr(codes), _ptr(scales), m, in_, out, _ptr(y))
    return y


def qlinear_q8_dx(dy, codes, scales, m: int, in_: int, out: int) -> np.ndarray:
    dy, codes, scales = _c(dy, np.float32), _c(codes, np.int8), _c(scales, np.float32)
    dx = np.empty(m * in_, np.float32)
    lib().rqo_qlinear_q8_dx(_ptr(dy), _ptr(codes), _ptr(scales), m, in_, out, _ptr(dx))
    return dx


# ---------------------------------------------------------------- Q4_0 / parametric
def quantize_weight(w, weight_bits: int, zero_point: int, nibble: bool):
    """raster.compiler.backend.cpu.quant/quantize-weight -> (wq u8, ws f32)."""
    w = _c(w, np.float32)
    n = w.size
    wq = np.empty(n // 2 if nibble else n, np.uint8)
    ws = np.empty(n // 32, np.float32)
    lib().rqo_quantize_weight(_ptr(w), n, weight_bits, zero_point, int(nibble), _ptr(wq), _ptr(ws))
    return wq, ws


def quantize_weight_q4(w):
    return quantize_weight(w, 4, 8, True)


def quantize_weight_q8u(w):
    return quantize_weight(w, 8, 128, False)


def dequant_weight(wq, ws, n: int, zero_point: int, nibble: bool) -> np.ndarray:
    wq, ws = _c(wq, np.uint8), _c(ws, np.float32)
    out = np.empty(n, np.float32)
    lib().rqo_dequant_weight(_ptr(wq), _ptr(ws), n, zero_point, int(nibble), _ptr(out))
    return out


def dequant_q4(wq, ws, in_: int, out: int) -> np.ndarray:
    """Row-major Q4_0 -> f32 W; ws is fp16 bits (uint16) or f32."""
    wq = _c(wq, np.uint8)
    W = np.empty(out * in_, np.float32)
    if np.asarray(ws).dtype == np.uint16:
        ws = _c(ws, np.uint16)
        lib().rqo_dequant_q4_f16(_ptr(wq), _ptr(ws), in_, out, _ptr(W))
    else:
        ws = _c(ws, np.float32)
        lib().rqo_dequant_q4_f32(_ptr(wq), _ptr(ws), in_, out, _ptr(W))
    return W


def qlinear_q4(x, wq, ws, m: int, in_: int, out: int) -> np.ndarray:
    x, wq = _c(x, np.float32), _c(wq, np.uint8)
    y = np.empty(m * out, np.float32)
    if np.asarray(ws).dtype == np.uint16:
        ws = _c(ws, np.uint16)
        lib().rqo_qlinear_q4(_ptr(x), _ptr(wq), _ptr(ws), None, m, in_, out, _ptr(y))
    else:
        ws = _c(ws, np.float32)
        lib().rqo_qlinear_q4(_ptr(x), _ptr(wq), None, _ptr(ws), m, in_, out, _ptr(y))
    return y


# ---------------------------------------------------------------- act quant + int GEMVs
def quantize_act_i8(x, M: int, in_: int):
    """raster.compiler.backend.cpu.quant/quantize-act-i8 -> (xq, xs, xsum)."""
    x = _c(x, np.float32)
    nb = M * (in_ // 32)
    xq = np.empty(M * in_, np.int8)
    xs = np.empty(nb, np.float32)
    xsum = np.empty(nb, np.int32)
    lib().rqo_quantize_act_i8(_ptr(x), M, in_, _ptr(xq), _ptr(xs), _ptr(xsum))
    return xq, xs, xsum


def qmatmul_q4_composable(xq, xs, xsum, wq, ws, in_: int, out: int) -> np.ndarray:
    xq, xs, xsum = _c(xq, np.int8), _c(xs, np.float32), _c(xsum, np.int32)
    wq, ws = _c(wq, np.uint8), _c(ws, np.float32)
    y = np.zeros(out, np.float32)
    lib().rqo_qmatmul_q4_composable(_ptr(xq), _ptr(xs), _ptr(xsum), _ptr(wq), _ptr(ws), _ptr(y),
                                    in_, out, 0, out)
    return y


def repack_x8(wq, ws, out: int, in_: int, nibble: bool):
    """raster.compiler.core.layout/repack (NC=8) -> (wqi, wsi)."""
    wq, ws = _c(wq, np.uint8), _c(ws, np.float32)
    nb = in_ // 32
    wqi = np.empty((out // 8) * nb * (128 if nibble else 256), np.uint8)
    wsi = np.empty((out // 8) * nb * 8, np.float32)
    if lib().rqo_repack_x8(_ptr(wq), _ptr(ws), out, in_, int(nibble), _ptr(wqi), _ptr(wsi)) != 0:
        raise AssertionError("repack needs out % 8 == 0 and in % 32 == 0")
    return wqi, wsi


def wi8_dot_x8(wqi, woff: int, xq, xoff: int, nibble: bool) -> np.ndarray:
    wqi, xq = _c(wqi, np.uint8), _c(xq, np.int8)
    out8 = np.empty(8, np.int32)
    fn = lib().rqo_wi8_dot_q4_x8 if nibble else lib().rqo_wi8_dot_q8_x8
    fn(_ptr(wqi), woff, _ptr(xq), xoff, _ptr(out8))
    return out8


def qmatmul_x8(xq, xs, xsum, wqi, wsi, in_: int, out: int, nibble: bool) -> np.ndarray:
    xq, xs, xsum = _c(xq, np.int8), _c(xs, np.float32), _c(xsum, np.int32)
    wqi, wsi = _c(wqi, np.uint8), _c(wsi, np.float32)
    y = np.zeros(out, np.float32)
    fn = lib().rqo_qmatmul_q4_x8 if nibble else lib().rqo_qmatmul_q8_x8
    fn(_ptr(xq), _ptr(xs), _ptr(xsum), _ptr(wqi), _ptr(wsi), _ptr(y), in_, out, 0, out // 8)
    return y


# ---------------------------------------------------------------- signed q8_0 prefill
def quantize_one_q8(W, in_: int, out: int):
    W = _c(W, np.float32)
    wp = np.empty(out * (in_ // 4), np.int32)
    ws = np.empty(out * (in_ // 32), np.float32)
    if lib().rqo_quantize_one_q8(_ptr(W), in_, out, _ptr(wp), _ptr(ws)) != 0:
        raise AssertionError(f"in={in_} not %32")
    return wp, ws


def quant_act_i8_rows(x, in_: int, nrows: int):
    x = _c(x, np.float32)
    xp = np.empty(nrows * (in_ // 4), np.int32)
    xs = np.empty(nrows * (in_ // 32), np.float32)
    lib().rqo_quant_act_i8_rows(_ptr(x), _ptr(xp), _ptr(xs), in_, nrows)
    return xp, xs


def qmatmul_i8_gemm(xp, xs, wp, ws, in_: int, out: int, nrows: int) -> np.ndarray:
    xp, xs, wp, ws = _c(xp, np.int32), _c(xs, np.float32), _c(wp, np.int32), _c(ws, np.float32)
    y = np.empty(nrows * out, np.float32)
    lib().rqo_qmatmul_i8_gemm(_ptr(xp), _ptr(xs), _ptr(wp), _ptr(ws), _ptr(y), in_, out, nrows)
    return y


def i8gemv_dp4a(wp, xp, kw: int, out: int) -> np.ndarray:
    wp, xp = _c(wp, np.int32), _c(xp, np.int32)
    y = np.empty(out, np.float32)
    lib().rqo_i8gemv_dp4a(_ptr(wp), _ptr(xp), _ptr(y), kw, out)
    return y


def dense_matmul_nt_f64(X, W, m: int, in_: int, out: int) -> np.ndarray:
    X, W = _c(X, np.float32), _c(W, np.float32)
    y = np.empty(m * out, np.float64)
    lib().rqo_dense_matmul_nt_f64(_ptr(X), _ptr(W), m, in_, out, _ptr(y))
    return y


def sgemm(trans_a: bool, trans_b: bool, A, B, Cm, m: int, k: int, n: int, alpha: float, beta: float) -> np.ndarray:
    """dgemm! / dgemm-tn! / dgemm-nt! float arm (rqo_sgemm): a new C."""
    A, B = _c(A, np.float32), _c(B, np.float32)
    out = _c(Cm, np.float32).copy()
    lib().rqo_sgemm(int(trans_a), int(trans_b), m, k, n, alpha, _ptr(A), _ptr(B), beta, _ptr(out))
    return out


def linear(x, W, b, batch: int, in_: int, out: int) -> np.ndarray:
    """nn/linear (rqo_linear): y[batch*out]."""
    x, W, b = _c(x, np.float32), _c(W, np.float32), _c(b, np.float32)
    y = np.zeros(max(batch, 0) * max(out, 0), np.float32)
    lib().rqo_linear(_ptr(x), _ptr(W), _ptr(b), _ptr(y), batch, in_, out)
    return y


# ---------------------------------------------------------------- decoder glue
def rms_norm(x, w, rows: int, features: int, eps: float, gain_offset: float) -> np.ndarray:
    """raster.dl.nn/rms-norm! (nn.clj:497-516)."""
    x, w = _c(x, np.float32), _c(w, np.float32)
    out = np.empty(rows * features, np.float32)
    lib().rqo_rms_norm(_ptr(x), _ptr(w), _ptr(out), rows, features, eps, gain_offset)
    return out


def rope_pos(x, seq_len: int, heads: int, head_dim: int, theta: float, pos_offset: int) -> np.ndarray:
    """raster.dl.attention/rope-pos (attention.clj:197-214)."""
    x = _c(x, np.float32)
    out = np.empty(seq_len * heads * head_dim, np.float32)
    lib().rqo_rope_pos(_ptr(x), _ptr(out), seq_len, heads, head_dim, theta, pos_offset)
    return out


def gqa_decode_attention(q, k, v, cache_len: int, n_q: int, n_kv: int, head_dim: int, scale: float) -> np.ndarray:
    """raster.dl.attention/gqa-decode-attention (attention.clj:248-287)."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    out = np.empty(n_q * head_dim, np.float32)
    sc = np.empty(max(cache_len, 1), np.float32)
    lib().rqo_gqa_decode_attention(_ptr(q), _ptr(k), _ptr(v), cache_len, n_q, n_kv, head_dim, scale, _ptr(out),
                                   _ptr(sc))
    return out


def silu_mul(gate, up, n: int) -> np.ndarray:
    """raster.dl.nn/silu-mul! (nn.clj:200-203)."""
    gate, up = _c(gate, np.float32), _c(up, np.float32)
    out = np.empty(n, np.float32)
    lib().rqo_silu_mul(_ptr(gate), _ptr(up), _ptr(out), n)
    return out


def residual_add(a, b, n: int) -> np.ndarray:
    """raster.dl.nn/residual-add! (nn.clj:217-219)."""
    a, b = _c(a, np.float32), _c(b, np.float32)
    out = np.empty(n, np.float32)
    lib().rqo_residual_add(_ptr(a), _ptr(b), _ptr(out), n)
    return out


def decoder_layer(x, weights, gain1, gain2, kcache, vcache, d: int, n_q: int, n_kv: int, head_dim: int, ffn: int,
                  cache_len: int, eps: float, theta: float):
    """One pre-norm decoder layer step (rqo_decoder_layer). weights: seven
    (codes, scales) pairs for q, k, v, o, gate, up, down. Returns (x_out,
    kcache, vcache) with the new position appended (copies; inputs untouched)."""
    x = _c(x, np.float32).copy()
    kc, vc = _c(kcache, np.float32).copy(), _c(vcache, np.float32).copy()
    codes = [_c(c, np.int8) for c, _ in weights]
    scales = [_c(s_, np.float32) for _, s_ in weights]
    wp = (C.c_void_p * 7)(*[c.ctypes.data for c in codes])
    sp = (C.c_void_p * 7)(*[s_.ctypes.data for s_ in scales])
    g1, g2 = _c(gain1, np.float32), _c(gain2, np.float32)
    scratch = np.empty(3 * d + 5 * n_q * head_dim + 3 * ffn + cache_len, np.float32)
    lib().rqo_decoder_layer(_ptr(x), C.cast(wp, C.c_void_p), C.cast(sp, C.c_void_p), _ptr(g1), _ptr(g2), _ptr(kc),
                            _ptr(vc), d, n_q, n_kv, head_dim, ffn, cache_len, eps, theta, _ptr(scratch))
    return x, kc, vc


def normwise_relerr(a, ref) -> float:
    """max|a-ref| / max|ref| (test/raster/dl/decoder_layer_gpu_test.clj:17)."""
    a = np.asarray(a, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    return float(np.max(np.abs(a - ref)) / max(1e-9, float(np.max(np.abs(ref)))))


# ---------------------------------------------------------------- K-quants
def quantize_weight_q4k(w):
    """raster.compiler.backend.cpu.quant/quantize-weight-q4k -> (wq, da, db, aq, bq)."""
    w = _c(w, np.float32)
    n = w.size
    wq = np.empty(n // 2, np.uint8)
    da, db = np.empty(n // 256, np.float32), np.empty(n // 256, np.float32)
    aq, bq = np.empty(n // 32, np.uint8), np.empty(n // 32, np.int8)
    lib().rqo_quantize_weight_q4k(_ptr(w), n, _ptr(wq), _ptr(da), _ptr(db), _ptr(aq), _ptr(bq))
    return wq, da, db, aq, bq


def nextpad(in_: int) -> int:
    """raster.quant.pack/nextpad: in rounded up to a multiple of 256."""
    return int(lib().rqo_nextpad(in_))


def q4k_of(W, out: int, in_: int):
    """raster.quant.pack/q4k-of -> (wq, da, db, aq, bq, inp): rows zero-padded to
    inp = nextpad(in), then quantize-weight-q4k; wq is the nibble bytes (the
    reference reinterprets them as little-endian int32 words)."""
    W = _c(W, np.float32)
    inp = nextpad(in_)
    n = out * inp
    wq = np.empty(n // 2, np.uint8)
    da, db = np.empty(n // 256, np.float32), np.empty(n // 256, np.float32)
    aq, bq = np.empty(n // 32, np.uint8), np.empty(n // 32, np.int8)
    got = lib().rqo_q4k_of(_ptr(W), out, in_, _ptr(wq), _ptr(da), _ptr(db), _ptr(aq), _ptr(bq))
    if got != inp:
        raise MemoryError("rqo_q4k_of failed")
    return wq, da, db, aq, bq, inp


def dequant_q4k(wq, da, db, aq, bq, n: int) -> np.ndarray:
    """dequant-q4k -> f32[n]."""
    out = np.empty(n, np.float32)
    lib().rqo_dequant_q4k(_ptr(_c(wq, np.uint8)), _ptr(_c(da, np.float32)), _ptr(_c(db, np.float32)),
                          _ptr(_c(aq, np.uint8)), _ptr(_c(bq, np.int8)), n, _ptr(out))
    return out


def quantize_weight_q6k(w):
    """quantize-weight-q6k -> (wq, sc, ds)."""
    w = _c(w, np.float32)
    n = w.size
    wq, sc, ds = np.empty(n, np.uint8), np.empty(n // 16, np.int8), np.empty(n // 256, np.float32)
    lib().rqo_quantize_weight_q6k(_ptr(w), n, _ptr(wq), _ptr(sc), _ptr(ds))
    return wq, sc, ds


def dequant_q6k(wq, sc, ds, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().rqo_dequant_q6k(_ptr(_c(wq, np.uint8)), _ptr(_c(sc, np.int8)), _ptr(_c(ds, np.float32)), n, _ptr(out))
    return out


def quantize_act_q8k(x, m: int, in_: int, sub: int):
    """quantize-act-q8k of m rows -> (xq, xs[m*in/256], bsums[m*in/sub])."""
    x = _c(x, np.float32)
    xq = np.empty(m * in_, np.int8)
    xs = np.empty(m * (in_ // 256), np.float32)
    bsums = np.empty(m * (in_ // sub), np.int32)
    lib().rqo_quantize_act_q8k(_ptr(x), m, in_, sub, _ptr(xq), _ptr(xs), _ptr(bsums))
    return xq, xs, bsums


def qmatmul_q4k(xq, xs, bsums, wq, da, db, aq, bq, m: int, in_: int, out: int) -> np.ndarray:
    """qmatmul-q4k-composable! for m rows -> y[m*out]."""
    y = np.empty(m * out, np.float32)
    lib().rqo_qmatmul_q4k(_ptr(_c(xq, np.int8)), _ptr(_c(xs, np.float32)), _ptr(_c(bsums, np.int32)),
                          _ptr(_c(wq, np.uint8)), _ptr(_c(da, np.float32)), _ptr(_c(db, np.float32)),
                          _ptr(_c(aq, np.uint8)), _ptr(_c(bq, np.int8)), m, in_, out, _ptr(y))
    return y


def qmatmul_q6k(xq, xs, bsums, wq, sc, ds, m: int, in_: int, out: int) -> np.ndarray:
    """qmatmul-q6k-composable! for m rows -> y[m*out]."""
    y = np.empty(m * out, np.float32)
    lib().rqo_qmatmul_q6k(_ptr(_c(xq, np.int8)), _ptr(_c(xs, np.float32)), _ptr(_c(bsums, np.int32)),
                          _ptr(_c(wq, np.uint8)), _ptr(_c(sc, np.int8)), _ptr(_c(ds, np.float32)), m, in_, out,
                          _ptr(y))
    return y
