"""Seeded synthetic inputs for the benchmark configurations (host numpy arrays).

Distributions follow the workload definitions (weights of Raster's Q8_0 /
Q4_0 formats, activations N(0, 1)); numpy's PCG64 generator makes them
identical on every machine for a given seed.
"""
from __future__ import annotations

import numpy as np

# (name, m values, K, N, format, activation dtype, output dtype)
CONFIGS = {
    "C1": dict(fmt="q8", m=(1,), k=4096, n=4096, x="f32", y="f32"),
    "C2": dict(fmt="q8", m=(512,), k=4096, n=11008, x="bf16", y="bf16"),
    "C3": dict(fmt="q4", m=(1, 4, 16), k=4096, n=14336, x="f32", y="f32"),
    "C5q8": dict(fmt="q8", m=(1, 32, 256), k=8192, n=28672, x="bf16", y="bf16"),
    "C5q4": dict(fmt="q4", m=(1, 32, 256), k=8192, n=28672, x="bf16", y="bf16"),
}


def q8_weights(out: int, in_: int, seed: int = 0):
    """int8 codes U{-127..127}, f32 scales U(0.002, 0.02) per 32-block."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(-127, 128, size=out * in_, dtype=np.int8)
    scales = rng.uniform(0.002, 0.02, size=out * (in_ // 32)).astype(np.float32)
    return codes, scales


def q4_weights(out: int, in_: int, seed: int = 0):
    """Packed nibbles U{0..15} (two per byte), fp16 scales U(0.005, 0.05) as uint16 bits."""
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, size=out * in_ // 2, dtype=np.uint8)
    scales = rng.uniform(0.005, 0.05, size=out * (in_ // 32)).astype(np.float16).view(np.uint16)
    return packed, scales


def q4k_weights(out: int, in_: int, seed: int = 0):
    """Synthetic Q4_K arrays in Raster's layout: nibbles U{0..15}, aq U{0..63},
    bq U{-32..31}, da / db U(0.0005, 0.002) per super-block."""
    rng = np.random.default_rng(seed)
    wq = rng.integers(0, 256, size=out * in_ // 2, dtype=np.uint8)
    da = rng.uniform(0.0005, 0.002, out * (in_ // 256)).astype(np.float32)
    db = rng.uniform(0.0005, 0.002, out * (in_ // 256)).astype(np.float32)
    aq = rng.integers(0, 64, size=out * (in_ // 32), dtype=np.uint8)
    bq = rng.integers(-32, 32, size=out * (in_ // 32), dtype=np.int8)
    return wq, da, db, aq, bq


def q6k_weights(out: int, in_: int, seed: int = 0):
    """Synthetic Q6_K arrays: codes U{0..63}, sc U{0..127}, ds U(0.00002, 0.0001)."""
    rng = np.random.default_rng(seed)
    wq = rng.integers(0, 64, size=out * in_, dtype=np.uint8)
    sc = rng.integers(0, 128, size=out * (in_ // 16), dtype=np.int8)
    ds = rng.uniform(0.00002, 0.0001, out * (in_ // 256)).astype(np.float32)
    return wq, sc, ds


def activations(m: int, in_: int, seed: int = 1, dtype: str = "f32") -> np.ndarray:
    """x ~ N(0, 1); for "bf16" the values are rounded to bf16 (returned as f32 values
    that are exactly representable in bf16)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(m * in_, dtype=np.float32)
    if dtype == "bf16":
        x = bf16_round(x)
    return x


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round f32 values to the nearest bf16 (ties to even), returned as f32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """bf16 bits of values already exactly representable in bf16."""
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


# The two-layer decode step: d_model 2048, 16 heads x 128, SwiGLU FFN 5632,
# Q8_0 linears, RMSNorm gains 1.0, batch 1 against 128 cached positions.
DECODER = dict(d=2048, n_q=16, n_kv=16, head_dim=128, ffn=5632, layers=2, cached=128, eps=1e-5, theta=1e4)


def decoder_weights(cfg=DECODER, seed: int = 0):
    """Per layer: seven (codes, scales) pairs (q, k, v, o, gate, up, down),
    RMSNorm gains (1.0), and K / V caches of cfg['cached'] positions ~ N(0, 1)
    with one free row for the new token. Returns (layers, x)."""
    d, hd, ffn = cfg["d"], cfg["head_dim"], cfg["ffn"]
    qd, kvd = cfg["n_q"] * hd, cfg["n_kv"] * hd
    shapes = ((qd, d), (kvd, d), (kvd, d), (d, qd), (ffn, d), (ffn, d), (d, ffn))
    layers = []
    for li in range(cfg["layers"]):
        ws = [q8_weights(o, i, seed=seed + 100 * li + j) for j, (o, i) in enumerate(shapes)]
        rng = np.random.default_rng(seed + 100 * li + 50)
        kc = np.zeros(((cfg["cached"] + 1), kvd), np.float32)
        vc = np.zeros(((cfg["cached"] + 1), kvd), np.float32)
        kc[:cfg["cached"]] = rng.standard_normal((cfg["cached"], kvd), dtype=np.float32)
        vc[:cfg["cached"]] = rng.standard_normal((cfg["cached"], kvd), dtype=np.float32)
        layers.append(dict(weights=ws, gain1=np.ones(d, np.float32), gain2=np.ones(d, np.float32), kcache=kc,
                           vcache=vc))
    x = np.random.default_rng(seed + 7).standard_normal(d, dtype=np.float32)
    return layers, x
