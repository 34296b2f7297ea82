"""Seeded rq_qmatmul shapes over every dispatch route, shared by the GPU sweep
and the no-alloc sweep (48 shapes: m bands 1, 2-4, 5-8, 9-16, 17-32, 33-64,
65-128, 129-600; in a multiple of 32; out 1-6000; Q8_0 / Q4_0; f32 / bf16 x
and y), plus 12 wide prefill shapes for the GPU sweep (m 129-1100, in a
multiple of 64, out 6000-30000, bf16 x: the tile cost model's 32x32x16
kernels, role-split 256 x 96 / 256 x 128 and 256 x 192)."""
import numpy as np


def shapes():
    rng = np.random.default_rng(20261202)
    bands = [(1, 1), (2, 4), (5, 8), (9, 16), (17, 32), (33, 64), (65, 128), (129, 600)]
    out = []
    for i in range(48):
        lo, hi = bands[i % len(bands)]
        m = int(rng.integers(lo, hi + 1))
        in_ = 32 * int(rng.choice([1, 3, 7, 32, 64, 129, 160, 256]))
        n = int(rng.choice([int(rng.integers(1, 300)), int(rng.integers(300, 6000))]))
        fmt = ["q8", "q4"][int(rng.integers(0, 2))]
        xdt = ["f32", "bf16"][int(rng.integers(0, 2))]
        ydt = ["f32", "bf16"][int(rng.integers(0, 2))]
        out.append((i, m, in_, n, fmt, xdt, ydt))
    return out


SHAPES = shapes()


def wide_shapes():
    rng = np.random.default_rng(20261203)
    out = []
    for i in range(12):
        m = int(rng.integers(129, 1101))
        in_ = 64 * int(rng.integers(1, 97))
        n = int(rng.integers(6000, 30001))
        fmt = ["q8", "q4"][i % 2]
        ydt = ["f32", "bf16"][(i // 2) % 2]
        out.append((100 + i, m, in_, n, fmt, "bf16", ydt))
    return out


WIDE_SHAPES = wide_shapes()
