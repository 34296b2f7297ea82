"""Format-keyed quantized matrices on the GPU: the mirror of raster.quant.core.

    register_quant(fmt, {"descriptor": ..., "quantize": fn, "apply": fn})
    registered_formats() -> set
    qmatrix(fmt, W, rows, cols) -> QMatrix
    matmul(qm, x) -> y[rows]

(raster/quant/core.clj:22-51). `quantize` is called as quantize(W, rows,
cols, descriptor) and returns the format's arrays; `apply` is called as
apply(qm, x) and returns y. The built-in formats carry the reference's keys
and descriptors (raster/quant/core.clj:55-75, descriptors from
raster/compiler/backend/cpu/quant.clj:85-90,206-212) and run on the device:

  q4_K : rq_q4k_of (quantize-weight-q4k on the device; rows of `cols` not a
         multiple of 256 are zero-padded as raster.quant.pack/q4k-of does),
         a resident Q4_K weight, then per call rq_qmatmul with f32 x, which
         quantizes x to q8_K and runs the K-quant GEMV in one call
         (quantize-act-q8k + qmatmul-q4k-composable!, bitwise the same as
         rq_quantize_act_q8k + rq_qmatmul_q8k);
  q6_K : the same with rq_quantize_weight_q6k and the Q6_K kernel;
  q8_0 : rq_q8_quantize (raster.quant.train/q8-quantize) into a resident Q8_0
         weight, then rq_qmatmul (qlinear-q8's numerics). Raster reaches this
         format through qlinear-q8 rather than the registry; it is registered
         here so one surface covers the formats librq runs.

`x` may be a host float32 array (y comes back as one) or a CUDA tensor (y
stays on the device). Weights stay resident until the QMatrix is released
(`release(qm)`) or its context closes.
"""
from __future__ import annotations

import threading
from dataclasses import dataclass, field
from typing import Any

import numpy as np

from .quant import QWeight, context, nextpad, q4k_of, q8_quantize, quantize_weight_q6k

# descriptors as data, as in raster/compiler/backend/cpu/quant.clj
Q4_K = {"name": "q4_K", "super-block": 256, "subblock": 32, "n-subblocks": 8, "weight-bits": 4, "scale-bits": 6,
        "has-dmin": True, "pack": "nibble-interleaved", "act-type": "i8-K"}
Q6_K = {"name": "q6_K", "super-block": 256, "subblock": 16, "n-subblocks": 16, "weight-bits": 6, "scale-bits": 8,
        "has-dmin": False, "zero-point": 32, "pack": "byte-direct", "act-type": "i8-K"}
Q8_0 = {"name": "q8_0", "block": 32, "weight-bits": 8, "symmetric": True, "signed": True, "act-type": "f32"}


@dataclass
class QMatrix:
    """raster.quant.core/QMatrix: format key, rows, cols and the format's arrays."""

    format: Any
    rows: int
    cols: int
    arrays: dict = field(default_factory=dict)


_lock = threading.Lock()
_registry: dict[Any, dict] = {}


def register_quant(fmt_key, spec: dict) -> None:
    """Register (or replace) a format: spec = {"descriptor", "quantize", "apply"}."""
    for k in ("quantize", "apply"):
        if not callable(spec.get(k)):
            raise ValueError(f"spec needs a callable {k!r}")
    with _lock:
        _registry[fmt_key] = dict(spec)


def registered_formats() -> set:
    with _lock:
        return set(_registry)


def _spec(fmt_key) -> dict:
    with _lock:
        spec = _registry.get(fmt_key)
    if spec is None:
        raise KeyError(f"unknown quant format {fmt_key!r}; known: {sorted(map(str, registered_formats()))}")
    return spec


def qmatrix(fmt_key, W, rows: int, cols: int) -> QMatrix:
    """Quantize a row-major weight [rows x cols] into a QMatrix of `fmt_key`."""
    spec = _spec(fmt_key)
    return QMatrix(fmt_key, rows, cols, spec["quantize"](W, rows, cols, spec.get("descriptor")))


def matmul(qm: QMatrix, x):
    """y = QMatrix . x: dispatches on the QMatrix's format to its `apply`."""
    return _spec(qm.format)["apply"](qm, x)


def release(qm: QMatrix) -> None:
    """Free a built-in QMatrix's resident weight."""
    w = qm.arrays.get("weight")
    if isinstance(w, QWeight):
        w.destroy()


# ---- built-in device formats ---------------------------------------------------

def _device_w(W, rows: int, cols: int):
    import torch

    if isinstance(W, torch.Tensor):
        t = W.detach().to(device="cuda", dtype=torch.float32).contiguous().reshape(-1)
    else:
        t = torch.from_numpy(np.ascontiguousarray(W, np.float32).reshape(-1)).cuda()
    if t.numel() != rows * cols:
        raise ValueError("W must hold rows * cols values")
    return t


def _device_x(x, cols: int, width: int):
    """x as an f32 CUDA tensor of m rows, zero-padded from cols to width columns;
    and whether the caller passed a host array."""
    import torch

    host = not isinstance(x, torch.Tensor)
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32)) if host else x.to(torch.float32)
    t = t.reshape(-1, cols)
    if width != cols:
        t = torch.nn.functional.pad(t, (0, width - cols))
    return t.contiguous().cuda(), host


def _finish(y, host: bool, x):
    import torch

    if host:
        torch.cuda.synchronize()
        y = y.cpu().numpy()
        return y.ravel() if np.ndim(x) == 1 else y
    return y


def _quantize_kquant(fmt: str):
    def quantize(W, rows, cols, _descriptor):
        ctx = context()
        if fmt == "q4_K":
            a = q4k_of(ctx, _device_w(W, rows, cols), rows, cols)
            host = {k: a[k].cpu().numpy() for k in ("wq", "da", "db", "aq", "bq")}
            w = QWeight.q4k(host["wq"], host["da"], host["db"], host["aq"], host["bq"], rows, a["in"], ctx)
            return {"weight": w, "in": a["in"]}
        inp = cols
        if cols % 256 != 0:
            raise ValueError("q6_K needs cols % 256 == 0 (quantize-weight-q6k has no padding)")
        wq, sc, ds = quantize_weight_q6k(ctx, _device_w(W, rows, cols), rows, cols)
        w = QWeight.q6k(wq.cpu().numpy(), sc.cpu().numpy(), ds.cpu().numpy(), rows, inp, ctx)
        return {"weight": w, "in": inp}

    return quantize


def _apply_kquant():
    def apply(qm: QMatrix, x):
        w: QWeight = qm.arrays["weight"]
        xt, host = _device_x(x, qm.cols, qm.arrays["in"])
        return _finish(w.matmul(xt.reshape(-1, qm.arrays["in"])), host, x)

    return apply


def _quantize_q8(W, rows, cols, _descriptor):
    ctx = context()
    codes, scales = q8_quantize(ctx, _device_w(W, rows, cols), rows, cols)
    w = QWeight.q8(codes.cpu().numpy(), scales.cpu().numpy(), rows, cols, ctx)
    return {"weight": w, "in": cols}


def _apply_q8(qm: QMatrix, x):
    w: QWeight = qm.arrays["weight"]
    xt, host = _device_x(x, qm.cols, qm.cols)
    return _finish(w.matmul(xt), host, x)


register_quant("q4_K", {"descriptor": Q4_K, "quantize": _quantize_kquant("q4_K"), "apply": _apply_kquant()})
register_quant("q6_K", {"descriptor": Q6_K, "quantize": _quantize_kquant("q6_K"), "apply": _apply_kquant()})
register_quant("q8_0", {"descriptor": Q8_0, "quantize": _quantize_q8, "apply": _apply_q8})

__all__ = ["QMatrix", "register_quant", "registered_formats", "qmatrix", "matmul", "release", "nextpad",
           "Q4_K", "Q6_K", "Q8_0"]
