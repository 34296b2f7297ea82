"""Decoder step over librq's quantized linears (the two-layer decode workload).

One pre-norm decoder layer for one token, the op chain of the reference's
resident decoder layer (test/raster/dl/decoder_layer_gpu_test.clj:25-83) in its
Llama form: RMSNorm, NeoX RoPE, SwiGLU, no q/k norms. The glue ops keep the
reference's names and math:

  rms_norm              raster/dl/nn.clj:497-516
  rope_pos              raster/dl/attention.clj:197-214
  gqa_decode_attention  raster/dl/attention.clj:248-287
  silu_mul              raster/dl/nn.clj:200-203
  residual_add          raster/dl/nn.clj:217-219
  kv_append             raster/dl/attention.clj:413-416

The seven linears (q, k, v, o, gate, up, down) run on librq's decode kernel
at m = 1. q, k and v share one resident weight (their rows stacked), and so do
gate and up, so a layer makes four matmul calls; stacking rows changes no
output element. Two ways to run the glue:

  fused (default)  five librq calls per layer, no torch op: the RMSNorms ride
                   in the q/k/v and gate/up matmuls (rq_qmatmul_fused), the
                   residual adds in the o and down matmuls, SwiGLU in the
                   gate/up epilogue (gate and up rows interleaved), and RoPE,
                   KV append and attention in rq_decode_attention.
  unfused          rq_qmatmul for the linears and the glue as f32 torch ops
                   on the same stream (the functions above, a plain
                   restatement kept as the second path of the parity tests).

A whole step can be captured in one HIP graph (no call allocates).
"""
from __future__ import annotations

import math

import numpy as np

from .quant import Context, QWeight, decode_attention


def rms_norm(torch, x, weight, eps: float, gain_offset: float = 0.0):
    """x * (mean(x^2) + eps)^-1/2 * (gain_offset + weight), per row of the last axis."""
    ms = torch.mean(x * x, dim=-1, keepdim=True)
    return x * torch.rsqrt(ms + eps) * (gain_offset + weight)


def rope_tables(torch, head_dim: int, theta: float, pos: int, device):
    """cos / sin of pos * theta^(-2i/head_dim), i < head_dim/2, formed in double."""
    half = head_dim // 2
    ln = math.log(theta)
    ang = np.array([pos * math.exp((-2.0 * i / head_dim) * ln) for i in range(half)], np.float64)
    return (torch.from_numpy(np.cos(ang).astype(np.float32)).to(device),
            torch.from_numpy(np.sin(ang).astype(np.float32)).to(device))


def rope_pos(torch, x, heads: int, head_dim: int, cos, sin):
    """NeoX half split: element i pairs with i + head_dim/2 of the same head."""
    h = x.view(heads, head_dim)
    half = head_dim // 2
    x0, x1 = h[:, :half], h[:, half:]
    return torch.cat([x0 * cos - x1 * sin, x1 * cos + x0 * sin], dim=1).reshape(-1)


def gqa_decode_attention(torch, q, kcache, vcache, cache_len: int, n_q: int, n_kv: int, head_dim: int,
                         scale: float):
    """Single-query attention of n_q heads over the first cache_len cached
    positions ([positions, n_kv * head_dim] each); query head h reads kv head
    h // (n_q / n_kv)."""
    group = n_q // n_kv
    k = kcache[:cache_len].view(cache_len, n_kv, head_dim).permute(1, 2, 0).contiguous()  # [n_kv, hd, len]
    v = vcache[:cache_len].view(cache_len, n_kv, head_dim).permute(1, 0, 2).contiguous()  # [n_kv, len, hd]
    qg = q.view(n_kv, group, head_dim)
    p = torch.softmax(torch.bmm(qg, k) * scale, dim=-1)  # [n_kv, group, len]
    return torch.bmm(p, v).reshape(-1)


def silu_mul(torch, gate, up):
    return gate * torch.sigmoid(gate) * up


def residual_add(a, b):
    return a + b


def kv_append(cache, src, pos: int):
    cache[pos].copy_(src)


class DecoderLayer:
    """A layer's resident Q8_0 weights and norm gains. `weights` is seven
    (codes int8[out*in], scales f32[out*in/32]) pairs in Raster's row-major
    layout for q, k, v, o, gate, up, down."""

    def __init__(self, ctx: Context, weights, gain1, gain2, d: int, n_q: int, n_kv: int, head_dim: int, ffn: int,
                 eps: float = 1e-5, theta: float = 1e4, fused: bool = True):
        import torch

        if n_q % n_kv:
            raise ValueError("n_q must be a multiple of n_kv")
        self.ctx, self.fused = ctx, fused
        self.d, self.n_q, self.n_kv, self.hd, self.ffn = d, n_q, n_kv, head_dim, ffn
        self.eps, self.theta = eps, theta
        qd, kvd = n_q * head_dim, n_kv * head_dim
        (cq, sq), (ck, sk), (cv, sv), (co, so), (cg, sg), (cu, su), (cd, sd) = weights
        self.w_qkv = QWeight.q8(np.concatenate([cq, ck, cv]), np.concatenate([sq, sk, sv]), qd + 2 * kvd, d, ctx)
        self.w_o = QWeight.q8(co, so, d, qd, ctx)
        if fused:
            # rows 2i / 2i+1 = gate row i / up row i: the SwiGLU epilogue pairs them
            gu = np.stack([np.asarray(cg).reshape(ffn, d), np.asarray(cu).reshape(ffn, d)], axis=1).reshape(-1)
            gus = np.stack([np.asarray(sg).reshape(ffn, -1), np.asarray(su).reshape(ffn, -1)], axis=1).reshape(-1)
            self.w_gu = QWeight.q8(np.ascontiguousarray(gu), np.ascontiguousarray(gus), 2 * ffn, d, ctx)
        else:
            self.w_gu = QWeight.q8(np.concatenate([cg, cu]), np.concatenate([sg, su]), 2 * ffn, d, ctx)
        self.w_d = QWeight.q8(cd, sd, d, ffn, ctx)
        dev = torch.device("cuda", ctx.device)
        self.g1 = torch.as_tensor(np.ascontiguousarray(gain1, np.float32), device=dev)
        self.g2 = torch.as_tensor(np.ascontiguousarray(gain2, np.float32), device=dev)
        self._rope = {}

    def step(self, x, kcache, vcache, pos: int):
        """x: f32 [d] on the device; kcache / vcache: f32 [>= pos+1, n_kv*head_dim].
        Appends this token's k / v at `pos`, attends positions 0..pos and
        returns the layer output [d]."""
        import torch

        qd, kvd = self.n_q * self.hd, self.n_kv * self.hd
        if self.fused:
            qkv = self.w_qkv.matmul_fused(x.view(1, -1), norm_gain=self.g1, norm_eps=self.eps).view(-1)
            at = decode_attention(self.ctx, qkv[:qd], qkv[qd:qd + kvd], qkv[qd + kvd:], kcache, vcache, pos,
                                  self.n_q, self.n_kv, self.hd, self.theta, 1.0 / math.sqrt(self.hd))
            x1 = self.w_o.matmul_fused(at.view(1, -1), residual=x.view(1, -1))
            h = self.w_gu.matmul_fused(x1, norm_gain=self.g2, norm_eps=self.eps, swiglu=True)
            return self.w_d.matmul_fused(h, residual=x1).view(-1)
        if pos not in self._rope:
            self._rope[pos] = rope_tables(torch, self.hd, self.theta, pos, x.device)
        cos, sin = self._rope[pos]
        xn = rms_norm(torch, x, self.g1, self.eps)
        qkv = self.w_qkv.matmul(xn.view(1, -1)).view(-1)
        q, k, v = qkv[:qd], qkv[qd:qd + kvd], qkv[qd + kvd:]
        kv_append(kcache, rope_pos(torch, k, self.n_kv, self.hd, cos, sin), pos)
        kv_append(vcache, v, pos)
        at = gqa_decode_attention(torch, rope_pos(torch, q, self.n_q, self.hd, cos, sin), kcache, vcache, pos + 1,
                                  self.n_q, self.n_kv, self.hd, 1.0 / math.sqrt(self.hd))
        x1 = residual_add(x, self.w_o.matmul(at.view(1, -1)).view(-1))
        gu = self.w_gu.matmul(rms_norm(torch, x1, self.g2, self.eps).view(1, -1)).view(-1)
        h = silu_mul(torch, gu[:self.ffn], gu[self.ffn:])
        return residual_add(x1, self.w_d.matmul(h.view(1, -1)).view(-1))

    def matmul_bytes(self) -> int:
        """Algorithmic weight bytes the step streams (codes + f32 scales)."""
        return sum(w.out * w.in_ + w.out * (w.in_ // 32) * 4 for w in (self.w_qkv, self.w_o, self.w_gu, self.w_d))

    def destroy(self):
        for w in (self.w_qkv, self.w_o, self.w_gu, self.w_d):
            w.destroy()
