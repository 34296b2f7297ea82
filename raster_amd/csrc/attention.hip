// attention.hip — one decode step of RoPE, KV-cache append and single-query
// attention (the glue between a decoder layer's q/k/v and o linears).
//
// Restates, for one token at position pos:
//   rope-pos               raster/dl/attention.clj:197-214 (NeoX half split)
//   kv-append!             raster/dl/attention.clj:413-416
//   gqa-decode-attention   raster/dl/attention.clj:248-287
// One workgroup per query head. It rotates its query and its KV head's new
// key (angles pos * theta^(-2i/head_dim) in double, as the reference), takes
// the scores of positions 0..pos (the new key from LDS, the older ones from
// the cache), their softmax, and the weighted sum of values. The first query
// head of each KV head writes the rotated key and the value into the caches
// at row pos; no workgroup reads row pos from memory, so none waits for
// another.
//
// Two kernels:
//   chunk kernel (head_dim a multiple of 4, at most 512): the cached rows
//     0..pos-1 stream through registers in chunks of rows, K and V of a chunk
//     loaded together as 16-byte vectors and the next chunk's loads in flight
//     while the current one is used. TPR lanes hold one row (4 or 8 of its
//     dimensions each), so a wave holds 64/TPR rows per load. Each wave keeps
//     its own running maximum, sum and weighted values (the usual online
//     softmax); the four waves' states are combined at the end. Memory
//     latency is paid about once per two chunks instead of once per row.
//     A short cache on few heads would leave most CUs idle, so the cached
//     rows are split into nsplit contiguous ranges, one workgroup per (head,
//     range): each writes its range's softmax state (running maximum, sum of
//     exponentials, weighted values) to a scratch record, and a second
//     kernel merges each head's records in range order.
//   generic kernel (any even head_dim): a wave per position for the scores,
//     a thread per dimension for the values; the scores sit in LDS, so the
//     cache length is bounded by it.
#include <algorithm>
#include <atomic>
#include <cmath>

#include "rq_internal.h"

namespace rq {

namespace {

constexpr int kAttnThreads = 256;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

}  // namespace

// LDS: qr[head_dim], kr[head_dim], vn[head_dim], sc[pos + 1], red[8]
__global__ __launch_bounds__(kAttnThreads) void decode_attention_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v, float* __restrict__ kcache,
    float* __restrict__ vcache, int pos, int n_q, int n_kv, int head_dim, double theta, float scale,
    float* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  float* qr = sm;
  float* kr = qr + head_dim;
  float* vn = kr + head_dim;
  float* sc = vn + head_dim;
  float* red = sc + pos + 1;
  const int hq = blockIdx.x, group = n_q / n_kv, hkv = hq / group;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = head_dim / 2, kvd = n_kv * head_dim;
  const double ln_theta = log(theta);

  // RoPE of this head's query and of the KV head's new key; the value as is
  for (int i = tid; i < half; i += kAttnThreads) {
    const double ang = (double)pos * exp((-2.0 * (double)i / (double)head_dim) * ln_theta);
    const double c = cos(ang), s = sin(ang);
    const double q0 = q[hq * head_dim + i], q1 = q[hq * head_dim + i + half];
    qr[i] = (float)(q0 * c - q1 * s);
    qr[i + half] = (float)(q1 * c + q0 * s);
    const double k0 = k[hkv * head_dim + i], k1 = k[hkv * head_dim + i + half];
    kr[i] = (float)(k0 * c - k1 * s);
    kr[i + half] = (float)(k1 * c + k0 * s);
  }
  for (int d = tid; d < head_dim; d += kAttnThreads) vn[d] = v[hkv * head_dim + d];
  __syncthreads();
  if (hq % group == 0) {
    for (int d = tid; d < head_dim; d += kAttnThreads) {
      kcache[(int64_t)pos * kvd + hkv * head_dim + d] = kr[d];
      vcache[(int64_t)pos * kvd + hkv * head_dim + d] = vn[d];
    }
  }

  // scores: a wave per position, lanes over the head dimension
  float mloc = -INFINITY;
  for (int j = wave; j <= pos; j += kAttnThreads / 64) {
    const float* kj = j == pos ? kr : kcache + (int64_t)j * kvd + hkv * head_dim;
    float dot = 0.0f;
    for (int d = lane; d < head_dim; d += 64) dot += qr[d] * kj[d];
    dot = wave_sum(dot) * scale;
    if (lane == 0) sc[j] = dot;
    mloc = fmaxf(mloc, dot);
  }
  if (lane == 0) red[wave] = mloc;
  __syncthreads();
  float mx = red[0];
  for (int w = 1; w < kAttnThreads / 64; w++) mx = fmaxf(mx, red[w]);
  __syncthreads();
  // softmax numerators and their sum
  float sloc = 0.0f;
  for (int j = tid; j <= pos; j += kAttnThreads) {
    const float e = expf(sc[j] - mx);
    sc[j] = e;
    sloc += e;
  }
  sloc = wave_sum(sloc);
  if (lane == 0) red[wave] = sloc;
  __syncthreads();
  float sum = 0.0f;
  for (int w = 0; w < kAttnThreads / 64; w++) sum += red[w];
  const float inv = 1.0f / sum;
  // weighted values: a thread per output element (threads past head_dim idle)
  for (int d = tid; d < head_dim; d += kAttnThreads) {
    float a = 0.0f;
    for (int j = 0; j < pos; j++) a += sc[j] * vcache[(int64_t)j * kvd + hkv * head_dim + d];
    a += sc[pos] * vn[d];
    out[hq * head_dim + d] = a * inv;
  }
}

namespace {

// lanes per row and 4-dimension vectors per lane of the chunk kernel, or 0
int chunk_tpr(int64_t head_dim) {
  if (head_dim % 4 != 0 || head_dim > 512) return 0;
  return head_dim <= 64 ? 16 : head_dim <= 128 ? 32 : 64;
}

constexpr int kMaxDims = 512;

}  // namespace

// TPR lanes per row, NV 4-dimension vectors per lane (dimension
// 4 (lane % TPR) + 4 TPR v), NP rows per lane per chunk
// Split records: per (head, range) kAttnRec header floats (maximum, sum) then
// head_dim weighted values.
constexpr int kAttnRec = 4;
constexpr int kMaxSplits = 64;

template <int TPR, int NV, int NP, int THREADS>
__global__ __launch_bounds__(THREADS) void decode_attention_chunk_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v, float* __restrict__ kcache,
    float* __restrict__ vcache, int pos, int n_q, int n_kv, int head_dim, double theta, float scale,
    float* __restrict__ out, int nsplit, int rps, float* __restrict__ part) {
  constexpr int WAVES = THREADS / 64;
  constexpr int RW = 64 / TPR;         // rows per wave per load
  constexpr int CH = WAVES * RW * NP;  // rows per chunk
  __shared__ __attribute__((aligned(16))) float qr[kMaxDims];
  __shared__ __attribute__((aligned(16))) float kr[kMaxDims];
  __shared__ __attribute__((aligned(16))) float vn[kMaxDims];
  __shared__ __attribute__((aligned(16))) float wacc[WAVES][kMaxDims];
  __shared__ float wm[WAVES], wl[WAVES];
  const int hq = (int)blockIdx.x % n_q, split = (int)blockIdx.x / n_q, group = n_q / n_kv, hkv = hq / group;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int sub = lane % TPR, rg = lane / TPR;
  const int half = head_dim / 2, kvd = n_kv * head_dim;
  // cached rows [r0, r1) of this range (rows 0..pos-1 are read from memory)
  const int r0 = min(split * rps, pos), r1 = min(r0 + rps, pos);
  const int nch = (r1 - r0 + CH - 1) / CH;
  const float* kb = kcache + hkv * head_dim;
  const float* vb = vcache + hkv * head_dim;

  // this lane's rows of chunk c: c CH + p WAVES RW + wave RW + rg. Loads are
  // unconditional at clamped rows / dimensions; the masks act at use.
  f32x4 kx[2][NP][NV], vx[2][NP][NV];
  auto load = [&](int slot, int c) {
#pragma unroll
    for (int p = 0; p < NP; p++) {
      const int row = min(r0 + c * CH + p * WAVES * RW + wave * RW + rg, r1 - 1);
#pragma unroll
      for (int nv = 0; nv < NV; nv++) {
        const int d = min(4 * sub + 4 * TPR * nv, head_dim - 4);
        kx[slot][p][nv] = *reinterpret_cast<const f32x4*>(kb + (int64_t)row * kvd + d);
        vx[slot][p][nv] = *reinterpret_cast<const f32x4*>(vb + (int64_t)row * kvd + d);
      }
    }
  };
  if (nch > 0) load(0, 0);

  // RoPE of this head's query and of the KV head's new key; the value as is
  const double ln_theta = log(theta);
  for (int i = tid; i < half; i += THREADS) {
    const double ang = (double)pos * exp((-2.0 * (double)i / (double)head_dim) * ln_theta);
    const double c = cos(ang), s = sin(ang);
    const double q0 = q[hq * head_dim + i], q1 = q[hq * head_dim + i + half];
    qr[i] = (float)(q0 * c - q1 * s);
    qr[i + half] = (float)(q1 * c + q0 * s);
    const double k0 = k[hkv * head_dim + i], k1 = k[hkv * head_dim + i + half];
    kr[i] = (float)(k0 * c - k1 * s);
    kr[i + half] = (float)(k1 * c + k0 * s);
  }
  for (int d = tid; d < head_dim; d += THREADS) vn[d] = v[hkv * head_dim + d];
  __syncthreads();
  if (hq % group == 0 && split == 0) {
    for (int d = tid; d < head_dim; d += THREADS) {
      kcache[(int64_t)pos * kvd + hkv * head_dim + d] = kr[d];
      vcache[(int64_t)pos * kvd + hkv * head_dim + d] = vn[d];
    }
  }
  // the lane's query dimensions (zero past head_dim)
  f32x4 q4[NV];
  bool dlive[NV];
#pragma unroll
  for (int nv = 0; nv < NV; nv++) {
    const int d = 4 * sub + 4 * TPR * nv;
    dlive[nv] = d < head_dim;
    const f32x4 t = *reinterpret_cast<const f32x4*>(qr + min(d, head_dim - 4));
    q4[nv] = dlive[nv] ? t : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  // the wave's online softmax state: running maximum m (wave-uniform), the
  // sum of exp(s - m) over the lane's row group, and the weighted values
  float m = -INFINITY, l = 0.0f;
  f32x4 acc[NV];
#pragma unroll
  for (int nv = 0; nv < NV; nv++) acc[nv] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto fold = [&](float (&s)[NP], f32x4 (&vv)[NP][NV]) {
    float mc = s[0];
#pragma unroll
    for (int p = 1; p < NP; p++) mc = fmaxf(mc, s[p]);
#pragma unroll
    for (int off = TPR; off < 64; off <<= 1) mc = fmaxf(mc, __shfl_xor(mc, off, 64));
    const float mn = fmaxf(m, mc);
    const float alpha = m == -INFINITY ? 0.0f : expf(m - mn);
    l *= alpha;
#pragma unroll
    for (int nv = 0; nv < NV; nv++) acc[nv] *= alpha;
#pragma unroll
    for (int p = 0; p < NP; p++) {
      const float e = s[p] == -INFINITY ? 0.0f : expf(s[p] - mn);
      l += e;
#pragma unroll
      for (int nv = 0; nv < NV; nv++) acc[nv] += e * vv[p][nv];
    }
    m = mn;
  };
  auto compute = [&](int slot, int c) {
    float s[NP];
#pragma unroll
    for (int p = 0; p < NP; p++) {
      float dot = 0.0f;
#pragma unroll
      for (int nv = 0; nv < NV; nv++) {
        const f32x4 kk = kx[slot][p][nv];
        dot += q4[nv][0] * kk[0] + q4[nv][1] * kk[1] + q4[nv][2] * kk[2] + q4[nv][3] * kk[3];
      }
#pragma unroll
      for (int off = TPR / 2; off >= 1; off >>= 1) dot += __shfl_xor(dot, off, 64);
      const int row = r0 + c * CH + p * WAVES * RW + wave * RW + rg;
      s[p] = row < r1 ? dot * scale : -INFINITY;
    }
    fold(s, vx[slot]);
  };
  for (int c = 0; c < nch; c += 2) {
    if (c + 1 < nch) load(1, c + 1);
    compute(0, c);
    if (c + 1 >= nch) break;
    if (c + 2 < nch) load(0, c + 2);
    compute(1, c + 1);
  }

  // the new row (pos) from LDS, folded into wave 0's state by its row group 0
  // (of the last range)
  if (wave == 0 && split == nsplit - 1) {
    float dot = 0.0f;
    f32x4 vv[NP][NV];
    float s[NP];
#pragma unroll
    for (int nv = 0; nv < NV; nv++) {
      const int d = min(4 * sub + 4 * TPR * nv, head_dim - 4);
      const f32x4 kk = *reinterpret_cast<const f32x4*>(kr + d);
      dot += q4[nv][0] * kk[0] + q4[nv][1] * kk[1] + q4[nv][2] * kk[2] + q4[nv][3] * kk[3];
      vv[0][nv] = *reinterpret_cast<const f32x4*>(vn + d);
    }
#pragma unroll
    for (int off = TPR / 2; off >= 1; off >>= 1) dot += __shfl_xor(dot, off, 64);
    s[0] = rg == 0 ? dot * scale : -INFINITY;
#pragma unroll
    for (int p = 1; p < NP; p++) {
      s[p] = -INFINITY;
#pragma unroll
      for (int nv = 0; nv < NV; nv++) vv[p][nv] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    fold(s, vv);
  }

  // the wave's row groups, then the waves
#pragma unroll
  for (int off = TPR; off < 64; off <<= 1) {
    l += __shfl_xor(l, off, 64);
#pragma unroll
    for (int nv = 0; nv < NV; nv++)
#pragma unroll
      for (int e = 0; e < 4; e++) acc[nv][e] += __shfl_xor(acc[nv][e], off, 64);
  }
  if (rg == 0) {
#pragma unroll
    for (int nv = 0; nv < NV; nv++)
      if (dlive[nv]) *reinterpret_cast<f32x4*>(&wacc[wave][4 * sub + 4 * TPR * nv]) = acc[nv];
  }
  if (lane == 0) {
    wm[wave] = m;
    wl[wave] = l;
  }
  __syncthreads();
  float mx = wm[0];
#pragma unroll
  for (int w = 1; w < WAVES; w++) mx = fmaxf(mx, wm[w]);
  float f[WAVES], sum = 0.0f;
#pragma unroll
  for (int w = 0; w < WAVES; w++) {
    f[w] = wm[w] == -INFINITY ? 0.0f : expf(wm[w] - mx);
    sum += f[w] * wl[w];
  }
  if (nsplit == 1) {
    const float inv = 1.0f / sum;
    for (int d = tid; d < head_dim; d += THREADS) {
      float a = 0.0f;
#pragma unroll
      for (int w = 0; w < WAVES; w++) a += f[w] * wacc[w][d];
      out[hq * head_dim + d] = a * inv;
    }
    return;
  }

  // this range's record; an empty range records maximum -inf and sum 0
  const int rstride = kAttnRec + head_dim;
  float* rec = part + ((int64_t)hq * nsplit + split) * rstride;
  for (int d = tid; d < head_dim; d += THREADS) {
    float a = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; w++) a += f[w] * wacc[w][d];
    rec[kAttnRec + d] = a;
  }
  if (tid == 0) {
    rec[0] = mx;
    rec[1] = sum;
  }
}

// Grouped-query form of the chunk kernel: one workgroup per (KV head, row
// range) serves all G query heads that read that KV head, so each cached row
// is loaded once instead of G times. Per row a lane forms the G partial dot
// products of its dimensions; each head keeps its own online softmax state.
// G query heads hkv G .. hkv G + G - 1; 4 waves; 2 rows per lane per chunk.
// LDS (dynamic): qr[G][hd], kr[hd], vn[hd], wacc[WAVES][G][hd], wm / wl[WAVES][G].
template <int TPR, int NV, int G>
__global__ __launch_bounds__(kAttnThreads) void decode_attention_gqa_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v, float* __restrict__ kcache,
    float* __restrict__ vcache, int pos, int n_q, int n_kv, int head_dim, double theta, float scale,
    float* __restrict__ out, int nsplit, int rps, float* __restrict__ part) {
  constexpr int WAVES = kAttnThreads / 64;
  constexpr int NP = 2;
  constexpr int RW = 64 / TPR;         // rows per wave per load
  constexpr int CH = WAVES * RW * NP;  // rows per chunk
  extern __shared__ __attribute__((aligned(16))) float gsm[];
  float* qr = gsm;                         // [G][head_dim]
  float* kr = qr + G * head_dim;           // [head_dim]
  float* vn = kr + head_dim;               // [head_dim]
  float* wacc = vn + head_dim;             // [WAVES][G][head_dim]
  float* wm = wacc + WAVES * G * head_dim;  // [WAVES][G]
  float* wl = wm + WAVES * G;               // [WAVES][G]
  const int hkv = (int)blockIdx.x % n_kv, split = (int)blockIdx.x / n_kv, hq0 = hkv * G;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int sub = lane % TPR, rg = lane / TPR;
  const int half = head_dim / 2, kvd = n_kv * head_dim;
  const int r0 = min(split * rps, pos), r1 = min(r0 + rps, pos);
  const int nch = (r1 - r0 + CH - 1) / CH;
  const float* kb = kcache + hkv * head_dim;
  const float* vb = vcache + hkv * head_dim;

  f32x4 kx[2][NP][NV], vx[2][NP][NV];
  auto load = [&](int slot, int c) {
#pragma unroll
    for (int p = 0; p < NP; p++) {
      const int row = min(r0 + c * CH + p * WAVES * RW + wave * RW + rg, r1 - 1);
#pragma unroll
      for (int nv = 0; nv < NV; nv++) {
        const int d = min(4 * sub + 4 * TPR * nv, head_dim - 4);
        kx[slot][p][nv] = *reinterpret_cast<const f32x4*>(kb + (int64_t)row * kvd + d);
        vx[slot][p][nv] = *reinterpret_cast<const f32x4*>(vb + (int64_t)row * kvd + d);
      }
    }
  };
  if (nch > 0) load(0, 0);

  // RoPE of the G queries and of the KV head's new key (the angle depends on
  // the dimension only); the value as is
  const double ln_theta = log(theta);
  for (int i = tid; i < half; i += kAttnThreads) {
    const double ang = (double)pos * exp((-2.0 * (double)i / (double)head_dim) * ln_theta);
    const double c = cos(ang), s = sin(ang);
#pragma unroll
    for (int g = 0; g < G; g++) {
      const double q0 = q[(hq0 + g) * head_dim + i], q1 = q[(hq0 + g) * head_dim + i + half];
      qr[g * head_dim + i] = (float)(q0 * c - q1 * s);
      qr[g * head_dim + i + half] = (float)(q1 * c + q0 * s);
    }
    const double k0 = k[hkv * head_dim + i], k1 = k[hkv * head_dim + i + half];
    kr[i] = (float)(k0 * c - k1 * s);
    kr[i + half] = (float)(k1 * c + k0 * s);
  }
  for (int d = tid; d < head_dim; d += kAttnThreads) vn[d] = v[hkv * head_dim + d];
  __syncthreads();
  if (split == 0) {
    for (int d = tid; d < head_dim; d += kAttnThreads) {
      kcache[(int64_t)pos * kvd + hkv * head_dim + d] = kr[d];
      vcache[(int64_t)pos * kvd + hkv * head_dim + d] = vn[d];
    }
  }
  f32x4 q4[G][NV];
  bool dlive[NV];
#pragma unroll
  for (int nv = 0; nv < NV; nv++) {
    const int d = 4 * sub + 4 * TPR * nv;
    dlive[nv] = d < head_dim;
#pragma unroll
    for (int g = 0; g < G; g++) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(qr + g * head_dim + min(d, head_dim - 4));
      q4[g][nv] = dlive[nv] ? t : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }

  float m[G], l[G];
  f32x4 acc[G][NV];
#pragma unroll
  for (int g = 0; g < G; g++) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int nv = 0; nv < NV; nv++) acc[g][nv] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  // fold the scores s[g][p] of NP rows (values vv) into head g's state
  auto fold = [&](int g, const float (&s)[NP], const f32x4 (&vv)[NP][NV]) {
    float mc = s[0];
#pragma unroll
    for (int p = 1; p < NP; p++) mc = fmaxf(mc, s[p]);
#pragma unroll
    for (int off = TPR; off < 64; off <<= 1) mc = fmaxf(mc, __shfl_xor(mc, off, 64));
    const float mn = fmaxf(m[g], mc);
    const float alpha = m[g] == -INFINITY ? 0.0f : expf(m[g] - mn);
    l[g] *= alpha;
#pragma unroll
    for (int nv = 0; nv < NV; nv++) acc[g][nv] *= alpha;
#pragma unroll
    for (int p = 0; p < NP; p++) {
      const float e = s[p] == -INFINITY ? 0.0f : expf(s[p] - mn);
      l[g] += e;
#pragma unroll
      for (int nv = 0; nv < NV; nv++) acc[g][nv] += e * vv[p][nv];
    }
    m[g] = mn;
  };
  auto compute = [&](int slot, int c) {
#pragma unroll
    for (int g = 0; g < G; g++) {
      float s[NP];
#pragma unroll
      for (int p = 0; p < NP; p++) {
        float dot = 0.0f;
#pragma unroll
        for (int nv = 0; nv < NV; nv++) {
          const f32x4 kk = kx[slot][p][nv];
          dot += q4[g][nv][0] * kk[0] + q4[g][nv][1] * kk[1] + q4[g][nv][2] * kk[2] + q4[g][nv][3] * kk[3];
        }
#pragma unroll
        for (int off = TPR / 2; off >= 1; off >>= 1) dot += __shfl_xor(dot, off, 64);
        const int row = r0 + c * CH + p * WAVES * RW + wave * RW + rg;
        s[p] = row < r1 ? dot * scale : -INFINITY;
      }
      fold(g, s, vx[slot]);
    }
  };
  for (int c = 0; c < nch; c += 2) {
    if (c + 1 < nch) load(1, c + 1);
    compute(0, c);
    if (c + 1 >= nch) break;
    if (c + 2 < nch) load(0, c + 2);
    compute(1, c + 1);
  }

  // the new row (pos) from LDS, folded into wave 0's states by its row group
  // 0 (of the last range)
  if (wave == 0 && split == nsplit - 1) {
    f32x4 vv[NP][NV], kk[NV];
#pragma unroll
    for (int nv = 0; nv < NV; nv++) {
      const int d = min(4 * sub + 4 * TPR * nv, head_dim - 4);
      kk[nv] = *reinterpret_cast<const f32x4*>(kr + d);
      vv[0][nv] = *reinterpret_cast<const f32x4*>(vn + d);
#pragma unroll
      for (int p = 1; p < NP; p++) vv[p][nv] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
      float dot = 0.0f;
#pragma unroll
      for (int nv = 0; nv < NV; nv++)
        dot += q4[g][nv][0] * kk[nv][0] + q4[g][nv][1] * kk[nv][1] + q4[g][nv][2] * kk[nv][2] +
               q4[g][nv][3] * kk[nv][3];
#pragma unroll
      for (int off = TPR / 2; off >= 1; off >>= 1) dot += __shfl_xor(dot, off, 64);
      float s[NP];
      s[0] = rg == 0 ? dot * scale : -INFINITY;
#pragma unroll
      for (int p = 1; p < NP; p++) s[p] = -INFINITY;
      fold(g, s, vv);
    }
  }

  // each head: the wave's row groups, then the waves
#pragma unroll
  for (int g = 0; g < G; g++) {
#pragma unroll
    for (int off = TPR; off < 64; off <<= 1) {
      l[g] += __shfl_xor(l[g], off, 64);
#pragma unroll
      for (int nv = 0; nv < NV; nv++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[g][nv][e] += __shfl_xor(acc[g][nv][e], off, 64);
    }
    if (rg == 0) {
#pragma unroll
      for (int nv = 0; nv < NV; nv++)
        if (dlive[nv])
          *reinterpret_cast<f32x4*>(&wacc[(wave * G + g) * head_dim + 4 * sub + 4 * TPR * nv]) = acc[g][nv];
    }
    if (lane == 0) {
      wm[wave * G + g] = m[g];
      wl[wave * G + g] = l[g];
    }
  }
  __syncthreads();
  const int rstride = kAttnRec + head_dim;
  for (int idx = tid; idx < G * head_dim; idx += kAttnThreads) {
    const int g = idx / head_dim, d = idx - g * head_dim;
    float mx = wm[g];
#pragma unroll
    for (int w = 1; w < WAVES; w++) mx = fmaxf(mx, wm[w * G + g]);
    float a = 0.0f, sum = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; w++) {
      const float f = wm[w * G + g] == -INFINITY ? 0.0f : expf(wm[w * G + g] - mx);
      sum += f * wl[w * G + g];
      a += f * wacc[(w * G + g) * head_dim + d];
    }
    const int hq = hq0 + g;
    if (nsplit == 1) {
      out[hq * head_dim + d] = a * (1.0f / sum);
    } else {
      float* rec = part + ((int64_t)hq * nsplit + split) * rstride;
      rec[kAttnRec + d] = a;
      if (d == 0) {
        rec[0] = mx;
        rec[1] = sum;
      }
    }
  }
}

size_t decode_attention_gqa_lds(int64_t head_dim, int g) {
  return (size_t)((g + 2) * head_dim + (kAttnThreads / 64) * (g * head_dim + 2 * g)) * sizeof(float);
}

// Merge of the nsplit range records of each head (one workgroup per head), in
// range order: out = sum_r e_r a_r / sum_r e_r l_r with e_r = exp(m_r - max m).
__global__ __launch_bounds__(kAttnThreads) void decode_attention_merge_kernel(const float* __restrict__ part,
                                                                              int nsplit, int head_dim,
                                                                              float* __restrict__ out) {
  __shared__ float fac[kMaxSplits], lw[kMaxSplits];
  __shared__ float inv;
  const int hq = (int)blockIdx.x, tid = (int)threadIdx.x;
  const int rstride = kAttnRec + head_dim;
  const float* hrec = part + (int64_t)hq * nsplit * rstride;
  if (tid < 64) {
    const float rm = tid < nsplit ? hrec[(int64_t)tid * rstride] : -INFINITY;
    float gm = rm;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) gm = fmaxf(gm, __shfl_xor(gm, off, 64));
    if (tid < nsplit) {
      const float fr = rm == -INFINITY ? 0.0f : expf(rm - gm);
      fac[tid] = fr;
      lw[tid] = fr * hrec[(int64_t)tid * rstride + 1];
    }
  }
  __syncthreads();
  if (tid == 0) {
    float gs = 0.0f;  // in range order
    for (int r = 0; r < nsplit; r++) gs += lw[r];
    inv = 1.0f / gs;
  }
  __syncthreads();
  for (int d = tid; d < head_dim; d += kAttnThreads) {
    float a = 0.0f;
    for (int r = 0; r < nsplit; r++) a += fac[r] * hrec[(int64_t)r * rstride + kAttnRec + d];
    out[hq * head_dim + d] = a * inv;
  }
}

size_t decode_attention_lds(int64_t pos, int64_t head_dim) {
  if (chunk_tpr(head_dim)) return (size_t)(3 + kAttnThreads / 64) * kMaxDims * sizeof(float);
  return (size_t)(3 * head_dim + pos + 1 + 8) * sizeof(float);
}

// Row ranges per head of the chunk kernel. Measured on MI355X (hd 128, 16 or
// 32 heads): a launch costs about 3 us before it reads anything and the merge
// launch as much again, so a cache under ~256 rows stays in one workgroup per
// head (8 waves, 2 rows per lane per chunk: 6.4 us at 128 rows against 7.1
// with 4 waves); longer caches split into ranges of at least kMinSplitRows
// rows, about one workgroup per CU over all heads (16 heads: 512 rows 16 ->
// 8 us, 2048 rows 49 -> 11 us, 8192 rows 180 -> 28 us).
namespace {
constexpr int kMinSplitRows = 64;
constexpr int kAttnThreads1 = 512;  // threads of the single-range workgroup
}  // namespace

AttnSplit plan_decode_attention(int64_t pos, int64_t n_q, int64_t n_kv, int64_t head_dim, int cu_count) {
  AttnSplit p{1, (int)pos, kAttnThreads1, 2, 1, 0};
  if (!chunk_tpr(head_dim)) return p;
  // grouped-query heads (4 or 8 per KV head) on long caches: one workgroup
  // per KV head serves its G query heads, about two workgroups per CU.
  // Measured (hd 128, 256 CUs): 32 heads over 8, 2048 / 4096 rows 18.0 / 27.2
  // -> 15.6 / 19.5 us; 64 over 8, 4096 / 16384 rows 46.0 / 158 -> 27.8 / 64.2;
  // 32 over 4, 8192 rows 45.9 -> 35.9. Shorter caches and pairs of heads stay
  // with a workgroup per query head (1024 rows: 10.6 against 14.4; 16 over 8,
  // 2048 rows: 11.0 against 12.7).
  const int64_t g = n_q / n_kv;
  const bool gqa = (g == 4 || g == 8) && g * head_dim <= 1024 && pos >= 2048;
  if (gqa) p.group = (int)g;
  const int64_t want = gqa ? (2 * (int64_t)std::max(cu_count, 1) + n_kv - 1) / n_kv
                           : ((int64_t)std::max(cu_count, 1) + n_q - 1) / n_q;
  const int64_t ns = std::min<int64_t>({want, pos / kMinSplitRows, (int64_t)kMaxSplits});
  if (ns < 4) {
    // one range per head: beyond two chunks of 2 rows per lane, 8 rows per
    // lane keep more of the cache in flight (16 heads, hd 128, graph
    // replays: 128 rows 6.9 -> 6.2 us, 255 rows 9.3 -> 8.1; at two chunks
    // or fewer the larger chunk is slower: 64 rows 5.5 against 6.0)
    if (pos > 2 * (kAttnThreads1 / 64) * (64 / chunk_tpr(head_dim)) * 2) p.np = 8;
    return p;
  }
  p.nsplit = (int)ns;
  p.rps = (int)((pos + ns - 1) / ns);
  p.threads = 256;
  // small ranges take 2 rows per lane per chunk (a chunk is 4 waves x 64 / TPR x NP rows)
  p.np = p.rps <= 4 * (64 / chunk_tpr(head_dim)) * 2 ? 2 : 8;
  p.scratch_bytes = (size_t)n_q * (size_t)ns * (size_t)(kAttnRec + head_dim) * sizeof(float);
  return p;
}

namespace {

template <int TPR, int NV, int NP, int THREADS>
hipError_t launch_chunk(const float* q, const float* k, const float* v, float* kcache, float* vcache, int64_t pos,
                        int64_t n_q, int64_t n_kv, int64_t head_dim, double theta, double scale, float* out,
                        const AttnSplit& sp, float* part, hipStream_t stream) {
  const int ns = sp.nsplit;
  hipLaunchKernelGGL((decode_attention_chunk_kernel<TPR, NV, NP, THREADS>), dim3((unsigned)(n_q * ns)),
                     dim3(THREADS), 0, stream, q, k, v, kcache, vcache, (int)pos, (int)n_q, (int)n_kv, (int)head_dim,
                     theta, (float)scale, out, ns, sp.rps, part);
  if (hipError_t e = hipGetLastError()) return e;
  if (ns > 1)
    hipLaunchKernelGGL(decode_attention_merge_kernel, dim3((unsigned)n_q), dim3(kAttnThreads), 0, stream, part, ns,
                       (int)head_dim, out);
  return hipGetLastError();
}

// (threads, rows per lane) of the plan -> one instantiation
template <int TPR, int NV, int NPS, int NPL>
hipError_t launch_chunk_cfg(const float* q, const float* k, const float* v, float* kcache, float* vcache, int64_t pos,
                            int64_t n_q, int64_t n_kv, int64_t head_dim, double theta, double scale, float* out,
                            const AttnSplit& sp, float* part, hipStream_t stream) {
#define RQ_ATTN_ARGS q, k, v, kcache, vcache, pos, n_q, n_kv, head_dim, theta, scale, out, sp, part, stream
  if (sp.threads == 1024) return launch_chunk<TPR, NV, NPS, 1024>(RQ_ATTN_ARGS);
  if (sp.threads == 512)
    return sp.np == NPS ? launch_chunk<TPR, NV, NPS, 512>(RQ_ATTN_ARGS) : launch_chunk<TPR, NV, NPL, 512>(RQ_ATTN_ARGS);
  if (sp.np == NPS) return launch_chunk<TPR, NV, NPS, 256>(RQ_ATTN_ARGS);
  return launch_chunk<TPR, NV, NPL, 256>(RQ_ATTN_ARGS);
#undef RQ_ATTN_ARGS
}

}  // namespace

namespace {

template <int TPR, int NV, int G>
hipError_t launch_gqa(const float* q, const float* k, const float* v, float* kcache, float* vcache, int64_t pos,
                      int64_t n_q, int64_t n_kv, int64_t head_dim, double theta, double scale, float* out,
                      const AttnSplit& sp, float* part, hipStream_t stream) {
  const int ns = sp.nsplit;
  hipLaunchKernelGGL((decode_attention_gqa_kernel<TPR, NV, G>), dim3((unsigned)(n_kv * ns)), dim3(kAttnThreads),
                     (unsigned)decode_attention_gqa_lds(head_dim, G), stream, q, k, v, kcache, vcache, (int)pos,
                     (int)n_q, (int)n_kv, (int)head_dim, theta, (float)scale, out, ns, sp.rps, part);
  if (hipError_t e = hipGetLastError()) return e;
  if (ns > 1)
    hipLaunchKernelGGL(decode_attention_merge_kernel, dim3((unsigned)n_q), dim3(kAttnThreads), 0, stream, part, ns,
                       (int)head_dim, out);
  return hipGetLastError();
}

template <int TPR, int NV>
hipError_t launch_gqa_g(const float* q, const float* k, const float* v, float* kcache, float* vcache, int64_t pos,
                        int64_t n_q, int64_t n_kv, int64_t head_dim, double theta, double scale, float* out,
                        const AttnSplit& sp, float* part, hipStream_t stream) {
#define RQ_GQA_ARGS q, k, v, kcache, vcache, pos, n_q, n_kv, head_dim, theta, scale, out, sp, part, stream
  if (sp.group == 2) return launch_gqa<TPR, NV, 2>(RQ_GQA_ARGS);
  if (sp.group == 4) return launch_gqa<TPR, NV, 4>(RQ_GQA_ARGS);
  return launch_gqa<TPR, NV, 8>(RQ_GQA_ARGS);
#undef RQ_GQA_ARGS
}

}  // namespace

hipError_t launch_decode_attention(const float* q, const float* k, const float* v, float* kcache, float* vcache,
                                   int64_t pos, int64_t n_q, int64_t n_kv, int64_t head_dim, double theta,
                                   double scale, float* out, const AttnSplit& sp, void* scratch, hipStream_t stream) {
  float* part = static_cast<float*>(scratch);
#define RQ_ATTN_ARGS q, k, v, kcache, vcache, pos, n_q, n_kv, head_dim, theta, scale, out, sp, part, stream
  if (sp.group > 1) {
    switch (chunk_tpr(head_dim)) {
      case 16:
        return launch_gqa_g<16, 1>(RQ_ATTN_ARGS);
      case 32:
        return launch_gqa_g<32, 1>(RQ_ATTN_ARGS);
      case 64:
        if (head_dim <= 256) return launch_gqa_g<64, 1>(RQ_ATTN_ARGS);
        return launch_gqa_g<64, 2>(RQ_ATTN_ARGS);
      default:
        return hipErrorInvalidValue;
    }
  }
  switch (chunk_tpr(head_dim)) {
    case 16:
      return launch_chunk_cfg<16, 1, 2, 8>(RQ_ATTN_ARGS);
    case 32:
      return launch_chunk_cfg<32, 1, 2, 8>(RQ_ATTN_ARGS);
    case 64:
      if (head_dim <= 256) return launch_chunk_cfg<64, 1, 2, 8>(RQ_ATTN_ARGS);
      return launch_chunk_cfg<64, 2, 2, 4>(RQ_ATTN_ARGS);
    default:
      break;
  }
#undef RQ_ATTN_ARGS
  const size_t lds = decode_attention_lds(pos, head_dim);
  if (lds > 65536) {
    static std::atomic<uint64_t> attr_set{0};
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev)) return e;
    const uint64_t bit = uint64_t(1) << (dev & 63);
    if (!(attr_set.load(std::memory_order_acquire) & bit)) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&decode_attention_kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
      if (e != hipSuccess) return e;
      attr_set.fetch_or(bit, std::memory_order_acq_rel);
    }
  }
  hipLaunchKernelGGL(decode_attention_kernel, dim3((unsigned)n_q), dim3(kAttnThreads), (unsigned)lds, stream, q, k,
                     v, kcache, vcache, (int)pos, (int)n_q, (int)n_kv, (int)head_dim, theta, (float)scale, out);
  return hipGetLastError();
}

}  // namespace rq
