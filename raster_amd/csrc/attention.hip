// attention.hip — one decode step of RoPE, KV-cache append and single-query
// attention (the glue between a decoder layer's q/k/v and o linears).
//
// Restates, for one token at position pos:
//   rope-pos               raster/dl/attention.clj:197-214 (NeoX half split)
//   kv-append!             raster/dl/attention.clj:413-416
//   gqa-decode-attention   raster/dl/attention.clj:248-287
// One workgroup per query head. It rotates its query and its KV head's new
// key (angles pos * theta^(-2i/head_dim) in double, as the reference), takes
// the scores of positions 0..pos (the new key straight from registers, the
// older ones from the cache), their softmax, and the weighted sum of values.
// The first query head of each KV head writes the rotated key and the value
// into the caches at row pos; the others never read that row from memory, so
// no workgroup waits for another.
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

size_t decode_attention_lds(int64_t pos, int64_t head_dim) {
  return (size_t)(3 * head_dim + pos + 1 + 8) * sizeof(float);
}

hipError_t launch_decode_attention(const float* q, const float* k, const float* v, float* kcache, float* vcache,
                                   int64_t pos, int64_t n_q, int64_t n_kv, int64_t head_dim, double theta,
                                   double scale, float* out, hipStream_t stream) {
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
