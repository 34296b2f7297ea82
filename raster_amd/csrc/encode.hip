// encode.hip — weight encoders on the device: Raster's K-quant packers.
//
// quantize-weight-q4k (raster/compiler/backend/cpu/quant.clj:92-137), as
// q4k-of calls it (raster/quant/pack.clj:45-53: each row of W zero-padded to
// inp = nextpad(in), the padded matrix quantized as one array), and
// quantize-weight-q6k (quant.clj:214-239). Load-time work, run once per weight.
//
// Every step is the reference's arithmetic in double, in its order: the
// sub-block minimum / maximum (exact), the sub-block scale, the super-block
// scale of scales, the 6-bit codes of scale and minimum by Math/round (ties
// toward +infinity), and the weight codes against the quantized scale and
// minimum. Only maxima cross lanes, and a maximum does not depend on the order
// it is taken in, so the result is bitwise the reference's for finite input.
//
// Layout of the work: one lane per sub-block (Q4_K: 8 lanes of 32 elements per
// super-block, Q6_K: 16 lanes of 16), the super-block maxima by lane shuffles
// within the group. Padded columns read as 0.
#include "rq_internal.h"

namespace rq {

namespace {

constexpr int kEncThreads = 256;

// Math/round of a double, clamped to [lo, hi] (NaN -> 0 before the clamp).
__device__ __forceinline__ int java_round_clamp(double v, int lo, int hi) {
  if (!(v == v)) return lo > 0 ? lo : (hi < 0 ? hi : 0);
  const double f = floor(v);
  const double r = (v - f >= 0.5) ? f + 1.0 : f;
  return r > (double)hi ? hi : r < (double)lo ? lo : (int)r;
}

// Element c of row o of the zero-padded matrix.
__device__ __forceinline__ float padded(const float* W, int64_t o, int64_t c, int64_t in) {
  return c < in ? W[o * in + c] : 0.0f;
}

}  // namespace

// One lane per 32-element sub-block; 8 lanes per super-block.
__global__ __launch_bounds__(kEncThreads) void q4k_encode_kernel(const float* __restrict__ W, int64_t out, int64_t in,
                                                                 int64_t inp, uint8_t* __restrict__ wq,
                                                                 float* __restrict__ da, float* __restrict__ db,
                                                                 uint8_t* __restrict__ aq, int8_t* __restrict__ bq) {
  const int64_t nsb = out * (inp / 256);
  const int64_t t = (int64_t)blockIdx.x * kEncThreads + threadIdx.x;
  const int64_t sb_raw = t >> 3;
  const bool live = sb_raw < nsb;
  const int64_t sb = live ? sb_raw : nsb - 1;  // lanes past the end redo the last super-block, store nothing
  const int j = (int)(t & 7);
  const int64_t o = sb / (inp / 256);
  const int64_t c0 = (sb % (inp / 256)) * 256 + j * 32;
  float v[32];
#pragma unroll
  for (int i = 0; i < 32; i++) v[i] = padded(W, o, c0 + i, in);
  // 1. sub-block scale a = (max - min) / 15 and minimum b
  float lo = v[0], hi = v[0];
#pragma unroll
  for (int i = 1; i < 32; i++) {
    if (v[i] < lo) lo = v[i];
    if (v[i] > hi) hi = v[i];
  }
  const double as = ((double)hi - (double)lo) / 15.0;
  const double bs = (double)lo;
  // 2. super-block scale of scales and of minima (maxima over the 8 lanes)
  double amax = as > 0.0 ? as : 0.0;
  double bmax = fabs(bs);
#pragma unroll
  for (int s = 1; s < 8; s <<= 1) {
    const double oa = __shfl_xor(amax, s, 8);
    const double ob = __shfl_xor(bmax, s, 8);
    amax = oa > amax ? oa : amax;
    bmax = ob > bmax ? ob : bmax;
  }
  const double dav = amax / 63.0, dbv = bmax / 31.0;
  const double ida = dav == 0.0 ? 0.0 : 1.0 / dav;
  const double idb = dbv == 0.0 ? 0.0 : 1.0 / dbv;
  const int aqj = java_round_clamp(as * ida, 0, 63);
  const int bqj = java_round_clamp(bs * idb, -32, 31);
  const double a1 = dav * (double)aqj, b1 = dbv * (double)bqj;
  const double ia1 = a1 == 0.0 ? 0.0 : 1.0 / a1;
  // 3. the weights against the quantized scale and minimum: byte k holds
  // element k (low nibble) and element k + 16 (high nibble)
  u32x4 packed = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int k = 0; k < 16; k++) {
    const uint32_t q0 = (uint32_t)java_round_clamp(((double)v[k] - b1) * ia1, 0, 15);
    const uint32_t q1 = (uint32_t)java_round_clamp(((double)v[k + 16] - b1) * ia1, 0, 15);
    packed[k >> 2] |= (q0 | (q1 << 4)) << (8 * (k & 3));
  }
  if (live) {
    const int64_t sidx = sb * 8 + j;
    *reinterpret_cast<u32x4*>(wq + sidx * 16) = packed;
    aq[sidx] = (uint8_t)aqj;
    bq[sidx] = (int8_t)bqj;
    if (j == 0) {
      da[sb] = (float)dav;
      db[sb] = (float)dbv;
    }
  }
}

// One lane per 16-element sub-block; 16 lanes per super-block.
__global__ __launch_bounds__(kEncThreads) void q6k_encode_kernel(const float* __restrict__ W, int64_t nsb,
                                                                 uint8_t* __restrict__ wq, int8_t* __restrict__ sc,
                                                                 float* __restrict__ ds) {
  const int64_t t = (int64_t)blockIdx.x * kEncThreads + threadIdx.x;
  const int64_t sb_raw = t >> 4;
  const bool live = sb_raw < nsb;
  const int64_t sb = live ? sb_raw : nsb - 1;
  const int j = (int)(t & 15);
  const int64_t base = sb * 256 + j * 16;
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; i += 4) {
    const f32x4 q = *reinterpret_cast<const f32x4*>(W + base + i);
    v[i] = q[0];
    v[i + 1] = q[1];
    v[i + 2] = q[2];
    v[i + 3] = q[3];
  }
  double mx = 0.0;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const double a = fabsf(v[i]);
    if (a > mx) mx = a;
  }
  const double as = mx / 32.0;
  double amax = as;
#pragma unroll
  for (int s = 1; s < 16; s <<= 1) {
    const double o = __shfl_xor(amax, s, 16);
    amax = o > amax ? o : amax;
  }
  const double dv = amax / 127.0, idv = dv == 0.0 ? 0.0 : 1.0 / dv;
  const int scj = java_round_clamp(as * idv, 0, 127);
  const double a1 = dv * (double)scj, ia1 = a1 == 0.0 ? 0.0 : 1.0 / a1;
  u32x4 packed = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int k = 0; k < 16; k++) {
    // Math/round, + zero point 32, clamp to [0, 63]: the rounded value is
    // clamped to [-32, 31] first, which is the same result
    const uint32_t q = (uint32_t)(java_round_clamp((double)v[k] * ia1, -32, 31) + 32);
    packed[k >> 2] |= q << (8 * (k & 3));
  }
  if (live) {
    *reinterpret_cast<u32x4*>(wq + base) = packed;
    sc[sb * 16 + j] = (int8_t)scj;
    if (j == 0) ds[sb] = (float)dv;
  }
}

hipError_t launch_q4k_encode(const float* W, int64_t out, int64_t in, int64_t inp, uint8_t* wq, float* da, float* db,
                             uint8_t* aq, int8_t* bq, hipStream_t stream) {
  const int64_t lanes = out * (inp / 256) * 8;
  const int64_t grid = (lanes + kEncThreads - 1) / kEncThreads;
  hipLaunchKernelGGL(q4k_encode_kernel, dim3((unsigned)grid), dim3(kEncThreads), 0, stream, W, out, in, inp, wq, da,
                     db, aq, bq);
  return hipGetLastError();
}

hipError_t launch_q6k_encode(const float* W, int64_t out, int64_t in, uint8_t* wq, int8_t* sc, float* ds,
                             hipStream_t stream) {
  const int64_t nsb = out * (in / 256);
  const int64_t grid = (nsb * 16 + kEncThreads - 1) / kEncThreads;
  hipLaunchKernelGGL(q6k_encode_kernel, dim3((unsigned)grid), dim3(kEncThreads), 0, stream, W, nsb, wq, sc, ds);
  return hipGetLastError();
}

}  // namespace rq
