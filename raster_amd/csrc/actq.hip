// actq.hip — on-device activation quantizer: Raster's per-block symmetric int8
// activation format.
//
// quantize-act-i8 (raster/compiler/backend/cpu/quant.clj:282-305,399-415): per
// row and 32-element block,
//   d = max|x| / 127 (double), id = 1 / d (0 when d == 0),
//   q = clamp(round(x * id), -127, 127) with Java's Math/round (ties toward
//   +infinity), xs = (float) d, xsum = sum q.
// The int8 bytes are also the little-endian int32 words of the GPU prefill
// quantizer quant-act-i8-rows-gpu! (raster/quant/kernels_k.clj:326-355), which
// skips the clamp: |x * id| rounds to at most 127 for finite x, so the two
// agree on finite input.
//
// Eight lanes share a block (4 elements each): one 16-byte load per lane, the
// block maximum and sum over the 8 lanes by register shuffles, the per-element
// math in double as the reference does it (the quotient and the products
// round exactly as the CPU's), one 4-byte store per lane. HBM-bound: 4 bytes
// read and 1 + 8/32 bytes written per element.
#include "rq_internal.h"

namespace rq {

namespace {

constexpr int kActqThreads = 256;

}  // namespace

__global__ __launch_bounds__(kActqThreads) void quantize_act_i8_kernel(const float* __restrict__ x,
                                                                      int8_t* __restrict__ xq,
                                                                      float* __restrict__ xs,
                                                                      int32_t* __restrict__ xsum, int64_t nblk) {
  const int64_t blk = (int64_t)blockIdx.x * (kActqThreads / 8) + threadIdx.x / 8;
  const int part = threadIdx.x & 7;
  // lanes past the last block reread it (all 8 lanes of a group agree) and
  // store nothing
  const int64_t b = blk < nblk ? blk : nblk - 1;
  const f32x4 v = *reinterpret_cast<const f32x4*>(x + b * 32 + part * 4);
  // block maximum of |x| (NaN elements drop out of fmaxf, as they fail the
  // reference's `>` test)
  float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  a = fmaxf(a, __shfl_xor(a, 1, 8));
  a = fmaxf(a, __shfl_xor(a, 2, 8));
  a = fmaxf(a, __shfl_xor(a, 4, 8));
  const double d = (double)a / 127.0;
  const double id = d == 0.0 ? 0.0 : 1.0 / d;
  uint32_t word = 0u;
  int s = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int q = java_round_clamp127((double)v[i] * id);
    word |= (uint32_t)(q & 0xFF) << (8 * i);
    s += q;
  }
  s += __shfl_xor(s, 1, 8);
  s += __shfl_xor(s, 2, 8);
  s += __shfl_xor(s, 4, 8);
  if (blk < nblk) {
    *reinterpret_cast<uint32_t*>(xq + b * 32 + part * 4) = word;
    if (part == 0) {
      xs[b] = (float)d;
      if (xsum) xsum[b] = s;
    }
  }
}

hipError_t launch_quantize_act_i8(const float* x, int64_t m, int64_t in, int8_t* xq, float* xs, int32_t* xsum,
                                  hipStream_t stream) {
  const int64_t nblk = m * (in / 32);
  if (nblk == 0) return hipSuccess;
  const int64_t grid = (nblk + kActqThreads / 8 - 1) / (kActqThreads / 8);
  hipLaunchKernelGGL(quantize_act_i8_kernel, dim3((unsigned)grid), dim3(kActqThreads), 0, stream, x, xq, xs, xsum,
                     nblk);
  return hipGetLastError();
}

}  // namespace rq
