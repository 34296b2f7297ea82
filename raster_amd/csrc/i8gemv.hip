// i8gemv.hip — the raw int8 GEMV core of Raster's quant formats,
// i8gemv-dp4a! (raster/quant/kernels_k.clj:141-150):
//
//   y[o] = (float) sum_w dp4a(wp[o * kw + w], xp[w], 0)
//
// wp is [out x kw] int32 words, xp [kw] words, each word four little-endian
// signed int8 lanes (par/dp4a, raster/par.clj:421-440). Raster accumulates in
// a 64-bit long and converts the exact sum to float once; here each lane
// accumulates its words with v_dot4_i32_i8 in int32 (a lane takes at most
// ceil(kw / 64) words and one word's dot is at most 4 * 128 * 128 = 2^16 in
// magnitude, so with kw <= 2^20, the entry's limit, a lane's partial stays
// within 2^30) and the wave adds the lanes' partials in int64, then converts
// once (round to nearest even, as Java's (float) long).
//
// One wave per output row, four rows per workgroup; xp is read through the
// caches (it is kw * 4 bytes, shared by every row). Rows of wp stream as
// 16-byte loads per lane.
#include "rq_internal.h"

namespace rq {

namespace {

__device__ __forceinline__ int dot4(int a, int b, int acc) { return __builtin_amdgcn_sdot4(a, b, acc, false); }

}  // namespace

__global__ __launch_bounds__(256) void i8gemv_dp4a_kernel(const int32_t* __restrict__ wp,
                                                          const int32_t* __restrict__ xp, float* __restrict__ y,
                                                          int64_t kw, int64_t out) {
  const int lane = threadIdx.x & 63;
  const int64_t o = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (o >= out) return;
  const int32_t* row = wp + o * kw;
  int acc = 0;
  // 16-byte pieces where the row is 16-byte aligned, words otherwise
  const bool vec = ((reinterpret_cast<uintptr_t>(row) | reinterpret_cast<uintptr_t>(xp)) & 15) == 0;
  int64_t w = 0;
  if (vec) {
    const int64_t kw4 = kw / 4 * 4;
    for (w = 4 * lane; w < kw4; w += 256) {
      const i32x4 a = *reinterpret_cast<const i32x4*>(row + w);
      const i32x4 b = *reinterpret_cast<const i32x4*>(xp + w);
      acc = dot4(a[0], b[0], acc);
      acc = dot4(a[1], b[1], acc);
      acc = dot4(a[2], b[2], acc);
      acc = dot4(a[3], b[3], acc);
    }
    w = kw4 + lane;
  } else {
    w = lane;
  }
  for (; w < kw; w += 64) acc = dot4(row[w], xp[w], acc);
  // lanes' int32 partials summed in int64 (exact), then one conversion
  int64_t s = acc;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const int lo = __shfl_xor((int)(uint32_t)s, off);
    const int hi = __shfl_xor((int)(s >> 32), off);
    s += ((int64_t)hi << 32) | (uint32_t)lo;
  }
  if (lane == 0) y[o] = (float)s;
}

hipError_t launch_i8gemv_dp4a(const int32_t* wp, const int32_t* xp, float* y, int64_t kw, int64_t out,
                              hipStream_t stream) {
  hipLaunchKernelGGL(i8gemv_dp4a_kernel, dim3((unsigned)((out + 3) / 4)), dim3(256), 0, stream, wp, xp, y, kw, out);
  return hipGetLastError();
}

}  // namespace rq
