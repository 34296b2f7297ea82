// stream.hip — a plain streaming read, the HBM read ceiling the decode kernels
// are measured against. Not part of the matmul path: measurement only.
//
// Each thread reads 16-byte vectors in a grid-stride loop, four loads in
// flight per iteration, and folds them with XOR; a workgroup stores its fold
// only when it equals a value it cannot know in advance, so the loads cannot
// be removed and (almost) nothing is written.
#include "rq_internal.h"

namespace rq {

namespace {
constexpr int kStreamThreads = 256;
}

__global__ __launch_bounds__(kStreamThreads) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                                     uint32_t key, uint32_t* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * kStreamThreads;
  int64_t i = (int64_t)blockIdx.x * kStreamThreads + threadIdx.x;
  u32x4 a0 = {0u, 0u, 0u, 0u}, a1 = a0, a2 = a0, a3 = a0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 v0 = __builtin_nontemporal_load(src + i);
    const u32x4 v1 = __builtin_nontemporal_load(src + i + stride);
    const u32x4 v2 = __builtin_nontemporal_load(src + i + 2 * stride);
    const u32x4 v3 = __builtin_nontemporal_load(src + i + 3 * stride);
    a0 ^= v0;
    a1 ^= v1;
    a2 ^= v2;
    a3 ^= v3;
  }
  for (; i < n16; i += stride) a0 ^= src[i];
  const u32x4 a = a0 ^ a1 ^ a2 ^ a3;
  const uint32_t r = a[0] ^ a[1] ^ a[2] ^ a[3];
  if (r == key) sink[(int64_t)blockIdx.x * kStreamThreads + threadIdx.x] = r;
}

hipError_t launch_stream_read(const void* src, size_t bytes, int grid, uint32_t* sink, hipStream_t stream) {
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)grid), dim3(kStreamThreads), 0, stream,
                     static_cast<const u32x4*>(src), (int64_t)(bytes / 16), 0x9E3779B9u, sink);
  return hipGetLastError();
}

}  // namespace rq
