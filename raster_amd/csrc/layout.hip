// layout.hip — converts a weight from Raster's row-major arrays to the chunked
// device layout described in rq_internal.h (run once, at weight creation).
#include "rq_internal.h"

namespace rq {

// One thread per 16-byte piece of the chunked codes; padded rows read as zero.
template <int CB>
__global__ __launch_bounds__(256) void chunk_codes_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                         int64_t out, int64_t nb, int64_t npieces) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= npieces) return;
  constexpr int PPC = CB;  // 16-byte pieces per chunk (16 rows * CB bytes / 16)
  const int64_t chunk = p / PPC, within = p % PPC;
  const int64_t g = chunk / nb, b = chunk % nb;
  const int64_t r = within * 16 / CB, off = within * 16 % CB;
  const int64_t row = 16 * g + r;
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (row < out) v = *reinterpret_cast<const uint4*>(src + row * nb * CB + b * CB + off);
  *reinterpret_cast<uint4*>(dst + 16 * p) = v;
}

// block-major scales: element e = chunk * 16 + r
template <typename ST>
__global__ __launch_bounds__(256) void chunk_scales_kernel(const ST* __restrict__ src, ST* __restrict__ dst,
                                                          int64_t out, int64_t nb, int64_t n) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const int64_t chunk = e / 16, r = e % 16;
  const int64_t g = chunk / nb, b = chunk % nb;
  const int64_t row = 16 * g + r;
  dst[e] = row < out ? src[row * nb + b] : ST(0);
}

// row-batched scales: element e = scale_rb_group(g) + scale_rb_in_group(b, r)
template <typename ST>
__global__ __launch_bounds__(256) void batch_scales_kernel(const ST* __restrict__ src, ST* __restrict__ dst,
                                                          int64_t out, int64_t nb, int64_t n) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const int64_t per_group = scale_nb8(nb) * 16;
  const int64_t g = e / per_group, t = e % per_group;
  const int64_t b = (t / 128) * 8 + (t % 8), r = (t % 128) / 8;
  const int64_t row = 16 * g + r;
  dst[e] = row < out && b < nb ? src[row * nb + b] : ST(0);
}

hipError_t launch_chunk_weight(int format, int scale_dtype, const uint8_t* q_rm, const void* s_rm, int64_t out,
                               int64_t in, int64_t npad, uint8_t* q, void* s, void* s_rb, hipStream_t stream) {
  const int64_t nb = in / 32;
  const int cb = code_bytes(format);
  const int64_t npieces = npad * nb * cb / 16;
  const dim3 gq((unsigned)((npieces + 255) / 256));
  if (cb == 32)
    hipLaunchKernelGGL((chunk_codes_kernel<32>), gq, dim3(256), 0, stream, q_rm, q, out, nb, npieces);
  else
    hipLaunchKernelGGL((chunk_codes_kernel<16>), gq, dim3(256), 0, stream, q_rm, q, out, nb, npieces);
  const int64_t ns = npad * nb, nsb = npad * scale_nb8(nb);
  const dim3 gs((unsigned)((ns + 255) / 256)), gsb((unsigned)((nsb + 255) / 256));
  if (scale_dtype == RQ_F16) {
    hipLaunchKernelGGL((chunk_scales_kernel<uint16_t>), gs, dim3(256), 0, stream,
                       static_cast<const uint16_t*>(s_rm), static_cast<uint16_t*>(s), out, nb, ns);
    hipLaunchKernelGGL((batch_scales_kernel<uint16_t>), gsb, dim3(256), 0, stream,
                       static_cast<const uint16_t*>(s_rm), static_cast<uint16_t*>(s_rb), out, nb, nsb);
  } else {
    hipLaunchKernelGGL((chunk_scales_kernel<float>), gs, dim3(256), 0, stream, static_cast<const float*>(s_rm),
                       static_cast<float*>(s), out, nb, ns);
    hipLaunchKernelGGL((batch_scales_kernel<float>), gsb, dim3(256), 0, stream, static_cast<const float*>(s_rm),
                       static_cast<float*>(s_rb), out, nb, nsb);
  }
  return hipGetLastError();
}

}  // namespace rq
