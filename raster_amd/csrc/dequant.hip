// dequant.hip — writes the dequantized f32 weight W[out x in] (row-major, as
// Raster returns it) from a resident chunked weight, with the same decode helpers (q8_code / q4_nib / load_scale) the
// matmul kernels use. W[o, i] = scale[o, i/32] * code[o, i] is one IEEE f32
// multiply of two exactly-represented operands, the value dequant-q8-dense
// produces (raster/quant/train.clj:60-71: (float)(double scale * double code)
// rounds the exact product once). Q4_0: scale * (q - 8)
// (test/raster/compiler/backend/cpu/quant_encode_test.clj:19-20).
#include "rq_internal.h"

namespace rq {

template <int FMT, typename ST>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                                     float* __restrict__ w, int64_t out, int64_t in) {
  const int64_t rowbytes = FMT == RQ_Q8_0 ? in : in / 2;
  const int64_t nchunk = out * (rowbytes / 16);
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= nchunk) return;
  const int64_t row = c / (rowbytes / 16), cc = c % (rowbytes / 16);
  const int64_t nb = in / 32;
  // 16-byte piece cc of the row: Q8 half cc % 2 of block cc / 2, Q4 block cc
  const int64_t src = FMT == RQ_Q8_0 ? code_off<FMT>(row, cc / 2, nb) + 16 * (cc % 2) : code_off<FMT>(row, cc, nb);
  const uint4 raw = *reinterpret_cast<const uint4*>(q + src);
  const uint32_t d[4] = {raw.x, raw.y, raw.z, raw.w};
  if (FMT == RQ_Q8_0) {
    const float s = load_scale<ST>(sc, scale_off(row, cc / 2, nb));
    float4* dst = reinterpret_cast<float4*>(w + row * in + cc * 16);
#pragma unroll
    for (int i = 0; i < 4; i++)
      dst[i] = make_float4(s * q8_code(d[i], 0), s * q8_code(d[i], 1), s * q8_code(d[i], 2), s * q8_code(d[i], 3));
  } else {
    const float s = load_scale<ST>(sc, scale_off(row, cc, nb));
    float4* dst = reinterpret_cast<float4*>(w + row * in + cc * 32);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      dst[i] = make_float4(s * (q4_nib(d[i], 0, false) - 8.0f), s * (q4_nib(d[i], 1, false) - 8.0f),
                           s * (q4_nib(d[i], 2, false) - 8.0f), s * (q4_nib(d[i], 3, false) - 8.0f));
      dst[4 + i] = make_float4(s * (q4_nib(d[i], 0, true) - 8.0f), s * (q4_nib(d[i], 1, true) - 8.0f),
                               s * (q4_nib(d[i], 2, true) - 8.0f), s * (q4_nib(d[i], 3, true) - 8.0f));
    }
  }
}

hipError_t launch_dequant(const Weight& w, float* out, hipStream_t stream) {
  const int64_t rowbytes = w.format == RQ_Q8_0 ? w.in : w.in / 2;
  const int64_t nchunk = w.out * (rowbytes / 16);
  dim3 grid((unsigned)((nchunk + 255) / 256));
  if (w.format == RQ_Q8_0)
    hipLaunchKernelGGL((dequant_kernel<RQ_Q8_0, float>), grid, dim3(256), 0, stream, w.q,
                       static_cast<const float*>(w.scales), out, w.out, w.in);
  else if (w.scale_dtype == RQ_F16)
    hipLaunchKernelGGL((dequant_kernel<RQ_Q4_0, uint16_t>), grid, dim3(256), 0, stream, w.q,
                       static_cast<const uint16_t*>(w.scales), out, w.out, w.in);
  else
    hipLaunchKernelGGL((dequant_kernel<RQ_Q4_0, float>), grid, dim3(256), 0, stream, w.q,
                       static_cast<const float*>(w.scales), out, w.out, w.in);
  return hipGetLastError();
}

}  // namespace rq
