// dx.hip — backward-data of the quantized linear:
//   dx[m, i] = sum_o scale[o, i/32] * code[o, i] * dy[m, o]
// qlinear-q8-dx (raster/quant/train.clj:110-137), the pullback Raster emits for
// qlinear-q8 (train.clj:143-155), over the same resident chunked weight (Q8_0,
// or Q4_0 with code = nibble - 8). Per term the weight w = scale * code and
// the product w * dy are rounded to f32 as Raster does; the sum runs in f32
// (Raster: double).
//
// The reduction runs over `out`, across the 16-row chunks of one 32-column
// block b. A wave owns a block b and a slice of the 16-row groups: per chunk,
// one coalesced load (lane l: row l / 4 of the chunk, 8 columns 8 (l % 4) ..)
// and the row's scale; each lane keeps 8 columns x MB rows of dy in registers
// over all of its slice, then the 16 lanes of a column quad are summed by
// shuffles. Slices write partial sums that a second kernel adds in slice
// order (deterministic); with one slice the first kernel writes dx.
// HBM-bound for small m (the weight is read once per MB rows of dy).
#include <algorithm>

#include "rq_internal.h"

namespace rq {

namespace {

constexpr int kDxThreads = 256;
constexpr int kDxRows = 4;  // dy rows per pass over the weight (MB)

}  // namespace

template <int FMT, typename ST>
__global__ __launch_bounds__(kDxThreads) void dx_kernel(const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                                       const float* __restrict__ dy, float* __restrict__ out_buf,
                                                       int M, int K, int N, int npad, int gps) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int nb = K / 32, ngroups = npad / 16;
  const int b = (int)blockIdx.x * (kDxThreads / 64) + wave;  // column block
  if (b >= nb) return;                                        // wave-uniform, no barrier follows
  const int s = (int)blockIdx.y;                              // slice of row groups
  const int g0 = s * gps, g1 = min(ngroups, g0 + gps);
  const int r = lane >> 2, p = lane & 3;  // chunk row, column quad
  float* dst = gridDim.y == 1 ? out_buf : out_buf + (int64_t)s * M * K;
  for (int m0 = 0; m0 < M; m0 += kDxRows) {
    float acc[kDxRows][8];
#pragma unroll
    for (int mi = 0; mi < kDxRows; mi++)
#pragma unroll
      for (int k = 0; k < 8; k++) acc[mi][k] = 0.0f;
    for (int g = g0; g < g1; g++) {
      const int64_t chunk = (int64_t)g * nb + b;
      u32x2 v;
      if (FMT == RQ_Q8_0)
        v = *reinterpret_cast<const u32x2*>(q + chunk * 512 + r * 32 + 8 * p);
      else
        v = *reinterpret_cast<const u32x2*>(q + chunk * 256 + r * 16 + 8 * (p & 1));
      const float sv = load_scale<ST>(sc, chunk * 16 + r);
      const int o = 16 * g + r;
      float dyv[kDxRows];
#pragma unroll
      for (int mi = 0; mi < kDxRows; mi++) {
        const int m = min(m0 + mi, M - 1);
        const float t = dy[(int64_t)m * N + min(o, N - 1)];
        dyv[mi] = o < N ? t : 0.0f;  // padded rows: no term (their codes and scales are zero)
      }
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const uint32_t word = v[k >> 2];
        int code;
        if (FMT == RQ_Q8_0)
          code = (int)(int8_t)(word >> (8 * (k & 3)));
        else
          code = (int)((word >> (8 * (k & 3) + (p >= 2 ? 4 : 0))) & 0xFu) - 8;
        const float w = sv * (float)code;
#pragma unroll
        for (int mi = 0; mi < kDxRows; mi++) acc[mi][k] += w * dyv[mi];
      }
    }
    // sum the 16 rows of the chunk (lanes with the same column quad p)
#pragma unroll
    for (int mi = 0; mi < kDxRows; mi++)
#pragma unroll
      for (int k = 0; k < 8; k++) {
        float t = acc[mi][k];
        t += __shfl_xor(t, 4, 64);
        t += __shfl_xor(t, 8, 64);
        t += __shfl_xor(t, 16, 64);
        t += __shfl_xor(t, 32, 64);
        acc[mi][k] = t;
      }
    if (lane < 4) {
      // Q4_0 quads: p = 0, 1 hold elements 8p..8p+7, p = 2, 3 elements 16 + 8(p-2)..
      const int col = FMT == RQ_Q8_0 ? 8 * p : (p < 2 ? 8 * p : 16 + 8 * (p - 2));
#pragma unroll
      for (int mi = 0; mi < kDxRows; mi++) {
        const int m = m0 + mi;
        if (m >= M) break;
        float* d = dst + (int64_t)m * K + 32 * b + col;
        *reinterpret_cast<f32x4*>(d) = f32x4{acc[mi][0], acc[mi][1], acc[mi][2], acc[mi][3]};
        *reinterpret_cast<f32x4*>(d + 4) = f32x4{acc[mi][4], acc[mi][5], acc[mi][6], acc[mi][7]};
      }
    }
  }
}

// dx = sum over slices of the partial sums, in slice order (the slices'
// loads go out four at a time; the adds stay in order)
__global__ __launch_bounds__(256) void dx_reduce_kernel(const float* __restrict__ part, float* __restrict__ dx,
                                                       int64_t n4, int slices) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n4) return;
  const f32x4* p = reinterpret_cast<const f32x4*>(part);
  f32x4 t = p[e];
  int s = 1;
  for (; s + 3 < slices; s += 4) {
    const f32x4 a = p[(int64_t)s * n4 + e], b = p[(int64_t)(s + 1) * n4 + e];
    const f32x4 c = p[(int64_t)(s + 2) * n4 + e], d = p[(int64_t)(s + 3) * n4 + e];
    t += a;
    t += b;
    t += c;
    t += d;
  }
  for (; s < slices; s++) t += p[(int64_t)s * n4 + e];
  reinterpret_cast<f32x4*>(dx)[e] = t;
}

int dx_slices(int64_t in, int64_t npad, int cu_count) {
  // about 8 waves per CU: column blocks times slices of the row groups
  const int64_t nb = in / 32, ngroups = npad / 16;
  const int64_t want = (int64_t)cu_count * 8;
  return (int)std::max<int64_t>(1, std::min<int64_t>(ngroups, (want + nb - 1) / nb));
}

template <int FMT, typename ST>
static hipError_t launch_dx_t(const Weight& w, const float* dy, float* dx, int64_t m, float* part, int slices,
                              hipStream_t stream) {
  const int64_t nb = w.in / 32, ngroups = w.npad / 16;
  const int gps = (int)((ngroups + slices - 1) / slices);
  const dim3 grid((unsigned)((nb + 3) / 4), (unsigned)slices);
  hipLaunchKernelGGL((dx_kernel<FMT, ST>), grid, dim3(kDxThreads), 0, stream, w.q, static_cast<const ST*>(w.scales),
                     dy, slices == 1 ? dx : part, (int)m, (int)w.in, (int)w.out, (int)w.npad, gps);
  if (hipError_t e = hipGetLastError()) return e;
  if (slices > 1) {
    const int64_t n4 = m * w.in / 4;
    hipLaunchKernelGGL(dx_reduce_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, stream, part, dx, n4,
                       slices);
  }
  return hipGetLastError();
}

hipError_t launch_dx(const Weight& w, const float* dy, float* dx, int64_t m, float* part, int slices,
                     hipStream_t stream) {
  if (w.format == RQ_Q8_0) return launch_dx_t<RQ_Q8_0, float>(w, dy, dx, m, part, slices, stream);
  if (w.scale_dtype == RQ_F16) return launch_dx_t<RQ_Q4_0, uint16_t>(w, dy, dx, m, part, slices, stream);
  return launch_dx_t<RQ_Q4_0, float>(w, dy, dx, m, part, slices, stream);
}

}  // namespace rq
