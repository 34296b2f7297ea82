// gemv.hip — decode-regime (m <= 16) block-quantized GEMV for gfx950.
//
// y[m, o] = sum_b scale[o, b] * sum_{k in block b} code[o, k] * x[m, k]
// (the staged form of qlinear-q8, raster/quant/train.clj:77-108: the f32 scale
// multiplies the f32 block partial instead of every element; the product of
// an integer code and x is exact, so the per-element dequantized weight is the
// same number, only the summation order differs).
//
// HBM-bound. Mapping: one wave owns ROWS consecutive output rows; its 64 lanes
// stride along K in 16-byte chunks (Q8: 16 codes = half a block, Q4: 16 bytes =
// one 32-block). A group of G wave-steps issues every 128-bit load of codes and
// scales before any arithmetic, so each lane keeps G*ROWS*16 bytes in flight.
// x is read through L1/L2 (it is shared by every wave). Lane partials are
// reduced across the wave at the end.
#include "rq_internal.h"

namespace rq {

// Loads N consecutive activations starting at element `off` as f32.
template <int XT, int N>
__device__ __forceinline__ void load_x(const void* x, int64_t off, float* out) {
  if (XT == RQ_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + off);
#pragma unroll
    for (int i = 0; i < N / 4; i++) {
      float4 v = p[i];
      out[4 * i + 0] = v.x;
      out[4 * i + 1] = v.y;
      out[4 * i + 2] = v.z;
      out[4 * i + 3] = v.w;
    }
  } else {
    const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + off);
#pragma unroll
    for (int i = 0; i < N / 8; i++) {
      uint4 v = p[i];
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        out[8 * i + 2 * j] = __uint_as_float(w[j] << 16);
        out[8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
      }
    }
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int FMT, typename ST, int XT, int MT, int ROWS, int G>
__global__ __launch_bounds__(256) void gemv_kernel(const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                                  const void* __restrict__ x, void* __restrict__ y, int M,
                                                  int K, int N, int y_dtype) {
  constexpr int EPC = FMT == RQ_Q8_0 ? 16 : 32;  // weight elements per 16-byte chunk
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * ROWS;
  if (row0 >= N) return;  // wave-uniform
  const int nb = K / 32;
  const int64_t rowbytes = FMT == RQ_Q8_0 ? (int64_t)K : (int64_t)K / 2;
  const int nchunks = (int)(rowbytes / 16);

  float acc[MT][ROWS];
#pragma unroll
  for (int m = 0; m < MT; m++)
#pragma unroll
    for (int r = 0; r < ROWS; r++) acc[m][r] = 0.0f;

  for (int c0 = 0; c0 < nchunks; c0 += 64 * G) {
    uint4 raw[G][ROWS];
    float s[G][ROWS];
#pragma unroll
    for (int g = 0; g < G; g++) {
      const int c = c0 + g * 64 + lane;
#pragma unroll
      for (int r = 0; r < ROWS; r++) {
        const int row = row0 + r;
        if (c < nchunks && row < N) {
          const int64_t off = FMT == RQ_Q8_0 ? code_off<FMT>(row, c / 2, nb) + 16 * (c % 2) : code_off<FMT>(row, c, nb);
          raw[g][r] = *reinterpret_cast<const uint4*>(q + off);
          s[g][r] = load_scale<ST>(sc, scale_off(row, FMT == RQ_Q8_0 ? c / 2 : c, nb));
        } else {
          raw[g][r] = make_uint4(0, 0, 0, 0);
          s[g][r] = 0.0f;
        }
      }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
      const int c = c0 + g * 64 + lane;
      if (c >= nchunks) continue;
      const int64_t k0 = (int64_t)c * EPC;
      // decode the chunk of every row once; reused for all m
      float w[ROWS][EPC];
#pragma unroll
      for (int r = 0; r < ROWS; r++) {
        const uint32_t d[4] = {raw[g][r].x, raw[g][r].y, raw[g][r].z, raw[g][r].w};
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int j = 0; j < 4; j++) {
            if (FMT == RQ_Q8_0) {
              w[r][4 * i + j] = q8_code(d[i], j);
            } else {
              w[r][4 * i + j] = q4_nib(d[i], j, false);
              w[r][16 + 4 * i + j] = q4_nib(d[i], j, true);
            }
          }
      }
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if (m < M) {
        float xv[EPC];
        load_x<XT, EPC>(x, (int64_t)m * K + k0, xv);
        float xs = 0.0f;
        if (FMT == RQ_Q4_0) {
#pragma unroll
          for (int e = 0; e < EPC; e++) xs += xv[e];
        }
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
          float p = 0.0f;
#pragma unroll
          for (int e = 0; e < EPC; e++) p = fmaf(w[r][e], xv[e], p);
          if (FMT == RQ_Q4_0) p = fmaf(-8.0f, xs, p);  // zero-point 8
          acc[m][r] = fmaf(s[g][r], p, acc[m][r]);
        }
        }
      }
    }
  }

#pragma unroll
  for (int m = 0; m < MT; m++) {
    if (m < M) {
#pragma unroll
      for (int r = 0; r < ROWS; r++) {
        const float v = wave_sum(acc[m][r]);
        const int row = row0 + r;
        if (lane == 0 && row < N) {
          if (y_dtype == RQ_F32)
            static_cast<float*>(y)[(int64_t)m * N + row] = v;
          else
            static_cast<uint16_t*>(y)[(int64_t)m * N + row] = (uint16_t)f32_to_bf16_bits(v);
        }
      }
    }
  }
}

template <int FMT, typename ST, int XT, int MT>
static hipError_t launch_t(const MatmulArgs& a) {
  constexpr int ROWS = FMT == RQ_Q8_0 ? 4 : 2;
  constexpr int G = FMT == RQ_Q8_0 ? 4 : 4;
  const int rows_per_block = 4 * ROWS;
  dim3 grid((unsigned)((a.n + rows_per_block - 1) / rows_per_block));
  hipLaunchKernelGGL((gemv_kernel<FMT, ST, XT, MT, ROWS, G>), grid, dim3(256), 0, a.stream, a.q,
                     static_cast<const ST*>(a.scales), a.x, a.y, (int)a.m, (int)a.k, (int)a.n, a.y_dtype);
  return hipGetLastError();
}

template <int FMT, typename ST, int XT>
static hipError_t launch_m(const MatmulArgs& a) {
  if (a.m <= 1) return launch_t<FMT, ST, XT, 1>(a);
  if (a.m <= 2) return launch_t<FMT, ST, XT, 2>(a);
  if (a.m <= 4) return launch_t<FMT, ST, XT, 4>(a);
  if (a.m <= 8) return launch_t<FMT, ST, XT, 8>(a);
  return launch_t<FMT, ST, XT, 16>(a);
}

template <int FMT, typename ST>
static hipError_t launch_x(const MatmulArgs& a) {
  return a.x_dtype == RQ_F32 ? launch_m<FMT, ST, RQ_F32>(a) : launch_m<FMT, ST, RQ_BF16>(a);
}

hipError_t launch_gemv(const MatmulArgs& a) {
  if (a.format == RQ_Q8_0) return launch_x<RQ_Q8_0, float>(a);
  if (a.scale_dtype == RQ_F16) return launch_x<RQ_Q4_0, uint16_t>(a);
  return launch_x<RQ_Q4_0, float>(a);
}

}  // namespace rq
