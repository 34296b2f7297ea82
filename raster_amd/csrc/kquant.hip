// kquant.hip — Raster's K-quant formats (Q4_K, Q6_K) on the device: the q8_K
// activation quantizer, the K-quant GEMV, and dequantization.
//
// Formats (raster/compiler/backend/cpu/quant.clj:78-280, Raster's own layout,
// each weight row its own 256-element super-blocks):
//   Q4_K  x = (da*aq)*q + (db*bq): nibbles q (w[k] low, w[k+16] high per
//         32-sub-block), per super-block f32 da / db, per sub-block 6-bit aq
//         (0..63) and bq (-32..31).
//   Q6_K  x = (ds*sc)*(q - 32): one byte q (0..63) per element, per
//         16-sub-block int8 sc, per super-block f32 ds.
// Resident form: the codes as Raster stores them (row-major), the super-block
// scales per (row, super-block) (Q4_K: da and db side by side), the sub-block
// scales per (row, sub-block) (Q4_K: aq and bq side by side).
//
// Activations are q8_K (quantize-act-q8k, quant.clj:158-176, and its GPU form
// quant-act-q8k-gpu!, raster/quant/kernels_k.clj:93-134): per 256-element
// super-block d = max|x| / 127 and int8 codes, plus per-sub-block sums bsums
// (32-element for Q4_K, 16 for Q6_K).
//
// The GEMV is the K dot of qmatmul-q4k-dp4a! / qmatmul-q6k-dp4a!
// (kernels_k.clj:186-297): per super-block
//   Q4_K  d_act * sum_j [(da*aq_j) * dot_j + (db*bq_j) * bsum_j]
//   Q6_K  ds * d_act * sum_j sc_j * (dot_j - 32 * bsum_j)
// with the sub-block dots exact in int32 (v_dot4 over packed bytes: nibbles
// and 6-bit codes are non-negative int8). The terms are added in f32 (Raster
// adds in double). HBM-bound on the codes: a wave takes kKqRows rows at a time,
// its lanes one sub-block each (16 code bytes, one load) strided by 64, the
// activations of up to 4 rows staged in LDS once per workgroup.
#include <algorithm>
#include <atomic>

#include "rq_internal.h"

namespace rq {

namespace {

constexpr int kKqThreads = 256;
// weight rows a wave takes at a time (14336 x 4096, m = 1, cold, rows 1 / 2 /
// 4 / 8: Q4_K 12.1 / 10.3 / 11.3 / 12.7 us, Q6_K 15.7 / 12.5 / 13.8 / 14.4 us;
// m = 4 likewise best at 2)
constexpr int kKqRows = 2;

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace

// ---- q8_K activation quantizer: one wave per 256-element super-block, four
// elements per lane; SUB-element sub-block sums over SUB/4 lanes.
template <int SUB>
__global__ __launch_bounds__(kKqThreads) void quantize_act_q8k_kernel(const float* __restrict__ x,
                                                                     int8_t* __restrict__ xq, float* __restrict__ xs,
                                                                     int32_t* __restrict__ bsums, int64_t nsb) {
  const int lane = threadIdx.x & 63;
  const int64_t sb = (int64_t)blockIdx.x * (kKqThreads / 64) + (threadIdx.x >> 6);
  const int64_t b = sb < nsb ? sb : nsb - 1;  // waves past the end reread the last one and store nothing
  const f32x4 v = *reinterpret_cast<const f32x4*>(x + b * 256 + lane * 4);
  float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 64));
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
#pragma unroll
  for (int off = 1; off < SUB / 4; off <<= 1) s += __shfl_xor(s, off, 64);
  if (sb < nsb) {
    *reinterpret_cast<uint32_t*>(xq + b * 256 + lane * 4) = word;
    if (lane == 0) xs[b] = (float)d;
    if (lane % (SUB / 4) == 0) bsums[b * (256 / SUB) + lane / (SUB / 4)] = s;
  }
}

hipError_t launch_quantize_act_q8k(const float* x, int64_t m, int64_t in, int sub, int8_t* xq, float* xs,
                                   int32_t* bsums, hipStream_t stream) {
  const int64_t nsb = m * (in / 256);
  if (nsb == 0) return hipSuccess;
  const dim3 grid((unsigned)((nsb + kKqThreads / 64 - 1) / (kKqThreads / 64)));
  if (sub == 32)
    hipLaunchKernelGGL((quantize_act_q8k_kernel<32>), grid, dim3(kKqThreads), 0, stream, x, xq, xs, bsums, nsb);
  else
    hipLaunchKernelGGL((quantize_act_q8k_kernel<16>), grid, dim3(kKqThreads), 0, stream, x, xq, xs, bsums, nsb);
  return hipGetLastError();
}

// Q6_K codes on the device: each 16-code sub-block packed into 12 bytes.
// Bytes 0..7: byte j holds code j (low nibble) and code j + 8 (high nibble),
// their low 4 bits; bytes 8..11: byte j holds bits 4..5 of codes j, j + 4,
// j + 8, j + 12 in its bit pairs 0, 1, 2, 3. p0, p1, p2 are bytes 0..3, 4..7,
// 8..11 as little-endian words; the result holds codes 4 k .. 4 k + 3 as
// bytes in word k.
__device__ __forceinline__ u32x4 unpack_q6k(uint32_t p0, uint32_t p1, uint32_t p2) {
  return u32x4{(p0 & 0x0F0F0F0Fu) | ((p2 & 0x03030303u) << 4), (p1 & 0x0F0F0F0Fu) | (((p2 >> 2) & 0x03030303u) << 4),
               ((p0 >> 4) & 0x0F0F0F0Fu) | (((p2 >> 4) & 0x03030303u) << 4),
               ((p1 >> 4) & 0x0F0F0F0Fu) | (((p2 >> 6) & 0x03030303u) << 4)};
}

// ---- K-quant GEMV: y[t][o] for MT activation rows t. FMT RQ_Q4_K / RQ_Q6_K.
// LDS: xq[MT][K] codes, bsums[MT][K/SUB], xs[MT][K/256].
template <int FMT, int MT, int D>
__global__ __launch_bounds__(kKqThreads) void kquant_gemv_kernel(
    const uint8_t* __restrict__ wq, const void* __restrict__ sup, const void* __restrict__ subsc,
    const int8_t* __restrict__ xq, const float* __restrict__ xs, const int32_t* __restrict__ bsums,
    void* __restrict__ y, int M, int K, int N, int y_dtype) {
  constexpr int SUB = FMT == RQ_Q4_K ? 32 : 16;  // elements per sub-block (16 code bytes either way)
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int nsub = K / SUB, nsb = K / 256;
  int8_t* lx = reinterpret_cast<int8_t*>(smem);
  int32_t* lb = reinterpret_cast<int32_t*>(smem + MT * K);
  float* ls = reinterpret_cast<float*>(smem + MT * K + MT * nsub * 4);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // ---- this wave's work: row groups gi = 0 .. ng-1 (rows o0 = 4 (gw + gi
  // nwaves) ..), each swept in nit steps (lane: sub-block lane + 64 si). The
  // steps stream through a D-step register ring of raw code and scale bits
  // across row groups (steps padded to whole ring turns); nothing converts or
  // tests loaded bits before the step computes, and refills are unconditional
  // at clamped addresses, so the compiler keeps D steps of loads in flight.
  // D = 1 measured best (14336 x 4096, m = 1: Q4_K 11.7 / 12.2 / 13.5 /
  // 15.5 us and Q6_K 16.9 / 17.4 / 18.9 / 19.0 us at D = 1 .. 4; before this
  // stream, loading each step only when it was computed: 15.0 and 16.3 us).
  const int gw = (int)blockIdx.x * (kKqThreads / 64) + wave, nwaves = (int)gridDim.x * (kKqThreads / 64);
  const int ngrp = (N + kKqRows - 1) / kKqRows;
  const int ng = gw < ngrp ? (ngrp - 1 - gw) / nwaves + 1 : 0;
  const int nit = (nsub + 63) / 64, nitp = (nit + D - 1) / D * D;
  // code bytes per row: K / 2 (Q4_K nibbles), 3 K / 4 (Q6_K, 12 bytes per 16-code sub-block)
  const int64_t row_bytes = FMT == RQ_Q4_K ? K / 2 : K / 4 * 3;
  struct Slot {
    u32x4 w[kKqRows];
    uint32_t a[kKqRows], b[kKqRows], c[kKqRows];  // Q4_K: da, db bits, aq | bq << 8; Q6_K: ds bits, sc
  };
  Slot ring[D];
  auto load = [&](int slot, int gi, int si) {
    if (gi >= ng) {  // past the end: the last step again
      gi = ng - 1;
      si = nitp - 1;
    }
    const int o0 = (gw + gi * nwaves) * kKqRows;
    const int sb = min(lane + 64 * min(si, nit - 1), nsub - 1);
#pragma unroll
    for (int r = 0; r < kKqRows; r++) {
      const int o = min(o0 + r, N - 1);
      if (FMT == RQ_Q4_K) {
        ring[slot].w[r] = *reinterpret_cast<const u32x4*>(wq + (int64_t)o * row_bytes + sb * 16);
      } else {  // 12 bytes, unpacked when the step computes
        const uint32_t* p = reinterpret_cast<const uint32_t*>(wq + (int64_t)o * row_bytes + sb * 12);
        ring[slot].w[r] = u32x4{p[0], p[1], p[2], 0u};
      }
      if (FMT == RQ_Q4_K) {
        const u32x2 d2 = static_cast<const u32x2*>(sup)[(int64_t)o * nsb + sb / 8];
        ring[slot].a[r] = d2[0];
        ring[slot].b[r] = d2[1];
        ring[slot].c[r] = static_cast<const uint16_t*>(subsc)[(int64_t)o * nsub + sb];
      } else {
        ring[slot].a[r] = static_cast<const uint32_t*>(sup)[(int64_t)o * nsb + sb / 16];
        ring[slot].c[r] = (uint32_t)(uint8_t)static_cast<const int8_t*>(subsc)[(int64_t)o * nsub + sb];
      }
    }
  };
  int lg = 0, ls_ = 0;
  auto advance = [&](int& gi, int& si) {
    if (++si == nitp) {
      si = 0;
      ++gi;
    }
  };
  // the first weight loads go out before the activations are staged, so
  // their latency overlaps the staging (14336 x 4096, m = 1, cold: Q4_K
  // 11.65 -> 11.19 us; Q6_K unchanged at 16.9)
  if (ng > 0) {
#pragma unroll
    for (int i = 0; i < D; i++) {
      load(i, lg, ls_);
      advance(lg, ls_);
    }
  }

  // stage the activations (rows past M as zeros)
  for (int i = tid; i < MT * K / 16; i += kKqThreads) {
    const int t = i / (K / 16);
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (t < M) v = reinterpret_cast<const u32x4*>(xq + (int64_t)t * K)[i % (K / 16)];
    reinterpret_cast<u32x4*>(lx)[i] = v;
  }
  for (int i = tid; i < MT * nsub; i += kKqThreads) lb[i] = i / nsub < M ? bsums[(int64_t)i] : 0;
  for (int i = tid; i < MT * nsb; i += kKqThreads) ls[i] = i / nsb < M ? xs[(int64_t)i] : 0.0f;
  __syncthreads();
  if (ng == 0) return;  // wave-uniform; no barrier follows

  float acc[kKqRows][MT];
#pragma unroll
  for (int r = 0; r < kKqRows; r++)
#pragma unroll
    for (int t = 0; t < MT; t++) acc[r][t] = 0.0f;
  for (int gi = 0; gi < ng; gi++) {
    for (int si0 = 0; si0 < nitp; si0 += D) {
#pragma unroll
      for (int i = 0; i < D; i++) {
        const int si = si0 + i;
        const Slot cur = ring[i];
        load(i, lg, ls_);
        advance(lg, ls_);
        const int sraw = lane + 64 * si;
        if (si < nit) {  // wave-uniform: padding steps compute nothing
          const bool live = sraw < nsub;
          const int s = min(sraw, nsub - 1);
          float f0[kKqRows], f1[kKqRows];
#pragma unroll
          for (int r = 0; r < kKqRows; r++) {
            if (FMT == RQ_Q4_K) {
              f0[r] = __uint_as_float(cur.a[r]) * (float)(int)(cur.c[r] & 0xFFu);        // da * aq
              f1[r] = __uint_as_float(cur.b[r]) * (float)(int)(int8_t)(cur.c[r] >> 8);   // db * bq
            } else {
              f0[r] = __uint_as_float(cur.a[r]) * (float)(int)(int8_t)cur.c[r];          // ds * sc
              f1[r] = 0.0f;
            }
          }
          // Q6_K: the rows' 16 codes as bytes, unpacked once for all MT rows
          u32x4 cw[kKqRows];
#pragma unroll
          for (int r = 0; r < kKqRows; r++)
            cw[r] = FMT == RQ_Q6_K ? unpack_q6k(cur.w[r][0], cur.w[r][1], cur.w[r][2]) : cur.w[r];
#pragma unroll
          for (int t = 0; t < MT; t++) {
            const u32x4 xa = reinterpret_cast<const u32x4*>(lx + t * K)[s * SUB / 16];
            const int bs = lb[t * nsub + s];
            const float dact = ls[t * nsb + s * SUB / 256];
            if (FMT == RQ_Q4_K) {
              const u32x4 xb = reinterpret_cast<const u32x4*>(lx + t * K)[s * 2 + 1];
#pragma unroll
              for (int r = 0; r < kKqRows; r++) {
                int dp = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                  dp = __builtin_amdgcn_sdot4((int)(cur.w[r][k] & 0x0F0F0F0Fu), (int)xa[k], dp, false);
                  dp = __builtin_amdgcn_sdot4((int)((cur.w[r][k] >> 4) & 0x0F0F0F0Fu), (int)xb[k], dp, false);
                }
                const float v = fmaf(dact, f0[r] * (float)dp + f1[r] * (float)bs, acc[r][t]);
                acc[r][t] = live ? v : acc[r][t];
              }
            } else {
#pragma unroll
              for (int r = 0; r < kKqRows; r++) {
                int dp = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) dp = __builtin_amdgcn_sdot4((int)cw[r][k], (int)xa[k], dp, false);
                const float v = fmaf(dact * f0[r], (float)(dp - 32 * bs), acc[r][t]);
                acc[r][t] = live ? v : acc[r][t];
              }
            }
          }
        }
      }
    }
    // ---- row group gi: sum the lanes, store
    const int o0 = (gw + gi * nwaves) * kKqRows;
#pragma unroll
    for (int r = 0; r < kKqRows; r++)
#pragma unroll
      for (int t = 0; t < MT; t++) {
        const float v = wave_sum64(acc[r][t]);
        acc[r][t] = 0.0f;
        const int o = o0 + r;
        if (lane == 0 && o < N && t < M) {
          if (y_dtype == RQ_F32)
            static_cast<float*>(y)[(int64_t)t * N + o] = v;
          else
            static_cast<uint16_t*>(y)[(int64_t)t * N + o] = (uint16_t)f32_to_bf16_bits(v);
        }
      }
  }
}
size_t kquant_gemv_lds(int format, int64_t k, int mt) {
  const int64_t sub = format == RQ_Q4_K ? 32 : 16;
  return (size_t)mt * (size_t)(k + 4 * (k / sub) + 4 * (k / 256));
}

template <int FMT, int MT, int D = 1>
static hipError_t launch_kq_t(const Weight& w, const int8_t* xq, const float* xs, const int32_t* bsums, void* y,
                              int y_dtype, int64_t m, int cu_count, hipStream_t stream) {
  auto kernel = &kquant_gemv_kernel<FMT, MT, D>;
  const size_t lds = kquant_gemv_lds(FMT, w.in, MT);
  if (lds > 65536) {
    static std::atomic<uint64_t> attr_set{0};
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev)) return e;
    const uint64_t bit = uint64_t(1) << (dev & 63);
    if (!(attr_set.load(std::memory_order_acquire) & bit)) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
      if (e != hipSuccess) return e;
      attr_set.fetch_or(bit, std::memory_order_acq_rel);
    }
  }
  // a wave per row group, all of them launched at once: at 14336 x 4096,
  // m = 1, cold, Q4_K 10.9 us and Q6_K 17.4 us against 11.1-11.3 / 18.5 with
  // at most 8 waves per CU (each then taking ~2 groups one after another)
  const int64_t groups = (w.out + kKqRows - 1) / kKqRows;
  const int64_t wg = (groups + 3) / 4;
  (void)cu_count;
  hipLaunchKernelGGL(kernel, dim3((unsigned)std::max<int64_t>(wg, 1)), dim3(kKqThreads), (unsigned)lds, stream, w.q,
                     w.scales, w.sub_scales, xq, xs, bsums, y, (int)m, (int)w.in, (int)w.out, y_dtype);
  return hipGetLastError();
}

hipError_t launch_kquant_gemv(const Weight& w, const int8_t* xq, const float* xs, const int32_t* bsums, void* y,
                              int y_dtype, int64_t m, int cu_count, hipStream_t stream) {
  const int64_t nsub = w.in / (w.format == RQ_Q4_K ? 32 : 16), nsb = w.in / 256;
  const size_t ysz = y_dtype == RQ_F32 ? 4 : 2;
  // four activation rows per launch
  for (int64_t t0 = 0; t0 < m; t0 += 4) {
    const int64_t mt = std::min<int64_t>(4, m - t0);
    const int8_t* xq_t = xq + t0 * w.in;
    const float* xs_t = xs + t0 * nsb;
    const int32_t* bs_t = bsums + t0 * nsub;
    void* y_t = static_cast<uint8_t*>(y) + (size_t)(t0 * w.out) * ysz;
    hipError_t e;
    if (w.format == RQ_Q4_K)
      e = mt == 1 ? launch_kq_t<RQ_Q4_K, 1>(w, xq_t, xs_t, bs_t, y_t, y_dtype, mt, cu_count, stream)
                  : launch_kq_t<RQ_Q4_K, 4>(w, xq_t, xs_t, bs_t, y_t, y_dtype, mt, cu_count, stream);
    else
      e = mt == 1 ? launch_kq_t<RQ_Q6_K, 1>(w, xq_t, xs_t, bs_t, y_t, y_dtype, mt, cu_count, stream)
                  : launch_kq_t<RQ_Q6_K, 4>(w, xq_t, xs_t, bs_t, y_t, y_dtype, mt, cu_count, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// ---- dequantization, bitwise as dequant-q4k / dequant-q6k (the products are
// exact in double, one rounding of the sum, one narrowing)
template <int FMT>
__global__ __launch_bounds__(256) void kquant_dequant_kernel(const uint8_t* __restrict__ wq,
                                                            const void* __restrict__ sup,
                                                            const void* __restrict__ subsc, float* __restrict__ out,
                                                            int64_t K, int64_t n) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const int64_t o = e / K, k = e % K, nsb = K / 256;
  if (FMT == RQ_Q4_K) {
    const int64_t s = k / 32, j = k % 32;
    const uint32_t b = wq[o * (K / 2) + s * 16 + (j % 16)];
    const uint32_t q = j < 16 ? (b & 0xFu) : (b >> 4);
    const f32x2 d2 = static_cast<const f32x2*>(sup)[o * nsb + s / 8];
    const uint32_t ab = static_cast<const uint16_t*>(subsc)[o * (K / 32) + s];
    const double a1 = (double)d2[0] * (double)(int)(ab & 0xFFu);
    const double b1 = (double)d2[1] * (double)(int)(int8_t)(ab >> 8);
    out[e] = (float)(a1 * (double)q + b1);
  } else {
    const double a1 = (double)static_cast<const float*>(sup)[o * nsb + k / 256] *
                      (double)static_cast<const int8_t*>(subsc)[o * (K / 16) + k / 16];
    const int64_t s = k / 16, j = k % 16;
    const uint8_t* sbp = wq + o * (K / 4 * 3) + s * 12;
    const uint32_t lo = (sbp[j % 8] >> (j < 8 ? 0 : 4)) & 0xFu, hi = (sbp[8 + j % 4] >> (2 * (j / 4))) & 3u;
    out[e] = (float)(a1 * (double)((int)(lo | (hi << 4)) - 32));
  }
}

hipError_t launch_kquant_dequant(const Weight& w, float* out, hipStream_t stream) {
  const int64_t n = w.out * w.in;
  if ((n + 255) / 256 > INT32_MAX) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (w.format == RQ_Q4_K)
    hipLaunchKernelGGL((kquant_dequant_kernel<RQ_Q4_K>), grid, dim3(256), 0, stream, w.q, w.scales, w.sub_scales,
                       out, w.in, n);
  else
    hipLaunchKernelGGL((kquant_dequant_kernel<RQ_Q6_K>), grid, dim3(256), 0, stream, w.q, w.scales, w.sub_scales,
                       out, w.in, n);
  return hipGetLastError();
}

}  // namespace rq
