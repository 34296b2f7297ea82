// gemm_i8.hip — int8-activation GEMM on CDNA4 int8 MFMA (prefill regime).
//
// y[t, o] = sum_b ws[o, b] * xs[t, b] * (dot_b(code[o], xq[t]) [- 8 xsum[t, b]])
// qmatmul-i8-gemm! (raster/quant/kernels_k.clj:357-370) for Q8_0 weights and
// the int-activation Q4_0 form of qmatmul-q4-composable
// (raster/quant/kernels.clj:140-184), with activations from
// rq_quantize_act_i8. v_mfma_i32_16x16x32_i8 takes one 32-element block per
// instruction, so the integer block dot is exact; each block's 16 x 16 int32
// tile is then scaled by ws[o, b] * xs[t, b] and added to f32 accumulators
// (Raster adds in double; the f32 sum differs from it by rounding only).
//
// Operands: A = weights (16 rows o x 32 k, one chunk of the chunked layout,
// 8 bytes per lane, one coalesced load), B = activations (32 k x 16 rows t,
// 8 bytes per lane from row-major xq). Lane (t = lane % 16, q = lane / 16)
// of the result holds y[t][o0 + 4q .. 4q + 3]: four outputs of one
// activation row, stored together.
//
// Workgroup: 4 waves in a 2 x 2 arrangement over a 64 (o) x 64 (t) tile, each
// wave 2 x 2 MFMA tiles; the next block's operands and scales are loaded
// while the current block's MFMAs and scaling run.
#include "rq_internal.h"

namespace rq {

namespace {

constexpr int kI8Threads = 256;

typedef long i64x1;

}  // namespace

template <int FMT, typename ST>
__global__ __launch_bounds__(kI8Threads) void gemm_i8_kernel(const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                                            const int8_t* __restrict__ xq,
                                                            const float* __restrict__ xs,
                                                            const int32_t* __restrict__ xsum, void* __restrict__ y,
                                                            int M, int K, int N, int npad, int y_dtype,
                                                            int tiles_t) {
  const int nb = K / 32;
  // tile order: the activation tiles of one weight tile adjacent, and each
  // XCD (workgroups are dealt round-robin by id) given a contiguous run
  const int nblk = (int)gridDim.x, bid = (int)blockIdx.x;
  const int xcd = bid & 7, per = nblk >> 3, rem = nblk & 7;
  const int tord = xcd * per + (xcd < rem ? xcd : rem) + (bid >> 3);
  const int tt = tord % tiles_t, to = tord / tiles_t;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, kg = lane >> 4;  // operand row / column, 8-element k group
  const int g_last = npad / 16 - 1;
  // this wave's two weight groups and two activation tiles
  int grp[2], trow[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    grp[i] = min(to * 4 + (wave & 1) * 2 + i, g_last);
    trow[i] = min(tt * 64 + (wave >> 1) * 32 + 16 * i + li, M - 1);  // B operand row of this lane
  }
  constexpr int CB = FMT == RQ_Q8_0 ? 32 : 16;  // code bytes per row and block

  struct Ops {
    uint64_t a[2], b[2];
    f32x4 ws[2];
    float xs[2];
    int xsum[2];
  };
  // block b's operands: weight rows of lane (li) for k group kg, activation
  // row trow for k group kg; the scales of the 4 weight rows this lane's
  // results cover (4 kg .. 4 kg + 3 of the group) and of its activation rows
  auto load = [&](Ops& o, int b) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const uint8_t* ch = q + ((int64_t)grp[i] * nb + b) * (16 * CB) + li * CB;
      if (FMT == RQ_Q8_0) {
        o.a[i] = *reinterpret_cast<const uint64_t*>(ch + 8 * kg);
      } else {
        // k group kg: low nibbles of bytes 0..7 / 8..15, then high nibbles
        const uint64_t w = *reinterpret_cast<const uint64_t*>(ch + 8 * (kg & 1));
        o.a[i] = (w >> (4 * (kg >> 1))) & 0x0F0F0F0F0F0F0F0Full;
      }
      o.b[i] = *reinterpret_cast<const uint64_t*>(xq + (int64_t)trow[i] * K + 32 * b + 8 * kg);
      const ST* s4 = sc + ((int64_t)grp[i] * nb + b) * 16 + 4 * kg;
      if (sizeof(ST) == 4) {
        o.ws[i] = *reinterpret_cast<const f32x4*>(s4);
      } else {
        const u32x2 h = *reinterpret_cast<const u32x2*>(s4);
        o.ws[i] = f32x4{f16_bits_to_f32((uint16_t)(h[0] & 0xFFFFu)), f16_bits_to_f32((uint16_t)(h[0] >> 16)),
                        f16_bits_to_f32((uint16_t)(h[1] & 0xFFFFu)), f16_bits_to_f32((uint16_t)(h[1] >> 16))};
      }
      o.xs[i] = xs[(int64_t)trow[i] * nb + b];
      o.xsum[i] = FMT == RQ_Q4_0 ? xsum[(int64_t)trow[i] * nb + b] : 0;
    }
  };

  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](const Ops& o) {
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x32_i8((i64x1)o.a[i], (i64x1)o.b[j], i32x4{0, 0, 0, 0}, 0,
                                                              0, 0);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int v = FMT == RQ_Q4_0 ? d[e] - 8 * o.xsum[j] : d[e];
          acc[i][j][e] = fmaf((float)v, o.ws[i][e] * o.xs[j], acc[i][j][e]);
        }
      }
  };

  Ops op[2];
  load(op[0], 0);
  for (int b = 0; b < nb; b += 2) {
    load(op[1], min(b + 1, nb - 1));
    compute(op[0]);
    if (b + 1 >= nb) break;
    load(op[0], min(b + 2, nb - 1));
    compute(op[1]);
  }

  // lane (li, kg) holds y[t = row of tile j][o = 16 grp_i + 4 kg + e]
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int t = tt * 64 + (wave >> 1) * 32 + 16 * j + li;
    if (t >= M) continue;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int o0 = (to * 4 + (wave & 1) * 2 + i) * 16 + 4 * kg;
      if (o0 >= N) continue;
      if (o0 + 3 < N && (N & 3) == 0) {
        if (y_dtype == RQ_F32) {
          *reinterpret_cast<f32x4*>(static_cast<float*>(y) + (int64_t)t * N + o0) = acc[i][j];
        } else {
          const uint32_t p0 = pack2_bf16(acc[i][j][0], acc[i][j][1]), p1 = pack2_bf16(acc[i][j][2], acc[i][j][3]);
          *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(y) + (int64_t)t * N + o0) = u32x2{p0, p1};
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          if (o0 + e >= N) break;
          if (y_dtype == RQ_F32)
            static_cast<float*>(y)[(int64_t)t * N + o0 + e] = acc[i][j][e];
          else
            static_cast<uint16_t*>(y)[(int64_t)t * N + o0 + e] = (uint16_t)f32_to_bf16_bits(acc[i][j][e]);
        }
      }
    }
  }
}

template <int FMT, typename ST>
static hipError_t launch_i8_t(const MatmulArgs& a) {
  const int tiles_t = (int)((a.m + 63) / 64), tiles_o = (int)((a.npad / 16 + 3) / 4);
  const int64_t grid = (int64_t)tiles_t * tiles_o;
  if (grid > INT32_MAX) return hipErrorInvalidValue;
  hipExtLaunchKernelGGL((gemm_i8_kernel<FMT, ST>), dim3((unsigned)grid), dim3(kI8Threads), 0, a.stream, a.ev_main[0],
                        a.ev_main[1], 0, a.q, static_cast<const ST*>(a.scales), static_cast<const int8_t*>(a.x),
                        a.ops.act_scale, a.ops.act_sum, a.y, (int)a.m, (int)a.k, (int)a.n, (int)a.npad, a.y_dtype,
                        tiles_t);
  return hipGetLastError();
}

hipError_t launch_gemm_i8(const MatmulArgs& a, int cu_count) {
  (void)cu_count;
  if (a.format == RQ_Q8_0) return launch_i8_t<RQ_Q8_0, float>(a);
  if (a.scale_dtype == RQ_F16) return launch_i8_t<RQ_Q4_0, uint16_t>(a);
  return launch_i8_t<RQ_Q4_0, float>(a);
}

}  // namespace rq
