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
// 8 bytes per lane, one coalesced load), B = activations (32 k x 16 rows t).
// A packing pass first rewrites xq / xs / xsum fragment-major: per 16-row
// tile and block, the 512 code bytes in operand-lane order, then the 16 rows'
// xs and xsum (640 bytes), so every activation load is contiguous (row-major
// fragments would touch 16 cache lines per load). Lane (t = lane % 16,
// q = lane / 16) of the result holds y[t][o0 + 4q .. 4q + 3]: four outputs of
// one activation row, stored together.
//
// Workgroup: 4 waves in a 2 x 2 arrangement, each wave TO x TT MFMA tiles
// (16 rows each along o and t); a ring of R blocks keeps the loads of the next
// R - 1 blocks in flight while a block's MFMAs and scaling run.
#include "rq_internal.h"

namespace rq {

namespace {

constexpr int kI8Threads = 256;
// per-wave tile along t (16-row MFMA tiles) and blocks in flight; the tile
// along o is chosen per shape (launch_gemm_i8)
constexpr int kI8Tt = 4, kI8Ring = 4;

typedef long i64x1;

}  // namespace

constexpr int kI8Frag = 640;  // packed bytes per (16-row tile, block)

// Fragment-major copy of int8 activations: one thread per (tile, block, lane):
// the 8 codes of row 16 tile + lane % 16, k group lane / 16, then (lanes < 16)
// the row's xs and xsum. Rows past M are zero.
__global__ __launch_bounds__(256) void pack_i8_kernel(const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                     const int32_t* __restrict__ xsum, uint8_t* __restrict__ xp,
                                                     int M, int K, int64_t nfrag) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t f = i >> 6;
  if (f >= nfrag) return;
  const int lane = (int)(i & 63), nb = K / 32;
  const int64_t tile = f / nb;
  const int b = (int)(f % nb);
  const int64_t t = tile * 16 + (lane & 15);
  uint8_t* dst = xp + f * kI8Frag;
  u32x2 v = u32x2{0u, 0u};
  if (t < M) v = *reinterpret_cast<const u32x2*>(xq + t * K + 32 * b + 8 * (lane >> 4));
  *reinterpret_cast<u32x2*>(dst + lane * 8) = v;
  if (lane < 16) {
    reinterpret_cast<float*>(dst + 512)[lane] = t < M ? xs[t * nb + b] : 0.0f;
    reinterpret_cast<int32_t*>(dst + 576)[lane] = t < M && xsum ? xsum[t * nb + b] : 0;
  }
}

template <int FMT, typename ST, int TO, int TT, int R>
__global__ __launch_bounds__(kI8Threads) void gemm_i8_kernel(const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                                            const uint8_t* __restrict__ xp, void* __restrict__ y,
                                                            int M, int K, int N, int npad, int y_dtype,
                                                            int tiles_t) {
  constexpr int BO = 2 * 16 * TO, BT = 2 * 16 * TT;  // workgroup tile: 2 x 2 waves
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
  const int o_base = to * BO + (wave & 1) * 16 * TO, t_base = tt * BT + (wave >> 1) * 16 * TT;
  // this wave's weight groups and (clamped) packed activation tiles
  const int t_last = (M + 15) / 16 - 1;
  int grp[TO];
  const uint8_t* xt[TT];
#pragma unroll
  for (int i = 0; i < TO; i++) grp[i] = min(o_base / 16 + i, g_last);
#pragma unroll
  for (int j = 0; j < TT; j++) xt[j] = xp + (int64_t)min(t_base / 16 + j, t_last) * nb * kI8Frag;
  constexpr int CB = FMT == RQ_Q8_0 ? 32 : 16;  // code bytes per row and block

  struct Ops {
    uint64_t a[TO], b[TT];
    f32x4 ws[TO];
    float xs[TT];
    int xsum[TT];
  };
  // block b's operands: weight rows of lane li for k group kg, activation row
  // trow for k group kg, the scales of the 4 weight rows this lane's results
  // cover (4 kg .. 4 kg + 3 of the group) and of its activation rows
  auto load = [&](Ops& o, int b) {
#pragma unroll
    for (int i = 0; i < TO; i++) {
      const uint8_t* ch = q + ((int64_t)grp[i] * nb + b) * (16 * CB) + li * CB;
      if (FMT == RQ_Q8_0) {
        o.a[i] = *reinterpret_cast<const uint64_t*>(ch + 8 * kg);
      } else {
        // k group kg: low nibbles of bytes 0..7 / 8..15, then high nibbles
        const uint64_t w = *reinterpret_cast<const uint64_t*>(ch + 8 * (kg & 1));
        o.a[i] = (w >> (4 * (kg >> 1))) & 0x0F0F0F0F0F0F0F0Full;
      }
      const ST* s4 = sc + ((int64_t)grp[i] * nb + b) * 16 + 4 * kg;
      if (sizeof(ST) == 4) {
        o.ws[i] = *reinterpret_cast<const f32x4*>(s4);
      } else {
        const u32x2 h = *reinterpret_cast<const u32x2*>(s4);
        o.ws[i] = f32x4{f16_bits_to_f32((uint16_t)(h[0] & 0xFFFFu)), f16_bits_to_f32((uint16_t)(h[0] >> 16)),
                        f16_bits_to_f32((uint16_t)(h[1] & 0xFFFFu)), f16_bits_to_f32((uint16_t)(h[1] >> 16))};
      }
    }
#pragma unroll
    for (int j = 0; j < TT; j++) {
      const uint8_t* fr = xt[j] + (int64_t)b * kI8Frag;
      o.b[j] = *reinterpret_cast<const uint64_t*>(fr + lane * 8);
      o.xs[j] = reinterpret_cast<const float*>(fr + 512)[li];
      o.xsum[j] = FMT == RQ_Q4_0 ? reinterpret_cast<const int32_t*>(fr + 576)[li] : 0;
    }
  };

  f32x4 acc[TO][TT];
#pragma unroll
  for (int i = 0; i < TO; i++)
#pragma unroll
    for (int j = 0; j < TT; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](const Ops& o) {
#pragma unroll
    for (int i = 0; i < TO; i++)
#pragma unroll
      for (int j = 0; j < TT; j++) {
        const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x32_i8((i64x1)o.a[i], (i64x1)o.b[j], i32x4{0, 0, 0, 0}, 0,
                                                              0, 0);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int v = FMT == RQ_Q4_0 ? d[e] - 8 * o.xsum[j] : d[e];
          acc[i][j][e] = fmaf((float)v, o.ws[i][e] * o.xs[j], acc[i][j][e]);
        }
      }
  };

  // a ring of R blocks: block b computes from slot b % R while the loads of
  // blocks b + 1 .. b + R - 1 are in flight (loads past the last block reread
  // it and are not used)
  Ops op[R];
#pragma unroll
  for (int u = 0; u < R - 1; u++) load(op[u], min(u, nb - 1));
  for (int b0 = 0; b0 < nb; b0 += R) {
#pragma unroll
    for (int u = 0; u < R; u++) {
      const int b = b0 + u;
      if (b >= nb) break;
      load(op[(u + R - 1) % R], min(b + R - 1, nb - 1));
      compute(op[u]);
    }
  }

  // lane (li, kg) holds y[t = row li of tile j][o = 16 grp_i + 4 kg + e]
#pragma unroll
  for (int j = 0; j < TT; j++) {
    const int t = t_base + 16 * j + li;
    if (t >= M) continue;
#pragma unroll
    for (int i = 0; i < TO; i++) {
      const int o0 = o_base + 16 * i + 4 * kg;
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

template <int FMT, typename ST, int TO, int TT, int R>
static hipError_t launch_i8_t(const MatmulArgs& a) {
  constexpr int BO = 32 * TO, BT = 32 * TT;
  const int tiles_t = (int)((a.m + BT - 1) / BT), tiles_o = (int)((a.npad + BO - 1) / BO);
  const int64_t grid = (int64_t)tiles_t * tiles_o;
  if (grid > INT32_MAX) return hipErrorInvalidValue;
  // pack (its end is the timing start: see the bf16 GEMM), then the GEMM
  const int64_t nfrag = (a.m + 15) / 16 * (a.k / 32);
  hipExtLaunchKernelGGL(pack_i8_kernel, dim3((unsigned)((nfrag * 64 + 255) / 256)), dim3(256), 0, a.stream, nullptr,
                        a.ev_main[0], 0, static_cast<const int8_t*>(a.x), a.ops.act_scale, a.ops.act_sum,
                        static_cast<uint8_t*>(a.scratch), (int)a.m, (int)a.k, nfrag);
  if (hipError_t e = hipGetLastError()) return e;
  hipExtLaunchKernelGGL((gemm_i8_kernel<FMT, ST, TO, TT, R>), dim3((unsigned)grid), dim3(kI8Threads), 0, a.stream,
                        nullptr, a.ev_main[1], 0, a.q, static_cast<const ST*>(a.scales),
                        static_cast<const uint8_t*>(a.scratch), a.y, (int)a.m, (int)a.k, (int)a.n, (int)a.npad,
                        a.y_dtype, tiles_t);
  return hipGetLastError();
}

// The per-wave tile along o (TO 16-row tiles, TT = 4 along t): the kernel
// holds two workgroups per CU, and a grid that needs a second, partial round
// leaves CUs idle. TO in {2, 3, 4} minimizing rounds x TO (the time of a
// round grows with TO). Measured at M = 512, K = 4096, N = 11008 (Q8):
// 32 x 64 tiles 119-134 us (688 workgroups, two rounds), 48 x 64 101 us
// (460, one round), 64 x 64 125 us (344); 64 x 32 and 32 x 32 were slower.
hipError_t launch_gemm_i8(const MatmulArgs& a, int cu_count) {
  const int64_t slots = 2 * (int64_t)cu_count, tiles_t = (a.m + 32 * kI8Tt - 1) / (32 * kI8Tt);
  int best = 2;
  int64_t best_cost = INT64_MAX;
  for (int to = 2; to <= 4; to++) {
    const int64_t wgs = tiles_t * ((a.npad + 32 * to - 1) / (32 * to));
    const int64_t cost = (wgs + slots - 1) / slots * to;
    if (cost < best_cost) best_cost = cost, best = to;
  }
#define RQ_I8(FMT_, ST_)                                                               \
  return best == 2 ? launch_i8_t<FMT_, ST_, 2, kI8Tt, kI8Ring>(a)                      \
         : best == 3 ? launch_i8_t<FMT_, ST_, 3, kI8Tt, kI8Ring>(a)                    \
                     : launch_i8_t<FMT_, ST_, 4, kI8Tt, kI8Ring>(a);
  if (a.format == RQ_Q8_0) { RQ_I8(RQ_Q8_0, float) }
  if (a.scale_dtype == RQ_F16) { RQ_I8(RQ_Q4_0, uint16_t) }
  RQ_I8(RQ_Q4_0, float)
#undef RQ_I8
}

}  // namespace rq
