// gemm_sm.hip — bf16-activation GEMM for 16 < m <= 64: HBM-bound, the weight
// stream must keep many bytes in flight.
//
// y[m, o] = sum_k x[m, k] * W[o, k], W = scale * code dequantized exactly to
// bf16 as in gemm_bf16.hip, f32 accumulation (v_mfma_f32_16x16x32_bf16).
//
// At these m each weight element feeds only m/16 MFMAs, so the kernel is a
// weight stream. The per-wave-weights GEMM keeps the weights WD steps ahead,
// but its activation loads are consumed 3 steps after issue, and loads
// complete in issue order: waiting for an activation load also waits for
// every older weight load, so the weights get ~3 steps of slack whatever WD
// is. Here the activations (the fragment-major copy of pack_x_kernel) come in
// chunks of KC k-steps staged in LDS (double-buffered, one burst of loads per
// chunk, consumed a whole chunk after issue), so the weight ring can be
// WD = 2 KC steps deep. Each wave owns NTW 16-row weight fragments; the 4
// waves of a workgroup cover 64 NTW columns and all of m (MT 16-row tiles).
// K may be cut into ks slices (grid.y) whose f32 partial sums a second kernel
// adds in slice order (deterministic), for more waves in flight.
#include <algorithm>

#include "rq_internal.h"

namespace rq {

namespace {

struct WCodesSm {
  u32x2 v;
  uint32_t s;  // scale bits, converted at dequantization
};

template <int FMT, typename ST>
__device__ __forceinline__ void load_wc(WCodesSm& c, const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                        int64_t chunk, int fr, int fg) {
  if (FMT == RQ_Q8_0)
    c.v = *reinterpret_cast<const u32x2*>(q + chunk * 512 + fr * 32 + 8 * fg);
  else
    c.v = *reinterpret_cast<const u32x2*>(q + chunk * 256 + fr * 16 + 8 * (fg & 1));
  c.s = load_scale_bits<ST>(sc, chunk * 16 + fr);
}

// 8 bf16 of the lane's fragment share: exact f32 scale * code, one RNE
// rounding (the dequant of gemm_bf16.hip)
template <int FMT, typename ST>
__device__ __forceinline__ bf16x8 dequant_sm(const WCodesSm& c, int fg) {
  const float s = scale_from_bits<ST>(c.s);
  uint32_t d[2];
  float off;
  if (FMT == RQ_Q8_0) {
    d[0] = c.v[0] ^ 0x80808080u;
    d[1] = c.v[1] ^ 0x80808080u;
    off = -128.0f * s;
  } else {
    const int sh = fg >= 2 ? 4 : 0;
    d[0] = (c.v[0] >> sh) & 0x0F0F0F0Fu;
    d[1] = (c.v[1] >> sh) & 0x0F0F0F0Fu;
    off = -8.0f * s;
  }
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    o[2 * i] = pack2_bf16(fmaf((float)(d[i] & 0xFFu), s, off), fmaf((float)((d[i] >> 8) & 0xFFu), s, off));
    o[2 * i + 1] = pack2_bf16(fmaf((float)((d[i] >> 16) & 0xFFu), s, off), fmaf((float)(d[i] >> 24), s, off));
  }
  return __builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]});
}

}  // namespace

template <int FMT, typename ST, int MT, int NTW, int KC>
__global__ __launch_bounds__(256) void gemm_sm_kernel(const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                                     const uint16_t* __restrict__ xf, void* __restrict__ y,
                                                     float* __restrict__ part, int M, int K, int N, int npad,
                                                     int y_dtype) {
  constexpr int WD = 2 * KC;             // weight ring depth (steps)
  constexpr int AP = KC * MT / 4;        // 16-byte activation pieces per thread per chunk
  __shared__ __attribute__((aligned(16))) bf16x8 As[2][KC][MT][64];
  const int nkb = K / 32;
  const int ks = (int)gridDim.y, sl = (int)blockIdx.y;
  // this workgroup's K-slice: steps [kb0, kb0 + nst), a whole number of chunks
  const int spl = ((nkb + ks - 1) / ks + KC - 1) / KC * KC;
  const int kb0 = min(nkb, sl * spl), nst = min(nkb, kb0 + spl) - kb0;
  const int nch = (nst + KC - 1) / KC;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, fg = lane >> 4;
  const int n0 = (int)blockIdx.x * 64 * NTW;
  const int g_last = npad / 16 - 1, mt_last = (M + 15) / 16 - 1;
  int64_t wchunk[NTW];
#pragma unroll
  for (int j = 0; j < NTW; j++) wchunk[j] = (int64_t)min(n0 / 16 + wave * NTW + j, g_last) * nkb;

  // activation pieces of a chunk: piece p = tid + 256 i is step p / (64 MT),
  // tile (p / 64) % MT, lane p % 64 (tiles past the packed rows are clamped:
  // they only feed outputs that are never stored)
  u32x4 areg[AP];
  auto load_a = [&](int c) {
#pragma unroll
    for (int i = 0; i < AP; i++) {
      const int p = tid + 256 * i, u = p / (64 * MT), t = (p / 64) % MT, l = p % 64;
      const int kb = min(kb0 + min(c * KC + u, max(nst - 1, 0)), nkb - 1);
      areg[i] = *reinterpret_cast<const u32x4*>(xf + (((int64_t)min(t, mt_last) * nkb + kb) * 64 + l) * 8);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < AP; i++) {
      const int p = tid + 256 * i;
      reinterpret_cast<u32x4*>(&As[buf][0][0][0])[p] = areg[i];
    }
  };
  WCodesSm wc[WD][NTW];
  auto load_w = [&](int slot, int s) {  // step s of the slice (clamped)
    const int kb = min(kb0 + min(s, max(nst - 1, 0)), nkb - 1);
#pragma unroll
    for (int j = 0; j < NTW; j++) load_wc<FMT, ST>(wc[slot][j], q, sc, wchunk[j] + kb, fr, fg);
  };

  f32x4 acc[MT][NTW];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NTW; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // prologue: chunk 0 in LDS buffer 0, chunk 1 in registers, weights of
  // steps 0 .. WD-1 in the ring
  load_a(0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < WD; s++) load_w(s, s);
  __builtin_amdgcn_sched_barrier(0);
  store_a(0);
  if (nch > 1) load_a(1);
  __syncthreads();

  // chunk c (LDS buffer c % 2, ring slots (c % 2) KC ..): first stage chunk
  // c+1 (in registers since chunk c-1) into the other buffer and load chunk
  // c+2; then its steps, each computing from the LDS activations and the
  // weights in its ring slot, whose refill (step s + WD) goes out at once;
  // one barrier at the end (the other buffer is complete, this one is free).
  auto chunk = [&](int c, const int buf) {
    if (c + 1 < nch) {
      store_a(buf ^ 1);
      if (c + 2 < nch) load_a(c + 2);
    }
#pragma unroll
    for (int u = 0; u < KC; u++) {
      const int s = c * KC + u;
      if (s >= nst) break;
      const int slot = buf * KC + u;
      bf16x8 wf[NTW];
#pragma unroll
      for (int j = 0; j < NTW; j++) wf[j] = dequant_sm<FMT, ST>(wc[slot][j], fg);
      load_w(slot, s + WD);
      bf16x8 af[MT];
#pragma unroll
      for (int i = 0; i < MT; i++) af[i] = As[buf][u][i][lane];
#pragma unroll
      for (int j = 0; j < NTW; j++)
#pragma unroll
        for (int i = 0; i < MT; i++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[j], af[i], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  };
  for (int c = 0; c < nch; c += 2) {
    chunk(c, 0);
    if (c + 1 >= nch) break;
    chunk(c + 1, 1);
  }

  // acc[i][j] holds y[m][n .. n+3] with m = row fr of tile i, n = 4 fg of
  // this wave's fragment j
  const bool vec = (N & 3) == 0 && (ks > 1 || (reinterpret_cast<uintptr_t>(y) & 15) == 0);
#pragma unroll
  for (int i = 0; i < MT; i++) {
    const int m = i * 16 + fr;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < NTW; j++) {
      const int n = n0 + (wave * NTW + j) * 16 + 4 * fg;
      const f32x4 v = acc[i][j];
      if (ks > 1) {
        float* d = part + ((int64_t)sl * M + m) * N + n;
        if (vec && n + 3 < N) {
          *reinterpret_cast<f32x4*>(d) = v;
        } else {
#pragma unroll
          for (int r = 0; r < 4; r++)
            if (n + r < N) d[r] = v[r];
        }
      } else if (vec && n + 3 < N) {
        if (y_dtype == RQ_F32)
          *reinterpret_cast<f32x4*>(static_cast<float*>(y) + (int64_t)m * N + n) = v;
        else
          *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(y) + (int64_t)m * N + n) =
              u32x2{pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3])};
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          if (n + r >= N) break;
          if (y_dtype == RQ_F32)
            static_cast<float*>(y)[(int64_t)m * N + n + r] = v[r];
          else
            static_cast<uint16_t*>(y)[(int64_t)m * N + n + r] = (uint16_t)f32_to_bf16_bits(v[r]);
        }
      }
    }
  }
}

// y = sum over K-slices of the partial sums part[s * n + e], in slice order
__global__ __launch_bounds__(256) void gemm_sm_reduce_kernel(const float* __restrict__ part, void* __restrict__ y,
                                                            int64_t n, int ks, int y_dtype) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  float t = part[e];
  for (int s = 1; s < ks; s++) t += part[(int64_t)s * n + e];
  if (y_dtype == RQ_F32)
    static_cast<float*>(y)[e] = t;
  else
    static_cast<uint16_t*>(y)[e] = (uint16_t)f32_to_bf16_bits(t);
}

hipError_t launch_split_reduce(const float* part, void* y, int64_t n, int ks, int y_dtype, hipStream_t stream,
                               hipEvent_t stop) {
  hipExtLaunchKernelGGL(gemm_sm_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, nullptr, stop,
                        0, part, y, n, ks, y_dtype);
  return hipGetLastError();
}

template <int FMT, typename ST, int MT>
static hipError_t launch_sm_t(const MatmulArgs& a, int ks) {
  constexpr int NTW = 1, KC = 8;
  if (hipError_t e = launch_pack_x(a)) return e;
  const dim3 grid((unsigned)((a.npad / 16 + 4 * NTW - 1) / (4 * NTW)), (unsigned)ks);
  hipExtLaunchKernelGGL((gemm_sm_kernel<FMT, ST, MT, NTW, KC>), grid, dim3(256), 0, a.stream, nullptr,
                        ks > 1 ? nullptr : a.ev_main[1], 0, a.q, static_cast<const ST*>(a.scales),
                        static_cast<const uint16_t*>(a.scratch), a.y, a.part, (int)a.m, (int)a.k, (int)a.n,
                        (int)a.npad, a.y_dtype);
  if (hipError_t e = hipGetLastError()) return e;
  if (ks > 1) return launch_split_reduce(a.part, a.y, a.m * a.n, ks, a.y_dtype, a.stream, a.ev_main[1]);
  return hipSuccess;
}

// K-slices: about 24 waves per CU at m <= 32 (12 above: the 4-tile kernel
// holds fewer per CU), 4 per 64 output columns times the slices; each slice
// keeps at least 8 chunks of K. Measured (Q4, bf16 x): M = 32, K = 8192,
// N = 28672: 1 / 2 / 4 slices 66.8 / 60.4 / 58.7 us; M = 64: 1 / 2 slices
// 83.6 / 90.6 us; M = 17, K = 4096, N = 14336: 1 / 2 slices 27.1 / 20.8 us.
int gemm_sm_slices(int64_t m, int64_t k, int64_t npad, int cu_count) {
  const int64_t waves = (npad / 64) * 4, want = (int64_t)cu_count * (m <= 32 ? 24 : 12);
  int64_t ks = std::max<int64_t>(1, want / std::max<int64_t>(waves, 1));
  ks = std::min<int64_t>(ks, std::max<int64_t>(1, (k / 32) / 64));
  return (int)std::min<int64_t>(ks, 8);
}

// Q4_0 only: for Q8_0 (twice the bytes per step) the per-wave-weights GEMM
// measured ahead (64 vs 67 us at M = 32, K = 8192, N = 28672).
bool gemm_sm_takes(int format, int64_t m) { return format == RQ_Q4_0 && m > 16 && m <= 64; }

hipError_t launch_gemm_sm(const MatmulArgs& a, int ks) {
  if (a.m <= 16 || a.m > 64) return hipErrorInvalidValue;
#define RQ_SM(FMT_, ST_) return a.m <= 32 ? launch_sm_t<FMT_, ST_, 2>(a, ks) : launch_sm_t<FMT_, ST_, 4>(a, ks);
  if (a.format == RQ_Q8_0) { RQ_SM(RQ_Q8_0, float) }
  if (a.scale_dtype == RQ_F16) { RQ_SM(RQ_Q4_0, uint16_t) }
  RQ_SM(RQ_Q4_0, float)
#undef RQ_SM
}

}  // namespace rq
