// gemv1.hip — decode GEMV (MR activation rows, planned for m = 1; plain
// rq_qmatmul calls, f32 or bf16 x) on v_dot4_i32_i8, with the numerics of the
// int8-level decode kernel
// (gemv.hip): each 32-block of x is a 16-bit block fixed point X =
// rint(x * 2^(15-e)) split into two int8 levels X = 256 L0 + L1, and the
// weight codes enter the integer dots exactly (Q4_0 nibbles 0..15 with the
// zero point folded as -8 * sum X). Per block: the int32 dot 256 C0 + C1
// (- 8 sum X), then f32 (2^(e-15) * scale) times it. Int8 activations
// (rq_qmatmul_i8: Raster's quantize-act-i8 blocks) are the single level L1,
// with their block scale as the factor and their code sum as sum X; with
// act_i8 the kernel makes those blocks itself from f32 / bf16 x, by the math
// of quantize_act_i8_kernel (bitwise its codes, scales and sums).
//
// Memory: one load instruction moves 1 KB of codes. A Q4_0 lane takes the
// 16-byte row r of one chunk (4 consecutive chunks per wave, lane
// (r, j) = (lane % 16, lane / 16)); a Q8_0 lane takes half of a 32-byte row
// (2 chunks per wave, lane (r, h, j) = (lane % 16, lane / 16 % 2, lane / 32)).
// The lane's codes then go straight into sdot4 against the block's levels in
// LDS (read by 16 lanes at once: one broadcast per address). Per KB of codes
// this is about 30 (Q4) or 12 (Q8) VALU instructions per wave, against ~70 and
// ~35 for the MFMA variant scheme of gemv.hip, whose per-window epilogue
// bounds it at m = 1.
//
// Work: a workgroup decomposes x into LDS once, then takes 16-row groups
// g = blockIdx.x + i * gridDim.x; its W waves split each group's blocks
// (steps of BPL blocks, interleaved: wave w takes steps w, w + W, ..., so the
// W waves read adjacent kilobytes at a time; measured 1-3% per call against
// contiguous runs per wave at K = 8192, N = 28672; spw per wave, padded to
// whole turns of a D-step register ring). The ring streams loads across group boundaries; a group
// ends with a shuffle over the lanes of a row, one LDS exchange between the
// waves (double-buffered, one barrier) and the store, in wave order.
#include <algorithm>
#include <atomic>

#include "rq_internal.h"

namespace rq {

namespace {

template <typename ST>
struct G1Codes {
  u32x4 v;  // 16 code bytes
  ST s;     // the row's block scale, as stored
};

}  // namespace

// LDS: levels [mr][nb][64] (L0 then L1, 32 bytes each), factor [mr][nb] f32,
// level sum [mr][nb] i32, partial sums [2][W][mr][16] f32
__host__ __device__ inline int g1_lds_bytes(int nb, int waves, int mr) {
  return mr * nb * 72 + 2 * waves * mr * 16 * 4;
}

template <int FMT, typename ST, int XT, int W, int D, int MR, bool AQ>
__global__ __launch_bounds__(64 * W) void gemv1_kernel(const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                                      const void* __restrict__ x, const float* __restrict__ axs,
                                                      const int32_t* __restrict__ axsum,
                                                      void* __restrict__ y, int M, int K, int N, int npad,
                                                      int y_dtype) {
  constexpr int BPL = FMT == RQ_Q4_0 ? 4 : 2;  // blocks per load instruction
  constexpr int CB = FMT == RQ_Q4_0 ? 256 : 512;  // chunk bytes
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int nb = K / 32, ngroups = npad / 16;
  int8_t* lev = reinterpret_cast<int8_t*>(smem);
  float* fac = reinterpret_cast<float*>(smem + MR * nb * 64);
  int* sx = reinterpret_cast<int*>(smem + MR * nb * 68);
  float* red = reinterpret_cast<float*>(smem + MR * nb * 72);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15;
  const int j = FMT == RQ_Q4_0 ? lane >> 4 : lane >> 5;  // block of the load
  const int h = FMT == RQ_Q4_0 ? 0 : (lane >> 4) & 1;    // half of the row (Q8)
  const int lofs = j * CB + r * (CB / 16) + 16 * h;      // lane's bytes within a load

  // ---- this workgroup's groups and this wave's steps
  const int nsteps = (nb + BPL - 1) / BPL;           // load steps per group
  const int spw = (nsteps + W - 1) / W;              // per wave
  const int spp = (spw + D - 1) / D * D;             // padded to whole ring turns
  const int ng = (ngroups - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;  // groups of this workgroup
  G1Codes<ST> wc[D];
  auto load_w = [&](int slot, int gi, int u) {
    if (gi >= ng) {  // past the end: the last step again (addresses stay valid)
      gi = ng - 1;
      u = spp - 1;
    }
    const int g = (int)blockIdx.x + gi * (int)gridDim.x;
    const int st = min(min(u, spw - 1) * W + wave, nsteps - 1);
    const int b0 = min(st * BPL, nb - BPL);  // first block of the load (a short tail rereads)
    const int64_t chunk = (int64_t)g * nb + b0;
    wc[slot].v = *reinterpret_cast<const u32x4*>(q + chunk * (CB / 16) * 16 + lofs);
    wc[slot].s = sc[(chunk + j) * 16 + r];
  };
  int lg = 0, lu = 0;
  auto advance = [&](int& gi, int& u) {
    if (++u == spp) {
      u = 0;
      ++gi;
    }
  };

  // ---- x into LDS (first round of loads before the weight ring's). Item it:
  // row it / (8 nb), 4 elements; rows past M decompose as zeros.
  constexpr int XI = 4;
  const int nitems = MR * nb * 8, stride = 64 * W;
  float xv[XI][4];
  auto load_items = [&](int base) {
#pragma unroll
    for (int i = 0; i < XI; i++) {
      if (base + stride * i >= nitems) break;  // workgroup-uniform
      const int it = min(base + tid + stride * i, nitems - 1);
      const int mr = it / (nb * 8), rem = it - mr * nb * 8;
      load_x4<XT>(x, (int64_t)mr * K + rem * 4, mr < M, xv[i]);
      if (XT == kXtI8) {
        // the block's scale and code sum ride along in v[1], v[2], loaded
        // with the codes (not at the conversion, one more round trip)
        xv[i][1] = mr < M ? axs[it >> 3] : 0.0f;
        xv[i][2] = __int_as_float(mr < M && axsum ? axsum[it >> 3] : 0);
      }
    }
  };
  auto convert_items = [&](int base) {
#pragma unroll
    for (int i = 0; i < XI; i++) {
      if (base + stride * i >= nitems) break;
      const int it0 = base + tid + stride * i;
      const int it = min(it0, nitems - 1);
      const int b = it >> 3, part = it & 7;  // b counts the rows' blocks in turn: mr * nb + block
      if (XT == kXtI8) {
        if (it0 < nitems) {
          *reinterpret_cast<uint32_t*>(lev + b * 64 + part * 4) = 0u;
          *reinterpret_cast<uint32_t*>(lev + b * 64 + 32 + part * 4) = __float_as_uint(xv[i][0]);
          if (part == 0) {
            fac[b] = xv[i][1];
            sx[b] = __float_as_int(xv[i][2]);
          }
        }
        continue;
      }
      const float* v = xv[i];
      if (AQ) {
        const float qmax = max8(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
        const double d = (double)qmax / 127.0;
        const double id = d == 0.0 ? 0.0 : 1.0 / d;
        uint32_t word = 0u;
        int s = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const int qv = java_round_clamp127((double)v[k] * id);
          word |= (uint32_t)(qv & 0xFF) << (8 * k);
          s += qv;
        }
        s = sum8(s);
        if (it0 < nitems) {
          *reinterpret_cast<uint32_t*>(lev + b * 64 + part * 4) = 0u;
          *reinterpret_cast<uint32_t*>(lev + b * 64 + 32 + part * 4) = word;
          if (part == 0) {
            fac[b] = (float)d;
            sx[b] = s;
          }
        }
        continue;
      }
      float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
      int bad = !(fabsf(v[0]) <= 3.402823466e38f && fabsf(v[1]) <= 3.402823466e38f &&
                  fabsf(v[2]) <= 3.402823466e38f && fabsf(v[3]) <= 3.402823466e38f);
      amax = max8(amax);
      bad = or8(bad);
      const bool finite = !bad;
      int e = 0;
      (void)frexpf(amax, &e);
      e = ldexpf(amax, 15 - e) > 32639.0f ? e + 1 : e;
      uint32_t l0 = 0u, l1 = 0u;
      int sum = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int X = finite ? (int)rintf(ldexpf(v[k], 15 - e)) : 0;
        const int a = (X + 128) >> 8, c = X - 256 * a;
        l0 |= (uint32_t)(a & 0xFF) << (8 * k);
        l1 |= (uint32_t)(c & 0xFF) << (8 * k);
        sum += X;
      }
      sum = sum8(sum);
      if (it0 < nitems) {
        *reinterpret_cast<uint32_t*>(lev + b * 64 + part * 4) = l0;
        *reinterpret_cast<uint32_t*>(lev + b * 64 + 32 + part * 4) = l1;
        if (part == 0) {
          fac[b] = finite ? ldexpf(1.0f, e - 15) : __builtin_nanf("");
          sx[b] = sum;
        }
      }
    }
  };
  load_items(0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < D; i++) {
    load_w(i, lg, lu);
    advance(lg, lu);
  }
  __builtin_amdgcn_sched_barrier(0);
  for (int base = 0; base < nitems; base += stride * XI) {
    if (base > 0) load_items(base);
    convert_items(base);
  }
  __syncthreads();

  // ---- the stream
  float acc[MR];
#pragma unroll
  for (int mr = 0; mr < MR; mr++) acc[mr] = 0.0f;
  for (int gi = 0; gi < ng; gi++) {
    for (int u0 = 0; u0 < spp; u0 += D) {
#pragma unroll
      for (int i = 0; i < D; i++) {
        const int u = u0 + i;
        const u32x4 w = wc[i].v;
        const float s = scale_value(wc[i].s);
        load_w(i, lg, lu);
        advance(lg, lu);
        const int st = u * W + wave;
        if (u < spw && st < nsteps) {
          const int b = min(st * BPL, nb - BPL) + j;
          // a short tail load (shifted back to stay inside the row) rereads
          // blocks of the previous step: count each block once
          const bool fresh = st * BPL <= nb - BPL || b >= st * BPL;
          int lo[4], hi[4];
#pragma unroll
          for (int k = 0; k < 4; k++) {
            lo[k] = FMT == RQ_Q4_0 ? (int)(w[k] & 0x0F0F0F0Fu) : (int)w[k];
            hi[k] = (int)((w[k] >> 4) & 0x0F0F0F0Fu);
          }
#pragma unroll
          for (int mr = 0; mr < MR; mr++) {
            const int bb = mr * nb + b;
            int c0 = 0, c1 = 0;
            if (FMT == RQ_Q4_0) {
              const i32x4 a0 = *reinterpret_cast<const i32x4*>(lev + bb * 64);
              const i32x4 a1 = *reinterpret_cast<const i32x4*>(lev + bb * 64 + 16);
              const i32x4 a2 = *reinterpret_cast<const i32x4*>(lev + bb * 64 + 32);
              const i32x4 a3 = *reinterpret_cast<const i32x4*>(lev + bb * 64 + 48);
#pragma unroll
              for (int k = 0; k < 4; k++) {
                if (XT != kXtI8) {  // int8 activations: level 0 is zero
                  c0 = __builtin_amdgcn_sdot4(lo[k], a0[k], c0, false);
                  c0 = __builtin_amdgcn_sdot4(hi[k], a1[k], c0, false);
                }
                c1 = __builtin_amdgcn_sdot4(lo[k], a2[k], c1, false);
                c1 = __builtin_amdgcn_sdot4(hi[k], a3[k], c1, false);
              }
              c1 -= 8 * sx[bb];
            } else {
              const i32x4 a0 = *reinterpret_cast<const i32x4*>(lev + bb * 64 + 16 * h);
              const i32x4 a2 = *reinterpret_cast<const i32x4*>(lev + bb * 64 + 32 + 16 * h);
#pragma unroll
              for (int k = 0; k < 4; k++) {
                if (XT != kXtI8) c0 = __builtin_amdgcn_sdot4(lo[k], a0[k], c0, false);
                c1 = __builtin_amdgcn_sdot4(lo[k], a2[k], c1, false);
              }
            }
            const float t = (float)((c0 << 8) + c1);  // |256 C0 + C1| < 2^24: exact in f32
            if (fresh) acc[mr] = fmaf(t, fac[bb] * s, acc[mr]);
          }
        }
      }
    }
    // ---- group gi: the row's lanes, then the waves (in wave order)
    float* rb = red + (gi & 1) * W * MR * 16;
#pragma unroll
    for (int mr = 0; mr < MR; mr++) {
      float t = acc[mr];
      t += __shfl_xor(t, 16, 64);
      t += __shfl_xor(t, 32, 64);
      if (lane < 16) rb[(wave * MR + mr) * 16 + lane] = t;
      acc[mr] = 0.0f;
    }
    __syncthreads();
    if (wave == 0 && lane < 16) {
      const int o = 16 * ((int)blockIdx.x + gi * (int)gridDim.x) + lane;
#pragma unroll
      for (int mr = 0; mr < MR; mr++) {
        float t = rb[mr * 16 + lane];
#pragma unroll
        for (int ww = 1; ww < W; ww++) t += rb[(ww * MR + mr) * 16 + lane];
        if (mr < M && o < N) {
          if (y_dtype == RQ_F32)
            static_cast<float*>(y)[(int64_t)mr * N + o] = t;
          else
            static_cast<uint16_t*>(y)[(int64_t)mr * N + o] = (uint16_t)f32_to_bf16_bits(t);
        }
      }
    }
  }
}

// One configuration (the lab and the dispatcher): gcols workgroups.
// AQ: quantize x to int8 blocks in the kernel (rq_fused_ops.act_i8; a
// template parameter, as a run-time switch costs the plain path ~0.4 us)
template <int FMT, typename ST, int XT, int W, int D, int MR, bool AQ = false>
hipError_t launch_gemv1_t(const MatmulArgs& a, int gcols) {
  static_assert(!(AQ && XT == kXtI8), "int8 input is quantized already");
  auto kernel = &gemv1_kernel<FMT, ST, XT, W, D, MR, AQ>;
  const int nb = (int)(a.k / 32);
  constexpr int BPL = FMT == RQ_Q4_0 ? 4 : 2;
  if (a.m < 1 || a.m > MR || nb < BPL || gcols < 1) return hipErrorInvalidValue;
  if (XT == kXtI8 && !a.ops.act_scale) return hipErrorInvalidValue;
  const int lds = g1_lds_bytes(nb, W, MR);
  if (lds > 163840) return hipErrorInvalidValue;
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
  const int ngroups = (int)(a.npad / 16);
  hipExtLaunchKernelGGL(kernel, dim3((unsigned)std::min(gcols, ngroups)), dim3(64 * W), (unsigned)lds, a.stream,
                        a.ev_main[0], a.ev_main[1], 0, a.q, static_cast<const ST*>(a.scales), a.x, a.ops.act_scale,
                        a.ops.act_sum, a.y, (int)a.m, (int)a.k, (int)a.n, (int)a.npad, a.y_dtype);
  return hipGetLastError();
}

}  // namespace rq

namespace rq {

// Plan (m = 1, Q4_0, f32 / bf16 x). Measured cold against the int8-level
// decode kernel (which keeps Q8_0, where this kernel only ties it at C1 and
// trails it at K = 8192, N = 28672): K = 4096, N = 14336: 9.3 against 12.0 us;
// K = 8192, N = 28672: 25.5 against 31.4 us; K = 2048, N = 5632: 4.5 against
// 5.8 us; K = 14336, N = 4096: 10.3 against 14.1 us. 8 waves (16 from
// K = 12288: 10.3 against 10.8 us), a 2-step ring while a wave has at most 4
// steps per group, else 4 (deeper rings measured slower), and up to two
// workgroups per CU (one with 16 waves). The dot work grows with the rows:
// at K = 4096, N = 14336, m = 2 took 12.1 against 12.9 us and m = 4 17.2 to
// 19.4 against 14.5 us, so m > 1 stays with the int8-level kernel.
G1Plan plan_gemv1(int64_t m, int64_t k, int64_t npad, int x_dtype, int format, int cu_count) {
  G1Plan p{};
  if (m != 1 || format != RQ_Q4_0 || (x_dtype != RQ_F32 && x_dtype != RQ_BF16 && x_dtype != kXtI8) || k % 32 != 0)
    return p;
  const int64_t nb = k / 32, ngroups = npad / 16;
  if (nb < 4) return p;
  const int64_t nsteps = (nb + 3) / 4;
  p.waves = nsteps >= 96 ? 16 : 8;
  if (g1_lds_bytes((int)nb, p.waves, 1) > 163840) return p;
  const int64_t spw = (nsteps + p.waves - 1) / p.waves;
  p.ring = spw <= 4 ? 2 : 4;
  p.gcols = (int)std::min<int64_t>(ngroups, (int64_t)cu_count * (p.waves == 16 ? 1 : 2));
  p.ok = p.gcols >= 1;
  return p;
}

template <typename ST, int XT, bool AQ>
static hipError_t launch_g1_x(const MatmulArgs& a, const G1Plan& p) {
  if (p.waves == 8 && p.ring == 2) return launch_gemv1_t<RQ_Q4_0, ST, XT, 8, 2, 1, AQ>(a, p.gcols);
  if (p.waves == 8 && p.ring == 4) return launch_gemv1_t<RQ_Q4_0, ST, XT, 8, 4, 1, AQ>(a, p.gcols);
  if (p.waves == 16 && p.ring == 2) return launch_gemv1_t<RQ_Q4_0, ST, XT, 16, 2, 1, AQ>(a, p.gcols);
  if (p.waves == 16 && p.ring == 4) return launch_gemv1_t<RQ_Q4_0, ST, XT, 16, 4, 1, AQ>(a, p.gcols);
  return hipErrorInvalidValue;
}

template <typename ST, int XT>
static hipError_t launch_g1_q(const MatmulArgs& a, const G1Plan& p) {
  return a.ops.act_i8 ? launch_g1_x<ST, XT, true>(a, p) : launch_g1_x<ST, XT, false>(a, p);
}

template <typename ST>
static hipError_t launch_g1_s(const MatmulArgs& a, const G1Plan& p) {
  if (a.x_dtype == kXtI8) return launch_g1_x<ST, kXtI8, false>(a, p);
  return a.x_dtype == RQ_F32 ? launch_g1_q<ST, RQ_F32>(a, p) : launch_g1_q<ST, RQ_BF16>(a, p);
}

hipError_t launch_gemv1(const MatmulArgs& a, const G1Plan& p) {
  if (!p.ok || a.format != RQ_Q4_0) return hipErrorInvalidValue;
  return a.scale_dtype == RQ_F16 ? launch_g1_s<uint16_t>(a, p) : launch_g1_s<float>(a, p);
}

}  // namespace rq
