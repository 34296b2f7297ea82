// gemm.hip — prefill-regime (m > 16) block-quantized GEMM on CDNA4 MFMA.
//
// y[m, o] = sum_b scale[o, b] * P_b[m, o],  P_b = sum_{k in block b} x[m, k] * code[o, k]
//
// Raster's staged contraction (raster/compiler/ir/contract_stages.clj:25-31):
// the inner sum over one 32-element block runs on v_mfma_f32_16x16x32_bf16 whose
// K is exactly one quant block; the codes enter the MFMA as bf16 integers, which
// is exact (|code| <= 128 needs 8 significand bits), so the dequantized tile in
// LDS is bit-exact and every product is exact in f32. The f32 block scale then
// multiplies the f32 partial (one FMA per output per block).
//
// f32 activations are split into bf16 hi + lo (x = hi + lo + O(2^-17 |x|)) and
// take two MFMAs per tile. This is the f32-activation path; bf16 activations
// take gemm_bf16_kernel.
//
// Tiling: 256 threads = 4 waves (2 x 2), block tile 128 (m) x 128 (o), each wave
// 64 x 64 = 4 x 4 MFMA tiles. Weights are the B operand so each lane's four
// outputs of a tile share one column o and one scale. LDS is double-buffered:
// the next block's global loads are in flight while the current one computes.
// Block ids are remapped so the m-tiles that share a weight tile run on the same
// XCD (one L2 fetch of the weight tile per XCD).
#include "rq_internal.h"

namespace rq {

constexpr int GBM = 128, GBN = 128;
constexpr int LDA = 40;  // bf16 per LDS row: 32 + 8 padding (80 B stride spreads banks)

__device__ __forceinline__ uint32_t pack_bf16_exact(float lo, float hi) {
  // lo/hi are small integers: the bf16 is the top half of the f32, exactly
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
}

template <int FMT, typename ST, int XT>
__global__ __launch_bounds__(256) void gemm_kernel(const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                                  const void* __restrict__ x, void* __restrict__ y, int M,
                                                  int K, int N, int y_dtype, int tiles_m) {
  constexpr int NA = XT == RQ_F32 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][NA][GBM * LDA];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][GBN * LDA];
  __shared__ float Ss[2][GBN];

  // XCD-aware order: block b runs on XCD b % 8; give each XCD a contiguous run.
  const int nblk = gridDim.x, b = blockIdx.x;
  const int xcd = b & 7, per = nblk >> 3, rem = nblk & 7;
  const int tile = xcd * per + (xcd < rem ? xcd : rem) + (b >> 3);
  const int tn = tile / tiles_m, tm = tile - tn * tiles_m;
  const int m0 = tm * GBM, n0 = tn * GBN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int nkb = K / 32;
  const int lrow = tid >> 1, lhalf = tid & 1;

  // staging registers
  uint4 a_raw[XT == RQ_F32 ? 4 : 2];
  uint4 b_raw;
  float s_raw = 0.0f;

  auto gload = [&](int kb) {
    const int am = m0 + lrow;
    if (am < M) {
      if (XT == RQ_F32) {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const float*>(x) + (int64_t)am * K +
                                                        (int64_t)kb * 32 + 16 * lhalf);
#pragma unroll
        for (int i = 0; i < (XT == RQ_F32 ? 4 : 2); i++) a_raw[i] = p[i];
      } else {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + (int64_t)am * K +
                                                        (int64_t)kb * 32 + 16 * lhalf);
#pragma unroll
        for (int i = 0; i < 2; i++) a_raw[i] = p[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < (XT == RQ_F32 ? 4 : 2); i++) a_raw[i] = make_uint4(0, 0, 0, 0);
    }
    const int bn = n0 + lrow;
    if (bn < N) {
      const int64_t off = code_off<FMT>(bn, kb, nkb) + (FMT == RQ_Q8_0 ? 16 * lhalf : 0);
      b_raw = *reinterpret_cast<const uint4*>(q + off);
      s_raw = load_scale<ST>(sc, scale_off(bn, kb, nkb));
    } else {
      b_raw = make_uint4(0, 0, 0, 0);
      s_raw = 0.0f;
    }
  };

  auto lstore = [&](int buf) {
    // A -> bf16 (hi[/lo]) rows
    if (XT == RQ_F32) {
      uint32_t hi[8], lo[8];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float v[4] = {__uint_as_float(a_raw[i].x), __uint_as_float(a_raw[i].y),
                            __uint_as_float(a_raw[i].z), __uint_as_float(a_raw[i].w)};
        uint32_t h[4], l[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          h[j] = f32_to_bf16_bits(v[j]);
          l[j] = f32_to_bf16_bits(v[j] - bf16_bits_to_f32(h[j]));
        }
        hi[2 * i] = h[0] | (h[1] << 16);
        hi[2 * i + 1] = h[2] | (h[3] << 16);
        lo[2 * i] = l[0] | (l[1] << 16);
        lo[2 * i + 1] = l[2] | (l[3] << 16);
      }
      uint4* dh = reinterpret_cast<uint4*>(&As[buf][0][lrow * LDA + 16 * lhalf]);
      dh[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
      dh[1] = make_uint4(hi[4], hi[5], hi[6], hi[7]);
      uint4* dl = reinterpret_cast<uint4*>(&As[buf][NA - 1][lrow * LDA + 16 * lhalf]);
      dl[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
      dl[1] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
    } else {
      uint4* d = reinterpret_cast<uint4*>(&As[buf][0][lrow * LDA + 16 * lhalf]);
      d[0] = a_raw[0];
      d[1] = a_raw[1];
    }
    // B -> exact bf16 codes, elements [16*lhalf, 16*lhalf + 16) of the block
    const uint32_t w[4] = {b_raw.x, b_raw.y, b_raw.z, b_raw.w};
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float c[4];
#pragma unroll
      for (int j = 0; j < 4; j++)
        c[j] = FMT == RQ_Q8_0 ? q8_code(w[i], j) : q4_nib(w[i], j, lhalf != 0) - 8.0f;
      o[2 * i] = pack_bf16_exact(c[0], c[1]);
      o[2 * i + 1] = pack_bf16_exact(c[2], c[3]);
    }
    uint4* db = reinterpret_cast<uint4*>(&Bs[buf][lrow * LDA + 16 * lhalf]);
    db[0] = make_uint4(o[0], o[1], o[2], o[3]);
    db[1] = make_uint4(o[4], o[5], o[6], o[7]);
    if (lhalf == 0) Ss[buf][lrow] = s_raw;
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};

  gload(0);
  lstore(0);
  __syncthreads();
  const int fr = lane & 15, fk = 8 * (lane >> 4);
  for (int kb = 0; kb < nkb; kb++) {
    const int buf = kb & 1;
    if (kb + 1 < nkb) gload(kb + 1);
    bf16x8 af[NA][4], bfr[4];
    float sj[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int h = 0; h < NA; h++)
        af[h][i] = *reinterpret_cast<const bf16x8*>(&As[buf][h][(wm * 64 + i * 16 + fr) * LDA + fk]);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      bfr[j] = *reinterpret_cast<const bf16x8*>(&Bs[buf][(wn * 64 + j * 16 + fr) * LDA + fk]);
      sj[j] = Ss[buf][wn * 64 + j * 16 + fr];
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[0][i], bfr[j], zero, 0, 0, 0);
        if (NA == 2) p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[NA - 1][i], bfr[j], p, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) acc[i][j][r] = fmaf(sj[j], p[r], acc[i][j][r]);
      }
    if (kb + 1 < nkb) lstore(buf ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds column fr of each 16x16 tile, rows 4*(lane>>4) + r
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + wn * 64 + j * 16 + fr;
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + r;
        if (m >= M) continue;
        if (y_dtype == RQ_F32)
          static_cast<float*>(y)[(int64_t)m * N + n] = acc[i][j][r];
        else
          static_cast<uint16_t*>(y)[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_bits(acc[i][j][r]);
      }
    }
}

// f32 activations only: bf16 activations take gemm_bf16_kernel (gemm_bf16.hip).
template <int FMT, typename ST>
static hipError_t launch_x(const MatmulArgs& a) {
  if (a.x_dtype != RQ_F32) return hipErrorInvalidValue;
  const int tiles_m = (int)((a.m + GBM - 1) / GBM), tiles_n = (int)((a.n + GBN - 1) / GBN);
  dim3 grid((unsigned)(tiles_m * tiles_n));
  hipExtLaunchKernelGGL((gemm_kernel<FMT, ST, RQ_F32>), grid, dim3(256), 0, a.stream, a.ev_main[0], a.ev_main[1],
                        0, a.q, static_cast<const ST*>(a.scales), a.x, a.y, (int)a.m, (int)a.k, (int)a.n,
                        a.y_dtype, tiles_m);
  return hipGetLastError();
}

hipError_t launch_gemm(const MatmulArgs& a, int cu_count) {
  (void)cu_count;
  if (a.format == RQ_Q8_0) return launch_x<RQ_Q8_0, float>(a);
  if (a.scale_dtype == RQ_F16) return launch_x<RQ_Q4_0, uint16_t>(a);
  return launch_x<RQ_Q4_0, float>(a);
}

}  // namespace rq
