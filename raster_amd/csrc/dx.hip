// dx.hip — backward-data of the quantized linear for small m:
//   dx[m, i] = sum_o scale[o, i/32] * code[o, i] * dy[m, o]
// qlinear-q8-dx (raster/quant/train.clj:110-137), the pullback Raster emits for
// qlinear-q8 (train.clj:143-155), over the same resident chunked weight (Q8_0,
// or Q4_0 with code = nibble - 8). Each weight w = scale * code is rounded to
// f32 as Raster does; the products w * dy are formed and summed in f32 by the
// MFMA (Raster: each product rounded to f32, summed in double).
//
// The reduction runs over `out`, the row index of the resident weight. Slices
// of the 16-row groups write partial sums that dx_reduce_kernel adds in slice
// order (deterministic); with one slice the first kernel writes dx.
#include <algorithm>

#include "rq_internal.h"

namespace rq {

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

// ---- dx on f32 MFMA (small m): the weight in its stored layout as the B
// operand of v_mfma_f32_16x16x4_f32, so no transpose of the codes is needed.
//
// D[i][j] += sum_k A[i][k] B[k][j] with i = dy row (16 per pass), k = weight
// row o (4 per MFMA), j = a column of dx. Lane l = 16 kq + j supplies
// A[j][kq] and B[kq][j]; its k is row 4 kq + qd of the 16-row group for the
// row quad qd = 0..3, and its B values are the 16 weights of that row in
// columns [32 b + 16 h, +16) of block b = b0 + j / 2, h = j % 2: one 16-byte
// load (Q8: codes 16 h .. 16 h + 15 of the row; Q4: the row's 16 packed bytes,
// low nibbles for h = 0, high for h = 1). MFMA t (t = 0..15) takes the t-th of
// those weights, so accumulator t collects dx[m][32 b0 + 16 j + t]: a wave
// owns a 16-row x 256-column tile of dx. Every B value is Raster's dequantized
// weight scale * code, one IEEE f32 rounding (fma(u, s, -OFF s) with the
// offset code u = code + OFF exact); the MFMA forms the products w * dy in
// f32 and sums them in f32 (Raster: w * dy rounded to f32, summed in double).
//
// A workgroup of 8 waves owns one column tile and one slice of the row
// groups; wave w takes groups g0 + w, g0 + w + 8, ..., the next group's
// loads in flight while the current one's 64 MFMAs run. The eight tiles are
// added in wave order through LDS, and the workgroup writes dx (one slice)
// or its partial sum (several slices; dx_reduce_kernel adds them in slice
// order). grid.z runs over 16-row tiles of dy, each re-reading the weight.
// MFMA-bound: per 16 dy rows, 2 * 16 * out * in flop at 157 TFLOP/s f32
// (measured with the dequantization about 38 clocks per MFMA against 35
// without; at the C2 layer, in 4096 x out 11008, about 17 us per 16 dy rows
// plus about 10 us of slice sums, reduction launch and ramp).
namespace {
constexpr int kFmWaves = 8;
constexpr int kFmBlocks = 8;  // 32-column blocks per column tile (256 columns)

// one row group's operands for one lane: the 16-byte code pieces of its four
// row quads, their scale bits and the four dy values
struct FmSlot {
  u32x4 w[4];
  uint32_t s[4];
  float a[4];
};
}  // namespace

template <int FMT, typename ST>
__global__ __launch_bounds__(64 * kFmWaves) void dx_fm_kernel(const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                                             const float* __restrict__ dy, float* __restrict__ out_buf,
                                                             int M, int K, int N, int npad, int gps) {
  // the eight waves' tiles: [wave][r][lane][4 f32x4], the f32x4 index swizzled
  // by (lane >> 1) & 3 so that eight consecutive lanes' writes hit distinct banks
  __shared__ f32x4 red[kFmWaves * 4 * 64 * 4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nb = K / 32, ngroups = npad / 16;
  const int b0 = (int)blockIdx.x * kFmBlocks;
  const int s = (int)blockIdx.y, mt = (int)blockIdx.z;
  const int g0 = s * gps, g1 = min(ngroups, g0 + gps);
  const int j = lane & 15, kq = lane >> 4, h = j & 1;
  const int64_t bj = min(b0 + (j >> 1), nb - 1);  // blocks past K reread the last one (not stored)
  const float* dyr = dy + (int64_t)min(mt * 16 + j, M - 1) * N;  // rows past M reread row M - 1 (not stored)

  // Loads are unconditional at clamped addresses: a condition on them would
  // make the compiler wait for every load in flight. Rows past N (padding
  // rows: zero codes and scales) read dy at N - 1 and get a zero factor.
  auto load = [&](FmSlot& sl, int g) {
    g = min(g, ngroups - 1);
    const int64_t chunk = (int64_t)g * nb + bj;
#pragma unroll
    for (int qd = 0; qd < 4; qd++) {
      const int row = 4 * kq + qd;
      if (FMT == RQ_Q8_0)
        sl.w[qd] = *reinterpret_cast<const u32x4*>(q + chunk * 512 + row * 32 + 16 * h);
      else
        sl.w[qd] = *reinterpret_cast<const u32x4*>(q + chunk * 256 + row * 16);
      sl.s[qd] = load_scale_bits<ST>(sc, chunk * 16 + row);
      const int o = 16 * g + row;
      sl.a[qd] = dyr[min(o, N - 1)];
    }
  };

  f32x4 acc[16];
#pragma unroll
  for (int t = 0; t < 16; t++) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](const FmSlot& cur, int g) {
#pragma unroll
    for (int qd = 0; qd < 4; qd++) {
      const float sv = scale_from_bits<ST>(cur.s[qd]);
      const float a = g < g1 && 16 * g + 4 * kq + qd < N ? cur.a[qd] : 0.0f;
      const u32x4 wv = cur.w[qd];
      float off;
      uint32_t u[4];
      if (FMT == RQ_Q8_0) {
        // offset code u = code + 128 (byte ^ 0x80): fma(u, s, -128 s) = s * code, rounded once
        off = -128.0f * sv;
#pragma unroll
        for (int e = 0; e < 4; e++) u[e] = wv[e] ^ 0x80808080u;
      } else {
        // nibble n, zero-point 8: fma(n, s, -8 s) = s * (n - 8), rounded once
        off = -8.0f * sv;
#pragma unroll
        for (int e = 0; e < 4; e++) u[e] = (wv[e] >> (4 * h)) & 0x0F0F0F0Fu;
      }
      // the row quad's 16 weights first, then its 16 MFMAs: interleaved one
      // to one, each MFMA waits on its own conversion (measured 43 against
      // 38 clocks per MFMA)
      float w[16];
#pragma unroll
      for (int t = 0; t < 16; t++) w[t] = fmaf((float)((u[t >> 2] >> (8 * (t & 3))) & 0xFFu), sv, off);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < 16; t++) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, w[t], acc[t], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // two slots, alternating; the scheduling fences keep each refill ahead of
  // the other slot's MFMAs (without them the compiler moves the loads down to
  // their first use and every group waits for its own loads). The second
  // slot is computed unconditionally, with a zero factor past the slice (a
  // conditional use lets the compiler sink its loads into the condition).
  FmSlot s0, s1;
  int g = g0 + wave;
  load(s0, g);
  for (; g < g1; g += 2 * kFmWaves) {
    load(s1, g + kFmWaves);
    __builtin_amdgcn_sched_barrier(0);
    compute(s0, g);
    __builtin_amdgcn_sched_barrier(0);
    load(s0, g + 2 * kFmWaves);
    __builtin_amdgcn_sched_barrier(0);
    compute(s1, g + kFmWaves);
    __builtin_amdgcn_sched_barrier(0);
  }

  // the eight waves' tiles, added in wave order; acc[t][r] is
  // dx[16 mt + 4 kq + r][32 b0 + 16 j + t]
  const int swz = (lane >> 1) & 3;
#pragma unroll
  for (int r = 0; r < 4; r++)
#pragma unroll
    for (int t4 = 0; t4 < 4; t4++)
      red[((wave * 4 + r) * 64 + lane) * 4 + (t4 ^ swz)] =
          f32x4{acc[4 * t4][r], acc[4 * t4 + 1][r], acc[4 * t4 + 2][r], acc[4 * t4 + 3][r]};
  __syncthreads();
  float* dst = gridDim.y == 1 ? out_buf : out_buf + (int64_t)s * M * K;
#pragma unroll
  for (int p = 0; p < 2; p++) {
    const int u = tid + 64 * kFmWaves * p;  // f32x4 unit: (r, lane, t4)
    const int r = u >> 8, ln = (u >> 2) & 63, t4 = u & 3;
    const int at = (r * 64 + ln) * 4 + (t4 ^ ((ln >> 1) & 3));
    f32x4 v = red[at];
#pragma unroll
    for (int w = 1; w < kFmWaves; w++) v += red[w * 4 * 64 * 4 + at];
    const int m = mt * 16 + 4 * (ln >> 4) + r;
    const int jj = ln & 15;
    if (m < M && b0 + (jj >> 1) < nb)
      *reinterpret_cast<f32x4*>(dst + (int64_t)m * K + 32 * b0 + 16 * jj + 4 * t4) = v;
  }
}

int dx_fm_slices(int64_t m, int64_t in, int64_t npad, int cu_count) {
  // at most one workgroup per CU (the LDS of the tile sum allows one):
  // column tiles x dy-row tiles x slices, each wave of a slice at least one
  // row group
  const int64_t tiles = (in / 32 + kFmBlocks - 1) / kFmBlocks * ((m + 15) / 16);
  const int64_t ngroups = npad / 16;
  const int64_t want = (int64_t)std::max(cu_count, 1) / tiles;
  return (int)std::max<int64_t>(1, std::min<int64_t>(want, ngroups / kFmWaves));
}

template <int FMT, typename ST>
static hipError_t launch_dx_fm_t(const Weight& w, const float* dy, float* dx, int64_t m, float* part, int slices,
                                 hipStream_t stream) {
  const int64_t nb = w.in / 32, ngroups = w.npad / 16;
  const int gps = (int)((ngroups + slices - 1) / slices);
  const dim3 grid((unsigned)((nb + kFmBlocks - 1) / kFmBlocks), (unsigned)slices, (unsigned)((m + 15) / 16));
  hipLaunchKernelGGL((dx_fm_kernel<FMT, ST>), grid, dim3(64 * kFmWaves), 0, stream, w.q,
                     static_cast<const ST*>(w.scales), dy, slices == 1 ? dx : part, (int)m, (int)w.in, (int)w.out,
                     (int)w.npad, gps);
  if (hipError_t e = hipGetLastError()) return e;
  if (slices > 1) {
    const int64_t n4 = m * w.in / 4;
    hipLaunchKernelGGL(dx_reduce_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, stream, part, dx, n4,
                       slices);
  }
  return hipGetLastError();
}

hipError_t launch_dx_fm(const Weight& w, const float* dy, float* dx, int64_t m, float* part, int slices,
                        hipStream_t stream) {
  if (w.format == RQ_Q8_0) return launch_dx_fm_t<RQ_Q8_0, float>(w, dy, dx, m, part, slices, stream);
  if (w.scale_dtype == RQ_F16) return launch_dx_fm_t<RQ_Q4_0, uint16_t>(w, dy, dx, m, part, slices, stream);
  return launch_dx_fm_t<RQ_Q4_0, float>(w, dy, dx, m, part, slices, stream);
}

}  // namespace rq
