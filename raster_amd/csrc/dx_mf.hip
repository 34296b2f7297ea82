// dx_mf.hip — backward-data GEMM of the quantized linear for many dy rows, on
// bf16 MFMA:
//   dx[m, i] = sum_o dy[m, o] * w[o, i],   w[o, i] = scale[o, i/32] * code[o, i]
// (qlinear-q8-dx, raster/quant/train.clj:110-137, at training batch sizes).
//
// The reduction runs over `out`, the row index of the resident weight, so a
// weight tile enters the MFMA transposed and with a scale that changes along
// the reduction. Each workgroup owns a 128-row x 128-column tile of dx (four
// 32-column blocks) and walks the weight's 16-row groups two at a time:
//  * the eight waves dequantize the step's 8 chunks, a chunk a wave (each
//    lane 2 rows x 4 columns: w = fma(u, s, -OFF s), Raster's single f32
//    rounding of scale * code) and write them to LDS, transposed into the
//    32x32x16 B-operand order (lane = column + 32 (row / 8), 8 rows a lane),
//    as bf16 hi = RNE(w) and lo = RNE(w - hi);
//  * dy enters as A from a fragment-major copy made by dx_pack_kernel (hi and
//    lo bf16 of each element, the 32x32x16 A-operand order), read straight
//    into registers a few groups ahead;
//  * per group and 32x32 output tile three MFMAs accumulate
//    dy_hi w_hi + dy_hi w_lo + dy_lo w_hi in f32.
// hi + lo carries each operand to a relative 2^-16, so each product is within
// about 3 * 2^-16 of the f32 product (the dropped dy_lo w_lo is below 2^-16);
// the sums run in f32 in a fixed order. The weight is read once per 128 dy
// rows instead of once per few rows; when that leaves CUs idle the reduction
// is cut into slices whose partial sums a second kernel adds in slice order.
// Waves: 4 along m (32 rows each, all four column blocks); waves w and w + 4
// share a SIMD and the rows, and split the reduction: wave w takes the first
// 16-row group of each step, wave w + 4 the second, so no two waves load the
// same dy fragments (with the waves split along the columns instead, two
// waves loaded each fragment: M = 512, K = 4096, N = 11008, one slice, 238 ->
// 225 us; M = 1024 273 -> 260; K = 11008, N = 4096 189 -> 181). The two
// partial sums are added through LDS at the end.
#include <algorithm>

#include "rq_internal.h"

namespace rq {

namespace {

constexpr int kDxmThreads = 512;
constexpr int kDxmBM = 128;  // dx rows per workgroup
constexpr int kDxmNB = 4;    // 32-column blocks per workgroup
constexpr int kDxmG = 2;     // 16-row weight groups per pipeline step
constexpr int kDxmDB = 4;    // steps of weight loads in flight (register ring slots)
constexpr int kDxmAR = 8;    // groups of dy fragments in flight per wave
constexpr int kDxmFrag = 512;  // uint16 per 64-lane fragment (64 x 8 bf16)

// LDS slot (16 bytes) of B-operand lane L in a fragment: L with its bits 0, 1
// flipped by its bits 3, 5 (see store_b)
__device__ __forceinline__ int dxm_slot(int L) { return L ^ (((L >> 3) & 1) | (((L >> 5) & 1) << 1)); }

}  // namespace

// dy f32 [M][N] -> dyf: per 32-row tile mt and 16-row group g, fragments hi
// then lo (1 KB each): lane l holds rows m = 32 mt + l % 32, o = 16 g +
// 8 (l / 32) + j (j < 8) as bf16 hi = RNE(dy), lo = RNE(dy - hi). Rows
// m >= M and o >= N are zero.
__global__ __launch_bounds__(256) void dx_pack_kernel(const float* __restrict__ dy, uint16_t* __restrict__ dyf, int M,
                                                      int N, int ngroups, int64_t nthreads, int vec) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= nthreads) return;
  const int l = (int)(t & 63);
  const int64_t f = t >> 6;  // mt * ngroups + g
  const int g = (int)(f % ngroups), mt = (int)(f / ngroups);
  const int m = 32 * mt + (l & 31), o0 = 16 * g + 8 * (l >> 5);
  float v[8];
  if (m < M && vec && o0 + 8 <= N) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(dy + (int64_t)m * N + o0);
    const f32x4 b = *reinterpret_cast<const f32x4*>(dy + (int64_t)m * N + o0 + 4);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[j] = a[j];
      v[4 + j] = b[j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = (m < M && o0 + j < N) ? dy[(int64_t)m * N + o0 + j] : 0.0f;
  }
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    hi[j] = pack2_bf16(v[2 * j], v[2 * j + 1]);
    lo[j] = pack2_bf16(v[2 * j] - __uint_as_float(hi[j] << 16), v[2 * j + 1] - __uint_as_float(hi[j] & 0xFFFF0000u));
  }
  *reinterpret_cast<u32x4*>(dyf + (f * 2) * kDxmFrag + l * 8) = u32x4{hi[0], hi[1], hi[2], hi[3]};
  *reinterpret_cast<u32x4*>(dyf + (f * 2 + 1) * kDxmFrag + l * 8) = u32x4{lo[0], lo[1], lo[2], lo[3]};
}

template <int FMT, typename ST>
__global__ __launch_bounds__(kDxmThreads) void dx_mf_kernel(const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                                            const uint16_t* __restrict__ dyf, float* __restrict__ dx,
                                                            float* __restrict__ part, int M, int K, int npad,
                                                            int tiles_m, int gps) {
  constexpr float OFF = FMT == RQ_Q8_0 ? 128.0f : 8.0f;
  // B fragments: [buffer][group][block][hi, lo][64 lanes x 8 bf16]
  __shared__ __attribute__((aligned(16))) uint16_t bs[2][kDxmG][kDxmNB][2][kDxmFrag];

  const int nkb = K / 32, ngroups = npad / 16, mt_n = (M + 31) / 32;
  // Tile order: column strip major, the row tiles of a strip (which read the
  // same weight chunks) consecutive, each XCD a contiguous run of that order
  const int nblk = (int)gridDim.x, bid = (int)blockIdx.x;
  const int xcd = bid & 7, per = nblk >> 3, rem = nblk & 7;
  const int tord = xcd * per + (xcd < rem ? xcd : rem) + (bid >> 3);
  const int tm = tord % tiles_m, ti = tord / tiles_m;
  // this workgroup's slice of the reduction: groups [g0, g0 + ng)
  const int sl = (int)blockIdx.y, g0 = min(sl * gps, npad / 16), ng = min(npad / 16 - g0, gps);
  const int tid = (int)threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 3, kh = wave >> 2;  // 32-row tile, group parity within a step
  const int mt = tm * 4 + wm;          // this wave's 32-row tile
  const int mtc = min(mt, mt_n - 1);   // clamped for loads (rows past M are never stored)
  const int b0 = ti * kDxmNB;          // the workgroup's first column block

  // ---- weight producer: wave -> chunk (group gs of the step, block cb);
  // lane -> rows 2 rp, 2 rp + 1 and columns 4 cq .. 4 cq + 3 of it
  const int gs = wave >> 2, cb = wave & 3, rp = lane >> 3, cq = lane & 7;
  const int bcol = min(b0 + cb, nkb - 1);  // a block past K is computed, never stored
  uint32_t wv[kDxmDB][2];  // [ring slot][row]: the 4 codes (Q8) / the byte holding them (Q4)
  uint32_t sv[kDxmDB][2];  // [ring slot][row]: scale bits as stored
  auto load_b = [&](int slot, int step) {
    const int g = g0 + min(step * kDxmG + gs, ng - 1);
    const int64_t chunk = (int64_t)g * nkb + bcol;
#pragma unroll
    for (int rr = 0; rr < 2; rr++) {
      const int row = 2 * rp + rr;
      // Q4: byte j of a row holds column j (low nibble) and j + 16 (high)
      wv[slot][rr] = FMT == RQ_Q8_0
                         ? *reinterpret_cast<const uint32_t*>(q + chunk * 512 + row * 32 + 4 * cq)
                         : *reinterpret_cast<const uint32_t*>(q + chunk * 256 + row * 16 + 4 * (cq & 3));
      sv[slot][rr] = load_scale_bits<ST>(sc, chunk * 16 + row);
    }
  };
  // Dequantize the slot's 8 elements and write them, transposed, into
  // buffer `buf`: element (row, col) of the chunk belongs to B-operand lane
  // L = col + 32 (row / 8), position row % 8 (rows 2 rp, 2 rp + 1 share a
  // dword). Lane L's 16 bytes sit in slot L ^ swz(L), swz(L) = bit 3 of L |
  // bit 5 of L << 1: the readers' 8-lane groups still cover 8 distinct slots
  // of a 128-byte window, and the 64 writers of a chunk hit 32 distinct banks.
  auto store_b = [&](int slot, int buf) {
    float s[2];
    uint32_t d[2];
#pragma unroll
    for (int rr = 0; rr < 2; rr++) {
      s[rr] = scale_from_bits<ST>(sv[slot][rr]);
      d[rr] = FMT == RQ_Q8_0 ? wv[slot][rr] ^ 0x80808080u                           // u = code + 128
                             : (wv[slot][rr] >> (cq >= 4 ? 4 : 0)) & 0x0F0F0F0Fu;  // u = code + 8
    }
    uint32_t* hib = reinterpret_cast<uint32_t*>(&bs[buf][gs][cb][0][0]);
    uint32_t* lob = reinterpret_cast<uint32_t*>(&bs[buf][gs][cb][1][0]);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float w0 = fmaf((float)((d[0] >> (8 * e)) & 0xFFu), s[0], -OFF * s[0]);
      const float w1 = fmaf((float)((d[1] >> (8 * e)) & 0xFFu), s[1], -OFF * s[1]);
      const uint32_t hp = pack2_bf16(w0, w1);  // RNE, the hardware conversion
      const uint32_t lp = pack2_bf16(w0 - __uint_as_float(hp << 16), w1 - __uint_as_float(hp & 0xFFFF0000u));
      const int L = 4 * cq + e + 32 * (rp >> 2);
      const int dw = 4 * dxm_slot(L) + (rp & 3);
      hib[dw] = hp;
      lob[dw] = lp;
    }
  };

  // ---- dy fragments of this wave: ring of kDxmAR groups
  const uint16_t* abase = dyf + (int64_t)mtc * ngroups * 2 * kDxmFrag + lane * 8;
  constexpr int AR = kDxmAR / kDxmG;  // this wave's groups in flight (every other group)
  bf16x8 ah[AR], al[AR];
  auto load_a = [&](int ri, int g) {
    const int gc = g0 + min(g, ng - 1);
    ah[ri] = *reinterpret_cast<const bf16x8*>(abase + (int64_t)gc * 2 * kDxmFrag);
    al[ri] = *reinterpret_cast<const bf16x8*>(abase + ((int64_t)gc * 2 + 1) * kDxmFrag);
  };

  f32x16 acc[kDxmNB];
#pragma unroll
  for (int c = 0; c < kDxmNB; c++)
#pragma unroll
    for (int e = 0; e < 16; e++) acc[c][e] = 0.0f;

  // Step s (groups 2 s, 2 s + 1 of the slice) reads LDS buffer s & 1; the
  // weights of step s + 1 sit in ring slot (s + 1) % kDxmDB, loaded kDxmDB
  // steps earlier; dy group g in ring entry g % kDxmAR, loaded kDxmAR / 2
  // steps earlier. The loop runs whole turns of kDxmDB steps, unrolled, so
  // that every register index is a compile-time constant, and every load is
  // unconditional (clamped past the slice): a conditional load leaves the
  // compiler unsure how many loads are in flight, and it then waits for all
  // of them. Steps past the slice compute nothing. (A third LDS buffer that
  // lets the fragments be read a step ahead measured slower: 175 against
  // 160 us at M = 512, K = 4096, N = 11008.)
  const int nsteps = (ng + kDxmG - 1) / kDxmG;
#pragma unroll
  for (int k = 0; k < kDxmDB; k++) load_b(k, k);
#pragma unroll
  for (int r = 0; r < AR; r++) load_a(r, kDxmG * r + kh);
  store_b(0, 0);
  load_b(0, kDxmDB);

  auto step = [&](int s, int P) {  // P = s % kDxmDB
    __syncthreads();  // buffer s & 1 complete; buffer (s + 1) & 1 no longer read
    const int buf = P & 1;
    bf16x8 bh[kDxmNB], bl[kDxmNB];
#pragma unroll
    for (int c = 0; c < kDxmNB; c++) {
      bh[c] = *reinterpret_cast<const bf16x8*>(&bs[buf][kh][c][0][dxm_slot(lane) * 8]);
      bl[c] = *reinterpret_cast<const bf16x8*>(&bs[buf][kh][c][1][dxm_slot(lane) * 8]);
    }
    // the next step's weights into the other buffer, then that ring slot's
    // refill (step s + 1 + kDxmDB)
    store_b((P + 1) % kDxmDB, buf ^ 1);
    load_b((P + 1) % kDxmDB, s + 1 + kDxmDB);
    {
      const int g = s * kDxmG + kh, ri = P % AR;
      const bf16x8 a_h = ah[ri], a_l = al[ri];
      if (g < ng) {  // wave-uniform
#pragma unroll
        for (int c = 0; c < kDxmNB; c++) {
          acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_h, bh[c], acc[c], 0, 0, 0);
          acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_h, bl[c], acc[c], 0, 0, 0);
          acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_l, bh[c], acc[c], 0, 0, 0);
        }
      }
      load_a(ri, g + kDxmG * AR);
    }
  };
  for (int s = 0; s < nsteps; s += kDxmDB) {
#pragma unroll
    for (int P = 0; P < kDxmDB; P++) step(s + P, P);
  }
  static_assert(kDxmDB == 4 && kDxmG == 2 && kDxmDB % AR == 0, "ring indices");

  // the pair's sum: the odd-group waves pass their accumulators through LDS,
  // two column blocks a round; the even-group waves add and store.
  // D layout: lane l holds column l % 32 of the 32x32 tile, rows
  // (r / 4) 8 + 4 (l / 32) + r % 4
  f32x16* red = reinterpret_cast<f32x16*>(&bs[0][0][0][0][0]);
  static_assert(sizeof(bs) >= 4 * 2 * 64 * sizeof(f32x16), "reduction fits");
  float* dst = gridDim.y == 1 ? dx : part + (int64_t)sl * M * K;
#pragma unroll
  for (int h = 0; h < kDxmNB / 2; h++) {
    __syncthreads();
    if (kh == 1) {
#pragma unroll
      for (int c = 0; c < 2; c++) red[(wm * 2 + c) * 64 + lane] = acc[2 * h + c];
    }
    __syncthreads();
    if (kh == 0 && mt < mt_n) {
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const int b = b0 + 2 * h + c;
        if (b >= nkb) continue;
        const f32x16 v = acc[2 * h + c] + red[(wm * 2 + c) * 64 + lane];
        const int col = 32 * b + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int m = 32 * mt + (r >> 2) * 8 + 4 * (lane >> 5) + (r & 3);
          if (m < M) dst[(int64_t)m * K + col] = v[r];
        }
      }
    }
  }
}

size_t dx_mf_pack_bytes(int64_t m, int64_t npad) { return (size_t)((m + 31) / 32) * (size_t)npad * 32 * 2 * 2; }

// Slices of the reduction: about one workgroup (8 waves) per CU, each slice
// at least 32 groups (512 rows of the weight).
int dx_mf_slices(int64_t m, int64_t in, int64_t npad, int cu_count) {
  const int64_t tiles = (m + kDxmBM - 1) / kDxmBM * ((in / 32 + kDxmNB - 1) / kDxmNB);
  const int64_t ngroups = npad / 16;
  const int64_t want = ((int64_t)std::max(cu_count, 1) + tiles - 1) / tiles;
  return (int)std::max<int64_t>(1, std::min<int64_t>(want, ngroups / 32));
}

template <int FMT, typename ST>
static hipError_t launch_dx_mf_t(const Weight& w, const float* dy, float* dx, int64_t m, void* pack, float* part,
                                 int slices, hipStream_t stream) {
  const int ngroups = (int)(w.npad / 16), nkb = (int)(w.in / 32);
  const int64_t mt_n = (m + 31) / 32;
  const int64_t nthreads = mt_n * ngroups * 64;
  const int vec = (w.out % 4 == 0 && (reinterpret_cast<uintptr_t>(dy) & 15) == 0) ? 1 : 0;
  uint16_t* dyf = static_cast<uint16_t*>(pack);
  hipLaunchKernelGGL(dx_pack_kernel, dim3((unsigned)((nthreads + 255) / 256)), dim3(256), 0, stream, dy, dyf, (int)m,
                     (int)w.out, ngroups, nthreads, vec);
  if (hipError_t e = hipGetLastError()) return e;
  const int tiles_m = (int)((m + kDxmBM - 1) / kDxmBM), tiles_i = (nkb + kDxmNB - 1) / kDxmNB;
  const int gps = (ngroups + slices - 1) / slices;
  hipLaunchKernelGGL((dx_mf_kernel<FMT, ST>), dim3((unsigned)(tiles_m * tiles_i), (unsigned)slices),
                     dim3(kDxmThreads), 0, stream, w.q, static_cast<const ST*>(w.scales), dyf, dx, part, (int)m,
                     (int)w.in, (int)w.npad, tiles_m, gps);
  if (hipError_t e = hipGetLastError()) return e;
  if (slices > 1) return launch_split_reduce(part, dx, m * w.in, slices, RQ_F32, stream, nullptr, nullptr);
  return hipSuccess;
}

hipError_t launch_dx_mf(const Weight& w, const float* dy, float* dx, int64_t m, void* pack, float* part, int slices,
                        hipStream_t stream) {
  if (w.format == RQ_Q8_0) return launch_dx_mf_t<RQ_Q8_0, float>(w, dy, dx, m, pack, part, slices, stream);
  if (w.scale_dtype == RQ_F16) return launch_dx_mf_t<RQ_Q4_0, uint16_t>(w, dy, dx, m, pack, part, slices, stream);
  return launch_dx_mf_t<RQ_Q4_0, float>(w, dy, dx, m, pack, part, slices, stream);
}

}  // namespace rq
