// gemm_bf16.hip — prefill-regime GEMM for bf16 activations on CDNA4 bf16 MFMA.
//
// y[m, o] = sum_k x[m, k] * W[o, k],  W[o, k] = scale[o, k/32] * code[o, k]
//
// The weight tile is dequantized once per workgroup into LDS: the f32 product
// scale * code is formed exactly as Raster's dequant (one IEEE f32 rounding of
// the exact product, raster/quant/train.clj:60-71) and rounded to bf16 (RNE)
// for the MFMA operand; accumulation is f32 over the whole K. With the scale
// folded into the operand there is no per-block epilogue, so the inner loop is
// MFMA plus a small dequant that overlaps it. (The f32-activation GEMM in
// gemm.hip keeps integer codes as operands and applies the scale per block,
// which is exact but costs one FMA per output per 32-block.)
//
// Mapping: 256 threads = 4 waves stacked along M, each wave WM x 16 rows and
// the whole BN-column tile (BN/16 MFMA column tiles). Activations are not
// shared between waves, so each wave loads its A fragments straight from global
// memory into registers (2 k-steps ahead); only the dequantized weight tile,
// which all four waves read, goes through LDS (three buffers, one barrier per
// 32-wide k-step): while step s runs its MFMAs, step s+1's fragments are read
// from LDS and step s+2's codes are dequantized into the third buffer.
#include "rq_internal.h"

namespace rq {

namespace {

constexpr int LDB = 40;  // bf16 per LDS weight row: 32 + 8 pad (80-byte stride)

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  bf16x2_t v = {(__bf16)a, (__bf16)b};  // v_cvt_pk_bf16_f32, round to nearest even
  return __builtin_bit_cast(uint32_t, v);
}

// One loader thread's share of a 32-wide k-step of the weight tile: 16 elements
// of one row. Q8: bytes [16h, 16h+16) of the row's block. Q4: bytes [8h, 8h+8)
// of the 16-byte block, i.e. elements [8h, 8h+8) (low nibbles) and
// [16+8h, 16+8h+8) (high nibbles).
template <int FMT>
struct BChunk {
  uint4 v;
  float s;
};

// Loads are unconditional: out-of-range rows and k-steps are clamped to valid
// addresses so the pipelined loop has no branches (the compiler can then wait
// for exactly the load it needs instead of every outstanding one). A clamped
// weight row only feeds output columns that are never stored. In the chunked
// layout the 2*BN loader threads of a k-step read whole 512-byte (Q8) or
// 256-byte (Q4) chunks: one wave instruction covers two chunks.
template <int FMT, typename ST>
__device__ __forceinline__ void load_bchunk(BChunk<FMT>& c, const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                            int row, int half, int kb, int nkb) {
  if (FMT == RQ_Q8_0) {
    c.v = *reinterpret_cast<const uint4*>(q + code_off<FMT>(row, kb, nkb) + 16 * half);
  } else {
    const uint2 t = *reinterpret_cast<const uint2*>(q + code_off<FMT>(row, kb, nkb) + 8 * half);
    c.v = make_uint4(t.x, t.y, 0u, 0u);
  }
  c.s = load_scale<ST>(sc, scale_off(row, kb, nkb));
}

// Dequantize a chunk (exact f32 scale*code, then bf16 RNE) into an LDS row.
template <int FMT>
__device__ __forceinline__ void store_bchunk(const BChunk<FMT>& c, uint16_t* __restrict__ brow, int half) {
  const float s = c.s;
  if (FMT == RQ_Q8_0) {
    // signed code c = u - 128 with u = byte ^ 0x80; fma(u, s, -128 s) = s * c exactly rounded once
    const float off = -128.0f * s;
    const uint32_t d[4] = {c.v.x ^ 0x80808080u, c.v.y ^ 0x80808080u, c.v.z ^ 0x80808080u, c.v.w ^ 0x80808080u};
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float w0 = fmaf((float)(d[i] & 0xFFu), s, off);
      const float w1 = fmaf((float)((d[i] >> 8) & 0xFFu), s, off);
      const float w2 = fmaf((float)((d[i] >> 16) & 0xFFu), s, off);
      const float w3 = fmaf((float)(d[i] >> 24), s, off);
      o[2 * i] = pack2_bf16(w0, w1);
      o[2 * i + 1] = pack2_bf16(w2, w3);
    }
    uint4* dst = reinterpret_cast<uint4*>(brow + 16 * half);
    dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
    dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
  } else {
    // nibble q, zero-point 8: fma(q, s, -8 s) = s * (q - 8) exactly rounded once
    const float off = -8.0f * s;
    const uint32_t lo[2] = {c.v.x & 0x0F0F0F0Fu, c.v.y & 0x0F0F0F0Fu};
    const uint32_t hi[2] = {(c.v.x >> 4) & 0x0F0F0F0Fu, (c.v.y >> 4) & 0x0F0F0F0Fu};
    uint32_t ol[4], oh[4];
#pragma unroll
    for (int i = 0; i < 2; i++) {
      ol[2 * i] = pack2_bf16(fmaf((float)(lo[i] & 0xFFu), s, off), fmaf((float)((lo[i] >> 8) & 0xFFu), s, off));
      ol[2 * i + 1] =
          pack2_bf16(fmaf((float)((lo[i] >> 16) & 0xFFu), s, off), fmaf((float)(lo[i] >> 24), s, off));
      oh[2 * i] = pack2_bf16(fmaf((float)(hi[i] & 0xFFu), s, off), fmaf((float)((hi[i] >> 8) & 0xFFu), s, off));
      oh[2 * i + 1] =
          pack2_bf16(fmaf((float)((hi[i] >> 16) & 0xFFu), s, off), fmaf((float)(hi[i] >> 24), s, off));
    }
    *reinterpret_cast<uint4*>(brow + 8 * half) = make_uint4(ol[0], ol[1], ol[2], ol[3]);
    *reinterpret_cast<uint4*>(brow + 16 + 8 * half) = make_uint4(oh[0], oh[1], oh[2], oh[3]);
  }
}

// Instruction order inside one k-step: global loads first, then the LDS
// fragment reads, then each MFMA followed by two VALU instructions (the
// dequant of a later step hides under the MFMA pipeline), LDS writes last.
template <int NVMEM, int NDSR, int NMFMA>
__device__ __forceinline__ void rq_step_schedule() {
  __builtin_amdgcn_sched_group_barrier(0x020, NVMEM, 0);  // VMEM reads
  __builtin_amdgcn_sched_group_barrier(0x100, NDSR, 0);   // DS reads
#pragma unroll
  for (int i = 0; i < NMFMA; i++) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
  }
  __builtin_amdgcn_sched_group_barrier(0x200, 2, 0);  // DS writes
}

}  // namespace

template <int FMT, typename ST, int WM, int BN>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                                       const uint16_t* __restrict__ x, void* __restrict__ y, int M,
                                                       int K, int N, int npad, int y_dtype, int tiles_m) {
  constexpr int BM = 4 * WM * 16;
  constexpr int NT = BN / 16;
  // Three weight-tile buffers of 128 rows whatever BN is: threads beyond 2*BN
  // dequantize a clamped duplicate row into rows BN..127, which no wave reads.
  __shared__ __attribute__((aligned(16))) uint16_t Bs[3][128 * LDB];

  // XCD-aware order: workgroup b runs on XCD b % 8; give each XCD a contiguous
  // run of tiles, m-tiles of one weight tile adjacent (one L2 fill per XCD).
  const int nblk = gridDim.x, b = blockIdx.x;
  const int xcd = b & 7, per = nblk >> 3, rem = nblk & 7;
  const int tile = xcd * per + (xcd < rem ? xcd : rem) + (b >> 3);
  const int tn = tile / tiles_m, tm = tile - tn * tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, fg = lane >> 4;
  const int nkb = K / 32;

  // A fragment rows of this lane (rows past M are clamped: they only feed
  // output rows that are never stored)
  const uint16_t* arow[WM];
#pragma unroll
  for (int i = 0; i < WM; i++) {
    const int m = min(m0 + wave * WM * 16 + i * 16 + fr, M - 1);
    arow[i] = x + (int64_t)m * K + 8 * fg;
  }
  // weight loader role: 2 threads per tile row
  const int brow_l = tid >> 1, bhalf = tid & 1;
  const int brow_g = min(n0 + min(brow_l, BN - 1), npad - 1);
  const int bst = brow_l * LDB;            // this thread's LDS row
  const int bfo = fr * LDB + 8 * fg;       // this lane's fragment offset in a tile

  f32x4 acc[WM][NT];
#pragma unroll
  for (int i = 0; i < WM; i++)
#pragma unroll
    for (int j = 0; j < NT; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  bf16x8 ar[3][WM];   // A fragments of steps s, s+1, s+2
  bf16x8 bf[2][NT];   // weight fragments of steps s, s+1
  BChunk<FMT> bc[2];  // weight codes of steps s+2, s+3
#define RQ_LOAD_A(slot, kb_)                                                              \
  do {                                                                                    \
    const int64_t ko_ = (int64_t)min((kb_), nkb - 1) * 32;                                \
    _Pragma("unroll") for (int i = 0; i < WM; i++) ar[slot][i] =                          \
        *reinterpret_cast<const bf16x8*>(arow[i] + ko_);                                  \
  } while (0)
#define RQ_LOAD_B(slot, kb_) load_bchunk<FMT, ST>(bc[slot], q, sc, brow_g, bhalf, min((kb_), nkb - 1), nkb)
#define RQ_READ_F(slot, buf)                                                              \
  do {                                                                                    \
    _Pragma("unroll") for (int j = 0; j < NT; j++) bf[slot][j] =                          \
        *reinterpret_cast<const bf16x8*>(&Bs[buf][bfo + j * 16 * LDB]);                   \
  } while (0)

  RQ_LOAD_A(0, 0);
  RQ_LOAD_A(1, 1);
  RQ_LOAD_B(0, 0);
  RQ_LOAD_B(1, 1);
  store_bchunk<FMT>(bc[0], &Bs[0][bst], bhalf);
  RQ_LOAD_B(0, 2);
  store_bchunk<FMT>(bc[1], &Bs[1][bst], bhalf);
  RQ_LOAD_B(1, 3);
  __syncthreads();
  RQ_READ_F(0, 0);

  // k-step s (32 wide), software-pipelined across steps:
  //   A:      prefetch step s+2 from global into ar[(s+2) % 3]
  //   weight: read step s+1's fragments from LDS buffer (s+1) % 3 into bf[(s+1) % 2]
  //   MFMA:   ar[s % 3] x bf[s % 2]
  //   dequant the codes of step s+2 (bc[s % 2]) into LDS buffer (s+2) % 3 and
  //   refill bc[s % 2] with the codes of step s+4.
  // One barrier per step; a buffer is rewritten two steps after its fragments
  // were read. The scheduling barrier stops the compiler from hoisting the
  // dequant of a just-issued load into the step that issued it.
#define RQ_STEP(kb_, u_)                                                                  \
  do {                                                                                    \
    RQ_LOAD_A(((u_) + 2) % 3, (kb_) + 2);                                                 \
    RQ_READ_F(((u_) + 1) % 2, ((u_) + 1) % 3);                                            \
    _Pragma("unroll") for (int i = 0; i < WM; i++)                                        \
    _Pragma("unroll") for (int j = 0; j < NT; j++) acc[i][j] =                            \
        __builtin_amdgcn_mfma_f32_16x16x32_bf16(ar[(u_) % 3][i], bf[(u_) % 2][j], acc[i][j], 0, 0, 0); \
    store_bchunk<FMT>(bc[(u_) % 2], &Bs[((u_) + 2) % 3][bst], bhalf);                     \
    RQ_LOAD_B((u_) % 2, (kb_) + 4);                                                       \
    rq_step_schedule<WM + 2, NT, WM * NT>();                                                          \
    __syncthreads();                                                                      \
    __builtin_amdgcn_sched_barrier(0);                                                    \
  } while (0)

  int kb = 0;
  for (; kb + 6 <= nkb; kb += 6) {
    RQ_STEP(kb + 0, 0);
    RQ_STEP(kb + 1, 1);
    RQ_STEP(kb + 2, 2);
    RQ_STEP(kb + 3, 3);
    RQ_STEP(kb + 4, 4);
    RQ_STEP(kb + 5, 5);
  }
  if (kb + 0 < nkb) RQ_STEP(kb + 0, 0);
  if (kb + 1 < nkb) RQ_STEP(kb + 1, 1);
  if (kb + 2 < nkb) RQ_STEP(kb + 2, 2);
  if (kb + 3 < nkb) RQ_STEP(kb + 3, 3);
  if (kb + 4 < nkb) RQ_STEP(kb + 4, 4);
#undef RQ_STEP
#undef RQ_LOAD_A
#undef RQ_LOAD_B
#undef RQ_READ_F

  // epilogue: lane holds column fr of each 16x16 tile, rows 4*fg + r
#pragma unroll
  for (int i = 0; i < WM; i++)
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const int n = n0 + j * 16 + fr;
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + wave * WM * 16 + i * 16 + 4 * fg + r;
        if (m >= M) continue;
        if (y_dtype == RQ_F32)
          static_cast<float*>(y)[(int64_t)m * N + n] = acc[i][j][r];
        else
          static_cast<uint16_t*>(y)[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_bits(acc[i][j][r]);
      }
    }
}

// Tile choice: BM = 256 (4 waves x 64 rows) for M > 128, else 64 or 128;
// BN from {64, 96, 128} (two loader threads per weight row) minimising
// rounds(tiles / CUs) * (BN + 32), i.e. wave quantisation across the chip
// plus a fixed per-tile overhead.
template <int FMT, typename ST, int WM, int BN>
static hipError_t launch_t(const MatmulArgs& a) {
  constexpr int BM = 4 * WM * 16;
  const int tiles_m = (int)((a.m + BM - 1) / BM), tiles_n = (int)((a.n + BN - 1) / BN);
  dim3 grid((unsigned)(tiles_m * tiles_n));
  hipLaunchKernelGGL((gemm_bf16_kernel<FMT, ST, WM, BN>), grid, dim3(256), 0, a.stream, a.q,
                     static_cast<const ST*>(a.scales), static_cast<const uint16_t*>(a.x), a.y, (int)a.m, (int)a.k,
                     (int)a.n, (int)a.npad, a.y_dtype, tiles_m);
  return hipGetLastError();
}

template <int FMT, typename ST, int WM>
static hipError_t launch_bn(const MatmulArgs& a, int cu_count) {
  constexpr int BM = 4 * WM * 16;
  const int64_t tiles_m = (a.m + BM - 1) / BM;
  const int cands[3] = {64, 96, 128};
  int best = 128;
  int64_t best_cost = -1;
  for (int bn : cands) {
    const int64_t tiles = tiles_m * ((a.n + bn - 1) / bn);
    const int64_t rounds = (tiles + cu_count - 1) / cu_count;
    const int64_t cost = rounds * (bn + 32);
    if (best_cost < 0 || cost < best_cost) {
      best_cost = cost;
      best = bn;
    }
  }
  switch (best) {
    case 64: return launch_t<FMT, ST, WM, 64>(a);
    case 96: return launch_t<FMT, ST, WM, 96>(a);
    default: return launch_t<FMT, ST, WM, 128>(a);
  }
}

template <int FMT, typename ST>
static hipError_t launch_wm(const MatmulArgs& a, int cu_count) {
  if (a.m <= 64) return launch_bn<FMT, ST, 1>(a, cu_count);
  if (a.m <= 128) return launch_bn<FMT, ST, 2>(a, cu_count);
  return launch_bn<FMT, ST, 4>(a, cu_count);
}

hipError_t launch_gemm_bf16(const MatmulArgs& a, int cu_count) {
  if (a.format == RQ_Q8_0) return launch_wm<RQ_Q8_0, float>(a, cu_count);
  if (a.scale_dtype == RQ_F16) return launch_wm<RQ_Q4_0, uint16_t>(a, cu_count);
  return launch_wm<RQ_Q4_0, float>(a, cu_count);
}

}  // namespace rq
