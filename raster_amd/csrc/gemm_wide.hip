// gemm_wide.hip — prefill GEMMs for bf16 activations on 32x32x16 bf16 MFMA:
// gemm_wide_kernel (one wave per SIMD, 256 x 192 tiles over the whole K,
// M >= 1024 at N = 11008) and gemm_rs_kernel (256 x 96 / 256 x 128 tiles,
// eight waves split into MFMA consumers and dequantizing producers: C2 and
// C5 at M = 256). Both read the activations from the pack_x32 copy.
//
// y[m, o] = sum_k x[m, k] * W[o, k],  W[o, k] = scale[o, k/32] * code[o, k]
//
// Each weight element is dequantized once per workgroup, exactly as the other
// bf16 GEMMs do it: the f32 product scale * code with one IEEE rounding
// (Raster's dequant, raster/quant/train.clj:60-71), then RNE to bf16.
//
// Why 256 x 192 (gemm_wide_kernel). Per CU the global-load return path delivers ~50 B/clk and
// the LDS ~114 B/clk (measured on MI355X). A 256-row x 192-column tile pulls
// 256 x 64 B of activations and 192 x 36 B of weights per 32-k step, against
// 256 * 192 * 64 flop: 30 B/clk at the full MFMA rate (a 256 x 96 tile needs
// 52). The four waves each own 64 rows (two 32-row activation fragments,
// loaded straight into registers, never shared) and all 192 columns, so every
// dequantized weight fragment in LDS is read by the four waves once per
// k-step (78 B/clk at the full rate). A 64 x 192 f32 accumulator tile is 192
// registers per lane: one wave per SIMD, accumulators in AGPRs. 32x32x16
// MFMAs leave room for the dequantization's VALU work between them
// (measured: 4 VALU per MFMA cost ~2% with 32x32x16, ~24% with 16x16x32).
//
// Activations: pack_x32_kernel first copies x (row-major bf16) into the
// operand order of the 32x32x16 MFMA: per 32-row tile, 32-k step and half j,
// one contiguous kilobyte in which lane l holds row l % 32, k = 16 (l / 32) +
// 8 j + 0..7. The weight fragments use the same k order: a lane loads 16
// codes of its column, k = 16 (l / 32) + 0..15, codes 0..7 feed half 0 and
// 8..15 half 1, so no lane exchange is needed.
//
// Output: the accumulator layout puts one row in each lane, so direct stores
// write 8 or 16 bytes into 32 rows per instruction (partial cache lines,
// ~9 us of 92 at M 1024); the tile goes through LDS instead, 32 rows at a
// time, and leaves as whole-row 16-byte pieces.
#include "rq_internal.h"

namespace rq {

namespace {

// Buffer resources over whole arrays. Offsets are 32-bit: a per-lane part
// fixed for the kernel (clamped once, at the start) in a VGPR and the k
// offset of the step, uniform, in an SGPR, so a load costs no VALU work.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t wd_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// One 32-column x 32-k weight unit for one lane: 16 elements of its column
struct WdCodes {
  u32x4 v;     // Q8: codes k = 16 g + 0..15 of the lane's column; Q4: the column's 16 packed bytes
  uint32_t s;  // scale bits
};

// lo / so: the lane's byte offsets of its column's chunk row (codes) and
// scale at block 0; kb: the 32-k block (uniform)
template <int FMT, typename ST>
__device__ __forceinline__ void wd_load(WdCodes& c, __amdgpu_buffer_rsrc_t qr, __amdgpu_buffer_rsrc_t sr,
                                        uint32_t lo, uint32_t so, uint32_t kb) {
  constexpr uint32_t CB = FMT == RQ_Q8_0 ? 512 : 256;
  c.v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, (int)lo, (int)(kb * CB), 0));
  if (sizeof(ST) == 4)
    c.s = __builtin_amdgcn_raw_buffer_load_b32(sr, (int)so, (int)(kb * 64u), 0);
  else
    c.s = __builtin_amdgcn_raw_buffer_load_b16(sr, (int)so, (int)(kb * 32u), 0);
}

// the unit's two bf16x8 fragments (half 0: codes 0..7, half 1: codes 8..15)
template <int FMT, typename ST>
__device__ __forceinline__ void wd_dequant(const WdCodes& c, int g, bf16x8& f0, bf16x8& f1) {
  const float s = scale_from_bits<ST>(c.s);
  if (FMT == RQ_Q8_0) {
    u32x2 p[4];
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = q8_dword_bf16(c.v[i], s);
    f0 = __builtin_bit_cast(bf16x8, u32x4{p[0][0], p[0][1], p[1][0], p[1][1]});
    f1 = __builtin_bit_cast(bf16x8, u32x4{p[2][0], p[2][1], p[3][0], p[3][1]});
    return;
  }
  // Q4_0: lanes of half g = 0 take the low nibbles (elements 0..15 of the
  // block), g = 1 the high nibbles (16..31): fma(q, s, -8 s) = s * (q - 8)
  const int sh = 4 * g;
  uint32_t d[4];
#pragma unroll
  for (int i = 0; i < 4; i++) d[i] = (c.v[i] >> sh) & 0x0F0F0F0Fu;
  // opaque to the known-bits fold (a v_bfe per nibble): the byte-select
  // conversions below then read the bytes of d directly
  asm("" : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]));
  const float off = -8.0f * s;
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    o[2 * i] = pack2_bf16(fmaf((float)(d[i] & 0xFFu), s, off), fmaf((float)((d[i] >> 8) & 0xFFu), s, off));
    o[2 * i + 1] = pack2_bf16(fmaf((float)((d[i] >> 16) & 0xFFu), s, off), fmaf((float)(d[i] >> 24), s, off));
  }
  f0 = __builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]});
  f1 = __builtin_bit_cast(bf16x8, u32x4{o[4], o[5], o[6], o[7]});
}

}  // namespace

// x[M][K] (bf16) -> xf[M/32][K/32][2][64][8]: fragment (tile, kb, j), lane l =
// row l % 32 of the tile, k = 32 kb + 16 (l / 32) + 8 j + 0..7. Rows up to the
// next multiple of 32 are zero. A workgroup copies 32 rows x 64 k: thread t
// reads 16 bytes of row t / 8 (eight threads per 128 contiguous bytes).
__global__ __launch_bounds__(256) void pack_x32_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ xf,
                                                       int M, int K) {
  const int nkb = K / 32, nq = (nkb + 1) / 2;
  const int tile = blockIdx.x / nq, kb = (blockIdx.x % nq) * 2 + ((threadIdx.x & 7) >> 2);
  if (kb >= nkb) return;
  const int row = threadIdx.x >> 3, cc = threadIdx.x & 3;  // 8-k chunk cc of the k-step
  const int m = tile * 32 + row;
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (m < M) v = *reinterpret_cast<const uint4*>(x + (int64_t)m * K + 32 * kb + 8 * cc);
  const int j = cc & 1, lane = row + 32 * (cc >> 1);
  *reinterpret_cast<uint4*>(xf + ((((int64_t)tile * nkb + kb) * 2 + j) * 64 + lane) * 8) = v;
}

// One workgroup of four waves per tile. Tile: 256 rows x 32 NF
// columns; wave w owns rows 64 w .. 64 w + 63 (m fragments 0, 1).
// Macro step: two 32-k steps. Per macro step the 2 NF dequant units
// (n fragment c, k-step s) are dealt over the waves; each writes its two
// bf16x8 fragments to LDS buffer (step + 1) % 2, read by all four waves in
// the next macro step. Ring depths: activations RA - 1 macro steps ahead (RA
// register slots), weight codes RW - 1 ahead (RW slots). Loads complete in
// issue order, so each stream's distance also bounds the other's wait.
template <int FMT, typename ST, int NF, int RA, int RW>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1))) void gemm_wide_kernel(
    const uint8_t* __restrict__ q, const ST* __restrict__ sc, const uint16_t* __restrict__ xf, void* __restrict__ y,
    int M, int K, int N, int npad, int y_dtype, int tiles_m, uint32_t xf_bytes) {
  constexpr int NU = 2 * NF;           // dequant units per macro step
  constexpr int CW = (NU + 3) / 4;     // units per wave (at most)
  // unrolled macro steps: whole turns of every ring (LDS 2, RA, RW)
  constexpr int U = (RA == 3 || RW == 3) ? ((RA == 4 || RW == 4) ? 12 : 6) : 4;
  static_assert((RA == 2 || RA == 3 || RA == 4) && (RW == 2 || RW == 3 || RW == 4), "ring depths");
  static_assert(U % RA == 0 && U % RW == 0 && U % 2 == 0, "unroll covers the rings");
  // LDS: the dequantized weight ring Bs[buf][k-step][half][n frag][lane];
  // after the main loop, the output staging (4 waves x 32 rows x RS bytes)
  constexpr int RS = 400;
  constexpr int kRing = 2 * 2 * 2 * NF * 64 * 16, kStage = 4 * 32 * RS;
  __shared__ __attribute__((aligned(16))) uint8_t lds[kRing > kStage ? kRing : kStage];
  typedef bf16x8 RingT[2][2][NF][64];
  RingT* Bs = reinterpret_cast<RingT*>(lds);

  // tile order: the row tiles of a column tile adjacent, each XCD
  // (workgroup id % 8) a contiguous run of that order (one L2 fill of the
  // column tile's weights)
  const int nblk = (int)gridDim.x, bid = (int)blockIdx.x;
  const int xcd = bid & 7, per = nblk >> 3, rem = nblk & 7;
  const int tord = xcd * per + (xcd < rem ? xcd : rem) + (bid >> 3);
  const int tm = tord % tiles_m, tn = tord / tiles_m;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nkb = K / 32;
  const int steps = nkb / 2;  // macro steps of two 32-k steps
  const int m0 = tm * 256 + wave * 64;
  const int n0 = tn * 32 * NF;
  const int g = lane >> 5;  // k half of the lane inside a 32-k step

  // activation fragment (r32, kb, j) at byte ((r32 * nkb + kb) * 2 + j) * 1024
  // + 16 lane; this wave's m fragments are r32 = m0 / 32 + f, clamped to the
  // packed rows (rows past M only feed outputs that are never stored)
  const int r32_last = (M + 31) / 32 - 1;
  const __amdgpu_buffer_rsrc_t xr = wd_rsrc(xf, xf_bytes);
  const uint32_t a_lo = 16u * lane;
  uint32_t a_row[2];
#pragma unroll
  for (int f = 0; f < 2; f++)
    a_row[f] = (uint32_t)__builtin_amdgcn_readfirstlane(min(m0 / 32 + f, r32_last) * nkb);
  // weights: codes of npad/16 * nkb chunks, block-major scales npad * nkb
  constexpr uint32_t CB = FMT == RQ_Q8_0 ? 512u : 256u, RB = FMT == RQ_Q8_0 ? 32u : 16u;
  const __amdgpu_buffer_rsrc_t qr = wd_rsrc(q, (uint32_t)(npad / 16) * (uint32_t)nkb * CB);
  const __amdgpu_buffer_rsrc_t sr = wd_rsrc(sc, (uint32_t)npad * (uint32_t)nkb * (uint32_t)sizeof(ST));
  // this wave's dequant units u = wave + 4 i: n fragment u % NF, k-step u / NF.
  // The lane's column n0 + 32 c + lane % 32 is row lane % 16 of 16-row group
  // n0 / 16 + 2 c + (lane % 32) / 16 (clamped to the padded rows).
  const int g_last = npad / 16 - 1;
  uint32_t w_lo[CW], w_so[CW], w_ks[CW];
#pragma unroll
  for (int i = 0; i < CW; i++) {
    const int u = min(wave + 4 * i, NU - 1);
    const uint32_t grp = (uint32_t)min(n0 / 16 + 2 * (u % NF) + ((lane & 31) >> 4), g_last);
    w_lo[i] = grp * (uint32_t)nkb * CB + (uint32_t)(lane & 15) * RB + (FMT == RQ_Q8_0 ? 16u * (uint32_t)g : 0u);
    w_so[i] = (grp * (uint32_t)nkb * 16u + (uint32_t)(lane & 15)) * (uint32_t)sizeof(ST);
    w_ks[i] = (uint32_t)__builtin_amdgcn_readfirstlane(u / NF);  // uniform: keep it in an SGPR
  }

  f32x16 acc[2][NF];
#pragma unroll
  for (int f = 0; f < 2; f++)
#pragma unroll
    for (int c = 0; c < NF; c++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[f][c][e] = 0.0f;

  bf16x8 a[RA][2][2][2];  // [slot][m frag][k-step][half]
  WdCodes wc[RW][CW];
  bf16x8 b[2][NF];  // weight fragments of the current and the next phase

  // A macro step runs as four phases p = (k-step s, half j) = p / 2, p % 2,
  // each 2 NF MFMAs on the weight fragments read from LDS in the phase
  // before. Phases 0..2 also issue the next loads and dequantize this
  // wave's units of the next macro step; the barrier sits before phase 3,
  // after which phase 3 reads the next macro step's first fragments from the
  // other LDS buffer.
#define WD_LOAD_A(ms_, slot_, f_)                                                               \
  do {                                                                                          \
    const uint32_t so_ = (a_row[f_] + (uint32_t)(2 * min((ms_), steps - 1))) * 2048u;     \
    _Pragma("unroll") for (int s = 0; s < 2; s++)                                               \
      _Pragma("unroll") for (int j = 0; j < 2; j++) a[slot_][f_][s][j] = __builtin_bit_cast(    \
          bf16x8, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)(a_lo + 1024u * (2 * s + j)),  \
                                                        (int)so_, 0));                         \
  } while (0)
#define WD_LOAD_W(ms_, slot_)                                                                   \
  do {                                                                                          \
    const uint32_t kb_ = (uint32_t)(2 * min((ms_), steps - 1));                           \
    _Pragma("unroll") for (int i = 0; i < CW; i++)                                              \
        wd_load<FMT, ST>(wc[slot_][i], qr, sr, w_lo[i], w_so[i], kb_ + w_ks[i]);                \
  } while (0)
#define WD_DEQUANT1(slot_, i_, buf_)                                                            \
  do {                                                                                          \
    if ((i_) < CW) {                                                                            \
      bf16x8 f0_, f1_;                                                                          \
      wd_dequant<FMT, ST>(wc[slot_][(i_) < CW ? (i_) : 0], g, f0_, f1_);                        \
      const int u_ = wave + 4 * (i_);                                                           \
      if (4 * CW == NU || u_ < NU) {                                                            \
        Bs[buf_][u_ / NF][0][u_ % NF][lane] = f0_;                                              \
        Bs[buf_][u_ / NF][1][u_ % NF][lane] = f1_;                                              \
      }                                                                                         \
    }                                                                                           \
  } while (0)
#define WD_READ_B(buf_, p_, bb_)                                                                \
  do {                                                                                          \
    _Pragma("unroll") for (int c = 0; c < NF; c++) b[bb_][c] = Bs[buf_][(p_) / 2][(p_) % 2][c][lane]; \
  } while (0)
#define WD_MFMA(aslot_, p_, bb_)                                                                \
  do {                                                                                          \
    _Pragma("unroll") for (int c = 0; c < NF; c++)                                              \
      _Pragma("unroll") for (int f = 0; f < 2; f++) acc[f][c] =                                 \
          __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[bb_][c], a[aslot_][f][(p_) / 2][(p_) % 2],  \
                                                  acc[f][c], 0, 0, 0);                          \
  } while (0)
  // scheduling of one phase: its LDS reads and global loads first, then the
  // MFMAs with nv VALU instructions after each, then the LDS writes
#define WD_SCHED(nds_, nvm_, nv_, ndw_)                                                         \
  do {                                                                                          \
    __builtin_amdgcn_sched_group_barrier(0x100, (nds_), 0);                                     \
    __builtin_amdgcn_sched_group_barrier(0x020, (nvm_), 0);                                     \
    _Pragma("unroll") for (int i_ = 0; i_ < 2 * NF; i_++) {                                     \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                        \
      __builtin_amdgcn_sched_group_barrier(0x002, (nv_), 0);                                    \
    }                                                                                           \
    __builtin_amdgcn_sched_group_barrier(0x200, (ndw_), 0);                                     \
  } while (0)

  // prologue: activations of macro steps 0 .. RA-2, weight codes of
  // 0 .. RW-1, LDS buffer 0 dequantized, the first phase's fragments read
#pragma unroll
  for (int st = 0; st < RA - 1; st++) {
    WD_LOAD_A(st, st, 0);
    WD_LOAD_A(st, st, 1);
  }
#pragma unroll
  for (int st = 0; st < RW; st++) WD_LOAD_W(st, st);
#pragma unroll
  for (int i = 0; i < CW; i++) WD_DEQUANT1(0, i, 0);
  __syncthreads();
  WD_READ_B(0, 0, 0);

  // macro step ms (u = ms % U): activations of ms + RA - 1 (phases 0, 1),
  // weight codes of ms + RW (phase 2), units of ms + 1 dequantized into LDS
  // buffer (ms + 1) % 2 (phases 0..2)
  constexpr int NV = 48 / (2 * NF) + 1;  // VALU instructions between MFMAs (a unit is ~45)
#define WD_STEP(ms_, u_)                                                                        \
  do {                                                                                          \
    WD_READ_B((u_) % 2, 1, 1);                                                                  \
    WD_LOAD_A((ms_) + RA - 1, ((u_) + RA - 1) % RA, 0);                                         \
    WD_MFMA((u_) % RA, 0, 0);                                                                   \
    WD_DEQUANT1(((u_) + 1) % RW, 0, ((u_) + 1) % 2);                                            \
    WD_SCHED(NF, 4, NV, 2);                                                                     \
    __builtin_amdgcn_sched_barrier(0);                                                          \
    WD_READ_B((u_) % 2, 2, 0);                                                                  \
    WD_LOAD_A((ms_) + RA - 1, ((u_) + RA - 1) % RA, 1);                                         \
    WD_MFMA((u_) % RA, 1, 1);                                                                   \
    WD_DEQUANT1(((u_) + 1) % RW, 1, ((u_) + 1) % 2);                                            \
    WD_SCHED(NF, 4, NV, 2);                                                                     \
    __builtin_amdgcn_sched_barrier(0);                                                          \
    WD_READ_B((u_) % 2, 3, 1);                                                                  \
    WD_LOAD_W((ms_) + RW, (u_) % RW);                                                           \
    WD_MFMA((u_) % RA, 2, 0);                                                                   \
    WD_DEQUANT1(((u_) + 1) % RW, 2, ((u_) + 1) % 2);                                            \
    WD_DEQUANT1(((u_) + 1) % RW, 3, ((u_) + 1) % 2);                                            \
    WD_SCHED(NF, 2 * CW, CW > 3 ? 2 * NV : NV, 2 * (CW - 2));                                   \
    __builtin_amdgcn_sched_barrier(0);                                                          \
    __syncthreads();                                                                            \
    __builtin_amdgcn_sched_barrier(0);                                                          \
    WD_READ_B(((u_) + 1) % 2, 0, 0);                                                            \
    WD_MFMA((u_) % RA, 3, 1);                                                                   \
    __builtin_amdgcn_sched_barrier(0);                                                          \
  } while (0)

  int ms = 0;
  for (; ms + U <= steps; ms += U) {
#pragma unroll
    for (int u = 0; u < U; u++) WD_STEP(ms + u, u);
  }
#pragma unroll
  for (int u = 0; u < U - 1; u++)
    if (ms + u < steps) WD_STEP(ms + u, u);
#undef WD_STEP
#undef WD_SCHED
#undef WD_MFMA
#undef WD_READ_B
#undef WD_DEQUANT1
#undef WD_LOAD_W
#undef WD_LOAD_A

  // acc[f][c] register e: y[m][n] with m = m0 + 32 f + lane % 32 and
  // n = n0 + 32 c + 8 (e / 4) + 4 g + e % 4.
  const int mrow = lane & 31;
  const int ncols = min(32 * NF, N - n0);  // columns of this tile inside y
  const int ebytes = y_dtype == RQ_F32 ? 4 : 2;
  // staged through LDS when every row piece is a whole 16 bytes
  const bool staged = ((int64_t)N * ebytes) % 16 == 0 && (ncols * ebytes) % 16 == 0 &&
                      (reinterpret_cast<uintptr_t>(y) & 15) == 0;
  if (staged) {
    // per wave 12 KB of the LDS ring: 32 rows x (96 f32 or 192 bf16) columns,
    // rows 400 bytes apart (16 consecutive lanes then write 16 different bank
    // groups). f32 goes in two column halves.
    uint8_t* st = lds + wave * (32 * RS);
    const int halves = y_dtype == RQ_F32 ? 2 : 1;
    const int hcols = 32 * NF / halves;  // columns per round
    __syncthreads();  // every wave is done with the weight fragments in LDS
#pragma unroll
    for (int f = 0; f < 2; f++) {
      for (int hh = 0; hh < halves; hh++) {
#pragma unroll
        for (int c = 0; c < NF; c++) {
          if ((32 * c) / hcols != hh) continue;
#pragma unroll
          for (int qq = 0; qq < 4; qq++) {
            const int col = 32 * c + 8 * qq + 4 * g - hh * hcols;
            if (y_dtype == RQ_F32)
              *reinterpret_cast<f32x4*>(st + mrow * RS + col * 4) =
                  f32x4{acc[f][c][4 * qq], acc[f][c][4 * qq + 1], acc[f][c][4 * qq + 2], acc[f][c][4 * qq + 3]};
            else
              *reinterpret_cast<u32x2*>(st + mrow * RS + col * 2) =
                  u32x2{pack2_bf16(acc[f][c][4 * qq], acc[f][c][4 * qq + 1]),
                        pack2_bf16(acc[f][c][4 * qq + 2], acc[f][c][4 * qq + 3])};
          }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
        __builtin_amdgcn_wave_barrier();
        // 16-byte pieces, row by row: hcols * ebytes / 16 per row
        const int ppr = hcols * ebytes / 16;
        const int vcols = min(hcols, ncols - hh * hcols);  // columns of this round inside y
        const int vpr = vcols > 0 ? vcols * ebytes / 16 : 0;
        for (int p = lane; p < 32 * ppr; p += 64) {
          const int r = p / ppr, pc = p - r * ppr;
          const int m = m0 + 32 * f + r;
          if (m < M && pc < vpr) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(st + r * RS + pc * 16);
            // non-temporal, as in gemm_rs_kernel (M 1024: 82.2-83.4 -> 81.0-81.5 us)
            __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(static_cast<uint8_t*>(y) +
                                                                     ((int64_t)m * N + n0 + hh * hcols) * ebytes +
                                                                     pc * 16));
          }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
      }
    }
    return;
  }
  const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
#pragma unroll
  for (int f = 0; f < 2; f++) {
    const int m = m0 + 32 * f + mrow;
    if (m >= M) continue;
#pragma unroll
    for (int c = 0; c < NF; c++)
#pragma unroll
      for (int qq = 0; qq < 4; qq++) {
        const int n = n0 + 32 * c + 8 * qq + 4 * g;
        const float v[4] = {acc[f][c][4 * qq], acc[f][c][4 * qq + 1], acc[f][c][4 * qq + 2], acc[f][c][4 * qq + 3]};
        if (vec && n + 3 < N) {
          if (y_dtype == RQ_F32)
            *reinterpret_cast<float4*>(static_cast<float*>(y) + (int64_t)m * N + n) = make_float4(v[0], v[1], v[2], v[3]);
          else
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + (int64_t)m * N + n) =
                make_uint2(pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3]));
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

// Role-split variant of the 256 x 32 NF tile: eight waves, two per SIMD, one
// of each kind. Waves 0..3 (consumers) own rows 64 w .. + 63 and all of K: each
// issues only its activation loads (RA - 1 macro steps ahead, straight into
// registers, a quarter per 16-k sub-step), the LDS reads of the dequantized
// weight fragments (one sub-step ahead) and the MFMAs, so its SIMD's matrix
// pipe never waits behind dequantization. Waves 4..7 (producers) load the weight units RW - 1 macro
// steps ahead and dequantize the units of macro step s + 2 into LDS buffer
// (s + 2) % 3 while the consumers run step s; their VALU work issues beside the
// partner consumer's MFMAs. One barrier per macro step: a buffer is written two
// barriers before its first read and one barrier after its last, so the
// consumers also read the next step's first fragments before the barrier.
// The 2 NF units of a macro step (n fragment, k-step) go to producer p as
// units p and p + 4. At the end each consumer stages its tile through LDS, 32
// rows at a time, and it and its SIMD's producer each store 16 of the rows.
template <int FMT, typename ST, int NF, int RA, int RW>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2))) void gemm_rs_kernel(
    const uint8_t* __restrict__ q, const ST* __restrict__ sc, const uint16_t* __restrict__ xf, void* __restrict__ y,
    int M, int K, int N, int npad, int y_dtype, int tiles_m, uint32_t xf_bytes) {
  constexpr int NB = 3;
  constexpr int NU = 2 * NF;
  static_assert(NF == 3 || NF == 4, "column fragments per tile");
  static_assert(NU <= 8, "two units per producer at most");
  // unrolled macro steps: whole turns of the rings (lcm of the depths)
  constexpr int UC = RA % NB == 0 ? RA : RA * NB;
  constexpr int UP = RW % NB == 0 ? RW : RW * NB;
  static_assert(UC % RA == 0 && UC % NB == 0 && UP % RW == 0 && UP % NB == 0, "unroll covers the rings");
  constexpr int RS = 32 * NF * 4 + 16;
  constexpr int kRing = NB * 2 * 2 * NF * 64 * 16, kStage = 4 * 32 * RS;
  __shared__ __attribute__((aligned(16))) uint8_t lds[kRing + kStage];
  typedef bf16x8 RingT[2][2][NF][64];
  RingT* Bs = reinterpret_cast<RingT*>(lds);

  const int nblk = (int)gridDim.x, bid = (int)blockIdx.x;
  const int xcd = bid & 7, per = nblk >> 3, rem = nblk & 7;
  const int tord = xcd * per + (xcd < rem ? xcd : rem) + (bid >> 3);
  const int tm = tord % tiles_m, tn = tord / tiles_m;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 3;
  const int nkb = K / 32;
  const int steps = nkb / 2;
  const int m0 = tm * 256 + wm * 64;
  const int n0 = tn * 32 * NF;
  const int g = lane >> 5;
  const int mrow = lane & 31;
  const int ncols = min(32 * NF, N - n0);
  const int ebytes = y_dtype == RQ_F32 ? 4 : 2;
  const bool staged = ((int64_t)N * ebytes) % 16 == 0 && (ncols * ebytes) % 16 == 0 &&
                      (reinterpret_cast<uintptr_t>(y) & 15) == 0;
  uint8_t* st = lds + kRing + wm * (32 * RS);
  const int ppr = 32 * NF * ebytes / 16, vpr = ncols * ebytes / 16;

  if (wave < 4) {
    // ---- consumer ----
    const int r32_last = (M + 31) / 32 - 1;
    const __amdgpu_buffer_rsrc_t xr = wd_rsrc(xf, xf_bytes);
    const uint32_t a_lo = 16u * lane;
    uint32_t a_row[2];
#pragma unroll
    for (int f = 0; f < 2; f++)
      a_row[f] = (uint32_t)__builtin_amdgcn_readfirstlane(min(m0 / 32 + f, r32_last) * nkb * 2048);

    f32x16 acc[2][NF];
#pragma unroll
    for (int f = 0; f < 2; f++)
#pragma unroll
      for (int c = 0; c < NF; c++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[f][c][e] = 0.0f;
    bf16x8 a[RA][2][2][2];  // [slot][m frag][k-step][half]
    bf16x8 b[2][NF];

#define SC_LOAD_A(ms_, slot_, ks_)                                                              \
  do {                                                                                          \
    const uint32_t ko_ = (uint32_t)(2 * min((ms_), steps - 1) + (ks_)) * 2048u;                 \
    _Pragma("unroll") for (int f = 0; f < 2; f++)                                               \
      _Pragma("unroll") for (int j = 0; j < 2; j++) a[slot_][f][ks_][j] = __builtin_bit_cast(   \
          bf16x8, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)(a_lo + 1024u * j), (int)(a_row[f] + ko_), 0)); \
  } while (0)
#define SC_LOAD_A1(ms_, slot_, ks_, f_)                                                         \
  do {                                                                                          \
    const uint32_t ko_ = (uint32_t)(2 * min((ms_), steps - 1) + (ks_)) * 2048u;                 \
    _Pragma("unroll") for (int j = 0; j < 2; j++) a[slot_][f_][ks_][j] = __builtin_bit_cast(    \
        bf16x8, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)(a_lo + 1024u * j), (int)(a_row[f_] + ko_), 0)); \
  } while (0)
#define SC_READ_B(buf_, t_, bb_)                                                                \
  do {                                                                                          \
    _Pragma("unroll") for (int c = 0; c < NF; c++) b[bb_][c] = Bs[buf_][(t_) / 2][(t_) % 2][c][lane]; \
  } while (0)
#define SC_MFMA(slot_, t_, bb_)                                                                 \
  do {                                                                                          \
    _Pragma("unroll") for (int c = 0; c < NF; c++)                                              \
      _Pragma("unroll") for (int f = 0; f < 2; f++) acc[f][c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16( \
          b[bb_][c], a[slot_][f][(t_) / 2][(t_) % 2], acc[f][c], 0, 0, 0);                      \
  } while (0)
  // one 16-k sub-step: the next sub-step's LDS reads first, then a quarter of
  // the activation loads of macro step ms + RA - 1 (one m fragment of one
  // 32-k step: two kilobytes), then the MFMAs. Spread over the four sub-steps
  // the loads keep the CU's load-return path evenly busy; issued in two bursts
  // (the four consumers' 32 KB right after the barrier) the same kernel took
  // 46.3 against 43.7 us at C2 (bitwise the same output).
#define SC_SCHED(nvm_)                                                                          \
  do {                                                                                          \
    __builtin_amdgcn_sched_group_barrier(0x100, NF, 0);                                         \
    __builtin_amdgcn_sched_group_barrier(0x020, (nvm_), 0);                                     \
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * NF, 0);                                     \
  } while (0)
#define SC_STEP(ms_, u_)                                                                        \
  do {                                                                                          \
    SC_READ_B((u_) % NB, 1, 1);                                                                 \
    SC_LOAD_A1((ms_) + RA - 1, ((u_) + RA - 1) % RA, 0, 0);                                     \
    SC_MFMA((u_) % RA, 0, 0);                                                                   \
    SC_SCHED(2);                                                                                \
    __builtin_amdgcn_sched_barrier(0);                                                          \
    SC_READ_B((u_) % NB, 2, 0);                                                                 \
    SC_LOAD_A1((ms_) + RA - 1, ((u_) + RA - 1) % RA, 0, 1);                                     \
    SC_MFMA((u_) % RA, 1, 1);                                                                   \
    SC_SCHED(2);                                                                                \
    __builtin_amdgcn_sched_barrier(0);                                                          \
    SC_READ_B((u_) % NB, 3, 1);                                                                 \
    SC_LOAD_A1((ms_) + RA - 1, ((u_) + RA - 1) % RA, 1, 0);                                     \
    SC_MFMA((u_) % RA, 2, 0);                                                                   \
    SC_SCHED(2);                                                                                \
    __builtin_amdgcn_sched_barrier(0);                                                          \
    SC_READ_B(((u_) + 1) % NB, 0, 0);                                                           \
    SC_LOAD_A1((ms_) + RA - 1, ((u_) + RA - 1) % RA, 1, 1);                                     \
    SC_MFMA((u_) % RA, 3, 1);                                                                   \
    SC_SCHED(2);                                                                                \
    __builtin_amdgcn_sched_barrier(0);                                                          \
    __syncthreads();                                                                            \
    __builtin_amdgcn_sched_barrier(0);                                                          \
  } while (0)
#pragma unroll
    for (int s = 0; s < RA - 1; s++) {
      SC_LOAD_A(s, s, 0);
      SC_LOAD_A(s, s, 1);
    }
    __syncthreads();  // buffers 0 and 1 dequantized
    SC_READ_B(0, 0, 0);
    int ms = 0;
    for (; ms + UC <= steps; ms += UC) {
#pragma unroll
      for (int u = 0; u < UC; u++) SC_STEP(ms + u, u);
    }
#pragma unroll
    for (int u = 0; u < UC - 1; u++)
      if (ms + u < steps) SC_STEP(ms + u, u);
#undef SC_STEP
#undef SC_LOAD_A1
#undef SC_SCHED
#undef SC_MFMA
#undef SC_READ_B
#undef SC_LOAD_A

    // acc[f][c] register e: m = m0 + 32 f + lane % 32, n = n0 + 32 c + 8 (e / 4) + 4 g + e % 4
    if (staged) {
#pragma unroll
      for (int f = 0; f < 2; f++) {
        __syncthreads();  // the previous round's rows are stored
#pragma unroll
        for (int c = 0; c < NF; c++)
#pragma unroll
          for (int qq = 0; qq < 4; qq++) {
            const int col = 32 * c + 8 * qq + 4 * g;
            if (y_dtype == RQ_F32)
              *reinterpret_cast<f32x4*>(st + mrow * RS + col * 4) =
                  f32x4{acc[f][c][4 * qq], acc[f][c][4 * qq + 1], acc[f][c][4 * qq + 2], acc[f][c][4 * qq + 3]};
            else
              *reinterpret_cast<u32x2*>(st + mrow * RS + col * 2) =
                  u32x2{pack2_bf16(acc[f][c][4 * qq], acc[f][c][4 * qq + 1]),
                        pack2_bf16(acc[f][c][4 * qq + 2], acc[f][c][4 * qq + 3])};
          }
        __syncthreads();  // rows staged
        for (int p = lane; p < 16 * ppr; p += 64) {
          const int r = p / ppr, pc = p % ppr;
          const int m = m0 + 32 * f + r;
          if (m < M && pc < vpr) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(st + r * RS + pc * 16);
            // non-temporal: y is read by no one in this call, and kept out of L2
            // it costs the next call's activations and weights less
            // (C2: 44.6-44.8 -> 44.0-44.3 us, bitwise the same)
            __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(static_cast<uint8_t*>(y) +
                                                                     ((int64_t)m * N + n0) * ebytes + pc * 16));
          }
        }
      }
      return;
    }
    const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
#pragma unroll
    for (int f = 0; f < 2; f++) {
      const int m = m0 + 32 * f + mrow;
      if (m >= M) continue;
#pragma unroll
      for (int c = 0; c < NF; c++)
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
          const int n = n0 + 32 * c + 8 * qq + 4 * g;
          const float v[4] = {acc[f][c][4 * qq], acc[f][c][4 * qq + 1], acc[f][c][4 * qq + 2], acc[f][c][4 * qq + 3]};
          if (vec && n + 3 < N) {
            if (y_dtype == RQ_F32)
              *reinterpret_cast<float4*>(static_cast<float*>(y) + (int64_t)m * N + n) = make_float4(v[0], v[1], v[2], v[3]);
            else
              *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + (int64_t)m * N + n) =
                  make_uint2(pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3]));
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
    return;
  }

  // ---- producer ----
  const int p = wave - 4;
  constexpr uint32_t CB = FMT == RQ_Q8_0 ? 512u : 256u, RB = FMT == RQ_Q8_0 ? 32u : 16u;
  const __amdgpu_buffer_rsrc_t qr = wd_rsrc(q, (uint32_t)(npad / 16) * (uint32_t)nkb * CB);
  const __amdgpu_buffer_rsrc_t sr = wd_rsrc(sc, (uint32_t)npad * (uint32_t)nkb * (uint32_t)sizeof(ST));
  const bool has2 = p + 4 < NU;  // the second unit (waves 4, 5 at NF 3; all at NF 4)
  const int g_last = npad / 16 - 1;
  int uu[2];
  uint32_t w_lo[2], w_so[2], w_ks[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    uu[i] = min(p + 4 * i, NU - 1);
    const uint32_t grp = (uint32_t)min(n0 / 16 + 2 * (uu[i] % NF) + ((lane & 31) >> 4), g_last);
    w_lo[i] = grp * (uint32_t)nkb * CB + (uint32_t)(lane & 15) * RB + (FMT == RQ_Q8_0 ? 16u * (uint32_t)g : 0u);
    w_so[i] = (grp * (uint32_t)nkb * 16u + (uint32_t)(lane & 15)) * (uint32_t)sizeof(ST);
    w_ks[i] = (uint32_t)__builtin_amdgcn_readfirstlane(uu[i] / NF);
  }
  WdCodes wc[RW][2];
#define SP_LOAD(ms_, slot_)                                                                     \
  do {                                                                                          \
    _Pragma("unroll") for (int i = 0; i < 2; i++) wd_load<FMT, ST>(wc[slot_][i], qr, sr, w_lo[i], w_so[i], \
                                                                   (uint32_t)(2 * min((ms_), steps - 1)) + w_ks[i]); \
  } while (0)
#define SP_DEQUANT(slot_, buf_)                                                                 \
  do {                                                                                          \
    _Pragma("unroll") for (int i = 0; i < 2; i++) {                                             \
      if (i == 0 || has2) {                                                                     \
        bf16x8 f0_, f1_;                                                                        \
        wd_dequant<FMT, ST>(wc[slot_][i], g, f0_, f1_);                                         \
        Bs[buf_][uu[i] / NF][0][uu[i] % NF][lane] = f0_;                                        \
        Bs[buf_][uu[i] / NF][1][uu[i] % NF][lane] = f1_;                                        \
      }                                                                                         \
    }                                                                                           \
  } while (0)
#define SP_STEP(ms_, u_)                                                                        \
  do {                                                                                          \
    SP_LOAD((ms_) + RW - 1, ((u_) + RW - 1) % RW);                                              \
    SP_DEQUANT(((u_) + 2) % RW, ((u_) + 2) % NB);                                               \
    __builtin_amdgcn_sched_barrier(0);                                                          \
    __syncthreads();                                                                            \
    __builtin_amdgcn_sched_barrier(0);                                                          \
  } while (0)
#pragma unroll
  for (int s = 0; s < RW - 1; s++) SP_LOAD(s, s);
  SP_DEQUANT(0, 0);
  SP_DEQUANT(1, 1);
  __syncthreads();
  int ms = 0;
  for (; ms + UP <= steps; ms += UP) {
#pragma unroll
    for (int u = 0; u < UP; u++) SP_STEP(ms + u, u);
  }
#pragma unroll
  for (int u = 0; u < UP - 1; u++)
    if (ms + u < steps) SP_STEP(ms + u, u);
#undef SP_STEP
#undef SP_DEQUANT
#undef SP_LOAD
  if (!staged) return;
#pragma unroll
  for (int f = 0; f < 2; f++) {
    __syncthreads();
    __syncthreads();
    for (int pp = lane; pp < 16 * ppr; pp += 64) {
      const int r = 16 + pp / ppr, pc = pp % ppr;
      const int m = m0 + 32 * f + r;
      if (m < M && pc < vpr) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(st + r * RS + pc * 16);
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(static_cast<uint8_t*>(y) +
                                                                 ((int64_t)m * N + n0) * ebytes + pc * 16));
      }
    }
  }
}

// ---- planning and launch ---------------------------------------------------

// Taken where the 256 x 192 tiles fill their rounds of the CUs to at least 80%
// (M 1024, N 11008: 232 tiles, 92.5 us against 103 us for the 8-wave 256 x 96
// GEMM of gemm_bf16.hip, which keeps the other shapes). Splitting K in two to
// fill the CUs at M 512 (C2) measured slower (68 against 50 us): the partial
// tiles' round trip through memory, written back from one XCD's L2 and read
// after an invalidate on another, cost ~15 us. A 256 x 224 tile does not fit
// the register file without spilling.
WidePlan plan_gemm_wide(int64_t m, int64_t k, int64_t npad, int cu_count) {
  WidePlan p{};
  if (m <= 128 || cu_count <= 0 || k % 64 != 0) return p;
  const int64_t tiles_m = (m + 255) / 256, tiles_n = (npad + 191) / 192;
  const int64_t units = tiles_m * tiles_n, rounds = (units + cu_count - 1) / cu_count;
  if (units * 5 < rounds * cu_count * 4) return p;
  p.ok = true;
  p.tiles_m = (int)tiles_m;
  p.tiles_n = (int)tiles_n;
  return p;
}

size_t pack_x32_bytes(int64_t m, int64_t k) { return (size_t)((m + 31) / 32 * 32) * (size_t)k * 2; }

hipError_t launch_pack_x32(const MatmulArgs& a) {
  const int64_t blocks = (a.m + 31) / 32 * ((a.k / 32 + 1) / 2);
  hipExtLaunchKernelGGL(pack_x32_kernel, dim3((unsigned)blocks), dim3(256), 0, a.stream, nullptr, a.ev_main[0], 0,
                        static_cast<const uint16_t*>(a.x), static_cast<uint16_t*>(a.scratch), (int)a.m, (int)a.k);
  return hipGetLastError();
}

// Role-split ring depths: activation slots (loads RA - 1 macro steps ahead),
// weight units in flight (RW - 1 ahead). Measured at the C2 shape: RA 3
// against 4 (52.8 against 56.6 us kernel; at NF 4, RA 4 exceeds the
// register budget and spills).
constexpr int kRsRA = 3, kRsRW = 6;
template <int FMT, typename ST, int NF>
static hipError_t launch_rs_t(const MatmulArgs& a, int tiles_m, int tiles_n) {
  hipExtLaunchKernelGGL((gemm_rs_kernel<FMT, ST, NF, kRsRA, kRsRW>), dim3((unsigned)(tiles_m * tiles_n)), dim3(512), 0,
                        a.stream, nullptr, a.ev_main[1], 0, a.q, static_cast<const ST*>(a.scales),
                        static_cast<const uint16_t*>(a.scratch), a.y, (int)a.m, (int)a.k, (int)a.n, (int)a.npad,
                        a.y_dtype, tiles_m, (uint32_t)pack_x32_bytes(a.m, a.k));
  return hipGetLastError();
}

hipError_t launch_gemm_rs(const MatmulArgs& a, int nf) {
  if ((nf != 3 && nf != 4) || a.k % 64 != 0) return hipErrorInvalidValue;
  const int tiles_m = (int)((a.m + 255) / 256), tiles_n = (int)((a.npad + 32 * nf - 1) / (32 * nf));
  if (hipError_t e = launch_pack_x32(a)) return e;
#define RQ_RS(FMT_, ST_) \
  return nf == 3 ? launch_rs_t<FMT_, ST_, 3>(a, tiles_m, tiles_n) : launch_rs_t<FMT_, ST_, 4>(a, tiles_m, tiles_n);
  if (a.format == RQ_Q8_0) { RQ_RS(RQ_Q8_0, float) }
  if (a.scale_dtype == RQ_F16) { RQ_RS(RQ_Q4_0, uint16_t) }
  RQ_RS(RQ_Q4_0, float)
#undef RQ_RS
}

template <int FMT, typename ST>
static hipError_t launch_wide_t(const MatmulArgs& a, const WidePlan& p) {
  hipExtLaunchKernelGGL((gemm_wide_kernel<FMT, ST, 6, 2, 4>), dim3((unsigned)(p.tiles_m * p.tiles_n)), dim3(256), 0,
                        a.stream, nullptr, a.ev_main[1], 0, a.q, static_cast<const ST*>(a.scales),
                        static_cast<const uint16_t*>(a.scratch), a.y, (int)a.m, (int)a.k, (int)a.n, (int)a.npad,
                        a.y_dtype, p.tiles_m, (uint32_t)pack_x32_bytes(a.m, a.k));
  return hipGetLastError();
}

hipError_t launch_gemm_wide(const MatmulArgs& a, const WidePlan& p) {
  if (!p.ok) return hipErrorInvalidValue;
  if (hipError_t e = launch_pack_x32(a)) return e;
  if (a.format == RQ_Q8_0) return launch_wide_t<RQ_Q8_0, float>(a, p);
  if (a.scale_dtype == RQ_F16) return launch_wide_t<RQ_Q4_0, uint16_t>(a, p);
  return launch_wide_t<RQ_Q4_0, float>(a, p);
}

}  // namespace rq
