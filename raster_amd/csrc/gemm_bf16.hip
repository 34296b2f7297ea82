// gemm_bf16.hip — prefill-regime GEMM for bf16 activations on CDNA4 bf16 MFMA.
//
// y[m, o] = sum_k x[m, k] * W[o, k],  W[o, k] = scale[o, k/32] * code[o, k]
//
// Each weight element is dequantized once per workgroup: the f32 product
// scale * code is formed exactly as Raster's dequant (one IEEE f32 rounding of
// the exact product, raster/quant/train.clj:60-71) and rounded to bf16 (RNE)
// for the MFMA operand; accumulation is f32 over the whole K. With the scale
// folded into the operand there is no per-block epilogue, so the inner loop is
// MFMA plus a small dequant that overlaps it. (The f32-activation GEMM in
// gemm.hip keeps integer codes as operands and applies the scale per block,
// which is exact but costs one FMA per output per 32-block.)
//
// Data flow per workgroup (4 waves side by side along N; tile BM x BN with
// BM = 16*MT rows, BN = 4 * 16*NTW columns):
//  * activations: a pack kernel first writes x in fragment-major order (every
//    16-row x 32-k MFMA operand is one contiguous kilobyte, see pack_x_kernel).
//    All four waves need the same activation rows, so each k-step's BM x 32
//    tile is loaded once (coalesced), written to LDS in that same order and
//    read back linearly by every wave (no bank conflicts).
//  * weights: each wave owns its BN/4 columns. In the chunked device layout a
//    16-row x 32-k weight fragment is one 512-byte (Q8) / 256-byte (Q4)
//    chunk, so a wave loads its fragments straight into registers with one
//    coalesced instruction each and dequantizes them there; weights never
//    touch LDS and no element is dequantized twice.
// MFMA operands are swapped (weights = A, activations = B) so each lane's
// accumulator holds 4 consecutive outputs of one row (8/16-byte stores).
// The k-loop is software-pipelined and unrolled by 6 (see RQ_STEP).
#include "rq_internal.h"

namespace rq {

namespace {

// A lane's share of one 16-row x 32-k weight fragment: the 8 codes of row fr,
// elements [8 fg, 8 fg + 8) of the block, plus the row's block scale.
//  Q8: bytes [8 fg, 8 fg + 8) of the row's 32 codes.
//  Q4: bytes [8 (fg & 1), +8) of the row's 16 packed bytes; low nibbles are
//      elements 0..15 of the block, high nibbles 16..31 (Raster's packing),
//      so fg < 2 takes low nibbles and fg >= 2 high nibbles.
struct WCodes {
  u32x2 v;
  uint32_t s;  // scale bits, converted at dequantization
};

template <int FMT, typename ST>
__device__ __forceinline__ void load_wcodes(WCodes& c, const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                            int64_t chunk, int fr, int fg) {
  if (FMT == RQ_Q8_0)
    c.v = *reinterpret_cast<const u32x2*>(q + chunk * 512 + fr * 32 + 8 * fg);
  else
    c.v = *reinterpret_cast<const u32x2*>(q + chunk * 256 + fr * 16 + 8 * (fg & 1));
  c.s = load_scale_bits<ST>(sc, chunk * 16 + fr);
}

// Dequantized fragment (8 bf16): exact f32 scale * code, one RNE rounding to bf16.
template <int FMT, typename ST>
__device__ __forceinline__ bf16x8 dequant_frag(const WCodes& c, int fg) {
  const float s = scale_from_bits<ST>(c.s);
  if (FMT == RQ_Q8_0) {
    const u32x2 p0 = q8_dword_bf16(c.v[0], s), p1 = q8_dword_bf16(c.v[1], s);
    return __builtin_bit_cast(bf16x8, u32x4{p0[0], p0[1], p1[0], p1[1]});
  }
  // Q4_0: nibble q, zero-point 8: fma(q, s, -8 s) = s * (q - 8), rounded once
  const int sh = fg >= 2 ? 4 : 0;
  uint32_t d[2] = {(c.v[0] >> sh) & 0x0F0F0F0Fu, (c.v[1] >> sh) & 0x0F0F0F0Fu};
  // opaque to the known-bits fold (a v_bfe per nibble): the byte-select
  // conversions below then read the bytes of d directly
  asm("" : "+v"(d[0]), "+v"(d[1]));
  const float off = -8.0f * s;
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    o[2 * i] = pack2_bf16(fmaf((float)(d[i] & 0xFFu), s, off), fmaf((float)((d[i] >> 8) & 0xFFu), s, off));
    o[2 * i + 1] = pack2_bf16(fmaf((float)((d[i] >> 16) & 0xFFu), s, off), fmaf((float)(d[i] >> 24), s, off));
  }
  return __builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]});
}

}  // namespace

// Fragment-major copy of the activations: x[m][k] (bf16, row-major) to
// xf[m/16][k/32][lane][8] with lane = 16 * ((k % 32) / 8) + m % 16, i.e. the
// 16 bytes lane l of an MFMA operand fragment needs. Rows up to the next
// multiple of 16 are zero. Row-major fragment loads hit 16 rows one row
// stride apart (K*2 bytes, which aliases in L1) and use half of each cache
// line; from xf every fragment is one contiguous kilobyte.
// A wave copies one fragment: lane l loads its 16 bytes straight from x and
// stores them at position l, so the wave's store is one contiguous kilobyte;
// the four waves of a workgroup take four consecutive k-blocks of one 16-row
// tile (16 rows x 256 contiguous bytes read). At C2 (x 512 x 4096) this
// measured 2.6 us alone and 1.7 us less per pack + GEMM step than a
// transposing copy through LDS with four pieces per thread.
constexpr int kPackBlocks = 4;  // k-blocks per pack workgroup, one per wave
__global__ __launch_bounds__(256) void pack_x_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ xf, int M,
                                                    int K) {
  const int nb = K / 32, nq = (nb + kPackBlocks - 1) / kPackBlocks;
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int tile = blockIdx.x / nq, b = (blockIdx.x % nq) * kPackBlocks + w;
  if (b >= nb) return;
  const int m = tile * 16 + (l & 15);
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (m < M) v = *reinterpret_cast<const uint4*>(x + (int64_t)m * K + 32 * b + 8 * (l >> 4));
  *reinterpret_cast<uint4*>(xf + (((int64_t)tile * nb + b) * 64 + l) * 8) = v;
}

template <int FMT, typename ST, int MT, int NTW, int WD = 6>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                                       const uint16_t* __restrict__ xf, void* __restrict__ y, int M,
                                                       int K, int N, int npad, int y_dtype, int tiles_m) {
  constexpr int BM = 16 * MT, BN = 64 * NTW;
  constexpr int AP = MT / 4;  // 16-byte activation pieces each thread stages per k-step
  static_assert(MT % 4 == 0, "MT must be a multiple of 4");
  // three k-steps of activation fragments, fragment-major (1 KB per 16 rows)
  __shared__ __attribute__((aligned(16))) uint16_t As[3][MT * 512];

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

  // activation staging: piece p = tid + 256 i (i < AP) of the BM x 32 step
  // tile is fragment p / 64, lane position p % 64. Fragments past the padded
  // rows are clamped (they only feed output rows that are never stored).
  const int mt_last = (M + 15) / 16 - 1;
  const uint16_t* asrc[AP];
  int adst[AP];
#pragma unroll
  for (int i = 0; i < AP; i++) {
    const int p = tid + 256 * i;
    const int mt = min(m0 / 16 + p / 64, mt_last);
    asrc[i] = xf + (int64_t)mt * nkb * 512 + (p % 64) * 8;
    adst[i] = p * 8;
  }
  // this wave's weight chunks (16-row groups, clamped to the padded rows)
  const int g_last = npad / 16 - 1;
  int64_t wchunk[NTW];
#pragma unroll
  for (int j = 0; j < NTW; j++) wchunk[j] = (int64_t)min(n0 / 16 + wave * NTW + j, g_last) * nkb;

  f32x4 acc[MT][NTW];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NTW; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // Register rings (indices are compile-time inside the 6-step unrolled body):
  //   areg: staged activation pieces of steps s+2 .. s+4 (step s+2 is
  //         written to LDS at step s and its slot refilled with step s+5)
  //   afr:  activation fragments of steps s, s+1 (read from LDS one step ahead)
  //   wc:   weight codes of steps s+1 .. s+WD (loaded WD steps ahead: the
  //         weights come from HBM, whose latency a shallower ring leaves
  //         exposed)
  //   wf:   dequantized weight fragments of steps s, s+1
  u32x4 areg[3][AP];
  bf16x8 afr[2][MT];
  static_assert(WD == 3 || WD == 6, "the 6-step unrolled body indexes the ring modulo WD");
  WCodes wc[WD][NTW];
  bf16x8 wf[2][NTW];

#define RQ_LOAD_A(slot, kb_)                                                              \
  do {                                                                                    \
    const int64_t ko_ = (int64_t)min((kb_), nkb - 1) * 512;                               \
    _Pragma("unroll") for (int i = 0; i < AP; i++) areg[slot][i] =                        \
        *reinterpret_cast<const u32x4*>(asrc[i] + ko_);                                   \
  } while (0)
#define RQ_STORE_A(slot, buf)                                                             \
  do {                                                                                    \
    _Pragma("unroll") for (int i = 0; i < AP; i++)                                        \
        *reinterpret_cast<u32x4*>(&As[buf][adst[i]]) = areg[slot][i];                     \
  } while (0)
#define RQ_READ_A(slot, buf)                                                              \
  do {                                                                                    \
    _Pragma("unroll") for (int i = 0; i < MT; i++) afr[slot][i] =                         \
        *reinterpret_cast<const bf16x8*>(&As[buf][i * 512 + lane * 8]);                   \
  } while (0)
#define RQ_LOAD_W(slot, kb_)                                                              \
  do {                                                                                    \
    const int kk_ = min((kb_), nkb - 1);                                                  \
    _Pragma("unroll") for (int j = 0; j < NTW; j++)                                       \
        load_wcodes<FMT, ST>(wc[slot][j], q, sc, wchunk[j] + kk_, fr, fg);                \
  } while (0)

  // prologue: LDS buffers 0, 1 hold steps 0, 1; areg[s % 3] holds step s
  // for s = 2, 3, 4; afr[0] and wf[0] hold step 0; wc[1 .. WD-1] hold steps
  // 1 .. WD-1.
  RQ_LOAD_A(0, 0);
  RQ_LOAD_A(1, 1);
  RQ_LOAD_A(2, 2);
#pragma unroll
  for (int st = 0; st < WD; st++) RQ_LOAD_W(st, st);
  RQ_STORE_A(0, 0);
  RQ_STORE_A(1, 1);
  RQ_LOAD_A(0, 3);
  RQ_LOAD_A(1, 4);
#pragma unroll
  for (int j = 0; j < NTW; j++) wf[0][j] = dequant_frag<FMT, ST>(wc[0][j], fg);
  __syncthreads();
  RQ_READ_A(0, 0);

  // k-step s (u = s % 6), software-pipelined:
  //   LDS:    write areg[(u+2) % 3] (step s+2) into buffer (u+2) % 3;
  //           read step s+1's activation fragments from buffer (u+1) % 3
  //   global: activation pieces of step s+5 -> areg[(u+2) % 3];
  //           weight codes of step s+WD -> wc[u % WD]
  //   MFMA:   wf[u % 2] (A operand, weights) x afr[u % 2] (B operand, activations)
  //   VALU:   dequantize wc[(u+1) % WD] (step s+1) into wf[(u+1) % 2],
  //           interleaved with the MFMAs.
  // One barrier per step: a buffer is rewritten two steps after its last read.
  // Every load is consumed at least three steps after it is issued: the
  // loads complete in issue order, so a shorter distance for either stream
  // would make the wait for it also wait for the other's recent loads.
#define RQ_STEP(kb_, u_)                                                                  \
  do {                                                                                    \
    RQ_STORE_A(((u_) + 2) % 3, ((u_) + 2) % 3);                                           \
    RQ_LOAD_A(((u_) + 2) % 3, (kb_) + 5);                                                 \
    RQ_LOAD_W((u_) % WD, (kb_) + WD);                                                     \
    RQ_READ_A(((u_) + 1) % 2, ((u_) + 1) % 3);                                            \
    __builtin_amdgcn_sched_barrier(0);                                                    \
    _Pragma("unroll") for (int j = 0; j < NTW; j++) {                                     \
      _Pragma("unroll") for (int i = 0; i < MT; i++)                                      \
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[(u_) % 2][j], afr[(u_) % 2][i], \
                                                            acc[i][j], 0, 0, 0);          \
      wf[((u_) + 1) % 2][j] = dequant_frag<FMT, ST>(wc[((u_) + 1) % WD][j], fg);              \
      __builtin_amdgcn_sched_barrier(0);                                                  \
    }                                                                                     \
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
#undef RQ_STORE_A
#undef RQ_READ_A
#undef RQ_LOAD_W

  // epilogue: acc[i][j] holds y[m][n .. n+3] with m = row fr of activation
  // tile i, n = 4 fg of this wave's weight tile j: one 8-byte (bf16) or
  // 16-byte (f32) store per lane and tile when rows are 16-byte aligned.
  const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
#pragma unroll
  for (int i = 0; i < MT; i++) {
    const int m = m0 + i * 16 + fr;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < NTW; j++) {
      const int n = n0 + (wave * NTW + j) * 16 + 4 * fg;
      const f32x4 v = acc[i][j];
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

// Workgroup-shared weights: the W waves stack along M (MT 16-row activation
// fragments each, BM = 16 MT W rows) and share NT dequantized 16-row weight
// fragments (BN = 16 NT columns) through LDS. Per k-step every weight element
// is dequantized once per workgroup and each fragment feeds W MT MFMAs;
// activation fragments go from the fragment-major copy straight into
// registers (no LDS), since no two waves use the same rows.
// Pipeline per k-step s (unrolled by R so every ring index is compile-time):
//   VMEM: activation fragments of step s+R-1 -> ring slot (s+R-1) % R, weight
//         codes of step s+R -> slot s % R (loads complete in issue order, so
//         both streams get at least R-2 steps of slack)
//   LDS:  read step s+1's weight fragments (buffer (s+1) % L) into registers;
//         write step s+2's, dequantized, into buffer (s+2) % L (L = 4 LDS
//         buffers when R is a multiple of 4, else 3, so that R steps cover
//         whole turns of every ring)
//   MFMA: step s, with the weight fragments read during step s-1
//   one barrier
template <int FMT, typename ST, int MT, int NT, int R, int WPE, int W = 4>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(WPE))) void gemm_wl_kernel(
    const uint8_t* __restrict__ q, const ST* __restrict__ sc, const uint16_t* __restrict__ xf, void* __restrict__ y,
    int M, int K, int N, int npad, int y_dtype, int tiles_m) {
  constexpr int CW = (NT + W - 1) / W;  // weight fragments a wave dequantizes per step (at most)
  constexpr int L = R % 4 == 0 ? 4 : 3;
  static_assert(R >= 4 && R % L == 0 && R % 2 == 0, "ring depth: whole turns of the LDS and fragment rings");
  __shared__ __attribute__((aligned(16))) bf16x8 Bs[L][NT][64];

  // Tile order: column tile major, row tiles (which share the column tile's
  // weights) consecutive. Workgroups are dealt to the 8 XCDs round-robin by
  // id, so ids are remapped to give each XCD a contiguous run of that order:
  // the row tiles of a column tile then meet in one XCD's L2 instead of
  // fetching the weights from HBM once per XCD.
  const int nblk = (int)gridDim.x, bid = (int)blockIdx.x;
  const int xcd = bid & 7, per = nblk >> 3, rem = nblk & 7;
  const int tord = xcd * per + (xcd < rem ? xcd : rem) + (bid >> 3);
  const int tm = tord % tiles_m, tn = tord / tiles_m;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, fg = lane >> 4;
  const int nkb = K / 32;
  const int m0 = tm * (16 * MT * W) + wave * (16 * MT);  // this wave's first row
  const int n0 = tn * (16 * NT);

  // activation fragment i of this wave (rows m0 + 16 i ..): clamped to the
  // padded rows, whose outputs are never stored
  const int mt_last = (M + 15) / 16 - 1;
  const uint16_t* asrc[MT];
#pragma unroll
  for (int i = 0; i < MT; i++) asrc[i] = xf + (int64_t)min(m0 / 16 + i, mt_last) * nkb * 512 + lane * 8;
  // weight fragments this wave dequantizes: c = wave + W j < NT
  const int g_last = npad / 16 - 1;
  int64_t wchunk[CW];
#pragma unroll
  for (int j = 0; j < CW; j++) wchunk[j] = (int64_t)min(n0 / 16 + min(wave + W * j, NT - 1), g_last) * nkb;

  f32x4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int c = 0; c < NT; c++) acc[i][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  bf16x8 a[R][MT];
  WCodes wc[R][CW];
  bf16x8 b[2][NT];

#define WL_LOAD_A(kb_)                                                                            \
  do {                                                                                            \
    const int kk_ = min((kb_), nkb - 1);                                                          \
    _Pragma("unroll") for (int i = 0; i < MT; i++) a[(kb_) % R][i] =                              \
        *reinterpret_cast<const bf16x8*>(asrc[i] + (int64_t)kk_ * 512);                           \
  } while (0)
#define WL_LOAD_W(kb_)                                                                            \
  do {                                                                                            \
    const int kk_ = min((kb_), nkb - 1);                                                          \
    _Pragma("unroll") for (int j = 0; j < CW; j++)                                                \
        load_wcodes<FMT, ST>(wc[(kb_) % R][j], q, sc, wchunk[j] + kk_, fr, fg);                   \
  } while (0)
#define WL_DEQUANT(kb_)                                                                           \
  do {                                                                                            \
    _Pragma("unroll") for (int j = 0; j < CW; j++) {                                              \
      const bf16x8 d_ = dequant_frag<FMT, ST>(wc[(kb_) % R][j], fg);                                  \
      if (wave + W * j < NT) Bs[(kb_) % L][wave + W * j][lane] = d_;                              \
    }                                                                                             \
  } while (0)
#define WL_READ_B(kb_)                                                                            \
  do {                                                                                            \
    _Pragma("unroll") for (int c = 0; c < NT; c++) b[(kb_) % 2][c] = Bs[(kb_) % L][c][lane];      \
  } while (0)
#define WL_MFMA(kb_, c0, c1)                                                                      \
  do {                                                                                            \
    _Pragma("unroll") for (int c = (c0); c < (c1); c++)                                           \
      _Pragma("unroll") for (int i = 0; i < MT; i++)                                              \
        acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[(kb_) % 2][c], a[(kb_) % R][i], acc[i][c], 0, 0, 0); \
  } while (0)

  // prologue: a holds steps 0..R-2, wc steps 0..R-1; LDS buffers 0, 1
  // hold steps 0, 1 and b[0] step 0
#pragma unroll
  for (int st = 0; st < R - 1; st++) {
    WL_LOAD_A(st);
    WL_LOAD_W(st);
  }
  WL_LOAD_W(R - 1);
  WL_DEQUANT(0);
  WL_DEQUANT(1);
  __syncthreads();
  WL_READ_B(0);

  // the step body for kb_ with compile-time residue u_ = kb_ % R
#define WL_STEP(kb_, u_)                                                                          \
  do {                                                                                            \
    WL_LOAD_A_U((kb_) + R - 1, (u_) + R - 1);                                                     \
    WL_LOAD_W_U((kb_) + R, (u_) + R);                                                             \
    WL_READ_B_U((u_) + 1);                                                                        \
    __builtin_amdgcn_sched_barrier(0);                                                            \
    WL_MFMA_U(u_, 0, NT / 2);                                                                     \
    __builtin_amdgcn_sched_barrier(0);                                                            \
    WL_DEQUANT_U((u_) + 2);                                                                       \
    __builtin_amdgcn_sched_barrier(0);                                                            \
    WL_MFMA_U(u_, NT / 2, NT);                                                                    \
    __syncthreads();                                                                              \
    __builtin_amdgcn_sched_barrier(0);                                                            \
  } while (0)
// ring indices from the residue u (a multiple-of-R shift leaves every ring
// index unchanged); the load macros take the true step for address clamping
#define WL_LOAD_A_U(kb_, u_)                                                                      \
  do {                                                                                            \
    const int kk_ = min((kb_), nkb - 1);                                                          \
    _Pragma("unroll") for (int i = 0; i < MT; i++) a[(u_) % R][i] =                               \
        *reinterpret_cast<const bf16x8*>(asrc[i] + (int64_t)kk_ * 512);                           \
  } while (0)
#define WL_LOAD_W_U(kb_, u_)                                                                      \
  do {                                                                                            \
    const int kk_ = min((kb_), nkb - 1);                                                          \
    _Pragma("unroll") for (int j = 0; j < CW; j++)                                                \
        load_wcodes<FMT, ST>(wc[(u_) % R][j], q, sc, wchunk[j] + kk_, fr, fg);                    \
  } while (0)
#define WL_READ_B_U(u_) WL_READ_B(u_)
#define WL_DEQUANT_U(u_) WL_DEQUANT(u_)
#define WL_MFMA_U(u_, c0, c1) WL_MFMA(u_, c0, c1)

  int kb = 0;
  for (; kb + R <= nkb; kb += R) {
#pragma unroll
    for (int u = 0; u < R; u++) WL_STEP(kb + u, u);
  }
#pragma unroll
  for (int u = 0; u < R - 1; u++)
    if (kb + u < nkb) WL_STEP(kb + u, u);
#undef WL_STEP
#undef WL_LOAD_A_U
#undef WL_LOAD_W_U
#undef WL_READ_B_U
#undef WL_DEQUANT_U
#undef WL_MFMA_U
#undef WL_MFMA
#undef WL_READ_B
#undef WL_DEQUANT
#undef WL_LOAD_W
#undef WL_LOAD_A

  // epilogue: acc[i][c] holds y[m][n .. n+3], m = m0 + 16 i + fr,
  // n = n0 + 16 c + 4 fg
  const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
#pragma unroll
  for (int i = 0; i < MT; i++) {
    const int m = m0 + i * 16 + fr;
    if (m >= M) continue;
#pragma unroll
    for (int c = 0; c < NT; c++) {
      const int n = n0 + c * 16 + 4 * fg;
      const f32x4 v = acc[i][c];
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

// K-split wave pairs (8 waves, 256 x 16 NT tiles): waves w and w + 4 share a
// SIMD and own the same 64 rows (four 16-row activation fragments); wave w
// takes the even k-steps and wave w + 4 the odd ones. Per k-step each
// dequantized weight fragment in LDS is read by four waves instead of eight
// (24 KB of LDS reads per k-step at NT 6, against 48 KB when the eight waves
// stack along M), and one barrier serves two k-steps. The two waves' f32
// accumulators are added through LDS at the end (a different summation order
// from the one-wave-per-row-block kernel: two interleaved partial sums).
// Pipeline per macro step t (k-steps 2t, 2t+1; ring indices compile-time):
//   VMEM: this wave's activation fragments of macro step t+1 (two-slot ring),
//         weight codes of macro step t+R (2 NT dequant units per macro step,
//         (fragment, k parity), dealt over the 8 waves)
//   LDS:  read this wave's NT weight fragments of macro step t; write macro
//         step t+2's, dequantized, into LDS buffer (t+2) % 4
//   MFMA: 4 NT per wave, half before and half after the dequant
//   one barrier
// Measured at C2 (M 512, K 4096, N 11008): 50.1-50.8 us against 52.4-52.9 us
// for gemm_wl_kernel<.., 2, 6, 4, 2, 8>; C5 (M 256, K 8192, N 28672, NT 7):
// 121 against 123 us. Keeping the next macro step's weight fragments in
// registers (a second B buffer) measured the same at NT 6 and far slower at
// NT 7 (226 us); a four-slot activation ring 51.3-51.9 us.
template <int FMT, typename ST, int NT, int R>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void gemm_wk_kernel(
    const uint8_t* __restrict__ q, const ST* __restrict__ sc, const uint16_t* __restrict__ xf, void* __restrict__ y,
    int M, int K, int N, int npad, int y_dtype, int tiles_m) {
  constexpr int W = 8, MT = 4, L = 4, RA = 2;
  constexpr int NU = 2 * NT;            // dequant units (fragment, k parity) per macro step
  constexpr int CW = (NU + W - 1) / W;  // units per wave (at most)
  constexpr int RC = (L * 2 * NT) / (4 * MT);  // fragments per round of the final reduction
  static_assert(R >= 4 && R % L == 0, "ring depth: whole turns of the LDS ring");
  static_assert(RC >= 1, "the final reduction fits the LDS ring");
  __shared__ __attribute__((aligned(16))) bf16x8 Bs[L][2][NT][64];

  // tile order as gemm_wl_kernel: row tiles of a column tile on one XCD
  const int nblk = (int)gridDim.x, bid = (int)blockIdx.x;
  const int xcd = bid & 7, per = nblk >> 3, rem = nblk & 7;
  const int tord = xcd * per + (xcd < rem ? xcd : rem) + (bid >> 3);
  const int tm = tord % tiles_m, tn = tord / tiles_m;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 3, kh = wave >> 2;  // row block, k parity
  const int fr = lane & 15, fg = lane >> 4;
  const int nkb = K / 32;
  const int m0 = tm * (16 * MT * 4) + wm * (16 * MT);
  const int n0 = tn * (16 * NT);

  const int mt_last = (M + 15) / 16 - 1;
  const uint16_t* asrc[MT];
#pragma unroll
  for (int i = 0; i < MT; i++) asrc[i] = xf + (int64_t)min(m0 / 16 + i, mt_last) * nkb * 512 + lane * 8;
  // dequant unit u = wave + W j: k parity u / NT, weight fragment u % NT
  const int g_last = npad / 16 - 1;
  int64_t wchunk[CW];
  int upar[CW];
#pragma unroll
  for (int j = 0; j < CW; j++) {
    const int u = min(wave + W * j, NU - 1);
    upar[j] = u / NT;
    wchunk[j] = (int64_t)min(n0 / 16 + u % NT, g_last) * nkb;
  }

  f32x4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int c = 0; c < NT; c++) acc[i][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  bf16x8 a[RA][MT];
  WCodes wc[R][CW];
  bf16x8 b[NT];

#define WK_LOAD_A(t_, u_)                                                                         \
  do {                                                                                            \
    const int kk_ = min(2 * (t_) + kh, nkb - 1);                                                  \
    _Pragma("unroll") for (int i = 0; i < MT; i++) a[(u_) % RA][i] =                              \
        *reinterpret_cast<const bf16x8*>(asrc[i] + (int64_t)kk_ * 512);                           \
  } while (0)
#define WK_LOAD_W(t_, u_)                                                                         \
  do {                                                                                            \
    _Pragma("unroll") for (int j = 0; j < CW; j++) {                                              \
      const int kk_ = min(2 * (t_) + upar[j], nkb - 1);                                           \
      load_wcodes<FMT, ST>(wc[(u_) % R][j], q, sc, wchunk[j] + kk_, fr, fg);                      \
    }                                                                                             \
  } while (0)
#define WK_DEQUANT(u_)                                                                            \
  do {                                                                                            \
    _Pragma("unroll") for (int j = 0; j < CW; j++) {                                              \
      const bf16x8 d_ = dequant_frag<FMT, ST>(wc[(u_) % R][j], fg);                               \
      if (wave + W * j < NU) Bs[(u_) % L][upar[j]][(wave + W * j) % NT][lane] = d_;               \
    }                                                                                             \
  } while (0)
#define WK_READ_B(u_)                                                                             \
  do {                                                                                            \
    _Pragma("unroll") for (int c = 0; c < NT; c++) b[c] = Bs[(u_) % L][kh][c][lane];              \
  } while (0)
#define WK_MFMA(u_, c0, c1)                                                                       \
  do {                                                                                            \
    _Pragma("unroll") for (int c = (c0); c < (c1); c++)                                           \
      _Pragma("unroll") for (int i = 0; i < MT; i++)                                              \
        acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[c], a[(u_) % RA][i], acc[i][c], 0, 0, 0); \
  } while (0)
#define WK_STEP(t_, u_, live_)                                                                    \
  do {                                                                                            \
    WK_LOAD_A((t_) + RA - 1, (u_) + RA - 1);                                                      \
    WK_LOAD_W((t_) + R, (u_) + R);                                                                \
    WK_READ_B(u_);                                                                                \
    __builtin_amdgcn_sched_barrier(0);                                                            \
    if (live_) WK_MFMA(u_, 0, NT / 2);                                                            \
    __builtin_amdgcn_sched_barrier(0);                                                            \
    WK_DEQUANT((u_) + 2);                                                                         \
    __builtin_amdgcn_sched_barrier(0);                                                            \
    if (live_) WK_MFMA(u_, NT / 2, NT);                                                           \
    __syncthreads();                                                                              \
    __builtin_amdgcn_sched_barrier(0);                                                            \
  } while (0)

  // prologue: activations of macro step 0, weight codes of 0..R-1, LDS
  // buffers 0 and 1 dequantized
  WK_LOAD_A(0, 0);
#pragma unroll
  for (int st = 0; st < R; st++) WK_LOAD_W(st, st);
  WK_DEQUANT(0);
  WK_DEQUANT(1);
  __syncthreads();

  // macro steps with both k-steps present, then the rest (the last one may
  // hold only an even k-step: the odd-k waves skip its MFMAs, not its
  // barriers)
  const int nm = (nkb + 1) / 2, nfull = nkb / 2;
  int t = 0;
  for (; t + R <= nfull; t += R) {
#pragma unroll
    for (int u = 0; u < R; u++) WK_STEP(t + u, u, true);
  }
#pragma unroll
  for (int u = 0; u < R; u++)
    if (t + u < nm) WK_STEP(t + u, u, 2 * (t + u) + kh < nkb);
#undef WK_STEP
#undef WK_MFMA
#undef WK_READ_B
#undef WK_DEQUANT
#undef WK_LOAD_W
#undef WK_LOAD_A

  // the pair's sum through the LDS ring, RC fragments a round: the odd-k wave
  // writes its accumulators, the even-k wave adds them to its own and stores.
  // acc[i][c] holds y[m][n .. n+3], m = m0 + 16 i + fr, n = n0 + 16 c + 4 fg.
  f32x4* red = reinterpret_cast<f32x4*>(&Bs[0][0][0][0]);
  const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
#pragma unroll
  for (int h = 0; h < (NT + RC - 1) / RC; h++) {
    if (kh == 1) {
#pragma unroll
      for (int i = 0; i < MT; i++)
#pragma unroll
        for (int c = 0; c < RC; c++)
          if (h * RC + c < NT) red[((wm * MT + i) * RC + c) * 64 + lane] = acc[i][h * RC + c];
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
      for (int i = 0; i < MT; i++) {
        const int m = m0 + i * 16 + fr;
#pragma unroll
        for (int c = 0; c < RC; c++) {
          const int cc = h * RC + c;
          if (cc >= NT || m >= M) break;
          const f32x4 v = acc[i][cc] + red[((wm * MT + i) * RC + c) * 64 + lane];
          const int n = n0 + cc * 16 + 4 * fg;
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
    __syncthreads();
  }
}

// Kernel timing (a.ev_main set): the packing pass's end and the GEMM's end.
// A start event would put an extra packet, and an idle gap of a few
// microseconds, in front of the GEMM; the GEMM follows the packing pass
// directly, so its duration is the span between the two end events.
hipError_t launch_pack_x(const MatmulArgs& a) {
  const int64_t pack_blocks = (a.m + 15) / 16 * ((a.k / 32 + kPackBlocks - 1) / kPackBlocks);
  hipExtLaunchKernelGGL(pack_x_kernel, dim3((unsigned)pack_blocks), dim3(256), 0, a.stream, nullptr, a.ev_main[0], 0,
                        static_cast<const uint16_t*>(a.x), static_cast<uint16_t*>(a.scratch), (int)a.m, (int)a.k);
  return hipGetLastError();
}

template <int FMT, typename ST, int MT, int NTW>
static hipError_t launch_t(const MatmulArgs& a) {
  constexpr int BM = 16 * MT, BN = 64 * NTW;
  const int tiles_m = (int)((a.m + BM - 1) / BM), tiles_n = (int)((a.n + BN - 1) / BN);
  if (hipError_t e = launch_pack_x(a)) return e;
  dim3 grid((unsigned)(tiles_m * tiles_n));
  hipExtLaunchKernelGGL((gemm_bf16_kernel<FMT, ST, MT, NTW>), grid, dim3(256), 0, a.stream, nullptr,
                        a.ev_main[1], 0, a.q, static_cast<const ST*>(a.scales),
                        static_cast<const uint16_t*>(a.scratch), a.y, (int)a.m, (int)a.k, (int)a.n, (int)a.npad,
                        a.y_dtype, tiles_m);
  return hipGetLastError();
}

template <int FMT, typename ST, int MT, int NT, int R, int WPE, int W = 4>
static hipError_t launch_wl(const MatmulArgs& a) {
  const int tiles_m = (int)((a.m + 16 * MT * W - 1) / (16 * MT * W));
  const int tiles_n = (int)((a.npad / 16 + NT - 1) / NT);
  if (hipError_t e = launch_pack_x(a)) return e;
  hipExtLaunchKernelGGL((gemm_wl_kernel<FMT, ST, MT, NT, R, WPE, W>), dim3((unsigned)(tiles_m * tiles_n)), dim3(64 * W), 0,
                        a.stream, nullptr, a.ev_main[1], 0, a.q, static_cast<const ST*>(a.scales),
                        static_cast<const uint16_t*>(a.scratch), a.y, (int)a.m, (int)a.k, (int)a.n, (int)a.npad,
                        a.y_dtype, tiles_m);
  return hipGetLastError();
}

template <int FMT, typename ST, int NT>
static hipError_t launch_wk(const MatmulArgs& a) {
  const int tiles_m = (int)((a.m + 255) / 256);
  const int tiles_n = (int)((a.npad / 16 + NT - 1) / NT);
  if (hipError_t e = launch_pack_x(a)) return e;
  hipExtLaunchKernelGGL((gemm_wk_kernel<FMT, ST, NT, 4>), dim3((unsigned)(tiles_m * tiles_n)), dim3(512), 0, a.stream,
                        nullptr, a.ev_main[1], 0, a.q, static_cast<const ST*>(a.scales),
                        static_cast<const uint16_t*>(a.scratch), a.y, (int)a.m, (int)a.k, (int)a.n, (int)a.npad,
                        a.y_dtype, tiles_m);
  return hipGetLastError();
}

// Kernel and tile by M, measured with random data at M = 256, 512, 1024
// (K 4096 / 8192, N 11008 / 28672): for M > 128 the shared-weight kernel with
// 4-deep rings and two waves per SIMD is 8 to 25% faster than 128 x 128
// per-wave weights, whose tile suits smaller M. (Deeper rings make the
// compiler wait for every load.) Its tile comes from a cost model: a CU works
// through ceil(tiles / CUs) tiles on its critical path, whether side by side
// or one after another, so a tiling costs that count times the tile area.
// Candidates, ties to the first: 8 waves x 256 x 96 (two fragments of rows
// each, one workgroup per CU), 4 waves x 256 x 64 and 4 waves x 256 x 48 (two
// per CU), 8 waves x 256 x 112. (256 x 128 in this kernel would never be
// chosen: it costs at least what 256 x 64 does.) Measured (Q8, clocks settled): M = 512,
// K = 4096, N = 11008: 52.6 / 56.1 / 54.5 / 54.9 us (8 waves x 512 x 48, the
// same area: 54.8 us, its activation traffic from L2 twice that of 256 x 96);
// M = 256, K = 8192, N = 28672: 256 x 112 (256 tiles, one per CU) 122 us,
// 256 x 64 143, 256 x 48 197, 256 x 96 191, 256 x 128 123 (Q4, f16 scales:
// 256 x 112 113 us against 122 at 256 x 64);
// M = 1024: 256 x 96 103 us, 256 x 64 106 to 108 us. The model ranks them the
// same way. For M <= 64 the weight stream is latency-bound: 64 x 64 tiles
// (twice the workgroups of 64 x 128) measured 126 against 151 us (Q4) and 68
// against 81 us (Q8) at M = 32, K = 8192, N = 28672.
// The 32x32x16 kernels of gemm_wide.hip (K a multiple of 64) take the
// 256 x 96 tile and a fifth candidate, 256 x 128, at 0.85 of the cost of its
// area: at M = 256, K = 8192, N = 28672 (cold, same box) the 224 tiles of
// 256 x 128 took 125.5 us (Q8) / 121.5 us (Q4, f16 scales) in the K-pair
// kernel that preceded the role-split one, against 130.5 / 123.0 us for the
// 256 tiles of 256 x 112, 0.84 / 0.87 of the time per tile area; M = 300: 227
// against 235 us. The role-split kernel is 4-10% faster again there.
template <int FMT, typename ST>
static hipError_t launch_mt(const MatmulArgs& a, int cu_count) {
  if (a.m > 128) {
    const bool pair = a.k % 64 == 0;
    const int64_t bm[5] = {256, 256, 256, 256, 256}, bn[5] = {96, 64, 48, 112, 128};
    const int64_t pct[5] = {pair ? 85 : 100, 100, 100, 100, 85};
    int best = 0;
    int64_t best_cost = INT64_MAX;
    for (int i = 0; i < (pair ? 5 : 4); i++) {
      const int64_t tiles = (a.m + bm[i] - 1) / bm[i] * ((a.npad + bn[i] - 1) / bn[i]);
      const int64_t cost = (tiles + cu_count - 1) / std::max(cu_count, 1) * bm[i] * bn[i] * pct[i];
      if (cost < best_cost) {
        best_cost = cost;
        best = i;
      }
    }
    // 256 x 96: the role-split kernel on 32x32x16 MFMA (C2 step 52.5 against
    // 54.2 us for gemm_wk_kernel with its K-pair predecessor, same box and data)
    if (best == 0) return pair ? launch_gemm_rs(a, 3) : launch_wk<FMT, ST, 6>(a);
    if (best == 1) return launch_wl<FMT, ST, 4, 4, 4, 2>(a);
    if (best == 2) return launch_wl<FMT, ST, 4, 3, 4, 2>(a);
    if (best == 4) return launch_gemm_rs(a, 4);
    return launch_wk<FMT, ST, 7>(a);
  }
  if (a.m <= 64) return launch_t<FMT, ST, 4, 1>(a);
  return launch_t<FMT, ST, 8, 2>(a);
}

hipError_t launch_gemm_bf16(const MatmulArgs& a, int cu_count) {
  if (a.format == RQ_Q8_0) return launch_mt<RQ_Q8_0, float>(a, cu_count);
  if (a.scale_dtype == RQ_F16) return launch_mt<RQ_Q4_0, uint16_t>(a, cu_count);
  return launch_mt<RQ_Q4_0, float>(a, cu_count);
}

}  // namespace rq
