// gemv.hip — decode-regime (m <= 16) block-quantized matmul on CDNA4 int8 MFMA.
//
// y[m, o] = sum_b scale[o, b] * sum_{k in block b} code[o, k] * x[m, k]
// (qlinear-q8, raster/quant/train.clj:77-108, and its Q4_0 form: the f32 scale
// multiplies the block partial instead of every element).
//
// HBM-bound: the kernel must stream the weights at full bandwidth while doing
// as little VALU work per byte as possible. Weights go into
// v_mfma_i32_16x16x64_i8 as they are stored (Q8 codes as int8; Q4 nibbles
// unmasked to bytes 0..15 with zero-point 8 applied per block), so no weight
// is ever converted to floating point.
//
// Activations are made integer with a 16-bit block fixed point: per (row m,
// block b), with e from frexp(max |x|) (max |x| < 2^e), raised by one when
// max|x| * 2^(15-e) would round above 32639,
//   X_k = rne(x_k * 2^(15-e)),  |X_k| <= 32639,   x_k = 2^(e-15) X_k + d_k,
//   |d_k| <= 2^(e-16) <= 2^-15 max|x|  (2^-14 max|x| after the raise),
// and X_k = 256 L0_k + L1_k with int8 levels L0, L1 in [-128, 127]. Then
// sum_k code_k x_k = 2^(e-15) (256 C0 + C1) + sum_k code_k d_k with C0, C1
// the exact int32 dot products of the codes with each level: the products
// code_k * X_k are exact, so d_k is the only rounding beyond f32.
//
// MFMA shape: A (16 rows x 64 k) holds activation variants, B (64 k x 16
// columns) the weights of 16 output rows o for one 64-element window
// (two 32-blocks). Row r of A is (activation row 4 mg + r/4, level r & 1,
// block (r >> 1) & 1 of the window); a variant is zero on the k-slots of the
// other block. The int32 result lane (col o, quad q) then holds, for
// activation row 4 mg + q, the four partials C0/C1 of both blocks, and
//   acc += f32(256 C0_b + C1_b [- 8 XS_b for Q4]) * (scale[o, b] * 2^(e_b - 15))
// per block: about two VALU ops per block partial.
//
// A block of x holding Inf or NaN gets a NaN factor, so every output of that
// activation row is NaN (Raster's f32 loop gives +-Inf or NaN there).
//
// Mapping: a workgroup (8 waves) decomposes x into LDS once, then takes
// 16-row groups of the weight in turn (stride over the grid); each wave
// streams its share of a group's windows, 4 windows per batch with the next
// batch's loads in flight; the waves' partial sums meet in LDS. When the
// activations of all of K do not fit in LDS, K is cut into slices taken by
// different workgroups, and the last one to finish a group adds the slices'
// partial sums.
#include <algorithm>
#include <atomic>

#include "rq_internal.h"

namespace rq {

namespace {


// LDS layout (dynamic shared memory), offsets in bytes
struct SkinnyLds {
  int kp;       // k padded to whole windows
  int nbp;      // blocks, padded (= kp / 32)
  int lstr;     // bytes per lev row: kp + 32, so the rows of one MFMA operand read fall in different banks
  int xstr;     // elements per xsf / xs row: nbp + 2, for the same reason
  int lev;      // int8 lev[mt][2][lstr]
  int xsf;      // f32 xsf[mt + 1][xstr]: 2^(e-15), NaN for non-finite blocks; row mt zero
  int xs;       // i32 xs[mt + 1][xstr]: sum of X over the block (Q4 zero-point); row mt zero
  int zero;     // 16 zero bytes
  int red;      // f32 red[waves][mg][64]
  int nss;      // f32 nss[waves][mt]: the waves' partial sums of squares (input RMSNorm)
  int bytes;
  __host__ __device__ SkinnyLds(int mt, int k, int waves) {
    kp = (k + 63) / 64 * 64;
    nbp = kp / 32;
    lstr = kp + 32;
    xstr = nbp + 2;
    lev = 0;
    xsf = mt * 2 * lstr;
    xs = xsf + (mt + 1) * xstr * 4;
    zero = xs + (mt + 1) * xstr * 4;
    red = zero + 16;
    nss = red + waves * (mt / 4) * 64 * 4;
    bytes = nss + waves * mt * 4;
  }
};


// A row's 8 block scales of one batch of the row-batched scales.
template <typename ST>
struct ScaleBatch;
template <>
struct ScaleBatch<float> {
  f32x4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *reinterpret_cast<const f32x4*>(p);
    b = *reinterpret_cast<const f32x4*>(p + 4);
  }
  __device__ __forceinline__ float get(int j) const { return j < 4 ? a[j] : b[j - 4]; }
};
template <>
struct ScaleBatch<uint16_t> {
  u32x4 a;
  __device__ __forceinline__ void load(const uint16_t* p) { a = *reinterpret_cast<const u32x4*>(p); }
  __device__ __forceinline__ float get(int j) const {
    return f16_bits_to_f32((uint16_t)(a[j >> 1] >> (16 * (j & 1))));
  }
};

// Windows per K-slice of the decode kernel: a whole number of batches of nb
// windows (the host sizes LDS with the same count).
__host__ __device__ __forceinline__ int slice_windows(int nw, int ksplit, int nb) {
  return ((nw + ksplit - 1) / ksplit + nb - 1) / nb * nb;
}

// Decomposition of one item: 4 activations (row mm, elements k..k+3 of block
// b) of the 8 lanes sharing a block. Writes both int8 levels to LDS and, from
// the block's first lane, the block factor and level sum. All 8 lanes of a
// block run it together (the reductions cross lanes); `valid` (the same for
// the 8 lanes) only gates the LDS writes.
__device__ __forceinline__ void decompose_item(const float (&v)[4], bool valid, int mm, int b, int part, int k, int lstr,
                                               int xstr, int8_t* __restrict__ lev, float* __restrict__ xsf,
                                               int* __restrict__ xs) {
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  // fmaxf drops NaN operands, so non-finite values are flagged separately
  int bad = !(fabsf(v[0]) <= 3.402823466e38f && fabsf(v[1]) <= 3.402823466e38f && fabsf(v[2]) <= 3.402823466e38f &&
              fabsf(v[3]) <= 3.402823466e38f);
  amax = max8(amax);
  bad = or8(bad);
  const bool finite = !bad;
  int e = 0;
  (void)frexpf(amax, &e);  // 0 for amax == 0
  e = ldexpf(amax, 15 - e) > 32639.0f ? e + 1 : e;  // keeps |X| <= 32639: both levels fit int8
  uint32_t l0 = 0u, l1 = 0u;
  int sum = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int X = finite ? (int)rintf(ldexpf(v[i], 15 - e)) : 0;
    const int a = (X + 128) >> 8, c = X - 256 * a;
    l0 |= (uint32_t)(a & 0xFF) << (8 * i);
    l1 |= (uint32_t)(c & 0xFF) << (8 * i);
    sum += X;
  }
  sum = sum8(sum);
  if (valid) {
    *reinterpret_cast<uint32_t*>(lev + (mm * 2 + 0) * lstr + k) = l0;
    *reinterpret_cast<uint32_t*>(lev + (mm * 2 + 1) * lstr + k) = l1;
    if (part == 0) {
      xsf[mm * xstr + b] = finite ? ldexpf(1.0f, e - 15) : __builtin_nanf("");
      xs[mm * xstr + b] = sum;
    }
  }
}

// Int8 activation blocks (Raster's quantize-act-i8 format): level 0 is zero
// and level 1 holds the codes, so 256 C0 + C1 is the exact int8 block dot;
// the block factor is the activation scale xs and the level sum xsum (the
// Q4_0 zero-point fold of qmatmul-q4-composable).
__device__ __forceinline__ void store_int8_item(uint32_t word, bool valid, int mm, int b, int part, int k, int lstr,
                                                int xstr, int8_t* __restrict__ lev, float* __restrict__ xsf,
                                                int* __restrict__ xs, float scale, int sum) {
  if (valid) {
    *reinterpret_cast<uint32_t*>(lev + (mm * 2 + 0) * lstr + k) = 0u;
    *reinterpret_cast<uint32_t*>(lev + (mm * 2 + 1) * lstr + k) = word;
    if (part == 0) {
      xsf[mm * xstr + b] = scale;
      xs[mm * xstr + b] = sum;
    }
  }
}

// quantize-act-i8 of one item inside the kernel (the 8 lanes of a block run
// it together): the same math as quantize_act_i8_kernel, so the codes, scale
// and sum are bitwise those of rq_quantize_act_i8.
__device__ __forceinline__ void quantize_item_a5(const float (&v)[4], bool valid, int mm, int b, int part, int k,
                                                 int lstr, int xstr, int8_t* __restrict__ lev,
                                                 float* __restrict__ xsf, int* __restrict__ xs) {
  const float amax = max8(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  const double d = (double)amax / 127.0;
  const double id = d == 0.0 ? 0.0 : 1.0 / d;
  uint32_t word = 0u;
  int s = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int q = java_round_clamp127((double)v[i] * id);
    word |= (uint32_t)(q & 0xFF) << (8 * i);
    s += q;
  }
  store_int8_item(word, valid, mm, b, part, k, lstr, xstr, lev, xsf, xs, (float)d, sum8(s));
}

// The outputs of 16-row group g held by lane (r, g4) of one wave: v[mg] is
// y[4 mg + g4][16 g + r] before the fused epilogue, rinv[mg] that row's
// 1 / rms (input RMSNorm only). SwiGLU: lane r (even) holds the gate row,
// lane r + 1 the up row; y has N / 2 columns.
template <int MG>
__device__ __forceinline__ void store_group(const float (&v)[MG], const float (&rinv)[MG], int g, int lane, void* y,
                                            int M, int N, int y_dtype, const DecodeOps& ops) {
  const int r = lane & 15, g4 = lane >> 4;
  const int o = 16 * g + r;
  const int ny = ops.swiglu ? N / 2 : N, oy = ops.swiglu ? o / 2 : o;
#pragma unroll
  for (int mg = 0; mg < MG; mg++) {
    const int m = 4 * mg + g4;
    float out = v[mg];
    if (ops.norm_gain) out *= rinv[mg];
    if (ops.swiglu) {
      const float up = __shfl_down(out, 1, 64);
      out = out / (1.0f + expf(-out)) * up;
    }
    const bool mine = m < M && o < N && (!ops.swiglu || (r & 1) == 0);
    if (mine) {
      if (ops.residual)
        out += y_dtype == RQ_F32
                   ? *as_global(static_cast<const float*>(ops.residual) + (int64_t)m * ny + oy)
                   : bf16_bits_to_f32(*as_global(static_cast<const uint16_t*>(ops.residual) + (int64_t)m * ny + oy));
      if (y_dtype == RQ_F32)
        static_cast<float*>(y)[(int64_t)m * ny + oy] = out;
      else
        static_cast<uint16_t*>(y)[(int64_t)m * ny + oy] = (uint16_t)f32_to_bf16_bits(out);
    }
  }
}

}  // namespace

// NORM: input RMSNorm (ops.norm_gain set) as a compile-time switch, so that
// the calls without it issue no conditional loads ahead of the weights.
template <int FMT, typename ST, int XT, int MT, int WAVES, int NB, int RING, bool NORM>
__global__ __launch_bounds__(64 * WAVES) void skinny_kernel(const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                                           const void* __restrict__ x, void* __restrict__ y, int M,
                                                           int K, int N, int npad, int y_dtype, int ksplit,
                                                           float* __restrict__ part, DecodeOps ops) {
  constexpr int MG = MT / 4;                 // MFMAs per window (4 activation rows each)
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int nb = K / 32, nw = (K + 63) / 64;
  const int ngroups = npad / 16;
  // ---- this workgroup's K-slice: windows [s_beg, s_end), fixed for all its
  // groups. LDS holds the activations of the slice only (slice-relative).
  const int s = (int)blockIdx.x % ksplit;
  const int sw = slice_windows(nw, ksplit, NB);
  const int s_beg = min(nw, s * sw), s_end = min(nw, s_beg + sw);
  const SkinnyLds L(MT, 64 * sw, WAVES);
  int8_t* lev = reinterpret_cast<int8_t*>(smem + L.lev);
  float* xsf = reinterpret_cast<float*>(smem + L.xsf);
  int* xs = reinterpret_cast<int*>(smem + L.xs);
  float* red = reinterpret_cast<float*>(smem + L.red);
  float* nss = reinterpret_cast<float*>(smem + L.nss);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers and branches
  const int r = lane & 15, g4 = lane >> 4;

  // ---- per-lane A-fragment addressing. Lane (r, g4) supplies k-slots of
  // window block g4 >> 1; variant r = (row 4 mg + r/4, level r & 1, block
  // (r >> 1) & 1) is zero unless that block matches (and the row exists).
  const int lvl = r & 1, sel = (r >> 1) & 1;
  int aoff[MG];
#pragma unroll
  for (int mg = 0; mg < MG; mg++) {
    const int mm = 4 * mg + (r >> 2);
    const bool match = sel == (g4 >> 1) && mm < M;
    const int kin = FMT == RQ_Q8_0 ? 16 * g4 : 32 * (g4 >> 1) + 8 * (g4 & 1);
    aoff[mg] = match ? (mm * 2 + lvl) * L.lstr + kin : -1;
  }
  // this lane's activation row per MFMA (for xsf / xs), quad q = g4; rows
  // past M read the zero row
  int xrow[MG];
#pragma unroll
  for (int mg = 0; mg < MG; mg++) xrow[mg] = (4 * mg + g4 < M ? 4 * mg + g4 : MT) * L.xstr;

  // ---- wave's window range inside the slice (absolute window numbers); a
  // whole number of batches, so every batch starts on a scale batch
  const int per = ((sw + WAVES - 1) / WAVES + NB - 1) / NB * NB;
  const int wbeg = min(s_end, s_beg + wave * per), wend = min(s_end, wbeg + per);

  // weight bytes per 16-row chunk, and this lane's offset inside a window
  constexpr int CB = FMT == RQ_Q8_0 ? 32 : 16;
  const int wlo = (g4 >> 1) * CB * 16 + r * CB + (FMT == RQ_Q8_0 ? 16 : 8) * (g4 & 1);
  // last window this lane's block exists in (an odd block count leaves the
  // second block of the last window empty: its lanes reread a valid block,
  // which the zero A variants cancel)
  const int wmax = (nb - 1 - (g4 >> 1)) / 2;

  static_assert(NB == 4, "a batch is one 8-block scale batch");
  u32x4 wq[RING][NB];
  ScaleBatch<ST> sb[RING];
  const int nsb = scale_nb8(nb) / 8;  // scale batches per group
  // weight window w of group g: this lane's 16 (Q8) / 8 (Q4) code bytes, and
  // the row's 8 block scales of the batch in one or two 16-byte loads (zero
  // past the last block). All loads are unconditional at clamped addresses
  // and nothing here uses the loaded values: any condition or select on them
  // would make the compiler wait for the loads right here and lose the
  // overlap with the work that follows.
  auto load_batch = [&](int slot, int wb, int g) {
    const uint8_t* qg = q + (int64_t)g * nb * CB * 16;  // the group's chunks
#pragma unroll
    for (int i = 0; i < NB; i++) {
      const int w = min(wb + i, nw - 1);
      const int off = wlo + min(w, wmax) * 2 * CB * 16;
      if (FMT == RQ_Q8_0) {
        wq[slot][i] = *reinterpret_cast<const u32x4*>(qg + off);
      } else {
        const u32x2 t = *reinterpret_cast<const u32x2*>(qg + off);
        wq[slot][i] = u32x4{t[0], t[1], 0u, 0u};
      }
    }
    sb[slot].load(sc + scale_rb_group(g, nb) + scale_rb_in_group(8 * min(wb / NB, nsb - 1), r));
  };

  // ---- activation decomposition into LDS. A wave only ever reads the
  // activations of its own windows (wbeg..wend of every group), so each wave
  // decomposes just those into its own part of the LDS arrays: no workgroup
  // barrier. Items are 4 consecutive activations; a lane takes items lane,
  // lane + 64, ... in chunks of XJ whose loads all go out before any is used.
  // The first chunk's loads precede the first weight batch, so decomposing it
  // waits only for them (loads complete in issue order). Lanes past the
  // wave's last item reread it (same row) and do not write.
  const int nblk_w = 2 * (wend - wbeg);          // blocks of this wave's windows
  const int rb0 = 2 * (wbeg - s_beg);            // their first block, slice-relative
  const int witems = M * nblk_w * 8;             // 4-element items
  constexpr int XJ = 8;
  float xv[XJ][4];
  f32x4 gv[XJ];  // input RMSNorm: the gain of each item, loaded with it
  constexpr bool norm = NORM && XT != kXtI8;
  // Input RMSNorm needs each row's sum of squares over all of K. With one
  // K-slice and m <= 4 the waves sum the squares of the items they decompose
  // (together they cover K once); otherwise every workgroup reads the whole
  // rows once more.
  const bool ss_items = norm && MT == 4 && ksplit == 1;
  float ssl[MT];
#pragma unroll
  for (int r = 0; r < MT; r++) ssl[r] = 0.0f;
  // item slots j of a chunk that hold any item: a wave-uniform test, so the
  // loads and decompositions of empty slots are skipped by scalar branches
  auto load_chunk = [&](int base) {
#pragma unroll
    for (int j = 0; j < XJ; j++) {
      if (base + 64 * j >= witems) break;
      const int it = min(base + lane + 64 * j, witems - 1);
      const int mm = it / (nblk_w * 8), rb = rb0 + (it >> 3) % nblk_w;
      // columns past K (the missing half of a last window) reread in-row data
      const int k = min(32 * (2 * s_beg + rb) + 4 * (it & 7), K - 4);
      load_x4<XT>(x, (int64_t)mm * K + k, true, xv[j]);
      if (norm) gv[j] = *as_global(reinterpret_cast<const f32x4*>(ops.norm_gain + k));
      if (XT == kXtI8) {
        // the block's scale and level sum travel with its codes
        const int64_t bq = (int64_t)mm * nb + min(2 * s_beg + rb, nb - 1);
        xv[j][1] = ops.act_scale[bq];
        xv[j][2] = __int_as_float(ops.act_sum ? (int)ops.act_sum[bq] : 0);
      }
    }
  };
  auto decompose_chunk = [&](int base) {
#pragma unroll
    for (int j = 0; j < XJ; j++) {
      if (base + 64 * j >= witems) break;
      const int it0 = base + lane + 64 * j;
      const int it = min(it0, witems - 1);
      const int mm = it / (nblk_w * 8), rb = rb0 + (it >> 3) % nblk_w, pt = it & 7;
      if (norm) {
        if (ss_items) {
          // blocks past K (the missing half of a last window) reread data
          const bool ok = it0 < witems && 2 * s_beg + rb < nb;
          const float sq =
              ok ? xv[j][0] * xv[j][0] + xv[j][1] * xv[j][1] + xv[j][2] * xv[j][2] + xv[j][3] * xv[j][3] : 0.0f;
#pragma unroll
          for (int r = 0; r < MT; r++) ssl[r] += mm == r ? sq : 0.0f;
        }
        // the gain here; the row's 1 / rms factors out of the dot products
        // and is applied to the result
#pragma unroll
        for (int e = 0; e < 4; e++) xv[j][e] *= gv[j][e];
      }
      if (XT == kXtI8) {
        store_int8_item(__float_as_uint(xv[j][0]), it0 < witems, mm, rb, pt, 32 * rb + 4 * pt, L.lstr, L.xstr, lev,
                        xsf, xs, xv[j][1], __float_as_int(xv[j][2]));
      } else if (ops.act_i8) {
        quantize_item_a5(xv[j], it0 < witems, mm, rb, pt, 32 * rb + 4 * pt, L.lstr, L.xstr, lev, xsf, xs);
      } else {
        decompose_item(xv[j], it0 < witems, mm, rb, pt, 32 * rb + 4 * pt, L.lstr, L.xstr, lev, xsf, xs);
      }
    }
  };
  const int gcols = (int)gridDim.x / ksplit;  // workgroups per slice
  const int gfirst = (int)blockIdx.x / ksplit;
  load_chunk(0);
  // keep the scheduler from hoisting the weight loads above the activation
  // loads: the decomposition below waits for the activations only
  __builtin_amdgcn_sched_barrier(0);
  load_batch(0, wbeg, min(gfirst, ngroups - 1));
  __builtin_amdgcn_sched_barrier(0);
  // input RMSNorm without ss_items: sums of squares of the rows over all of K
  // (every workgroup reads the whole rows; they are small at m <= 16), a
  // partial per wave in nss, read after the first group's barrier. These
  // loads go out after the first weight batch.
  if (norm && !ss_items) {
    float ss[MT];
#pragma unroll
    for (int mm = 0; mm < MT; mm++) ss[mm] = 0.0f;
    for (int k = 4 * tid; k < K; k += 4 * 64 * WAVES) {
#pragma unroll
      for (int mm = 0; mm < MT; mm++) {
        if (mm >= M) break;
        float v[4];
        load_x4<XT>(x, (int64_t)mm * K + k, true, v);
        ss[mm] += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
      }
    }
#pragma unroll
    for (int mm = 0; mm < MT; mm++) {
      if (mm >= M) break;
      float t = ss[mm];
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) t += __shfl_xor(t, off, 64);
      if (lane == 0) nss[wave * MT + mm] = t;
    }
  }
  if (lane < 4) reinterpret_cast<uint32_t*>(smem + L.zero)[lane] = 0u;
  if (lane < nblk_w) {
    xsf[MT * L.xstr + rb0 + lane] = 0.0f;
    xs[MT * L.xstr + rb0 + lane] = 0;
  }
  decompose_chunk(0);
  for (int base = 64 * XJ; base < witems; base += 64 * XJ) {
    load_chunk(base);
    decompose_chunk(base);
  }
  if (ss_items) {
#pragma unroll
    for (int mm = 0; mm < MT; mm++) {
      if (mm >= M) break;
      float t = ssl[mm];
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) t += __shfl_xor(t, off, 64);
      if (lane == 0) nss[wave * MT + mm] = t;
    }
  }
  // the wave reads back what its own lanes wrote
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();

  float acc[MG];
#pragma unroll
  for (int mg = 0; mg < MG; mg++) acc[mg] = 0.0f;

  // Phases: every LDS read of the batch, then every MFMA, then every
  // epilogue, so LDS latency and MFMA latency overlap across windows.
  auto compute_batch = [&](int slot, int wb) {
    i32x4 af[NB][MG];
    float f0[NB][MG], f1[NB][MG];
    int x0[NB][MG], x1[NB][MG];
#pragma unroll
    for (int i = 0; i < NB; i++) {
      const int w = wb + i;
      const bool live = w < wend;  // wave-uniform
      const int rw = max(0, min(w, s_end - 1) - s_beg);  // slice-relative window
#pragma unroll
      for (int mg = 0; mg < MG; mg++) {
        const int ao = live && aoff[mg] >= 0 ? aoff[mg] + 64 * rw : L.zero - L.lev;
        if (FMT == RQ_Q8_0) {
          af[i][mg] = *reinterpret_cast<const i32x4*>(lev + ao);
        } else {
          // the zero slot is 16 bytes: both 8-byte halves read zeros there
          const int ao2 = live && aoff[mg] >= 0 ? ao + 16 : ao + 8;
          const u32x2 h0 = *reinterpret_cast<const u32x2*>(lev + ao);
          const u32x2 h1 = *reinterpret_cast<const u32x2*>(lev + ao2);
          af[i][mg] = i32x4{(int)h0[0], (int)h0[1], (int)h1[0], (int)h1[1]};
        }
        const f32x2 fv = *reinterpret_cast<const f32x2*>(xsf + xrow[mg] + 2 * rw);
        f0[i][mg] = live ? fv[0] : 0.0f;
        // a window's second block may not exist (odd block count)
        f1[i][mg] = live && 2 * w + 1 < nb ? fv[1] : 0.0f;
        if (FMT == RQ_Q4_0) {
          const i32x2 xv2 = *reinterpret_cast<const i32x2*>(xs + xrow[mg] + 2 * rw);
          x0[i][mg] = xv2[0];
          x1[i][mg] = xv2[1];
        }
      }
    }
    i32x4 c[NB][MG];
#pragma unroll
    for (int i = 0; i < NB; i++) {
      i32x4 bfrag;
      if (FMT == RQ_Q8_0) {
        bfrag = __builtin_bit_cast(i32x4, wq[slot][i]);
      } else {
        const uint32_t d0 = wq[slot][i][0], d1 = wq[slot][i][1];
        bfrag = i32x4{(int)(d0 & 0x0F0F0F0Fu), (int)(d1 & 0x0F0F0F0Fu), (int)((d0 >> 4) & 0x0F0F0F0Fu),
                      (int)((d1 >> 4) & 0x0F0F0F0Fu)};
      }
#pragma unroll
      for (int mg = 0; mg < MG; mg++)
        c[i][mg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i][mg], bfrag, i32x4{0, 0, 0, 0}, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < NB; i++)
#pragma unroll
      for (int mg = 0; mg < MG; mg++) {
        int t0 = (c[i][mg][0] << 8) + c[i][mg][1], t1 = (c[i][mg][2] << 8) + c[i][mg][3];
        if (FMT == RQ_Q4_0) {
          t0 -= 8 * x0[i][mg];
          t1 -= 8 * x1[i][mg];
        }
        acc[mg] = fmaf((float)t0, sb[slot].get(2 * i) * f0[i][mg], acc[mg]);
        acc[mg] = fmaf((float)t1, sb[slot].get(2 * i + 1) * f1[i][mg], acc[mg]);
      }
  };

  // ---- task stream: batch j of the wave's windows in group round i is task
  // t = i * nbg + j. The next task's loads (possibly the next group's) are in
  // flight while the current task computes and a finished group's partial
  // sums are combined.
  const int nbg = max(1, (per + NB - 1) / NB);  // batches per group
  const int rounds = gfirst < ngroups ? (ngroups - 1 - gfirst) / gcols + 1 : 0;
  const int ntask = rounds * nbg;
  auto task_load = [&](int slot, int t) {
    const int g = gfirst + (t / nbg) * gcols;
    load_batch(slot, wbeg + (t % nbg) * NB, min(g, ngroups - 1));
  };
  // Combine the waves' partial sums of the group in wave order; lane (r, g4)
  // of wave 0 owns y[4 mg + g4][16 g + r]. With one slice it stores y; with
  // several it stores the slice's partial sums, which skinny_reduce_kernel
  // adds in slice order (workgroup 0 also leaves the rows' sums of squares
  // there for the input RMSNorm).
  auto finish_group = [&](int t) {
    const int g = gfirst + (t / nbg) * gcols;
#pragma unroll
    for (int mg = 0; mg < MG; mg++) {
      red[(wave * MG + mg) * 64 + lane] = acc[mg];
      acc[mg] = 0.0f;
    }
    __syncthreads();
    if (wave == 0) {
      float v[MG], rinv[MG];
#pragma unroll
      for (int mg = 0; mg < MG; mg++) {
        v[mg] = 0.0f;
#pragma unroll
        for (int wv = 0; wv < WAVES; wv++) v[mg] += red[(wv * MG + mg) * 64 + lane];
        rinv[mg] = 1.0f;
        const int m = 4 * mg + g4;
        if (XT != kXtI8 && ops.norm_gain && m < M) {
          float ssum = 0.0f;
#pragma unroll
          for (int wv = 0; wv < WAVES; wv++) ssum += nss[wv * MT + m];
          rinv[mg] = 1.0f / sqrtf(ssum / (float)K + ops.norm_eps);
        }
      }
      if (ksplit == 1) {
        store_group<MG>(v, rinv, g, lane, y, M, N, y_dtype, ops);
      } else {
#pragma unroll
        for (int mg = 0; mg < MG; mg++) part[((int64_t)s * ngroups + g) * (MG * 64) + mg * 64 + lane] = v[mg];
        if (XT != kXtI8 && ops.norm_gain && blockIdx.x == 0 && lane < M) {
          float ssum = 0.0f;
#pragma unroll
          for (int wv = 0; wv < WAVES; wv++) ssum += nss[wv * MT + lane];
          part[(int64_t)ksplit * ngroups * (MG * 64) + lane] = ssum;
        }
      }
    }
    __syncthreads();
  };
  // a ring of RING batch slots: task t computes from slot t % RING while the
  // loads of tasks t + 1 .. t + RING - 1 are in flight. Task 0's batch went
  // out with the prologue; tasks 1 .. RING - 2 go out now.
#pragma unroll
  for (int u = 1; u < RING - 1; u++) task_load(u, u);
  for (int t0 = 0; t0 < ntask; t0 += RING) {
#pragma unroll
    for (int u = 0; u < RING; u++) {
      const int t = t0 + u;
      if (t >= ntask) break;
      task_load((u + RING - 1) % RING, t + RING - 1);
      compute_batch(u, wbeg + (t % nbg) * NB);
      if (t % nbg == nbg - 1) finish_group(t);
    }
  }
}

// y from the K-slices' partial sums of the decode kernel, added in slice
// order, then the fused epilogue; one wave per 16-row group
template <int MT>
__global__ __launch_bounds__(256) void skinny_reduce_kernel(const float* __restrict__ part, void* __restrict__ y, int M,
                                                            int K, int N, int ngroups, int ksplit, int y_dtype,
                                                            DecodeOps ops) {
  constexpr int MG = MT / 4;
  const int lane = threadIdx.x & 63;
  const int g = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  if (g >= ngroups) return;  // wave-uniform
  const float* ss = part + (int64_t)ksplit * ngroups * (MG * 64);
  float v[MG], rinv[MG];
#pragma unroll
  for (int mg = 0; mg < MG; mg++) {
    // the slices' loads four at a time, the adds in slice order
    auto ld = [&](int sl) { return part[((int64_t)sl * ngroups + g) * (MG * 64) + mg * 64 + lane]; };
    float t = 0.0f;
    int sl = 0;
    for (; sl + 3 < ksplit; sl += 4) {
      const float a = ld(sl), b = ld(sl + 1), c = ld(sl + 2), d = ld(sl + 3);
      t += a;
      t += b;
      t += c;
      t += d;
    }
    for (; sl < ksplit; sl++) t += ld(sl);
    v[mg] = t;
    const int m = 4 * mg + (lane >> 4);
    rinv[mg] = ops.norm_gain && m < M ? 1.0f / sqrtf(ss[m] / (float)K + ops.norm_eps) : 1.0f;
  }
  store_group<MG>(v, rinv, g, lane, y, M, N, y_dtype, ops);
}

constexpr int kBatch = 4;  // windows per batch
// batch slots in flight per wave
template <int FMT>
constexpr int kRing = 2;

// Split and grid for the decode kernel.
//  * waves per workgroup, measured with cold weights on the 4096 x 4096 Q8
//    and 14336 x 4096 Q4 shapes at m = 1..16 and warm on the decoder's
//    K = 2048 / 5632 shapes at m = 1: 16 waves for m <= 4 when there are more
//    16-row groups than CUs or m > 2, as long as every wave still gets a full
//    batch of windows (K >= 4096); 8 waves otherwise (at K = 2048 a 16-wave
//    workgroup leaves half of each batch empty: 7.1 against 5.0 us at
//    6144 x 2048). One workgroup per CU: a second one only repeats the
//    activation decomposition (measured no faster at 6144 and 11264 x 2048).
//  * A workgroup holds the activations of its K-range in LDS; when the whole
//    K does not fit, each 16-row group is cut into ksplit K-slices handled by
//    different workgroups; a second kernel adds their partial sums in slice
//    order. (Splitting only to create more workgroups does not pay: the
//    second launch and the partials' round trip cost more than they gain.)
DecodePlan plan_decode(int64_t m, int64_t k, int64_t npad, int cu_count) {
  DecodePlan p{};
  if (m < 1 || m > 16) return p;
  const int64_t nw = (k + 63) / 64, ngroups = npad / 16;
  p.mt = m <= 4 ? 4 : m <= 8 ? 8 : 16;
  p.waves = p.mt == 4 && (ngroups > cu_count || m > 2) && nw >= 16 * kBatch ? 16 : 8;
  const int per_cu_max = 1;
  int64_t ks = 1;
  while (SkinnyLds(p.mt, 64 * slice_windows((int)nw, (int)ks, kBatch), p.waves).bytes > 163840) {
    if (ks >= nw) return p;
    ks++;
  }
  const int lds = SkinnyLds(p.mt, 64 * slice_windows((int)nw, (int)ks, kBatch), p.waves).bytes;
  const int per_cu = std::max(1, std::min(163840 / lds, per_cu_max));
  const int64_t gcols = std::min<int64_t>(ngroups, std::max<int64_t>(1, (int64_t)per_cu * cu_count / ks));
  if (gcols * ks > INT32_MAX) return p;
  p.ksplit = (int)ks;
  p.grid = (int)(gcols * ks);
  p.lds_bytes = lds;
  // partial sums, then the rows' sums of squares (mt floats)
  p.part_bytes = ks > 1 ? ((size_t)ks * (size_t)ngroups * (size_t)(p.mt * 16) + (size_t)p.mt) * 4 : 0;
  p.ok = true;
  return p;
}

template <int FMT, typename ST, int XT, int MT, int WAVES, bool NORM>
static hipError_t launch_t(const MatmulArgs& a, const DecodePlan& p) {
  auto kernel = &skinny_kernel<FMT, ST, XT, MT, WAVES, kBatch, kRing<FMT>, NORM>;
  // dynamic LDS above 64 KB must be allowed once per kernel and device (bit d
  // of `attr_set`; setting it twice from racing threads is harmless)
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
  const bool split = p.ksplit > 1;
  hipExtLaunchKernelGGL(kernel, dim3((unsigned)p.grid), dim3(64 * WAVES), (unsigned)p.lds_bytes, a.stream,
                        a.ev_main[0], a.ev_main[1], 0, a.q, static_cast<const ST*>(a.scales_rb), a.x,
                        a.y, (int)a.m, (int)a.k, (int)a.n, (int)a.npad, a.y_dtype, p.ksplit, a.part, a.ops);
  if (hipError_t e = hipGetLastError()) return e;
  if (split) {
    const int ngroups = (int)(a.npad / 16);
    hipExtLaunchKernelGGL(skinny_reduce_kernel<MT>, dim3((unsigned)((ngroups + 3) / 4)), dim3(256), 0, a.stream,
                          a.ev_aux[0], a.ev_aux[1], 0, a.part, a.y, (int)a.m, (int)a.k, (int)a.n, ngroups, p.ksplit,
                          a.y_dtype, a.ops);
  }
  return hipGetLastError();
}

template <int FMT, typename ST, int XT, bool NORM>
static hipError_t launch_m(const MatmulArgs& a, const DecodePlan& p) {
  if (p.mt == 4)
    return p.waves == 16 ? launch_t<FMT, ST, XT, 4, 16, NORM>(a, p) : launch_t<FMT, ST, XT, 4, 8, NORM>(a, p);
  if (p.mt == 8) return launch_t<FMT, ST, XT, 8, 8, NORM>(a, p);
  return launch_t<FMT, ST, XT, 16, 8, NORM>(a, p);
}

template <int FMT, typename ST>
static hipError_t launch_x(const MatmulArgs& a, const DecodePlan& p) {
  if (a.x_dtype == kXtI8) return launch_m<FMT, ST, kXtI8, false>(a, p);
  if (a.ops.norm_gain)
    return a.x_dtype == RQ_F32 ? launch_m<FMT, ST, RQ_F32, true>(a, p) : launch_m<FMT, ST, RQ_BF16, true>(a, p);
  return a.x_dtype == RQ_F32 ? launch_m<FMT, ST, RQ_F32, false>(a, p) : launch_m<FMT, ST, RQ_BF16, false>(a, p);
}

hipError_t launch_gemv(const MatmulArgs& a, const DecodePlan& p) {
  if (!p.ok || (p.ksplit > 1 && !a.part)) return hipErrorInvalidValue;
  if (a.format == RQ_Q8_0) return launch_x<RQ_Q8_0, float>(a, p);
  if (a.scale_dtype == RQ_F16) return launch_x<RQ_Q4_0, uint16_t>(a, p);
  return launch_x<RQ_Q4_0, float>(a, p);
}

}  // namespace rq
