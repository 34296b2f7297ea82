// gemv_mf.hip — decode matmul (m <= 16; planned for 4 < m <= 16 with Q4_0
// weights, 8 < m <= 16 with Q8_0) of plain
// rq_qmatmul calls with f32 or bf16 activations, on bf16 MFMA with exact
// codes.
//
//   y[m, o] = sum_b s[o, b] * sum_{k in block b} x[m, k] * c[o, k]
//
// * f32 activations are split per element into bf16 hi + lo (hi = RNE(x),
//   lo = RNE(x - hi), so |x - hi - lo| <= 2^-17 |x|); bf16 activations are hi
//   alone.
// * Codes enter the MFMA exactly, with an offset: a Q4_0 nibble n as the bf16
//   128 + n (a byte permute with 0x43, the high byte of 128.0), a Q8_0 code c
//   as c + 128 (v_cvt_f32_ubyte of c ^ 0x80; every integer below 256 is a
//   bf16). Per block the MFMA adds sum x (c + OFF) in f32, OFF = 136 for Q4
//   (c = n - 8) and 128 for Q8, to an accumulator that starts at
//   -OFF * sum (hi + lo) (formed when the activations are staged, fed as the
//   MFMA's C operand), which leaves the block's dot product for the block
//   scale to multiply in f32. No rounding of scale * code is involved.
// * A workgroup has GW x KW waves and one K-slice (grid.x = columns x ks). It
//   stages its slice of x (all m rows, hi and lo) in LDS once; then each wave
//   streams the weight chunks of its 16-row groups through a WD-step register
//   ring: A = the activation fragment from LDS (lane (r, q): row r, k = 8q ..
//   8q+7; rows past m read row m - 1, whose products land only in outputs
//   that are never stored), B = the 16 x 32 chunk in the same
//   lane order, so lane (r, q) ends up holding y[4q + v][16 g + r], v < 4.
//   Q4_0 chunks come in fours: lane (r, q) loads the 16-byte row r of the
//   q-th chunk of a quad (a wave's load moves 1 KB, against 256 B of 8-byte
//   loads that two lanes share), and two lane-swap rounds across the 16-lane
//   rows (v_permlane32_swap, v_permlane16_swap) hand lane (r, q) dword q of
//   row r of each of the four chunks: bytes 4q .. 4q+3, i.e. k = 4q .. 4q+3
//   (low nibbles) and 4q+16 .. 4q+19 (high nibbles). The activation
//   fragments in LDS are laid out in that k order; the scales of the four
//   chunks are broadcast the same way.
//   The KW waves of a column split the slice's steps and add their partial
//   sums through LDS in wave order; with ks > 1 the slices' partial sums go
//   to `part` and gemm_sm_reduce_kernel adds them in slice order.
//   Deterministic either way.
#include <algorithm>
#include <atomic>

#include "rq_internal.h"

namespace rq {

namespace {

// One ring slot: the loaded bits only. Nothing may convert or test them at
// load time: that would make the compiler wait for the load right there.
template <typename ST>
struct MfCodes {
  u32x2 v;  // the lane's 8 code bytes (Q8) or 8 bytes holding its 8 nibbles (Q4)
  ST s;     // its row's block scale, as stored
};

// One ring slot of the Q4_0 quad stream: the lane's 16 loaded bytes (row r
// of chunk q of the quad) and that chunk's scale for row r, as stored.
template <typename ST>
struct MfQuad {
  u32x4 v;
  ST s;
};

// Lane (r, a) holds d[b] = dword b of row r of chunk a; afterwards d[j] =
// dword a of row r of chunk j. Swaps between the lane rows (16 lanes each):
// rows {2, 3} of d[0] with rows {0, 1} of d[2] (likewise d[1], d[3]), then
// rows {1, 3} of one with rows {0, 2} of the other.
__device__ __forceinline__ void mf_xpose4(uint32_t (&d)[4]) {
  const auto p02 = __builtin_amdgcn_permlane32_swap(d[0], d[2], false, false);
  const auto p13 = __builtin_amdgcn_permlane32_swap(d[1], d[3], false, false);
  const auto q01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
  const auto q23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
  d[0] = q01[0];
  d[1] = q01[1];
  d[2] = q23[0];
  d[3] = q23[1];
}

// Lane row a holds s (of chunk a); afterwards b[j] = lane row j's s, in
// every row.
__device__ __forceinline__ void mf_bcast4(uint32_t s, uint32_t (&b)[4]) {
  const auto p = __builtin_amdgcn_permlane32_swap(s, s, false, false);
  const auto b01 = __builtin_amdgcn_permlane16_swap(p[0], p[0], false, false);
  const auto b23 = __builtin_amdgcn_permlane16_swap(p[1], p[1], false, false);
  b[0] = b01[0];
  b[1] = b01[1];
  b[2] = b23[0];
  b[3] = b23[1];
}

// Dword a of a Q4_0 row (bytes 4a .. 4a+3) as the bf16 of 128 + nibble, in
// the k order k = 4a .. 4a+3, 4a+16 .. 4a+19
__device__ __forceinline__ bf16x8 mf_q4_dword(uint32_t d) {
  const uint32_t lo = d & 0x0F0F0F0Fu, hi = (d >> 4) & 0x0F0F0F0Fu;
  return __builtin_bit_cast(bf16x8, u32x4{__builtin_amdgcn_perm(0x43434343u, lo, 0x04010400u),
                                          __builtin_amdgcn_perm(0x43434343u, lo, 0x04030402u),
                                          __builtin_amdgcn_perm(0x43434343u, hi, 0x04010400u),
                                          __builtin_amdgcn_perm(0x43434343u, hi, 0x04030402u)});
}

__device__ __forceinline__ float mf_scale(float s) { return s; }
__device__ __forceinline__ float mf_scale(uint16_t s) { return f16_bits_to_f32(s); }

// the lane's 8 Q8_0 codes as bf16 of code + 128 (v_cvt_f32_ubyte of c ^ 0x80;
// the bf16 of an integer below 256 is the high half of its f32)
template <typename ST>
__device__ __forceinline__ bf16x8 mf_q8_codes(const MfCodes<ST>& c) {
  uint32_t o[4];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const uint32_t u = c.v[h] ^ 0x80808080u;
    const float f0 = (float)(u & 0xFFu), f1 = (float)((u >> 8) & 0xFFu);
    const float f2 = (float)((u >> 16) & 0xFFu), f3 = (float)(u >> 24);
    o[2 * h] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
    o[2 * h + 1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
  }
  return __builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]});
}

}  // namespace

// LDS bytes of a workgroup: x fragments (spl steps x P parts x m rows x 64 B),
// the offset sums (spl x 16 floats), a 16-byte zero slot, and with KW > 1 two
// sets of the waves' partial outputs
__host__ __device__ inline int mf_lds_bytes(int m, int spl, int parts, int kw, int gw) {
  return spl * parts * m * 64 + spl * 64 + 16 + (kw > 1 ? 2 * gw * kw * 1024 : 0);
}

template <int FMT, typename ST, int XT, int KW, int GW, int WD>
__global__ __launch_bounds__(64 * KW * GW) void gemv_mf_kernel(const uint8_t* __restrict__ q,
                                                               const ST* __restrict__ sc,
                                                               const void* __restrict__ x, void* __restrict__ y,
                                                               float* __restrict__ part, int M, int K, int N,
                                                               int npad, int y_dtype, int ks) {
  constexpr int WAVES = KW * GW, P = XT == RQ_F32 ? 2 : 1;
  constexpr float OFF = FMT == RQ_Q8_0 ? 128.0f : 136.0f;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int nkb = K / 32, ngroups = npad / 16;
  const int s = (int)blockIdx.x % ks, col = (int)blockIdx.x / ks, gcols = (int)gridDim.x / ks;
  const int spl = (nkb + ks - 1) / ks;
  const int kb0 = min(nkb, s * spl), nst = min(nkb, kb0 + spl) - kb0;  // this slice: steps kb0 .. kb0+nst-1
  const int xs_off = spl * P * M * 64, zero_off = xs_off + spl * 64, red_off = zero_off + 16;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kw = wave % KW, gw = wave / KW;
  const int r = lane & 15, qd = lane >> 4;

  // ---- activations of the slice into LDS. Item = 8 consecutive x of one
  // row (a quarter of a block); the 4 quarters of a block sit in adjacent
  // lanes, which add their sums by shuffles. The first round's loads go out
  // before the weight ring's, so converting them waits for them only.
  constexpr int XI = 4;
  const int nitems = M * nst * 4, stride = 64 * WAVES;
  float xv[XI][8];
  auto load_items = [&](int base) {
#pragma unroll
    for (int i = 0; i < XI; i++) {
      if (base + stride * i >= nitems) break;  // workgroup-uniform
      const int idx = min(base + tid + stride * i, nitems - 1);
      const int m = idx / (nst * 4), rem = idx - m * nst * 4;
      const int64_t off = (int64_t)m * K + 32 * (kb0 + (rem >> 2)) + 8 * (rem & 3);
      if (XT == RQ_F32) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(static_cast<const float*>(x) + off);
        const f32x4 b = *reinterpret_cast<const f32x4*>(static_cast<const float*>(x) + off + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          xv[i][e] = a[e];
          xv[i][4 + e] = b[e];
        }
      } else {
        const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(x) + off);
#pragma unroll
        for (int e = 0; e < 4; e++) xv[i][e] = __uint_as_float(w[e]);
      }
    }
  };
  auto convert_items = [&](int base) {
#pragma unroll
    for (int i = 0; i < XI; i++) {
      if (base + stride * i >= nitems) break;
      const int idx0 = base + tid + stride * i;
      const int idx = min(idx0, nitems - 1);
      const int m = idx / (nst * 4), rem = idx - m * nst * 4, u = rem >> 2, qq = rem & 3;
      uint32_t hi[4], lo[4];
      float sum = 0.0f;
      if (XT == RQ_F32) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float a = xv[i][2 * e], b = xv[i][2 * e + 1];
          hi[e] = pack2_bf16(a, b);
          const float ha = bf16_bits_to_f32(hi[e] & 0xFFFFu), hb = __uint_as_float(hi[e] & 0xFFFF0000u);
          lo[e] = pack2_bf16(a - ha, b - hb);
          const float la = bf16_bits_to_f32(lo[e] & 0xFFFFu), lb = __uint_as_float(lo[e] & 0xFFFF0000u);
          sum += (ha + la) + (hb + lb);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          hi[e] = __float_as_uint(xv[i][e]);
          sum += bf16_bits_to_f32(hi[e] & 0xFFFFu) + __uint_as_float(hi[e] & 0xFFFF0000u);
        }
      }
      sum += __shfl_xor(sum, 1, 64);
      sum += __shfl_xor(sum, 2, 64);
      if (idx0 < nitems) {
        uint8_t* f = smem + ((u * P) * M + m) * 64;
        if (FMT == RQ_Q4_0) {
          // k = 8qq .. 8qq+3 to lane group 2(qq&1), 8qq+4 .. 8qq+7 to the
          // next; the high half of the block to the upper 8 bytes of each
          const int o0 = 32 * (qq & 1) + 8 * (qq >> 1);
          *reinterpret_cast<u32x2*>(f + o0) = u32x2{hi[0], hi[1]};
          *reinterpret_cast<u32x2*>(f + o0 + 16) = u32x2{hi[2], hi[3]};
          if (P == 2) {
            *reinterpret_cast<u32x2*>(f + M * 64 + o0) = u32x2{lo[0], lo[1]};
            *reinterpret_cast<u32x2*>(f + M * 64 + o0 + 16) = u32x2{lo[2], lo[3]};
          }
        } else {
          *reinterpret_cast<u32x4*>(f + qq * 16) = u32x4{hi[0], hi[1], hi[2], hi[3]};
          if (P == 2) *reinterpret_cast<u32x4*>(f + M * 64 + qq * 16) = u32x4{lo[0], lo[1], lo[2], lo[3]};
        }
        if (qq == 0) *reinterpret_cast<float*>(smem + xs_off + (u * 16 + m) * 4) = -OFF * sum;
      }
    }
  };

  // ---- this wave's work: units j = 0 .. nunits-1 (group col GW + gw + j
  // gcols GW of the slice), each its share of the slice's steps (spw steps
  // from kw spw), padded to spp, a whole number of ring turns, so that the
  // unrolled ring loop holds steps only (a unit ends between turns; its
  // store code exists once: each wave runs the loop only a few times, and
  // a large unrolled body would be fetched from a cold instruction cache).
  // Flat step t = j spp + u; padding steps load their unit's last step
  // again and compute nothing.
  const int spw = (nst + KW - 1) / KW;
  const int spp = (spw + WD - 1) / WD * WD;
  const int nunits = (ngroups + gcols * GW - 1) / (gcols * GW);
  const int T = nunits * spp;
  static_assert(WD % 4 == 0, "the Q4_0 ring holds whole quads");
  MfCodes<ST> wc[FMT == RQ_Q4_0 ? 1 : WD];
  MfQuad<ST> wq[FMT == RQ_Q4_0 ? WD / 4 : 1];
  // Q4_0: quad slot of steps u .. u+3 (u a multiple of 4); lane (r, qd)
  // loads step u + qd, clamped to the wave's share (steps past it compute
  // nothing)
  auto load_q = [&](int slot, int j, int u) {
    if (j >= nunits) {  // past the end: the last quad again
      j = nunits - 1;
      u = spp - 4;
    }
    const int g = min(col * GW + gw + j * gcols * GW, ngroups - 1);
    const int kb = kb0 + min(kw * spw + min(u + qd, spw - 1), nst - 1);
    const int64_t chunk = (int64_t)g * nkb + kb;
    wq[slot].v = *reinterpret_cast<const u32x4*>(q + chunk * 256 + r * 16);
    wq[slot].s = sc[chunk * 16 + r];
  };
  // Q8_0: slot of step u, lane (r, qd) loading codes 8qd .. 8qd+7 of row r
  auto load_w = [&](int slot, int j, int u) {
    if (j >= nunits) {  // past the end: the last step again
      j = nunits - 1;
      u = spp - 1;
    }
    const int g = min(col * GW + gw + j * gcols * GW, ngroups - 1);
    const int kb = kb0 + min(kw * spw + min(u, spw - 1), nst - 1);
    const int64_t chunk = (int64_t)g * nkb + kb;
    wc[slot].v = *reinterpret_cast<const u32x2*>(q + chunk * 512 + r * 32 + 8 * qd);
    wc[slot].s = sc[chunk * 16 + r];
  };
  int lj = 0, lu = 0;  // next step to load
  auto advance = [&](int& j, int& u) {
    if (++u == spp) {
      u = 0;
      ++j;
    }
  };

  auto advance4 = [&](int& j, int& u) {
    u += 4;
    if (u == spp) {
      u = 0;
      ++j;
    }
  };

  load_items(0);
  __builtin_amdgcn_sched_barrier(0);
  // the ring's first WD steps, unconditionally (addresses are clamped; a
  // conditional here would leave the ring's indices to run time and put it
  // in scratch memory)
  if constexpr (FMT == RQ_Q4_0) {
#pragma unroll
    for (int t = 0; t < WD / 4; t++) {
      load_q(t, lj, lu);
      advance4(lj, lu);
    }
  } else {
#pragma unroll
    for (int i = 0; i < WD; i++) {
      load_w(i, lj, lu);
      advance(lj, lu);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  for (int base = 0; base < nitems; base += stride * XI) {
    if (base > 0) load_items(base);
    convert_items(base);
  }
  for (int i = tid; i < nst * (16 - M); i += stride) {
    const int u = i / (16 - M), m = M + i % (16 - M);
    *reinterpret_cast<float*>(smem + xs_off + (u * 16 + m) * 4) = 0.0f;
  }
  if (tid < 4) reinterpret_cast<uint32_t*>(smem + zero_off)[tid] = 0u;
  __syncthreads();

  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  auto store = [&](int j, const f32x4& v) {
    const int g = col * GW + gw + j * gcols * GW;
    const int o = 16 * g + r;
    if (g >= ngroups || o >= N) return;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int m = 4 * qd + e;
      if (m >= M) break;
      if (ks > 1)
        part[((int64_t)s * M + m) * N + o] = v[e];
      else if (y_dtype == RQ_F32)
        static_cast<float*>(y)[(int64_t)m * N + o] = v[e];
      else
        static_cast<uint16_t*>(y)[(int64_t)m * N + o] = (uint16_t)f32_to_bf16_bits(v[e]);
    }
  };
  auto finish = [&](int j) {
    if (KW > 1) {
      f32x4* red = reinterpret_cast<f32x4*>(smem + red_off);
      const int base = (j & 1) * GW * KW * 64 + gw * KW * 64;
      red[base + kw * 64 + lane] = acc;
      __syncthreads();
      if (kw == 0) {
        f32x4 t = red[base + lane];
#pragma unroll
        for (int k = 1; k < KW; k++) t += red[base + k * 64 + lane];
        store(j, t);
      }
    } else {
      store(j, acc);
    }
    acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  };

  // rows past m read row m - 1: their outputs are never stored, and the rows
  // stored do not depend on them
  const int aoff = min(r, M - 1) * 64 + qd * 16;
  // one step's MFMAs and block epilogue
  auto step = [&](int su, const bf16x8& bw, float sv) {
    const int ab = su * P * M * 64;
    const bf16x8 ah = *reinterpret_cast<const bf16x8*>(smem + ab + aoff);
    const f32x4 xo = *reinterpret_cast<const f32x4*>(smem + xs_off + (su * 16 + 4 * qd) * 4);
    f32x4 blk = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bw, xo, 0, 0, 0);
    if (P == 2) {
      const bf16x8 al = *reinterpret_cast<const bf16x8*>(smem + ab + M * 64 + aoff);
      blk = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bw, blk, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 4; e++) acc[e] = fmaf(sv, blk[e], acc[e]);
  };
  if constexpr (FMT == RQ_Q4_0) {
    for (int j = 0; j < nunits; j++) {
      for (int u0 = 0; u0 < spp; u0 += WD) {
#pragma unroll
        for (int t = 0; t < WD / 4; t++) {
          // one quad after the other: hoisting the next quad's lane swaps
          // above this quad's work would make the loop wait for the whole
          // ring at its head
          __builtin_amdgcn_sched_barrier(0);
          uint32_t d[4] = {wq[t].v[0], wq[t].v[1], wq[t].v[2], wq[t].v[3]};
          // the scale as f32 bits before the broadcast: a 16-bit scale's
          // zero extension would otherwise sit at the loop head and wait
          // for the whole ring there
          const uint32_t sb = __float_as_uint(scale_value(wq[t].s));
          mf_xpose4(d);
          uint32_t s4[4];
          mf_bcast4(sb, s4);
          // unconditional refill (past the end it rereads the last quad): a
          // conditional load leaves the compiler unsure how many loads are in
          // flight, and its waits then drain the ring once per turn. Issued
          // after the lane swaps have consumed the slot, so the slot's
          // registers need no copy.
          load_q(t, lj, lu);
          advance4(lj, lu);
          // the quad's four steps side by side: their LDS reads, then the
          // four MFMA chains, then the four block epilogues, so that neither
          // the LDS latency nor the MFMA latency is paid once per step. A
          // step past the share reads the slice's last step again and has
          // factor 0 (a finite block dot, or a row already non-finite).
          bf16x8 ah[4], al[4];
          f32x4 xo[4];
          float sv[4];
#pragma unroll
          for (int jj = 0; jj < 4; jj++) {
            const int u = u0 + 4 * t + jj;
            const bool live = u < spw && kw * spw + u < nst;  // workgroup-uniform
            const int su = min(kw * spw + u, nst - 1);
            const int ab = su * P * M * 64;
            ah[jj] = *reinterpret_cast<const bf16x8*>(smem + ab + aoff);
            if (P == 2) al[jj] = *reinterpret_cast<const bf16x8*>(smem + ab + M * 64 + aoff);
            xo[jj] = *reinterpret_cast<const f32x4*>(smem + xs_off + (su * 16 + 4 * qd) * 4);
            sv[jj] = live ? __uint_as_float(s4[jj]) : 0.0f;
          }
          f32x4 blk[4];
#pragma unroll
          for (int jj = 0; jj < 4; jj++)
            blk[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[jj], mf_q4_dword(d[jj]), xo[jj], 0, 0, 0);
          if (P == 2) {
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
              blk[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[jj], mf_q4_dword(d[jj]), blk[jj], 0, 0, 0);
          }
#pragma unroll
          for (int jj = 0; jj < 4; jj++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[e] = fmaf(sv[jj], blk[jj][e], acc[e]);
        }
      }
      finish(j);
    }
  } else {
  for (int j = 0; j < nunits; j++) {
    for (int u0 = 0; u0 < spp; u0 += WD) {
#pragma unroll
      for (int i = 0; i < WD; i++) {
        const int u = u0 + i;
        const bf16x8 bw = mf_q8_codes(wc[i]);
        const float sv = mf_scale(wc[i].s);
        // unconditional refill (past the end it rereads the last step): a
        // conditional load leaves the compiler unsure how many loads are in
        // flight, and its waits then drain the ring once per turn
        load_w(i, lj, lu);
        advance(lj, lu);
        const int su = kw * spw + u;
        if (u < spw && su < nst) step(su, bw, sv);
      }
    }
    finish(j);
  }
  }
}

hipError_t launch_split_reduce(const float* part, void* y, int64_t n, int ks, int y_dtype, hipStream_t stream,
                               hipEvent_t start, hipEvent_t stop);

// One configuration: ks K-slices, gcols workgroup columns per slice.
template <int FMT, typename ST, int XT, int KW, int GW, int WD>
hipError_t launch_gemv_mf_t(const MatmulArgs& a, int ks, int gcols) {
  constexpr int P = XT == RQ_F32 ? 2 : 1;
  auto kernel = &gemv_mf_kernel<FMT, ST, XT, KW, GW, WD>;
  const int nkb = (int)(a.k / 32);
  if (ks < 1 || ks > nkb || gcols < 1 || a.m < 1 || a.m > 16) return hipErrorInvalidValue;
  if (ks > 1 && !a.part) return hipErrorInvalidValue;
  const int spl = (nkb + ks - 1) / ks;
  if ((int64_t)(ks - 1) * spl >= nkb) return hipErrorInvalidValue;  // every slice holds steps
  const int lds = mf_lds_bytes((int)a.m, spl, P, KW, GW);
  if (lds > 163840) return hipErrorInvalidValue;
  // dynamic LDS above 64 KB is allowed once per kernel and device
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
  hipExtLaunchKernelGGL(kernel, dim3((unsigned)(gcols * ks)), dim3(64 * KW * GW), (unsigned)lds, a.stream,
                        a.ev_main[0], a.ev_main[1], 0, a.q, static_cast<const ST*>(a.scales),
                        a.x, a.y, a.part, (int)a.m, (int)a.k, (int)a.n, (int)a.npad, a.y_dtype, ks);
  if (hipError_t e = hipGetLastError()) return e;
  if (ks > 1) return launch_split_reduce(a.part, a.y, a.m * a.n, ks, a.y_dtype, a.stream, a.ev_aux[0], a.ev_aux[1]);
  return hipSuccess;
}

}  // namespace rq

namespace rq {

// Plan: taken for 4 < m <= 16 with Q4_0 weights, 8 < m <= 16 with Q8_0. There
// the int8 decode kernel spends most of its time forming its activation levels
// and in its per-window epilogue (K = 4096, N = 14336 Q4, f32 x: m = 6 / 8 /
// 16 21.4 / 23.6 / 38 us, this kernel 16.3 / 16.7 / 18 us); below it stays
// ahead (m = 2 / 4: 12.3 / 14.9 us against 15.6 / 16.0 us). The waves of a workgroup take different groups
// (splitting K between them measured slower at m = 16): Q4_0 16 waves with
// an 8-step ring (two quads; at that shape 17.9 us against 18.8 for 8 waves
// and 16 steps, and at K = 8192, N = 28672, bf16 x, 40.6 against 45.8),
// Q8_0 8 waves with a 16-step ring (32 steps: 30 us with 8-byte Q4 loads);
// ks: at least the fewest K-slices whose LDS fits two workgroups per CU, and
// enough workgroups for ~85% of the CUs (slices of at least 8 steps): at
// K = 4096, m = 16 both give 4 (18 us, against 20 at ks = 2 and 22 at 8); at
// m = 6 the LDS alone would allow 2 (23.3 us against 16.3 at 4).
MfPlan plan_gemv_mf(int64_t m, int64_t k, int64_t npad, int x_dtype, int format, int cu_count) {
  MfPlan p{};
  const int64_t m_min = format == RQ_Q4_0 ? 5 : 9;
  if (m < m_min || m > 16 || (x_dtype != RQ_F32 && x_dtype != RQ_BF16) || k % 32 != 0 || k < 32) return p;
  // Q8_0 (8-byte loads, no quads) only for small weights: at 4096 x 4096
  // m = 12 / 16 15.1 / 15.4 us against 26.9 for the int8-level kernel, at
  // K = 8192, N = 28672 81 / 90 / 101 us against 62 / 66 / 70 (m = 9 / 12 / 16)
  if (format == RQ_Q8_0 && npad * k > (int64_t(32) << 20)) return p;
  const int parts = x_dtype == RQ_F32 ? 2 : 1;
  const int64_t nkb = k / 32, ngroups = npad / 16;
  p.kw = 1;
  p.gw = format == RQ_Q4_0 ? 16 : 8;
  p.wd = format == RQ_Q4_0 ? 8 : 16;
  int64_t ks = 1;
  while (mf_lds_bytes((int)m, (int)((nkb + ks - 1) / ks), parts, p.kw, p.gw) > 81920 ||
         (ks - 1) * ((nkb + ks - 1) / ks) >= nkb) {
    if (++ks > nkb) return p;
  }
  p.gcols = (int)((ngroups + p.gw - 1) / p.gw);
  const int64_t fill = std::min<int64_t>(((int64_t)cu_count * 85 / 100 + p.gcols - 1) / p.gcols,
                                         std::max<int64_t>(1, nkb / 8));
  int64_t kf = std::max(ks, fill);
  // a power of two where the slices stay 8 steps long: even slices without
  // padded ring turns (K = 8192, N = 28672: m = 6 ks 3 / 4 49.9 / 41.0 us,
  // m = 16 ks 7 / 8 56.2 / 50.0 us)
  int64_t k2 = 1;
  while (k2 < kf) k2 *= 2;
  if (k2 * 8 <= nkb) kf = k2;
  while (kf > ks && (kf - 1) * ((nkb + kf - 1) / kf) >= nkb) --kf;  // no empty slice
  ks = kf;
  p.ks = (int)ks;
  if ((int64_t)p.gcols * ks > INT32_MAX) return p;
  p.ok = true;
  return p;
}

template <int FMT, typename ST, int XT>
static hipError_t launch_mf_x(const MatmulArgs& a, const MfPlan& p) {
  if constexpr (FMT == RQ_Q4_0) {
    if (p.kw == 1 && p.gw == 16 && p.wd == 8) return launch_gemv_mf_t<FMT, ST, XT, 1, 16, 8>(a, p.ks, p.gcols);
  } else {
    if (p.kw == 1 && p.gw == 8 && p.wd == 16) return launch_gemv_mf_t<FMT, ST, XT, 1, 8, 16>(a, p.ks, p.gcols);
  }
  return hipErrorInvalidValue;
}

template <int FMT, typename ST>
static hipError_t launch_mf_s(const MatmulArgs& a, const MfPlan& p) {
  return a.x_dtype == RQ_F32 ? launch_mf_x<FMT, ST, RQ_F32>(a, p) : launch_mf_x<FMT, ST, RQ_BF16>(a, p);
}

hipError_t launch_gemv_mf(const MatmulArgs& a, const MfPlan& p) {
  if (!p.ok) return hipErrorInvalidValue;
  if (a.format == RQ_Q8_0) return launch_mf_s<RQ_Q8_0, float>(a, p);
  if (a.scale_dtype == RQ_F16) return launch_mf_s<RQ_Q4_0, uint16_t>(a, p);
  return launch_mf_s<RQ_Q4_0, float>(a, p);
}

}  // namespace rq
