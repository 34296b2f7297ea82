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
// is. Here the activations come in chunks of KC k-steps staged in LDS
// (double-buffered, one burst of loads per chunk, consumed a whole chunk after
// issue), so the weight ring can be WD = 2 KC steps deep. They are read from
// row-major x itself, no packing pass: a wave's load takes 4 rows x 256
// contiguous bytes (the chunk's 4 blocks), and the LDS slots are rotated per
// lane group so that these stores, like the MFMA reads, hit every bank
// (against the packing kernel's fragment-major copy: C5 Q8_0 M = 32 61.5 ->
// 59.4 us per call, Q4_0 49.4 -> 48.2, K = 4096, N = 11008 Q8_0 M = 32 21.0 ->
// 19.0; Q4_0 at M = 64 61.1 -> 62.3). Loading 16 rows x 64 bytes per wave
// instead (each lane's natural piece) measured C5 Q8_0 M = 32 65.3 us, and
// 4 x 256 bytes without the rotated slots (4-way bank conflicts on the
// stores) Q4_0 M = 64 67.7. Each wave owns NTW 16-row weight fragments; the 4
// waves of a workgroup cover 64 NTW columns and all of m (MT 16-row tiles).
// K may be cut into ks slices (grid.y) whose f32 partial sums a second kernel
// adds in slice order (deterministic), for more waves in flight.
//
// Q4_0 weights stream in quads of chunks: lane (r, q) loads the 16-byte row r
// of chunk q of the quad (1 KB per wave load; 8-byte loads would have two
// lanes per address), and two rounds of lane-row swaps (v_permlane32_swap,
// v_permlane16_swap) hand lane (r, q) dword q of row r of each of the four
// chunks, k = 4q .. 4q+3 (low nibbles) and 4q+16 .. 4q+19 (high nibbles). The
// activation fragments are staged into LDS in that k order.
//
// Loads go through buffer resources (the workgroup's weight groups, the
// packed activations) with the k position and the group as uniform offsets:
// no 64-bit address arithmetic per load, and a load past a resource's end
// reads zeros. The loop is then bound by the dequantization's VALU work: at
// M = 32, K = 8192, N = 28672, Q4_0 it measured 64 VALU instructions per
// k-step and wave (80 with per-lane 64-bit addresses and per-nibble bit-field
// extracts) and 51.7 against 56.7 us per call.
#include <algorithm>

#include "rq_internal.h"

namespace rq {

namespace {

struct WCodesSm {
  u32x2 v;
  uint32_t s;  // scale bits, converted at dequantization
};

// buffer resource over bytes [p, p + bytes): loads past the end return zero
__device__ __forceinline__ __amdgpu_buffer_rsrc_t sm_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

struct WQuadSm {
  u32x4 v;     // row r of chunk q of the quad
  uint32_t s;  // that chunk's scale bits for row r
};

// Lane (r, a) holds d[b] = dword b of row r of chunk a; afterwards d[j] =
// dword a of row r of chunk j (swaps between the 16-lane rows: rows {2, 3}
// of d[0] with rows {0, 1} of d[2], likewise d[1], d[3]; then rows {1, 3} of
// one with rows {0, 2} of the other).
__device__ __forceinline__ void xpose4_rows(uint32_t (&d)[4]) {
  const auto p02 = __builtin_amdgcn_permlane32_swap(d[0], d[2], false, false);
  const auto p13 = __builtin_amdgcn_permlane32_swap(d[1], d[3], false, false);
  const auto q01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
  const auto q23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
  d[0] = q01[0];
  d[1] = q01[1];
  d[2] = q23[0];
  d[3] = q23[1];
}

// Lane row a holds s (of chunk a); afterwards b[j] = lane row j's s in every
// row.
__device__ __forceinline__ void bcast4_rows(uint32_t s, uint32_t (&b)[4]) {
  const auto p = __builtin_amdgcn_permlane32_swap(s, s, false, false);
  const auto b01 = __builtin_amdgcn_permlane16_swap(p[0], p[0], false, false);
  const auto b23 = __builtin_amdgcn_permlane16_swap(p[1], p[1], false, false);
  b[0] = b01[0];
  b[1] = b01[1];
  b[2] = b23[0];
  b[3] = b23[1];
}

// Dword a of a Q4_0 row (bytes 4a .. 4a+3) dequantized to bf16 in the k order
// k = 4a .. 4a+3, 4a+16 .. 4a+19: exact f32 scale * (n - 8), one RNE rounding
template <typename ST>
__device__ __forceinline__ bf16x8 dequant_q4_dword(uint32_t d, uint32_t sbits) {
  const float s = scale_from_bits<ST>(sbits), off = -8.0f * s;
  uint32_t lo = d & 0x0F0F0F0Fu, hi = (d >> 4) & 0x0F0F0F0Fu;
  // opaque to the known-bits fold, which would extract each nibble with its
  // own v_bfe before a byte-0 conversion: the byte-select conversions then
  // take the four bytes of lo and hi directly
  asm("" : "+v"(lo), "+v"(hi));
  auto two = [&](uint32_t v, int b) {
    return pack2_bf16(fmaf((float)((v >> (8 * b)) & 0xFFu), s, off), fmaf((float)((v >> (8 * b + 8)) & 0xFFu), s, off));
  };
  return __builtin_bit_cast(bf16x8, u32x4{two(lo, 0), two(lo, 2), two(hi, 0), two(hi, 2)});
}

// 8 bf16 of the lane's Q8_0 fragment share: exact f32 scale * code, one RNE
// rounding (the dequant of gemm_bf16.hip)
template <typename ST>
__device__ __forceinline__ bf16x8 dequant_sm_q8(const WCodesSm& c) {
  const float s = scale_from_bits<ST>(c.s);
  const u32x2 p0 = q8_dword_bf16(c.v[0], s), p1 = q8_dword_bf16(c.v[1], s);
  return __builtin_bit_cast(bf16x8, u32x4{p0[0], p0[1], p1[0], p1[1]});
}

// The 16-byte slot of lane (r, g) of the activation fragment of step u in
// LDS: within each 256-byte lane group the rows are rotated by 4 g + 4 (u % 2).
// The MFMA reads stay one permutation of each lane group (no bank conflicts),
// and a staging store of 4 rows x 4 lane groups x 4 steps (16 bytes each), or
// of their 8-byte halves (Q4_0), spreads over all banks.
__device__ __forceinline__ int sm_slot(int u, int g, int r) { return 16 * g + ((r + 4 * g + 4 * (u & 1)) & 15); }

}  // namespace

template <int FMT, typename ST, int MT, int NTW, int KC>
__global__ __launch_bounds__(256) void gemm_sm_kernel(const uint8_t* __restrict__ q, const ST* __restrict__ sc,
                                                     const uint16_t* __restrict__ x, void* __restrict__ y,
                                                     float* __restrict__ part, int M, int K, int N, int npad,
                                                     int y_dtype) {
  constexpr int WD = 2 * KC;             // weight ring depth (steps)
  constexpr int AP = KC * MT / 4;        // 16-byte activation pieces per thread per chunk
  __shared__ __attribute__((aligned(16))) bf16x8 As[2][KC][MT][64];
  const int nkb = K / 32;
  const int ks = (int)gridDim.y, sl = (int)blockIdx.y;
  // this workgroup's K-slice: steps [kb0, kb0 + nst); slices are whole pairs
  // of chunks (the last one may be shorter)
  const int spl = ((nkb + ks - 1) / ks + 2 * KC - 1) / (2 * KC) * (2 * KC);
  const int kb0 = min(nkb, sl * spl), nst = min(nkb, kb0 + spl) - kb0;
  const int nch = (nst + KC - 1) / KC;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, fg = lane >> 4;
  const int n0 = (int)blockIdx.x * 64 * NTW;
  const int g_last = npad / 16 - 1;
  // buffer resources: this workgroup's weight groups (codes, scales) and the
  // packed activations. A load's k position and group are uniform offsets;
  // groups past the last one read zeros (their outputs are never stored).
  constexpr uint32_t CB = FMT == RQ_Q8_0 ? 512u : 256u;
  const int gq0 = n0 / 16, ngr = min(4 * NTW, g_last + 1 - gq0);
  const __amdgpu_buffer_rsrc_t qr = sm_rsrc(q + (int64_t)gq0 * nkb * CB, (uint32_t)(ngr * nkb) * CB);
  const __amdgpu_buffer_rsrc_t sr =
      sm_rsrc(sc + (int64_t)gq0 * nkb * 16, (uint32_t)(ngr * nkb) * 16u * (uint32_t)sizeof(ST));
  const __amdgpu_buffer_rsrc_t xr = sm_rsrc(x, (uint32_t)M * (uint32_t)K * 2u);
  const int nstm = max(nst - 1, 0);
  uint32_t gofs[NTW];  // chunk row of group j (uniform)
#pragma unroll
  for (int j = 0; j < NTW; j++) gofs[j] = (uint32_t)__builtin_amdgcn_readfirstlane((wave * NTW + j) * nkb + kb0);

  // activation pieces of a chunk, straight from row-major x: piece
  // p = tid + 256 i holds the 16 bytes k = 32 kb + 8 g .. + 7 of row R = p / 16
  // (tile R / 16, row r = R % 16), kb the chunk's step u, with
  // (u, g) = (p % 16 / 4, p % 4): a wave's load reads 4 rows of 256
  // contiguous bytes each. Rows past m read zeros (they only feed outputs that
  // are never stored); steps past the slice reread its last step (zeroed when
  // staged).
  u32x4 areg[AP];
  auto load_a = [&](int c) {
#pragma unroll
    for (int i = 0; i < AP; i++) {
      const int p = tid + 256 * i, q = p & 15;
      const uint32_t kb = (uint32_t)(kb0 + min(c * KC + (q >> 2), nstm));
      areg[i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     xr, (int)((uint32_t)(p >> 4) * (uint32_t)K * 2u + kb * 64u + 16u * (uint32_t)(q & 3)), 0, 0));
    }
  };
  auto store_a = [&](int buf, int c) {
#pragma unroll
    for (int i = 0; i < AP; i++) {
      const int p = tid + 256 * i, q = p & 15, u = q >> 2, g = q & 3, t = p >> 8, r = (p >> 4) & 15;
      if (c * KC + u >= nst) areg[i] = u32x4{0u, 0u, 0u, 0u};  // a step past the slice adds nothing
      if (FMT == RQ_Q4_0) {
        // the piece of lane (r, g) holds k = 8g .. 8g+7: k = 8g .. 8g+3 go
        // to lane group 2 (g & 1), 8g+4 .. 8g+7 to the next one, the upper
        // half of the block (g >= 2) to the upper 8 bytes of each
        const int g0 = 2 * (g & 1);
        uint8_t* base = reinterpret_cast<uint8_t*>(&As[buf][u][t][0]) + 8 * (g >> 1);
        *reinterpret_cast<u32x2*>(base + 16 * sm_slot(u, g0, r)) = u32x2{areg[i][0], areg[i][1]};
        *reinterpret_cast<u32x2*>(base + 16 * sm_slot(u, g0 + 1, r)) = u32x2{areg[i][2], areg[i][3]};
      } else {
        *reinterpret_cast<u32x4*>(&As[buf][u][t][sm_slot(u, g, r)]) = areg[i];
      }
    }
  };
  static_assert(KC == 4, "a chunk is one Q4_0 quad, and 16 activation pieces per row");
  WCodesSm wc[FMT == RQ_Q4_0 ? 1 : WD][NTW];
  WQuadSm wq[FMT == RQ_Q4_0 ? WD / 4 : 1][NTW];
  auto load_w = [&](int slot, int s) {  // step s of the slice (clamped)
    if constexpr (FMT == RQ_Q4_0) {
      // quad slot / 4 of steps s .. s+3 (slot, s multiples of 4): lane
      // (fr, fg) loads step s + fg
      const uint32_t kl = (uint32_t)min(s + fg, nstm);
      const uint32_t vq = kl * 256u + (uint32_t)fr * 16u, vs = (kl * 16u + (uint32_t)fr) * (uint32_t)sizeof(ST);
#pragma unroll
      for (int j = 0; j < NTW; j++) {
        wq[slot / 4][j].v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, (int)vq, (int)(gofs[j] * 256u), 0));
        if constexpr (sizeof(ST) == 4)
          wq[slot / 4][j].s = __builtin_amdgcn_raw_buffer_load_b32(sr, (int)vs, (int)(gofs[j] * 64u), 0);
        else
          wq[slot / 4][j].s = __builtin_amdgcn_raw_buffer_load_b16(sr, (int)vs, (int)(gofs[j] * 32u), 0);
      }
    } else {
      const uint32_t kl = (uint32_t)min(s, nstm);  // uniform
      const uint32_t vq = (uint32_t)fr * 32u + 8u * (uint32_t)fg, vs = (uint32_t)fr * (uint32_t)sizeof(ST);
#pragma unroll
      for (int j = 0; j < NTW; j++) {
        wc[slot][j].v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(qr, (int)vq, (int)((gofs[j] + kl) * 512u), 0));
        if constexpr (sizeof(ST) == 4)
          wc[slot][j].s = __builtin_amdgcn_raw_buffer_load_b32(sr, (int)vs, (int)((gofs[j] + kl) * 64u), 0);
        else
          wc[slot][j].s = __builtin_amdgcn_raw_buffer_load_b16(sr, (int)vs, (int)((gofs[j] + kl) * 32u), 0);
      }
    }
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
  for (int s = 0; s < KC; s += FMT == RQ_Q4_0 ? 4 : 1) load_w(s, s);
  __builtin_amdgcn_sched_barrier(0);
  store_a(0, 0);
  load_a(1);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = KC; s < WD; s += FMT == RQ_Q4_0 ? 4 : 1) load_w(s, s);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();

  // chunk c (LDS buffer c % 2, ring slots (c % 2) KC ..): first stage chunk
  // c+1 (in registers since chunk c-1) into the other buffer and load chunk
  // c+2; then its steps, each computing from the LDS activations and the
  // weights in its ring slot, whose refill (step s + WD) goes out at once;
  // one barrier at the end (the other buffer is complete, this one is free).
  // Nothing in the loop is conditional: steps past the slice get zero
  // activations (store_a) and clamped weights, and an odd chunk count runs
  // one such chunk more. With conditional loads or early exits the compiler's
  // wait counts at the merges drained every load in flight once or twice per
  // loop turn (measured at C5, M = 32: Q4_0 51.0 -> 48.9 us per call with
  // even chunk counts, 50.7 -> 52.0 with the padded chunk of an odd count).
  // A padded step multiplies zeros by finite weights; a non-finite scale
  // already makes its column non-finite.
  auto chunk = [&](int c, const int buf) {
    // keeps the zeroing selects of store_a (pure VALU on the registers that
    // load_a filled a chunk ago) from being hoisted into the previous chunk,
    // where they would wait for those loads
    __builtin_amdgcn_sched_barrier(0);
    store_a(buf ^ 1, c + 1);
    __builtin_amdgcn_sched_barrier(0);
    load_a(c + 2);
    __builtin_amdgcn_sched_barrier(0);
    uint32_t dq[NTW][4], sq[NTW][4];  // the current quad, after the swaps
#pragma unroll
    for (int u = 0; u < KC; u++) {
      const int s = c * KC + u;
      const int slot = buf * KC + u;
      bf16x8 wf[NTW];
      if constexpr (FMT == RQ_Q4_0) {
        if (u % 4 == 0) {
#pragma unroll
          for (int j = 0; j < NTW; j++) {
#pragma unroll
            for (int b = 0; b < 4; b++) dq[j][b] = wq[slot / 4][j].v[b];
            // the scale as f32 before the broadcast: one conversion per
            // quad, and no zero-extension of the loaded half word ahead
            // of its use
            sq[j][0] = __float_as_uint(scale_from_bits<ST>(wq[slot / 4][j].s));
          }
#pragma unroll
          for (int j = 0; j < NTW; j++) {
            xpose4_rows(dq[j]);
            bcast4_rows(sq[j][0], sq[j]);
          }
        }
#pragma unroll
        for (int j = 0; j < NTW; j++) wf[j] = dequant_q4_dword<float>(dq[j][u % 4], sq[j][u % 4]);
      } else {
#pragma unroll
        for (int j = 0; j < NTW; j++) wf[j] = dequant_sm_q8<ST>(wc[slot][j]);
        load_w(slot, s + WD);
      }
      bf16x8 af[MT];
#pragma unroll
      for (int i = 0; i < MT; i++) af[i] = As[buf][u][i][sm_slot(u, fg, fr)];
#pragma unroll
      for (int j = 0; j < NTW; j++)
#pragma unroll
        for (int i = 0; i < MT; i++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[j], af[i], acc[i][j], 0, 0, 0);
      // Q4_0: the quad slot's refill after the quad's last step, when the
      // swapped copy is dead, so that the load can land in the same registers
      // (issued while the copy is live, it gets other registers, and the
      // loop's end copies them back, waiting for the load)
      if (FMT == RQ_Q4_0 && u % 4 == 3) load_w(slot - 3, s - 3 + WD);
    }
    __syncthreads();
  };
  for (int c = 0; c < nch; c += 2) {
    chunk(c, 0);
    chunk(c + 1, 1);  // past the end at an odd count: zero activations
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

// y = sum over K-slices of the partial sums part[s * n + e], in slice order.
// V elements per thread (4: 16-byte loads); the slices' loads go out four at
// a time (a loop over a run-time slice count would otherwise wait for each
// load before issuing the next), the adds stay in slice order.
template <int V>
__global__ __launch_bounds__(256) void gemm_sm_reduce_kernel(const float* __restrict__ part, void* __restrict__ y,
                                                            int64_t n, int ks, int y_dtype) {
  typedef float fv __attribute__((ext_vector_type(V)));
  const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V;
  if (e >= n) return;
  auto ld = [&](int s) { return *reinterpret_cast<const fv*>(part + (int64_t)s * n + e); };
  fv t = ld(0);
  int s = 1;
  for (; s + 3 < ks; s += 4) {
    const fv a = ld(s), b = ld(s + 1), c = ld(s + 2), d = ld(s + 3);
    t += a;
    t += b;
    t += c;
    t += d;
  }
  for (; s < ks; s++) t += ld(s);
  if (y_dtype == RQ_F32) {
    *reinterpret_cast<fv*>(static_cast<float*>(y) + e) = t;
  } else {
#pragma unroll
    for (int i = 0; i < V; i++) static_cast<uint16_t*>(y)[e + i] = (uint16_t)f32_to_bf16_bits(t[i]);
  }
}

hipError_t launch_split_reduce(const float* part, void* y, int64_t n, int ks, int y_dtype, hipStream_t stream,
                               hipEvent_t start, hipEvent_t stop) {
  const bool vec = n % 4 == 0 && (reinterpret_cast<uintptr_t>(part) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(y) & (y_dtype == RQ_F32 ? 15 : 1)) == 0;
  if (vec)
    hipExtLaunchKernelGGL(gemm_sm_reduce_kernel<4>, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, stream,
                          start, stop, 0, part, y, n, ks, y_dtype);
  else
    hipExtLaunchKernelGGL(gemm_sm_reduce_kernel<1>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, start,
                          stop, 0, part, y, n, ks, y_dtype);
  return hipGetLastError();
}

// Chunks of 4 k-steps (an 8-step weight ring). Weight fragments per wave:
// two (128 columns per workgroup) for Q4_0 and at m > 32: with the Q4_0
// quads, at M = 32 / 64, K = 8192, N = 28672 51.5 / 69.1 us against 55.7 /
// 78.1 us for one fragment and 8-step chunks; Q8_0 at m > 32: M = 48 / 64
// 72.7 / 75.1 us against 78.8 / 79.5 for one. Q8_0 at m <= 32 takes one
// fragment (64 columns, twice the workgroups, fewer K-slices: C5 M = 17 / 32
// in one slice, no reduction): K = 8192, N = 28672, M = 17 / 32 60.9 / 63.1
// -> 59.1 / 60.6 us per call; K = 4096, N = 11008, M = 32 23.4 -> 21.1;
// N = 14336, M = 24 24.8 -> 24.4.
constexpr int kSmKC = 4;
static int sm_ntw(int format, int64_t m) { return format == RQ_Q8_0 && m <= 32 ? 1 : 2; }

template <int FMT, typename ST, int MT, int NTW>
static hipError_t launch_sm_t(const MatmulArgs& a, int ks) {
  constexpr int KC = kSmKC;
  const dim3 grid((unsigned)((a.npad / 16 + 4 * NTW - 1) / (4 * NTW)), (unsigned)ks);
  hipExtLaunchKernelGGL((gemm_sm_kernel<FMT, ST, MT, NTW, KC>), grid, dim3(256), 0, a.stream, a.ev_main[0],
                        a.ev_main[1], 0, a.q, static_cast<const ST*>(a.scales), static_cast<const uint16_t*>(a.x),
                        a.y, a.part, (int)a.m, (int)a.k, (int)a.n, (int)a.npad, a.y_dtype);
  if (hipError_t e = hipGetLastError()) return e;
  if (ks > 1) return launch_split_reduce(a.part, a.y, a.m * a.n, ks, a.y_dtype, a.stream, a.ev_aux[0], a.ev_aux[1]);
  return hipSuccess;
}

// K-slices: about 24 waves per CU at m <= 32 (12 above: the 4-tile kernel
// holds fewer per CU), 4 per 64 NTW output columns times the slices; each
// slice keeps at least 8 chunks of K. Measured (Q4, bf16 x, two fragments per
// wave, 4-step chunks): M = 32, K = 8192, N = 28672: 3 / 4 / 6 / 8 slices
// 52.5 / 53.2 / 52.3 / 51.5 us; M = 64: 1 / 2 slices 82.9 / 69.1 us;
// M = 17, K = 4096, N = 14336: 2 / 4 slices 21.1 / 19.2 us. Q8_0 (cold,
// packing included), K = 8192, N = 28672: M = 17 2 / 3 / 4 / 6 slices 69.9 /
// 63.3 / 63.2 / 66.2 us, M = 32 75.3 / 67.1 / 69.5 / 71.3, M = 64 87.4 / 81.1 /
// 90.7 / 86.7.
int gemm_sm_slices(int format, int64_t m, int64_t k, int64_t npad, int cu_count) {
  // Q8_0 moves twice the bytes per step: 12 waves per CU at every m
  const int64_t waves = (npad / (64 * sm_ntw(format, m))) * 4;
  const int64_t want = (int64_t)cu_count * (format == RQ_Q8_0 || m > 32 ? 12 : 24);
  int64_t ks = std::max<int64_t>(1, want / std::max<int64_t>(waves, 1));
  ks = std::min<int64_t>(ks, std::max<int64_t>(1, (k / 32) / (8 * kSmKC)));
  // slices of whole chunk pairs: the nearest multiple of 2 KC steps to the
  // even split, then as many slices as that takes (C5 Q4_0 M = 32: 6 -> 7
  // slices of 40 steps; Q8_0 3 slices of 88)
  const int64_t nkb = k / 32, pair = 2 * kSmKC;
  const int64_t len = std::max<int64_t>(pair, ((nkb + ks - 1) / ks + pair / 2) / pair * pair);
  ks = (nkb + len - 1) / len;
  return (int)std::max<int64_t>(1, std::min<int64_t>(ks, 8));
}

// Q4_0 at 16 < m <= 64. Q8_0 at 16 < m <= 48, and up to 64 from K = 8192:
// measured cold against the per-wave-weights GEMM (Q8_0, bf16 x and y,
// packing included), K = 8192, N = 28672: m = 17 / 32 / 48 / 64 63 / 67 / 79 /
// 81 us against 92 / 84 / 88 / 87; K = 4096, N = 11008: m = 17 / 32 / 48 / 64
// 24.3 / 25.3 / 28.4 / 29.1 against 27.9 / 29.1 / 29.4 / 29.3; K = 4096,
// N = 14336: m = 17 / 32 / 64 26.5 / 27.7 / 32.5 against 30.3 / 30.1 / 31.0.
// The buffer offsets are 32-bit: K is bounded so that a workgroup's weight
// rows (8 groups x K/32 chunks of up to 512 bytes) and the packed activations
// (4 tiles x K/32 x 1 KB) stay far below 2^32 bytes.
constexpr int64_t kSmMaxK = int64_t(1) << 22;

bool gemm_sm_takes(int format, int64_t m, int64_t k) {
  if (m <= 16 || m > 64 || k > kSmMaxK) return false;
  return format == RQ_Q4_0 || m <= 48 || k >= 8192;
}

hipError_t launch_gemm_sm(const MatmulArgs& a, int ks) {
  if (a.m <= 16 || a.m > 64 || a.k > kSmMaxK) return hipErrorInvalidValue;
#define RQ_SM(FMT_, ST_) return a.m <= 32 ? launch_sm_t<FMT_, ST_, 2, 2>(a, ks) : launch_sm_t<FMT_, ST_, 4, 2>(a, ks);
  if (a.format == RQ_Q8_0)
    return a.m <= 32 ? launch_sm_t<RQ_Q8_0, float, 2, 1>(a, ks) : launch_sm_t<RQ_Q8_0, float, 4, 2>(a, ks);
  if (a.scale_dtype == RQ_F16) { RQ_SM(RQ_Q4_0, uint16_t) }
  RQ_SM(RQ_Q4_0, float)
#undef RQ_SM
}

}  // namespace rq
