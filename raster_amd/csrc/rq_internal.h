// rq_internal.h — shared definitions for librq's HIP translation units.
// gfx950 (CDNA4) only: wave64, MFMA bf16/i8, 160 KB LDS per CU.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/rq.h"

namespace rq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
// Register arrays use native vector types: HIP's uint2/uint4 are union-backed
// structs, and arrays of them can end up in scratch memory.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Resident weight in HBM, "chunked" layout. Rows are padded with zeros to
// npad = 16 * ceil(out / 16). Chunk (g, b) holds the 16 rows [16g, 16g+16) of
// the 32-element block b (nb = in / 32 blocks per row), chunks ordered g-major:
//   codes  : CB bytes per row and block, CB = 32 (Q8_0: int8 codes) or
//            16 (Q4_0: Raster's packing, byte j = lo nibble elem j | hi nibble
//            elem j+16); chunk (g, b) at byte (g*nb + b) * 16*CB, row r of the
//            chunk at + r*CB.
//   scales : 16 per chunk (f32, or fp16 bits), element (g*nb + b)*16 + r.
// A 16-row x 64-element window is then 1 KB (Q8) or 512 B (Q4) of contiguous
// codes and every weight load a kernel issues covers whole cache lines.
// Both arrays live in one allocation, each 256-byte aligned.
struct Weight {
  uint32_t magic;
  int format;       // RQ_Q8_0 / RQ_Q4_0
  int scale_dtype;  // RQ_F32 / RQ_F16
  int device;
  int64_t out, in, npad;
  void* base;       // device allocation
  uint8_t* q;       // chunked codes / packed nibbles
  void* scales;     // chunked scales, block-major (prefill kernels, dequant)
  void* scales_rb;  // the same scales row-batched (decode kernel)
  // K-quants (RQ_Q4_K / RQ_Q6_K) keep Raster's row-major codes in q, the
  // super-block scales in `scales` (Q4_K: da, db side by side) and these:
  void* sub_scales;  // per (row, sub-block): Q4_K aq, bq side by side; Q6_K sc
  size_t bytes;
  struct Ctx* ctx;
};

// bytes of codes per row and 32-element block
__host__ __device__ constexpr int code_bytes(int fmt) { return fmt == RQ_Q8_0 ? 32 : 16; }
__host__ __device__ __forceinline__ int64_t chunk_of(int64_t row, int64_t b, int64_t nb) { return (row >> 4) * nb + b; }
// byte offset of (row, block b) in the chunked codes
template <int FMT>
__host__ __device__ __forceinline__ int64_t code_off(int64_t row, int64_t b, int64_t nb) {
  return chunk_of(row, b, nb) * (16 * code_bytes(FMT)) + (row & 15) * code_bytes(FMT);
}
// Chunked scales are kept in two orders, each read by the kernels it suits:
//  * block-major: chunk (g, b) holds the 16 rows' scales of block b. A
//    prefill step reads one block of 16 rows: 64 contiguous bytes.
//  * row-batched: per 16-row group, the blocks in batches of 8 (4 windows of
//    64 elements), each batch stored row by row, [batch][row 0..15][8 blocks],
//    the last batch zero-padded. A decode lane gets all of its row's scales
//    for a batch in one 16-byte (f16) or two (f32) loads.
// element offset of (row, block b) in the block-major scales
__host__ __device__ __forceinline__ int64_t scale_off(int64_t row, int64_t b, int64_t nb) {
  return chunk_of(row, b, nb) * 16 + (row & 15);
}
__host__ __device__ __forceinline__ int64_t scale_nb8(int64_t nb) { return (nb + 7) / 8 * 8; }
// first row-batched scale of 16-row group g
__host__ __device__ __forceinline__ int64_t scale_rb_group(int64_t g, int64_t nb) { return g * scale_nb8(nb) * 16; }
// offset of (block b, row r) inside its group, row-batched
__host__ __device__ __forceinline__ int scale_rb_in_group(int b, int r) { return (b >> 3) * 128 + r * 8 + (b & 7); }

// Fused decode options (rq_qmatmul_fused); all off when zero.
struct DecodeOps {
  const float* norm_gain;  // RMSNorm of each x row first, times gain[k]
  float norm_eps;
  const void* residual;    // y = residual + product (y's dtype and shape)
  int swiglu;              // y[m][i] = silu(z[m][2i]) * z[m][2i+1]; y has n / 2 columns
  int act_i8;              // quantize x to Raster's int8 blocks in the kernel
  const float* act_scale;  // int8 input (x is int8): xs[m][b]
  const int32_t* act_sum;  // int8 input: xsum[m][b] (Q4_0)
};

// Activation dtype code of the decode kernel for int8 input quantized
// beforehand (not a public rq_dtype).
constexpr int kXtI8 = 3;

// Launch descriptor for the matmul kernels.
struct MatmulArgs {
  const uint8_t* q;
  const void* scales;     // block-major
  const void* scales_rb;  // row-batched
  int scale_dtype;
  int format;
  const void* x;
  int x_dtype;
  void* y;
  int y_dtype;
  int64_t m, k, n;  // m activation rows, k = in, n = out
  int64_t npad;     // n padded to a multiple of 16 (rows present in the chunked layout)
  hipStream_t stream;
  void* scratch;    // bf16 GEMM: ceil(m/16)*16 * k bf16 for the fragment-major activations
  float* part;      // decode with K-split: partial sums, DecodePlan::part_bytes
  DecodeOps ops = {nullptr, 0.0f, nullptr, 0, 0, nullptr, nullptr};
  // kernel timing: when set, the main kernel is launched with hipExtLaunchKernel
  // and these events take that dispatch's own start and end timestamps; on a
  // call whose partial sums a second kernel adds, ev_aux brackets that kernel
  hipEvent_t ev_main[2] = {nullptr, nullptr};
  hipEvent_t ev_aux[2] = {nullptr, nullptr};
  int slices = 1;  // K-slices of the small-m GEMM (partial sums in `part`)
};

// Decode kernel (m <= 16) launch plan: rows per MFMA group, waves per
// workgroup, K-slices per 16-row group, grid and LDS; ok is false when the
// decode kernel cannot take the shape (then the GEMM path runs).
struct DecodePlan {
  bool ok;
  int mt, waves, ksplit, grid, lds_bytes;
  size_t part_bytes;  // scratch for the slices' partial sums (ksplit > 1)
};
DecodePlan plan_decode(int64_t m, int64_t k, int64_t npad, int cu_count);

// Decode on bf16 MFMA with exact codes (gemv_mf.hip): plain calls, f32 / bf16
// x, 4 < m <= 16 (Q4_0) or 8 < m <= 16 (Q8_0) (the kernel takes m <= 16).
// kw x gw waves per workgroup,
// wd-step weight ring, ks K-slices, gcols workgroup columns per slice.
// Dense f32 GEMM (dense.hip, rocBLAS): a library handle per context, created
// on first use. Statuses are rocBLAS's (0 = success).
int dense_create(void** handle);
void dense_destroy(void* handle);
const char* dense_status_string(int st);
// C[m x n] = alpha op(A) op(B) + beta C, row-major; op(A) = A^T when trans_a
// (A stored [k x m]), op(B) = B^T when trans_b (B stored [n x k])
int dense_sgemm(void* handle, hipStream_t stream, int trans_a, int trans_b, int64_t m, int64_t n, int64_t k,
                float alpha, const float* a, const float* b, float beta, float* c);
// y[r, :] = b for r < rows
hipError_t launch_bias_rows(const float* b, float* y, int64_t rows, int64_t cols, hipStream_t stream);

struct MfPlan {
  bool ok;
  int kw, gw, wd, ks, gcols;
};
MfPlan plan_gemv_mf(int64_t m, int64_t k, int64_t npad, int x_dtype, int format, int cu_count);
hipError_t launch_gemv_mf(const MatmulArgs& a, const MfPlan& p);
// m = 1 decode on v_dot4_i32_i8 for Q4_0 weights (gemv1.hip): plain calls,
// f32 / bf16 x. waves per workgroup, ring depth, workgroups.
struct G1Plan {
  bool ok;
  int waves, ring, gcols;
};
G1Plan plan_gemv1(int64_t m, int64_t k, int64_t npad, int x_dtype, int format, int cu_count);
hipError_t launch_gemv1(const MatmulArgs& a, const G1Plan& p);

// y[e] = sum over s < ks of part[s * n + e] (f32 or bf16 y), in slice order
hipError_t launch_split_reduce(const float* part, void* y, int64_t n, int ks, int y_dtype, hipStream_t stream,
                               hipEvent_t start, hipEvent_t stop);

// Kernel launchers (each returns a hipError_t from hipGetLastError after launch).
hipError_t launch_gemv(const MatmulArgs& a, const DecodePlan& p);
hipError_t launch_gemm(const MatmulArgs& a, int cu_count);
hipError_t launch_gemm_bf16(const MatmulArgs& a, int cu_count);
// bf16 x, 16 < m <= 64, weight-stream GEMM with LDS-staged activations
// (gemm_sm.hip); K-slices and whether it takes a call
int gemm_sm_slices(int format, int64_t m, int64_t k, int64_t npad, int cu_count);
bool gemm_sm_takes(int format, int64_t m, int64_t k);
hipError_t launch_gemm_sm(const MatmulArgs& a, int ks);
// int8 activations (x_dtype kXtI8, scales / sums in a.ops), m > 16 (gemm_i8.hip)
hipError_t launch_gemm_i8(const MatmulArgs& a, int cu_count);
// bf16 x, m > 128: 256 x 192 tiles on 32x32x16 MFMA, one wave per SIMD
// (gemm_wide.hip), where its tiles fill their rounds of the CUs
struct WidePlan {
  bool ok;
  int tiles_m, tiles_n;
};
WidePlan plan_gemm_wide(int64_t m, int64_t k, int64_t npad, int cu_count);
// bytes of the 32x32x16 operand copy of x (rows rounded up to 32)
size_t pack_x32_bytes(int64_t m, int64_t k);
hipError_t launch_gemm_wide(const MatmulArgs& a, const WidePlan& p);
// 256 x 32 nf tiles, eight waves split into MFMA consumers and dequantizing
// producers (gemm_wide.hip); K a multiple of 64
hipError_t launch_gemm_rs(const MatmulArgs& a, int nf);  // nf: 3 or 4 column fragments
// Fragment-major copy of bf16 activations into a.scratch (gemm_bf16.hip).
hipError_t launch_pack_x(const MatmulArgs& a);
hipError_t launch_dequant(const Weight& w, float* out, hipStream_t stream);
hipError_t launch_quantize_act_i8(const float* x, int64_t m, int64_t in, int8_t* xq, float* xs, int32_t* xsum,
                                  hipStream_t stream);
// K-quants (kquant.hip)
hipError_t launch_quantize_act_q8k(const float* x, int64_t m, int64_t in, int sub, int8_t* xq, float* xs,
                                   int32_t* bsums, hipStream_t stream);
size_t kquant_gemv_lds(int format, int64_t k, int mt);
hipError_t launch_kquant_gemv(const Weight& w, const int8_t* xq, const float* xs, const int32_t* bsums, void* y,
                              int y_dtype, int64_t m, int cu_count, hipStream_t stream);
hipError_t launch_kquant_dequant(const Weight& w, float* out, hipStream_t stream);
// backward-data on f32 MFMA for m <= kDxFmMaxRows (dx.hip): the weight as
// stored feeds the MFMA's B operand; column tiles x dy-row tiles x slices of
// the row groups (part: slices * m * in f32 when slices > 1)
constexpr int64_t kDxFmMaxRows = 32;
int dx_fm_slices(int64_t m, int64_t in, int64_t npad, int cu_count);
hipError_t launch_dx_fm(const Weight& w, const float* dy, float* dx, int64_t m, float* part, int slices,
                        hipStream_t stream);
// backward-data on bf16 MFMA for m > kDxFmMaxRows (dx_mf.hip): dy packed
// into `pack` (dx_mf_pack_bytes), reduction slices (part: slices * m * in f32
// when slices > 1)
size_t dx_mf_pack_bytes(int64_t m, int64_t npad);
int dx_mf_slices(int64_t m, int64_t in, int64_t npad, int cu_count);
hipError_t launch_dx_mf(const Weight& w, const float* dy, float* dx, int64_t m, void* pack, float* part, int slices,
                        hipStream_t stream);
// RoPE + KV append + single-query attention for one decode step (attention.hip).
size_t decode_attention_lds(int64_t pos, int64_t head_dim);
// Cached rows split into nsplit ranges of rps rows per head; nsplit > 1 needs
// scratch_bytes of device scratch for the ranges' records.
struct AttnSplit {
  int nsplit, rps;
  int threads;  // workgroup size of the chunk kernel: 256, 512 or 1024
  int np;       // rows per lane per chunk at 256 threads (2, or the larger default)
  int group;    // > 1: the grouped-query kernel, a workgroup per KV head serving this many query heads
  size_t scratch_bytes;
};
AttnSplit plan_decode_attention(int64_t pos, int64_t n_q, int64_t n_kv, int64_t head_dim, int cu_count);
hipError_t launch_decode_attention(const float* q, const float* k, const float* v, float* kcache, float* vcache,
                                   int64_t pos, int64_t n_q, int64_t n_kv, int64_t head_dim, double theta,
                                   double scale, float* out, const AttnSplit& sp, void* scratch, hipStream_t stream);
// Weight encoders (encode.hip): q4k-of (rows zero-padded from in to inp) and
// quantize-weight-q6k (in % 256 == 0), device arrays in, device arrays out.
hipError_t launch_q4k_encode(const float* W, int64_t out, int64_t in, int64_t inp, uint8_t* wq, float* da, float* db,
                             uint8_t* aq, int8_t* bq, hipStream_t stream);
hipError_t launch_q6k_encode(const float* W, int64_t out, int64_t in, uint8_t* wq, int8_t* sc, float* ds,
                             hipStream_t stream);
// y[o] = (float) sum_w dp4a(wp[o * kw + w], xp[w]) (i8gemv.hip)
hipError_t launch_i8gemv_dp4a(const int32_t* wp, const int32_t* xp, float* y, int64_t kw, int64_t out,
                              hipStream_t stream);
// Streaming read of `bytes` (a multiple of 16) for the read-ceiling
// measurement (stream.hip): `grid` workgroups of 256 threads; sink holds
// grid * 256 words.
hipError_t launch_stream_read(const void* src, size_t bytes, int grid, uint32_t* sink, hipStream_t stream);
// Row-major (Raster's layout) -> chunked, for codes and scales (layout.hip).
hipError_t launch_chunk_weight(int format, int scale_dtype, const uint8_t* q_rm, const void* s_rm, int64_t out,
                               int64_t in, int64_t npad, uint8_t* q, void* s, void* s_rb, hipStream_t stream);

// ---- device helpers shared by every kernel that decodes weights -----------

// A pointer read from a by-value argument struct is generic to the compiler,
// so loads through it become flat loads; a flat load also counts against the
// LDS wait counter, and any LDS wait after it then waits for memory. This
// marks such a pointer as one into global memory.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* as_global(const T* p) {
  return (const __attribute__((address_space(1))) T*)p;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// Two f32 -> packed bf16, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  bf16x2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// A dword of Q8_0 codes (signed bytes) as two packed bf16 pairs: RNE of the
// f32 product scale * code (one rounding, as Raster's dequant). Each byte is
// converted with its sign by a byte-select conversion (v_cvt_f32_i32 with a
// sign-extended byte operand), so no bias or offset is needed.
__device__ __forceinline__ u32x2 q8_dword_bf16(uint32_t v, float s) {
  return u32x2{pack2_bf16(s * (float)(int8_t)v, s * (float)(int8_t)(v >> 8)),
               pack2_bf16(s * (float)(int8_t)(v >> 16), s * (float)(int8_t)(v >> 24))};
}

// Round-to-nearest-even f32 -> bf16 bits (NaN kept quiet).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// A block scale as loaded (f32 bits, or f16 bits zero-extended) and its value.
// Register rings of weights in flight keep the bits and convert when the step
// is computed: converting at load time makes the compiler wait for the load
// right there.
template <typename ST>
__device__ __forceinline__ uint32_t load_scale_bits(const ST* s, int64_t i);
template <>
__device__ __forceinline__ uint32_t load_scale_bits<float>(const float* s, int64_t i) { return __float_as_uint(s[i]); }
template <>
__device__ __forceinline__ uint32_t load_scale_bits<uint16_t>(const uint16_t* s, int64_t i) { return s[i]; }
template <typename ST>
__device__ __forceinline__ float scale_from_bits(uint32_t b);
template <>
__device__ __forceinline__ float scale_from_bits<float>(uint32_t b) { return __uint_as_float(b); }
template <>
__device__ __forceinline__ float scale_from_bits<uint16_t>(uint32_t b) { return f16_bits_to_f32((uint16_t)b); }

__device__ __forceinline__ float scale_value(float s) { return s; }
__device__ __forceinline__ float scale_value(uint16_t s) { return f16_bits_to_f32(s); }

template <typename ST>
__device__ __forceinline__ float load_scale(const ST* s, int64_t i);
template <>
__device__ __forceinline__ float load_scale<float>(const float* s, int64_t i) { return s[i]; }
template <>
__device__ __forceinline__ float load_scale<uint16_t>(const uint16_t* s, int64_t i) {
  return f16_bits_to_f32(s[i]);
}

// Four consecutive activations of a row as f32 (x_dtype f32 or bf16; for int8
// x the four codes travel as the bits of v[0]); zeros when !ok.
template <int XT>
__device__ __forceinline__ void load_x4(const void* x, int64_t off, bool ok, float (&v)[4]) {
  if (!ok) {
    v[0] = v[1] = v[2] = v[3] = 0.0f;
  } else if (XT == kXtI8) {
    // four int8 codes, carried as the bits of v[0]
    v[0] = __uint_as_float(*reinterpret_cast<const uint32_t*>(static_cast<const int8_t*>(x) + off));
    v[1] = v[2] = v[3] = 0.0f;
  } else if (XT == RQ_F32) {
    const f32x4 t = *reinterpret_cast<const f32x4*>(static_cast<const float*>(x) + off);
    v[0] = t[0];
    v[1] = t[1];
    v[2] = t[2];
    v[3] = t[3];
  } else {
    const u32x2 t = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(x) + off);
    v[0] = __uint_as_float(t[0] << 16);
    v[1] = __uint_as_float(t[0] & 0xFFFF0000u);
    v[2] = __uint_as_float(t[1] << 16);
    v[3] = __uint_as_float(t[1] & 0xFFFF0000u);
  }
}

// Reductions over the 8 lanes that share a block (lanes 8j..8j+7): swap
// neighbours, then pairs, then the two quads of the row half (DPP moves, no
// LDS traffic).
__device__ __forceinline__ int dpp_xor1(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ int dpp_xor2(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false); }
__device__ __forceinline__ int dpp_half_mirror(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false); }
__device__ __forceinline__ float max8(float v) {
  v = fmaxf(v, __int_as_float(dpp_xor1(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_xor2(__float_as_int(v))));
  return fmaxf(v, __int_as_float(dpp_half_mirror(__float_as_int(v))));
}
__device__ __forceinline__ int or8(int v) {
  v |= dpp_xor1(v);
  v |= dpp_xor2(v);
  return v | dpp_half_mirror(v);
}
__device__ __forceinline__ int sum8(int v) {
  v += dpp_xor1(v);
  v += dpp_xor2(v);
  return v + dpp_half_mirror(v);
}

// Math/round of a double clamped to [-127, 127] (the int8 quantizers'
// rounding, raster/compiler/backend/cpu/quant.clj:296-298): floor, plus one
// when the fraction is at least 1/2 (x - floor(x) is exact in double), so ties
// go toward +infinity. NaN gives 0.
__device__ __forceinline__ int java_round_clamp127(double v) {
  if (!(v == v)) return 0;
  const double f = floor(v);
  const double r = (v - f >= 0.5) ? f + 1.0 : f;
  return r > 127.0 ? 127 : r < -127.0 ? -127 : (int)r;
}

// Signed Q8 code j (0..3) of a little-endian dword, as an exact float.
__device__ __forceinline__ float q8_code(uint32_t d, int j) { return (float)(int8_t)(d >> (8 * j)); }
// Q4 nibble value q (0..15) of byte j of a dword; hi selects the high nibble.
__device__ __forceinline__ float q4_nib(uint32_t d, int j, bool hi) {
  return (float)((d >> (8 * j + (hi ? 4 : 0))) & 0xFu);
}

}  // namespace rq
