/*
 * rq_oracle.h — CPU restatement of Raster's block-quantized matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP kernels in
 * raster_amd/csrc: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. No product code path calls into it.
 *
 * Every function restates one reference function (Clojure, read as text from
 * replikativ/raster); the citation is the reference file:line it follows.
 * Numerics follow the JVM semantics of those functions:
 *   - Clojure arithmetic on float and double operands widens to double;
 *   - Math/round is Java Math.round(double): ties toward +infinity;
 *   - (float d) is one IEEE round-to-nearest-even narrowing.
 * Built with -O2 -ffp-contract=off and no fast-math so every rounding is the
 * one written.
 */
#ifndef RQ_ORACLE_H
#define RQ_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- java.util.Random (JDK LCG) — used to regenerate the reference tests'
 *      inputs (e.g. test/raster/quant/train_test.clj:14-16, pack_test.clj:9-12,
 *      tile_test.clj:10-11). nextGaussian uses the C library log/sqrt where
 *      the JDK uses StrictMath (fdlibm); the two can differ in the last bit on
 *      rare inputs, so Gaussian draws only feed tolerance-based checks. */
typedef struct {
  int64_t seed;
  double next_next_gaussian;
  int have_next_next_gaussian;
} rqo_jrandom;

void rqo_jrandom_init(rqo_jrandom* r, int64_t seed);
int32_t rqo_jrandom_next(rqo_jrandom* r, int bits);
int32_t rqo_jrandom_next_int(rqo_jrandom* r);
double rqo_jrandom_next_double(rqo_jrandom* r);
double rqo_jrandom_next_gaussian(rqo_jrandom* r);
void rqo_jrandom_next_bytes(rqo_jrandom* r, int8_t* out, int64_t n);
/* fill helpers matching the reference tests' generators */
void rqo_jfill_gauss(int64_t seed, double mult, float* out, int64_t n);       /* train_test.clj:14-16 */
void rqo_jfill_uniform_centered(int64_t seed, float* out, int64_t n);         /* pack_test.clj:9-12 */
void rqo_jfill_bytes(int64_t seed, int8_t* out, int64_t n);                   /* tile_test.clj:10-11 */

/* Java Math.round(double): floor(x + 0.5) evaluated exactly; NaN -> 0. */
int64_t rqo_java_round(double x);

/* ---- scalar conversions ---- */
float rqo_f16_to_f32(uint16_t h);          /* Float.float16ToFloat, raster/types/float16.clj:40-43 */
uint16_t rqo_f32_to_f16(float f);          /* Float.floatToFloat16 (RNE) */
float rqo_bf16_to_f32(uint16_t b);         /* exact widening */
uint16_t rqo_f32_to_bf16(float f);         /* RNE narrowing (NaN stays NaN) */

/* ---- int8 MAC seam ---- */
/* par/dp4a: raster/par.clj:421-440 (signed little-endian byte lanes). */
int64_t rqo_dp4a(int32_t a, int32_t b, int64_t acc);
/* wi8-dot-q4: raster/quant/kernels.clj:33-46 (16 packed bytes, lo=k, hi=k+16). */
int64_t rqo_wi8_dot_q4(const uint8_t* wq, int64_t woff, const int8_t* xq, int64_t xoff);
/* wi8-dot: raster/quant/kernels.clj:48-61 (unsigned byte x signed int8). */
int64_t rqo_wi8_dot(const uint8_t* wq, int64_t woff, const int8_t* xq, int64_t xoff, int64_t len);

/* ---- Q8_0 row-major (signed codes, f32 scale per 32) ---- */
/* q8-quantize: raster/quant/train.clj:34-58. Returns 0, or -1 if in % 32 != 0. */
int rqo_q8_quantize(const float* W, int64_t out, int64_t in, int8_t* codes, float* scales);
/* dequant-q8-dense: raster/quant/train.clj:60-71. */
void rqo_dequant_q8_dense(const int8_t* codes, const float* scales, int64_t in, int64_t out, float* W);
/* qlinear-q8: raster/quant/train.clj:77-108 (f32 products, f64 accumulator, f32 store). */
void rqo_qlinear_q8(const float* x, const int8_t* codes, const float* scales,
                    int64_t m, int64_t in, int64_t out, float* y);
/* qlinear-q8-dx: raster/quant/train.clj:110-137. */
void rqo_qlinear_q8_dx(const float* dy, const int8_t* codes, const float* scales,
                       int64_t m, int64_t in, int64_t out, float* dx);

/* ---- parametric unsigned-offset quantizer (Q4_0 / unsigned Q8_0) ---- */
/* quantize-weight: raster/compiler/backend/cpu/quant.clj:42-70. nibble != 0 selects
 * :nibble-interleaved (wq has len/2 bytes), else :byte-direct (len bytes). */
void rqo_quantize_weight(const float* w, int64_t len, int weight_bits, int zero_point,
                         int nibble, uint8_t* wq, float* ws);
/* Inverse used by test/raster/compiler/backend/cpu/quant_encode_test.clj:9-24. */
void rqo_dequant_weight(const uint8_t* wq, const float* ws, int64_t len, int zero_point,
                        int nibble, float* out);
/* Q4_0 rows with fp16 scales (the configs' storage): W[o,i] = f32(d)*(q-8), one rounding. */
void rqo_dequant_q4_f16(const uint8_t* wq, const uint16_t* ws_f16, int64_t in, int64_t out, float* W);
/* Q4_0 rows with f32 scales. */
void rqo_dequant_q4_f32(const uint8_t* wq, const float* ws, int64_t in, int64_t out, float* W);
/* f32-activation Q4_0 linear: qlinear-q8's loop (train.clj:92-107) over the Q4_0
 * dequant (quant_encode_test.clj:19-20); scale is fp16 when ws_f16 != NULL, else f32. */
void rqo_qlinear_q4(const float* x, const uint8_t* wq, const uint16_t* ws_f16, const float* ws_f32,
                    int64_t m, int64_t in, int64_t out, float* y);

/* ---- activation quantizer + int-activation GEMVs ---- */
/* quantize-act-blocks! / quantize-act-i8: cpu/quant.clj:282-305 (clamped, Java round). */
void rqo_quantize_act_i8(const float* x, int64_t M, int64_t in, int8_t* xq, float* xs, int32_t* xsum);
/* qmatmul-q4-composable!: raster/quant/kernels.clj:161-184 (row-major Q4_0, f32 scales). */
void rqo_qmatmul_q4_composable(const int8_t* xq, const float* xs, const int32_t* xsum,
                               const uint8_t* wq, const float* ws, float* y,
                               int64_t in, int64_t out, int64_t o_start, int64_t o_count);

/* ---- column-interleaved x8 layout (CPU stream-gemv layout) ---- */
/* repack: raster/compiler/core/layout.clj:246-286 (tile 8, k-group 4).
 * nibble: src wq row-major Q4_0 [out*in/2] -> wqi [(out/8)*(in/32)*128];
 * byte-direct: src wq unsigned bytes [out*in] -> wqi [(out/8)*(in/32)*256]. */
int rqo_repack_x8(const uint8_t* wq, const float* ws, int64_t out, int64_t in, int nibble,
                  uint8_t* wqi, float* wsi);
/* wi8-dot-q4-x8 / wi8-dot-q8-x8: raster/quant/kernels.clj:63-90, 258-278. */
void rqo_wi8_dot_q4_x8(const uint8_t* wqi, int64_t woff, const int8_t* xq, int64_t xoff, int32_t* out8);
void rqo_wi8_dot_q8_x8(const uint8_t* wqi, int64_t woff, const int8_t* xq, int64_t xoff, int32_t* out8);
/* qmatmul-q4-x8! / qmatmul-q8-x8!: raster/quant/kernels.clj:216-247, 308-333. */
void rqo_qmatmul_q4_x8(const int8_t* xq, const float* xs, const int32_t* xsum,
                       const uint8_t* wqi, const float* wsi, float* y,
                       int64_t in, int64_t out, int64_t g_start, int64_t g_count);
void rqo_qmatmul_q8_x8(const int8_t* xq, const float* xs, const int32_t* xsum,
                       const uint8_t* wqi, const float* wsi, float* y,
                       int64_t in, int64_t out, int64_t g_start, int64_t g_count);

/* ---- signed q8_0 x q8_0 prefill path ---- */
/* quantize-one-q8: raster/quant/pack.clj:55-81. Returns -1 if in % 32 != 0. */
int rqo_quantize_one_q8(const float* W, int64_t in, int64_t out, int32_t* wp, float* ws);
/* quant-act-i8-rows-gpu!: raster/quant/kernels_k.clj:309-342 (no clamp). */
void rqo_quant_act_i8_rows(const float* x, int32_t* xp, float* xs, int64_t in, int64_t nrows);
/* qmatmul-i8-gemm!: raster/quant/kernels_k.clj:344-370. */
void rqo_qmatmul_i8_gemm(const int32_t* xp, const float* xs, const int32_t* wp, const float* ws,
                         float* y, int64_t in, int64_t out, int64_t nrows);
/* i8gemv-dp4a!: raster/quant/kernels_k.clj:141-150. */
void rqo_i8gemv_dp4a(const int32_t* wp, const int32_t* xp, float* y, int64_t kw, int64_t out);

/* ---- decoder-step glue (f32 arrays, double arithmetic as on the JVM) ---- */
/* rms-norm!: raster/dl/nn.clj:497-516. */
void rqo_rms_norm(const float* x, const float* w, float* out, int64_t rows, int64_t features, double eps,
                  double gain_offset);
/* rope-pos: raster/dl/attention.clj:197-214. */
void rqo_rope_pos(const float* x, float* out, int64_t seq_len, int64_t heads, int64_t head_dim, double theta,
                  int64_t pos_offset);
/* gqa-decode-attention: raster/dl/attention.clj:248-287 (sc: cache_len floats of scratch). */
void rqo_gqa_decode_attention(const float* q, const float* k, const float* v, int64_t cache_len, int64_t n_q,
                              int64_t n_kv, int64_t head_dim, double scale, float* out, float* sc);
/* silu-mul!: raster/dl/nn.clj:200-203. */
void rqo_silu_mul(const float* gate, const float* up, float* out, int64_t n);
/* residual-add!: raster/dl/nn.clj:217-219. */
void rqo_residual_add(const float* a, const float* b, float* out, int64_t n);
/* kv-append!: raster/dl/attention.clj:413-416. */
void rqo_kv_append(const float* src, float* cache, int64_t kvrow, int64_t pos);
/* One pre-norm decoder layer for one token over Q8_0 linears (q, k, v, o,
 * gate, up, down); see rq_oracle.c. */
void rqo_decoder_layer(float* x, const int8_t* const* w, const float* const* s, const float* gain1,
                       const float* gain2, float* kcache, float* vcache, int64_t d, int64_t n_q, int64_t n_kv,
                       int64_t head_dim, int64_t ffn, int64_t cache_len, double eps, double theta,
                       float* scratch);

/* ---- K-quants (raster/compiler/backend/cpu/quant.clj:78-280; Raster's own
 * layout, not GGUF's) over a row-major [out x in] matrix, in % 256 == 0, each
 * row its own super-blocks (raster/quant/kernels_k.clj:1-10) ---- */
/* quantize-weight-q4k (quant.clj:92-137) of len values: wq[len/2] nibbles
 * (w[k] low, w[k+16] high per 32-sub-block), da/db[len/256], aq[len/32]
 * (0..63), bq[len/32] (-32..31). */
void rqo_quantize_weight_q4k(const float* w, int64_t len, uint8_t* wq, float* da, float* db, uint8_t* aq,
                             int8_t* bq);
/* nextpad (raster/quant/pack.clj:30-33): in rounded up to a multiple of 256 */
int64_t rqo_nextpad(int64_t in);
/* q4k-of (raster/quant/pack.clj:45-53): rows zero-padded to inp = nextpad(in),
 * then quantize-weight-q4k over out * inp values. Returns inp (-1: no memory). */
int64_t rqo_q4k_of(const float* W, int64_t out, int64_t in, uint8_t* wq, float* da, float* db, uint8_t* aq,
                   int8_t* bq);
/* dequant-q4k (quant.clj:139-156): x = (da*aq)*q + (db*bq), in double, one narrowing */
void rqo_dequant_q4k(const uint8_t* wq, const float* da, const float* db, const uint8_t* aq, const int8_t* bq,
                     int64_t len, float* out);
/* quantize-weight-q6k (quant.clj:214-239): wq[len] (0..63, zero point 32),
 * sc[len/16] (0..127), ds[len/256] */
void rqo_quantize_weight_q6k(const float* w, int64_t len, uint8_t* wq, int8_t* sc, float* ds);
/* dequant-q6k (quant.clj:241-252): x = (ds*sc)*(q-32) */
void rqo_dequant_q6k(const uint8_t* wq, const int8_t* sc, const float* ds, int64_t len, float* out);
/* quantize-act-q8k (quant.clj:158-176) of m rows of in: xq[m*in], xs[m*in/256]
 * (d = max|x|/127 per super-block), bsums[m*in/sub] (sub = 32 for Q4_K, 16 for Q6_K) */
void rqo_quantize_act_q8k(const float* x, int64_t m, int64_t in, int64_t sub, int8_t* xq, float* xs,
                          int32_t* bsums);
/* qmatmul-q4k-composable! (raster/quant/kernels_k.clj:15-46) for each of m
 * activation rows: y[t*out + o] */
void rqo_qmatmul_q4k(const int8_t* xq, const float* xs, const int32_t* bsums, const uint8_t* wq, const float* da,
                     const float* db, const uint8_t* aq, const int8_t* bq, int64_t m, int64_t in, int64_t out,
                     float* y);
/* qmatmul-q6k-composable! (raster/quant/kernels_k.clj:48-79) */
void rqo_qmatmul_q6k(const int8_t* xq, const float* xs, const int32_t* bsums, const uint8_t* wq, const int8_t* sc,
                     const float* ds, int64_t m, int64_t in, int64_t out, float* y);

/* ---- dense helpers (brute force, f64) used to pin the restatements ---- */
/* dense f32 GEMM surface (blas.clj float arms, nn/linear) */
void rqo_sgemm(int trans_a, int trans_b, int64_t m, int64_t k, int64_t n, float alpha, const float* A,
               const float* B, float beta, float* C);
void rqo_linear(const float* x, const float* W, const float* b, float* y, int64_t batch, int64_t in, int64_t out);
void rqo_dense_matmul_nt_f64(const float* X, const float* W, int64_t m, int64_t in, int64_t out,
                             double* y);

#ifdef __cplusplus
}
#endif
#endif
