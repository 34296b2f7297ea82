/*
 * rq.h — C ABI of librq, the MI355X (gfx950) block-quantized matmul library.
 *
 * Plain C: scalars, pointers and sizes only. A JVM caller binds these symbols
 * with Panama FFM downcalls (the reference reaches every native library that
 * way: raster/linalg/blas.clj:162-186, raster/gpu/ze_runtime.clj:40-64); a
 * Python caller uses ctypes. Reference paths below are inside replikativ/raster.
 *
 * Conventions
 *  - Every entry point returns an int status (RQ_OK == 0). On failure,
 *    rq_last_error() gives a message for the calling thread
 *    (mirrors ze-call! mapping non-zero driver status to ex-info,
 *    raster/gpu/ze_runtime.clj:281-291).
 *  - Weight layout is Raster's row-major [out x in] ("y = x . W^T"), one scale
 *    per 32 consecutive `in` elements, scales row-major [out x in/32]
 *    (raster/quant/train.clj:13-16, raster/compiler/backend/cpu/quant.clj:27-39).
 *  - "Device pointer" arguments are HIP device allocations (from rq_buf_alloc
 *    or any hipMalloc). "stream" is a hipStream_t passed as void*; NULL means
 *    the null stream. Compute entry points are asynchronous on that stream and
 *    never retain host pointers after they return.
 *  - bf16 and fp16 travel as raw uint16 bits (Raster's :half convention,
 *    raster/types/float16.clj:8). bf16 outputs are rounded to nearest even.
 *  - y is fully overwritten, never accumulated into (the :overwrite buffer
 *    write mode of raster/quant/op.clj:75-79).
 */
#ifndef RQ_H
#define RQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RQ_VERSION 1

/* status codes */
enum {
  RQ_OK = 0,
  RQ_ERR_SHAPE = 1,   /* in % 32 != 0, out % 8 != 0 for x8 layouts, non-positive dims */
  RQ_ERR_DTYPE = 2,   /* dtype/format not supported by this entry point */
  RQ_ERR_NULL = 3,    /* required pointer is NULL */
  RQ_ERR_OOM = 4,     /* device allocation failed */
  RQ_ERR_HIP = 5,     /* a HIP runtime call failed (message has the HIP error) */
  RQ_ERR_HANDLE = 6,  /* unknown, destroyed or foreign context / weight handle */
  RQ_ERR_DEVICE = 7   /* no gfx950 device with that id */
};

/* element types */
enum { RQ_F32 = 0, RQ_BF16 = 1, RQ_F16 = 2 };

/* weight formats */
enum {
  RQ_Q8_0 = 0, /* signed int8 codes, W = scale * code (raster/quant/train.clj:13-16) */
  RQ_Q4_0 = 1, /* unsigned nibbles, zero-point 8, lo = elem k, hi = elem k+16 of each
                  32-block (raster/compiler/backend/cpu/quant.clj:27-31) */
  RQ_Q4_K = 2, /* K-quant super-blocks of 256: x = (da*aq)*q + (db*bq) per 32-sub-block
                  (raster/compiler/backend/cpu/quant.clj:85-156) */
  RQ_Q6_K = 3  /* K-quant super-blocks of 256: x = (ds*sc)*(q-32) per 16-sub-block
                  (raster/compiler/backend/cpu/quant.clj:201-252) */
};

typedef struct rq_ctx_s* rq_ctx;
typedef struct rq_weight_s* rq_weight;

/* ---- library / context ------------------------------------------------- */
int rq_version(void);
const char* rq_status_string(int status);
const char* rq_last_error(void);
/* Binds a context to a HIP device (raster/gpu/core.clj:243-257 make-session). */
int rq_ctx_create(int device, rq_ctx* out);
/* Idempotent per handle; destroys weights still owned by the context
 * (raster/gpu/core.clj:259-293 close-session!). */
int rq_ctx_destroy(rq_ctx ctx);
/* Number of compute units and the wavefront size of the context's device. */
int rq_ctx_device_info(rq_ctx ctx, int* cu_count, int* wave_size, int* clock_khz);

/* Kernel timing for measurement harnesses. No counterpart in the reference,
 * whose microbench (raster/runtime/microbench.clj:20-60) times whole calls;
 * this one separates the main kernel of a call (the MFMA GEMM or the decode
 * kernel) from the small activation-packing pass of the bf16 GEMM.
 * While enabled, every rq_qmatmul on this context records a pair of HIP
 * events around its main kernel (hipExtLaunchKernel; not on a stream that is
 * being captured): for the bf16 prefill GEMM with a packing pass, the end of
 * that pass and the end of the GEMM, which follows it directly; for the other
 * kernels, the dispatch's own start and end. A call whose partial sums a second kernel
 * adds counts as one launch timed as the sum of its two kernels' own
 * durations (the gap between them excluded).
 * rq_ctx_kernel_time waits for the pending pairs, returns their summed
 * duration and count, and clears them. Disabling frees the events. */
int rq_ctx_set_kernel_timing(rq_ctx ctx, int enable);
int rq_ctx_kernel_time(rq_ctx ctx, double* total_ms, int64_t* launches);

/* A plain streaming read of `bytes` (a multiple of 16) from device memory at
 * src (16-byte aligned), by cu_count * wg_per_cu workgroups (1..16 per CU) of
 * 256 threads with 16-byte loads; sink (device, cu_count * wg_per_cu * 256
 * words) is written only by chance. No counterpart in the reference: it
 * measures the HBM read ceiling the HBM-bound kernels are compared with.
 * Timed like a matmul while kernel timing is enabled. */
int rq_stream_read(rq_ctx ctx, const void* src, size_t bytes, int wg_per_cu, uint32_t* sink, void* stream);

/* ---- device memory and streams (raster/gpu/ze_runtime.clj:765-787 DeviceBuffer) */
int rq_buf_alloc(rq_ctx ctx, size_t bytes, void** dptr);
int rq_buf_free(rq_ctx ctx, void* dptr);
int rq_upload(rq_ctx ctx, void* dst_dev, const void* src_host, size_t bytes, void* stream);
int rq_download(rq_ctx ctx, void* dst_host, const void* src_dev, size_t bytes, void* stream);
int rq_stream_create(rq_ctx ctx, void** stream);
int rq_stream_destroy(rq_ctx ctx, void* stream);
int rq_sync(rq_ctx ctx, void* stream);

/* ---- resident quantized weights ------------------------------------------
 * Created once from Raster's host arrays and kept in HBM (the :constant role of
 * resident weights, raster/gpu/core.clj:889-940). */

/* Q8_0 from qlinear-q8's arrays: codes int8[out*in], scales f32[out*in/32]
 * (raster/quant/train.clj:88-89). */
int rq_weight_create_q8(rq_ctx ctx, const int8_t* codes, const float* scales, int64_t out, int64_t in,
                        rq_weight* w);
/* Q8_0 from quantize-one-q8's packed words: wp int32[out*in/4] (4 little-endian
 * int8 lanes each), ws f32[out*in/32] (raster/quant/pack.clj:55-81). */
int rq_weight_create_q8_packed(rq_ctx ctx, const int32_t* wp, const float* ws, int64_t out, int64_t in,
                               rq_weight* w);
/* Q4_0 row-major: packed u8[out*in/2]; scales are f32 (Raster's Q4_0 ws,
 * raster/compiler/backend/cpu/quant.clj:42-70) or fp16 bits (scale_dtype RQ_F16). */
int rq_weight_create_q4(rq_ctx ctx, const uint8_t* packed, const void* scales, int scale_dtype, int64_t out,
                        int64_t in, rq_weight* w);
/* From the x8 column-interleaved repack-stream layout that raster.quant.op's
 * qlinear-i8! / qlinear-i8-q8! take (raster/compiler/core/layout.clj:246-286):
 * nibble = 1 for Q4_0 (wqi u8[(out/8)*(in/32)*128]), 0 for the unsigned
 * zero-point-128 Q8 (wqi u8[(out/8)*(in/32)*256]); wsi f32[(out/8)*(in/32)*8].
 * out % 8 == 0. Stored on the device in the row-major form. */
int rq_weight_create_x8(rq_ctx ctx, const uint8_t* wqi, const float* wsi, int nibble, int64_t out, int64_t in,
                        rq_weight* w);
int rq_weight_destroy(rq_weight w);
int rq_weight_info(rq_weight w, int* format, int64_t* out, int64_t* in, int* scale_dtype, size_t* device_bytes);
/* Device pointers to the resident codes/packed bytes and scales (read-only).
 * The resident form is NOT Raster's row-major layout: rows are padded to
 * npad = ceil(out/16)*16 and stored in 16-row x 32-element chunks, chunk
 * (r/16, b) at index (r/16)*(in/32) + b. A chunk holds the 16 rows' code blocks
 * back to back (16 x 32 B for Q8_0, 16 x 16 B for Q4_0, each block in Raster's
 * byte order) and the scales chunk holds the 16 rows' scales of block b.
 * Padded rows are zero codes with zero scales. The weight also holds a second
 * copy of the scales, ordered for the decode kernel (per 16-row group, batches
 * of 8 blocks stored row by row); device_bytes counts both. */
int rq_weight_device_ptrs(rq_weight w, const void** qdata, const void** scales);

/* ---- compute ---------------------------------------------------------------- */

/* y[m,o] = sum_i dequant(W)[o,i] * x[m,i] for a resident weight; x is
 * [m x in] of x_dtype (RQ_F32 or RQ_BF16), y is [m x out] of y_dtype (RQ_F32 or
 * RQ_BF16), both device pointers, row-major; x 16-byte aligned and y aligned
 * to its element (else RQ_ERR_SHAPE). Replaces qlinear-q8
 * (raster/quant/train.clj:77-108) and, for Q4_0, the f32-activation dequant
 * GEMV; m <= 16 runs the HBM-bound GEMV kernels, larger m the MFMA GEMM.
 * m == 0 is a no-op.
 *
 * Kernel by call (plain calls; every rq_qmatmul_fused call takes the int8-level
 * decode kernel):
 *  - m = 1, Q4_0: the v_dot4_i32_i8 GEMV;
 *  - m <= 16, MFMA decode (bf16 MFMA on exact codes): Q4_0 at 5 <= m <= 16,
 *    Q8_0 at 9 <= m <= 16 when out * in <= 32 Mi (2^25) elements;
 *  - every other m <= 16: the int8-level decode kernel (int8 MFMA on the raw
 *    codes, v_mfma_i32_16x16x64_i8);
 *  - m > 16: bf16 x: the bf16 MFMA GEMM (the weight-stream GEMM for Q4_0
 *    at 16 < m <= 64 and for Q8_0 at 16 < m <= 48, or <= 64 when
 *    in >= 8192; for m > 128 and in % 64 == 0, 256 x 192 tiles with one
 *    wave per SIMD where they fill their rounds of the CUs to 80%, else the
 *    cost model's tile, 256 x 96 on the role-split kernel); f32 x: the
 *    exact-code f32 GEMM;
 *  - Q4_K / Q6_K weights (f32 x only, any m; bf16 x fails with RQ_ERR_DTYPE):
 *    x is quantized to q8_K in scratch and the K-quant GEMV runs, the same two
 *    kernels as rq_quantize_act_q8k + rq_qmatmul_q8k and bit for bit their
 *    results (QMatrix apply of the built-in :q4_K / :q6_K formats,
 *    raster/quant/core.clj:55-75). The GEMV takes four activation rows per
 *    pass over the weight, so a call streams the weight ceil(m / 4) times:
 *    meant for decode (m <= 16); at prefill sizes (m = 512: 128 passes) its
 *    time grows with m.
 *
 * Numerics (all accumulation in f32):
 *  - v_dot4 GEMV and int8-level decode kernel: each 32-block of each
 *    activation row is held as a 16-bit block fixed-point value:
 *    X = rint(x * 2^(15-e)) with e the block's max exponent, |X| < 2^15, so
 *    the per-element error is <= 2^(e-16) (below 1.6e-5 relative to the block
 *    maximum); the integer dots are exact, the block scale applied in f32. An
 *    inf or NaN activation makes its row's outputs NaN.
 *  - MFMA decode: codes enter the bf16 MFMA exactly, offset to small
 *    non-negative integers (c + 136 for Q4_0, c + 128 for Q8_0), the offset
 *    times the block's activation sum subtracted and the block scale applied
 *    in f32; f32 x split into two bf16 terms (|x - hi - lo| <= 2^-17 |x|).
 *    Finite input range: a block whose largest |x| exceeds about 7e34 (Q4_0)
 *    or 4e34 (Q8_0) overflows the offset sums and makes its row's outputs
 *    NaN; a non-finite activation makes its row's outputs non-finite.
 *  - bf16 x, m > 16: weights are dequantized to bf16 (exact f32 product
 *    scale*code, then one round-to-nearest-even) and multiplied with bf16 MFMA;
 *    on the eight-wave 16x16x32 tiles (m > 128 where the tile cost model
 *    picks 256 x 112, or in % 64 != 0) K is summed as two f32 partial sums,
 *    of the even and of the odd 32-blocks, added at the end; the 32x32x16
 *    kernels (256 x 96 / 256 x 128 role-split, 256 x 192) keep one running
 *    sum over K.
 *  - f32 x, m > 16: exact codes as bf16 with the scale applied in f32 and x
 *    split into two bf16 terms (about 16 mantissa bits).
 *
 * Scratch (per stream, allocated on first use, grown on demand, freed by
 * rq_ctx_destroy; calls on one stream are ordered, calls on different streams
 * do not share it):
 *  - bf16 x with m > 16, except in the weight-stream GEMM (which reads x as
 *    it is): the packed activation tile, ceil(m/32)*32*in*2 bytes;
 *  - K-slices' partial sums, m * out * 4 bytes per slice, added in slice
 *    order by a second kernel: the int8-level decode kernel when a row of x
 *    does not fit one workgroup's LDS (in above 17472 at m <= 4, 8704 at
 *    m <= 8); the MFMA decode kernel when a slice of x would not fit two
 *    workgroups' LDS, and further until the grid covers about 85% of the CUs,
 *    rounded up to a power of two while each slice keeps 8 blocks (at most
 *    in / 32 slices); the weight-stream GEMM (bf16 x, 16 < m <= 64) on a
 *    thin grid (up to 8 slices);
 *  - Q4_K / Q6_K: the q8_K activations, m * (in + in/256*4 + in/sub*4)
 *    bytes (each part rounded up to 256), sub = 32 for Q4_K, 16 for Q6_K.
 * Under HIP graph capture nothing can be allocated: run the same (or a
 * larger) shape once on the capturing stream before capturing, otherwise the
 * call fails with RQ_ERR_SHAPE and a message saying so. A buffer that grows is
 * replaced but not freed until rq_ctx_destroy, so a graph captured before a
 * larger call still replays on its own (still allocated) buffers; graphs and
 * eager calls on one stream share a buffer only while it has not grown, and
 * are ordered by the stream.
 */
int rq_qmatmul(rq_ctx ctx, rq_weight w, const void* x, int x_dtype, void* y, int y_dtype, int64_t m,
               void* stream);

/* Bytes of the fixed device scratch behind rq_qmatmul_noalloc. */
#define RQ_NOALLOC_SCRATCH_MAX (32u << 20)

/* rq_qmatmul that allocates nothing. No counterpart in the reference: it is
 * for callers that cannot allocate device memory mid-stream (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments, kernels and results as rq_qmatmul, bit for bit; no kernel-timing
 * events are recorded. Where rq_qmatmul would use per-stream scratch (the
 * packed activations of the bf16 GEMM, K-slice partial sums, a K-quant
 * weight's q8_K activations) this call uses a
 * fixed device array of RQ_NOALLOC_SCRATCH_MAX bytes that each GPU holds from
 * the first context created on it until the process ends; a call that needs
 * more fails with RQ_ERR_SHAPE and a message saying so (for example bf16 x
 * with m * in above 16 Mi elements). Every call on one GPU shares that GPU's
 * array, whatever its context or stream: calls that may overlap on one GPU
 * (different streams, or different host threads) race and must be ordered
 * by the caller. Nothing in the array needs to start at zero: each call
 * writes every scratch byte it later reads. */
int rq_qmatmul_noalloc(rq_ctx ctx, rq_weight w, const void* x, int x_dtype, void* y, int y_dtype, int64_t m,
                       void* stream);

/* Options of rq_qmatmul_fused; a NULL / 0 field is off. They fold the
 * decoder glue around a linear into its decode kernel (Raster chains them as
 * separate ops, test/raster/dl/decoder_layer_gpu_test.clj:25-83):
 *  - norm_gain (device f32[in], 16-byte aligned): each row of x is first
 *    RMS-normalised, x * (mean(x^2) + norm_eps)^-1/2 * norm_gain[k]
 *    (rms-norm! with gain offset 0, raster/dl/nn.clj:497-516);
 *  - residual (device, y's dtype and shape): y = residual + x . W^T
 *    (residual-add!, raster/dl/nn.clj:217-219);
 *  - swiglu: weight rows 2i and 2i+1 are a gate row and an up row; y[m, i] =
 *    silu(z[m, 2i]) * z[m, 2i+1] for the product z, so y has out/2 columns
 *    (silu-mul!, raster/dl/nn.clj:200-203). Not combined with residual;
 *  - act_i8: the activations (after the norm's gain) are quantized in the
 *    kernel to Raster's int8 blocks exactly as rq_quantize_act_i8 does and
 *    multiplied as rq_qmatmul_i8 does, instead of the default 16-bit block
 *    fixed point: Raster's int-activation numerics (qmatmul-q4-composable,
 *    raster/quant/kernels.clj:140-184). Without a norm the result is bitwise
 *    that of rq_quantize_act_i8 followed by rq_qmatmul_i8. With a norm the
 *    row's 1/rms factor is applied to the result (it factors out of the
 *    dot products), so the blocks quantized are those of x * gain.
 * The epilogue math runs in f32. */
typedef struct {
  const float* norm_gain;
  float norm_eps;
  const void* residual;
  int swiglu;
  int act_i8;
} rq_fused_ops;

/* rq_qmatmul with fused options, for m <= 16 (the decode kernel); larger m
 * fails with RQ_ERR_SHAPE. No counterpart in the reference as one call: it
 * replaces the op sequences named in rq_fused_ops around a qlinear. */
int rq_qmatmul_fused(rq_ctx ctx, rq_weight w, const void* x, int x_dtype, void* y, int y_dtype, int64_t m,
                     const rq_fused_ops* ops, void* stream);

/* K-quant weights from Raster's arrays (Raster's own layout, each row of the
 * [out x in] matrix its own super-blocks, in % 256 == 0, in <= 32768 for
 * Q4_K and 32256 for Q6_K (the GEMV stages four activation rows in one
 * workgroup's LDS), else RQ_ERR_SHAPE; the encoders are
 * quantize-weight-q4k / quantize-weight-q6k, quant.clj:92-137,214-239):
 *  Q4_K: wq u8[out*in/2] nibbles (w[k] low, w[k+16] high per 32-sub-block),
 *        da, db f32[out*in/256], aq u8[out*in/32] (0..63), bq i8[out*in/32];
 *  Q6_K: wq u8[out*in] (0..63: a larger byte fails with RQ_ERR_SHAPE; the
 *        device keeps the codes packed, 16 to 12 bytes), sc i8[out*in/16],
 *        ds f32[out*in/256].
 * They take q8_K activations (rq_quantize_act_q8k, rq_qmatmul_q8k); rq_dequant
 * gives dequant-q4k / dequant-q6k bit for bit. rq_qmatmul and
 * rq_qmatmul_noalloc take them with f32 x (quantized to q8_K inside the call);
 * rq_qmatmul_fused and rq_qmatmul_i8 reject them with RQ_ERR_DTYPE. */
int rq_weight_create_q4k(rq_ctx ctx, const uint8_t* wq, const float* da, const float* db, const uint8_t* aq,
                         const int8_t* bq, int64_t out, int64_t in, rq_weight* w);
int rq_weight_create_q6k(rq_ctx ctx, const uint8_t* wq, const int8_t* sc, const float* ds, int64_t out, int64_t in,
                         rq_weight* w);

/* q8_K activations on the device (quantize-act-q8k, quant.clj:158-176, the
 * GPU quant-act-q8k-gpu! of raster/quant/kernels_k.clj:93-134): per row of x
 * f32[m*in] (in % 256 == 0) and 256-element super-block, d = max|x| / 127 in
 * double, xq int8[m*in] = clamp(Math/round(x / d), -127, 127), xs f32[m*in/256]
 * = (float) d, bsums int32[m*in/sub] the sums of sub consecutive codes (sub =
 * 32 for Q4_K, 16 for Q6_K). Bitwise equal to the reference on finite input. */
int rq_quantize_act_q8k(rq_ctx ctx, const float* x, int64_t m, int64_t in, int sub, int8_t* xq, float* xs,
                        int32_t* bsums, void* stream);

/* y[m, out] = the K dot of a Q4_K / Q6_K weight with q8_K activations
 * (qmatmul-q4k-dp4a! / qmatmul-q6k-dp4a!, raster/quant/kernels_k.clj:186-297):
 * exact int32 sub-block dots, the scale terms added in f32 (Raster: double).
 * bsums must use the weight's sub-block size. Decode-oriented: four activation
 * rows per pass over the weights. xq 16-byte aligned. */
int rq_qmatmul_q8k(rq_ctx ctx, rq_weight w, const int8_t* xq, const float* xs, const int32_t* bsums, void* y,
                   int y_dtype, int64_t m, void* stream);

/* The raw int8 GEMV core, i8gemv-dp4a! (raster/quant/kernels_k.clj:141-150):
 * y[o] = (float) sum_w dp4a(wp[o*kw + w], xp[w]) for o < out, where wp is
 * int32[out*kw] and xp int32[kw], each word four little-endian signed int8
 * lanes (par/dp4a, raster/par.clj:421-440). The sum is exact (Raster: a
 * 64-bit long) and converted to f32 once, round to nearest even. Unscaled:
 * no block scales, no zero point. Device pointers, 4-byte aligned (wp and
 * xp may be NULL when kw is 0: y is then all zeros); y fully overwritten;
 * kw <= 2^20. */
int rq_i8gemv_dp4a(rq_ctx ctx, const int32_t* wp, const int32_t* xp, float* y, int64_t kw, int64_t out,
                   void* stream);

/* Raster's activation quantizer on the device (quantize-act-i8,
 * raster/compiler/backend/cpu/quant.clj:282-305,399-415): per row of x
 * f32[m*in] and 32-element block b, d = max|x| / 127 (in double), q =
 * clamp(Math/round(x / d), -127, 127) (ties toward +infinity, 0 when d == 0),
 * xq int8[m*in], xs f32[m*in/32] = (float) d, xsum int32[m*in/32] = sum q
 * (xsum may be NULL). Bitwise equal to the reference on finite input; its
 * int8 bytes are also the packed words of quant-act-i8-rows-gpu!
 * (raster/quant/kernels_k.clj:326-355). x 16-byte and xq 4-byte aligned. */
int rq_quantize_act_i8(rq_ctx ctx, const float* x, int64_t m, int64_t in, int8_t* xq, float* xs, int32_t* xsum,
                       void* stream);

/* y[m, out] = sum_b xs[m, b] * scale[o, b] * (dot_b(codes[o], xq[m]) [- 8 *
 * xsum[m, b] for Q4_0]) with int8 activations from rq_quantize_act_i8: the
 * integer block dots are exact, the block terms are summed in f32 (Raster sums
 * in double). Q4_0 needs xsum (qmatmul-q4-composable,
 * raster/quant/kernels.clj:140-184); Q8_0 ignores it (qmatmul-i8-gemm!,
 * raster/quant/kernels_k.clj:357-370). m <= 16 runs the decode kernel, larger
 * m an int8-MFMA GEMM. xq 16-byte aligned. */
int rq_qmatmul_i8(rq_ctx ctx, rq_weight w, const int8_t* xq, const float* xs, const int32_t* xsum, void* y,
                  int y_dtype, int64_t m, void* stream);

/* One decode step of RoPE, KV-cache append and single-query attention, the
 * glue between a decoder layer's q/k/v and o linears, all on the device:
 * rope-pos (raster/dl/attention.clj:197-214, NeoX half split, angle
 * pos * theta^(-2i/head_dim)) of q f32[n_q*head_dim] and of k
 * f32[n_kv*head_dim]; kv-append! (attention.clj:413-416) of the rotated k and
 * of v f32[n_kv*head_dim] into row pos of kcache / vcache (f32, rows of
 * n_kv*head_dim); gqa-decode-attention (attention.clj:248-287) of the rotated
 * query over rows 0..pos with the given scale: out f32[n_q*head_dim]. Query
 * head h reads KV head h / (n_q/n_kv). head_dim a multiple of 4 up to 512:
 * any cache length; other even head_dim: pos + 1 <= about 40K positions
 * (the scores sit in one workgroup's LDS). With head_dim a multiple of 4 and
 * pos >= 32 the cached rows are split over several workgroups per head, whose
 * partial softmax states are merged in a fixed order (results do not depend
 * on scheduling); that uses per-stream scratch of the context, allocated by
 * the first such call on the stream and grown by larger ones (as for the bf16
 * GEMM: a call being captured into a graph that would need to grow it fails
 * with RQ_ERR_SHAPE, so run it once on the stream before capturing). Calls
 * on one stream run in order; calls on different streams do not share it. */
int rq_decode_attention(rq_ctx ctx, const float* q, const float* k, const float* v, float* kcache, float* vcache,
                        int64_t pos, int64_t n_q, int64_t n_kv, int64_t head_dim, double theta, double scale,
                        float* out, void* stream);

/* Writes the dequantized f32 weight W[out*in] (device pointer): the exact f32
 * product scale * code (one IEEE rounding; Q4_0: scale * (q - 8)). The bf16
 * GEMMs feed the MFMA this same value rounded to bf16 (RNE); the exact-code
 * kernels (decode, f32-x GEMM, int8 paths) multiply the codes exactly and
 * apply the scale to the block's partial sum instead. Replaces dequant-q8-dense
 * (raster/quant/train.clj:60-71) and the Q4_0 dequant
 * (test/raster/compiler/backend/cpu/quant_encode_test.clj:9-24). */
int rq_dequant(rq_ctx ctx, rq_weight w, float* w_out, void* stream);

/* Host-array convenience with qlinear-q8's exact argument list
 * (raster/quant/train.clj:88-89): uploads, runs rq_qmatmul, downloads, syncs. */
int rq_qlinear_q8(rq_ctx ctx, const float* x, const int8_t* codes, const float* scales, int64_t m, int64_t in,
                  int64_t out, float* y);

/* Backward-data of the quantized linear, qlinear-q8-dx
 * (raster/quant/train.clj:110-137, the pullback of qlinear-q8,
 * train.clj:143-155): dx[m, in] = dy[m, out] . dequant(W), i.e. dx[m, i] =
 * sum_o scale[o, i/32] * code[o, i] * dy[m, o], each w = scale * code
 * rounded to f32 as Raster does. m <= 32 (f32 MFMA on the weight as stored,
 * read once per 16 dy rows): the products w * dy formed and summed in f32
 * (Raster: each rounded to f32, summed in double). m > 32 (a bf16 MFMA GEMM
 * that reads the weight once per 128 dy rows): w and dy each carried as bf16
 * hi + lo (relative 2^-16), the products hi*hi + hi*lo + lo*hi summed in f32,
 * each within about 3 * 2^-16 of the f32 product. Q8_0 or Q4_0 (code =
 * nibble - 8) weights; device f32 buffers, dx 16-byte aligned, fully
 * overwritten; results do not depend on scheduling. Splits the reduction over
 * `out` into slices whose partial sums, like the m > 32 path's packed dy, use
 * per-stream scratch (grown outside capture only, like rq_qmatmul). */
int rq_qmatmul_dx(rq_ctx ctx, rq_weight w, const float* dy, float* dx, int64_t m, void* stream);

/* qlinear-q8-dx with its own argument list (dy codes scales m in out) on host
 * arrays: uploads a temporary weight, runs rq_qmatmul_dx, downloads dx. */
int rq_qlinear_q8_dx(rq_ctx ctx, const float* dy, const int8_t* codes, const float* scales, int64_t m, int64_t in,
                     int64_t out, float* dx);

/* ---- ingestion helpers and the int8 linear op ------------------------------ */

/* nextpad (raster/quant/pack.clj:30-33): *inp = in rounded up to a multiple of
 * 256, the K-quant super-block. q4k-of (pack.clj:45-53) zero-pads each row of
 * W to that width before quantize-weight-q4k and reports it as the weight's
 * `in`, so its buffer set goes to rq_weight_create_q4k with in = *inp; the
 * caller zero-pads x to the same width, and the padded columns then add
 * nothing (their q8_K codes and sums are 0). Host-only, no device work. */
int rq_nextpad(int64_t in, int64_t* inp);

/* q8-quantize (raster/quant/train.clj:34-58) on the device: a row-major f32
 * W[out*in] (device, 16-byte aligned, in % 32 == 0) to signed Q8_0 codes
 * int8[out*in] and scales f32[out*in/32] (device, 4-byte aligned): per row and
 * 32-block d = max|w| / 127 in double, code = clamp(Math/round(w / d), -127,
 * 127) (0 when d == 0), scale = (float) d. Bitwise equal to the reference on
 * finite input; the outputs feed rq_weight_create_q8 after a download, or
 * stay on the device. Asynchronous on `stream`. */
int rq_q8_quantize(rq_ctx ctx, const float* W, int64_t out, int64_t in, int8_t* codes, float* scales,
                   void* stream);

/* q4k-of (raster/quant/pack.clj:45-53) on the device: W f32[out*in]
 * (row-major, device) with each row zero-padded to *inp = nextpad(in), then
 * quantize-weight-q4k (raster/compiler/backend/cpu/quant.clj:92-137) over the
 * out * *inp values. Outputs (device): wq u8[out*inp/2] (16-byte aligned; the
 * bytes q4k-of reads as little-endian int32 words), da, db f32[out*inp/256],
 * aq u8[out*inp/32], bq i8[out*inp/32] -- the arrays rq_weight_create_q4k
 * takes with in = *inp. With in % 256 == 0 this is quantize-weight-q4k of W.
 * The reference's double arithmetic step for step (only maxima cross lanes):
 * bitwise equal on finite input. Asynchronous on `stream`; *inp is set on
 * return. */
int rq_q4k_of(rq_ctx ctx, const float* W, int64_t out, int64_t in, uint8_t* wq, float* da, float* db, uint8_t* aq,
              int8_t* bq, int64_t* inp, void* stream);

/* quantize-weight-q6k (raster/compiler/backend/cpu/quant.clj:214-239) on the
 * device over a row-major W f32[out*in] (in % 256 == 0, 16-byte aligned):
 * wq u8[out*in] (16-byte aligned), sc i8[out*in/16], ds f32[out*in/256], the
 * arrays rq_weight_create_q6k takes. Bitwise equal on finite input. */
int rq_quantize_weight_q6k(rq_ctx ctx, const float* W, int64_t out, int64_t in, uint8_t* wq, int8_t* sc, float* ds,
                           void* stream);

/* qlinear-i8! / qlinear-i8-q8! (raster/quant/op.clj:43-51,81-90) with their
 * argument list (x wqi wsi y in out) on host arrays: x f32[in], the x8
 * repack-stream weight (wqi, wsi as for rq_weight_create_x8; nibble = 1 for
 * the Q4_0 op qlinear-i8!, 0 for the zero-point-128 Q8 op qlinear-i8-q8!), y
 * f32[out] fully overwritten (:overwrite 3, op.clj:75-79). x is quantized
 * inside the kernel by quantize-act-i8's math (as quantize-act-i8-par,
 * cpu/quant.clj:399-415) and the exact int8 block dots are scaled and summed
 * in f32, which is the reference's numerics (qmatmul-q4-x8! / qmatmul-q8-x8!,
 * raster/quant/kernels.clj:216-247,308-333, sum their f32 lanes in another
 * order). Uploads a temporary weight per call and syncs; callers that call
 * again with the same weight keep it resident instead (rq_weight_create_x8
 * once, then rq_qmatmul_fused with act_i8 = 1 per call). */
int rq_qlinear_i8(rq_ctx ctx, const float* x, const uint8_t* wqi, const float* wsi, int nibble, float* y,
                  int64_t in, int64_t out);

/* Dense f32 GEMM, the float arms of raster/linalg/blas.clj (Raster's CPU
 * path hands them to cblas_sgemm of MKL / OpenBLAS), on device arrays,
 * row-major, asynchronous on `stream`; a plain library GEMM, so rocBLAS
 * computes it (f32 products and accumulation, deterministic). As in the
 * reference, a call with m, n or k not positive does nothing.
 *   rq_sgemm     C[m*n] = alpha A[m*k] B[k*n] + beta C     dgemm!    blas.clj:287-302
 *   rq_sgemm_tn  C[m*n] = alpha A^T B + beta C, A [k*m]     dgemm-tn! blas.clj:304-319
 *   rq_sgemm_nt  C[m*n] = alpha A B^T + beta C, B [n*k]     dgemm-nt! blas.clj:321-337
 * The first call on a context creates its library handle (device memory)
 * and fails under HIP graph capture; later calls are not meant for capture
 * either (the library may allocate or record memory operations there). */
int rq_sgemm(rq_ctx ctx, const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n, float alpha,
             float beta, void* stream);
int rq_sgemm_tn(rq_ctx ctx, const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n, float alpha,
                float beta, void* stream);
int rq_sgemm_nt(rq_ctx ctx, const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n, float alpha,
                float beta, void* stream);

/* linear! (raster/dl/nn.clj:161-183): y[batch*out_f] = x[batch*in_f]
 * W[out_f*in_f]^T + b[out_f], device arrays, as the reference computes it:
 * every row of y set to b, then rq_sgemm_nt with alpha = beta = 1. batch or
 * out_f not positive: nothing; in_f not positive: y = b in every row. */
int rq_linear(rq_ctx ctx, const float* x, const float* w, const float* b, float* y, int64_t batch, int64_t in_f,
              int64_t out_f, void* stream);

#ifdef __cplusplus
}
#endif
#endif
