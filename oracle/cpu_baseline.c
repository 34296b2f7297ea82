/*
 * cpu_baseline.c — timed CPU baseline for bench.py (TEST INFRASTRUCTURE ONLY).
 *
 * Two of Raster's CPU routes for the quantized matmul, restated in C and driven
 * by a pthread pool over disjoint output slices (the role of the spin-pool in
 * raster/compiler/backend/cpu/quant.clj:328-397):
 *
 *  B1  qlinear-q8 loop (raster/quant/train.clj:77-108): f32 scale*code*x
 *      products, f64 accumulation, f32 store. Compiled the way Raster compiles
 *      its CPU-C (-O3 -funroll-loops -ffast-math, cpu/codegen.clj:68-74).
 *  B2  the x8 dpbusd stream GEMV (quantize-act-i8 + qmatmul-q8-x8!,
 *      raster/quant/kernels.clj:258-333 with the C helper at :282-302):
 *      int8 activations, 8 column dots per vpdpbusd tile, f32 8-lane fold;
 *      and its Q4_0 form (qmatmul-q4-x8!, kernels.clj:216-247 with the C
 *      helper wi8-dot-q4-x8 at :116-138): nibbles unpacked to bytes, the same
 *      tile and fold with zero point 8.
 *
 * -march=native is NOT used: the library is built here and run on the GPU
 * box's host CPU, so the AVX-512-VNNI tile is compiled per function with a
 * target attribute and selected at run time (AVX2 maddubs otherwise).
 */
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef void (*slice_fn)(void* ctx, int64_t lo, int64_t hi);

/* A persistent pool of spinning workers released by a generation counter, as
 * Raster's spin-pool (raster/compiler/backend/cpu/quant.clj:339-388): a call
 * publishes one task, bumps the generation, runs slice 0 itself and spins
 * until every worker has reported. The pool is rebuilt when the thread count
 * changes; one dispatcher at a time (the caller serializes calls). */
#define RQB_MAX_THREADS 256
typedef struct {
  pthread_t th[RQB_MAX_THREADS];
  int nthreads;
  slice_fn fn;
  void* ctx;
  int64_t n;
  volatile int generation;
  volatile int done;
  volatile int stop;
  int start_generation; /* the generation workers created by pool_resize have seen */
} pool_t;

static pool_t g_pool;

static void pool_slice(int wid) {
  const int64_t chunk = (g_pool.n + g_pool.nthreads - 1) / g_pool.nthreads;
  const int64_t lo = (int64_t)wid * chunk;
  const int64_t hi = lo + chunk < g_pool.n ? lo + chunk : g_pool.n;
  if (lo < hi) g_pool.fn(g_pool.ctx, lo, hi);
}

static void* pool_worker(void* p) {
  const int wid = (int)(intptr_t)p;
  /* the generation at creation, not at thread start: a dispatch published
   * before this thread runs must still be taken */
  int seen = g_pool.start_generation;
  for (;;) {
    int g;
    while ((g = __atomic_load_n(&g_pool.generation, __ATOMIC_ACQUIRE)) == seen) {
      if (__atomic_load_n(&g_pool.stop, __ATOMIC_ACQUIRE)) return 0;
      __builtin_ia32_pause();
    }
    seen = g;
    pool_slice(wid);
    __atomic_add_fetch(&g_pool.done, 1, __ATOMIC_ACQ_REL);
  }
}

static void pool_resize(int nthreads) {
  if (g_pool.nthreads > 1) {
    __atomic_store_n(&g_pool.stop, 1, __ATOMIC_RELEASE);
    for (int w = 1; w < g_pool.nthreads; w++) pthread_join(g_pool.th[w], 0);
    __atomic_store_n(&g_pool.stop, 0, __ATOMIC_RELEASE);
  }
  g_pool.nthreads = nthreads;
  g_pool.start_generation = __atomic_load_n(&g_pool.generation, __ATOMIC_ACQUIRE);
  for (int w = 1; w < nthreads; w++) pthread_create(&g_pool.th[w], 0, pool_worker, (void*)(intptr_t)w);
}

static void run_pool(slice_fn fn, void* ctx, int64_t n, int nthreads) {
  if (nthreads > RQB_MAX_THREADS) nthreads = RQB_MAX_THREADS;
  if (nthreads <= 1) {
    fn(ctx, 0, n);
    return;
  }
  if (g_pool.nthreads != nthreads) pool_resize(nthreads);
  g_pool.fn = fn;
  g_pool.ctx = ctx;
  g_pool.n = n;
  __atomic_store_n(&g_pool.done, 0, __ATOMIC_RELEASE);
  __atomic_add_fetch(&g_pool.generation, 1, __ATOMIC_ACQ_REL);
  pool_slice(0);
  while (__atomic_load_n(&g_pool.done, __ATOMIC_ACQUIRE) != nthreads - 1) __builtin_ia32_pause();
}

/* Stops and joins the pool's workers (bench.py calls it after its legs). */
void rqb_pool_shutdown(void) {
  if (g_pool.nthreads > 1) pool_resize(1);
  g_pool.nthreads = 0;
}

/* ---------------- B1: qlinear-q8 loop ---------------- */
typedef struct {
  const float* x;
  const int8_t* codes;
  const float* scales;
  int64_t m, in, out;
  float* y;
} b1_ctx;

static void b1_slice(void* p, int64_t lo, int64_t hi) {
  b1_ctx* c = (b1_ctx*)p;
  int64_t nb = c->in / 32;
  for (int64_t o = lo; o < hi; o++) {
    const int8_t* wr = c->codes + o * c->in;
    const float* sr = c->scales + o * nb;
    for (int64_t mi = 0; mi < c->m; mi++) {
      const float* xr = c->x + mi * c->in;
      double acc = 0.0;
      for (int64_t i = 0; i < c->in; i++) acc += (double)((sr[i / 32] * (float)wr[i]) * xr[i]);
      c->y[mi * c->out + o] = (float)acc;
    }
  }
}

void rqb_qlinear_q8(const float* x, const int8_t* codes, const float* scales, int64_t m, int64_t in,
                    int64_t out, float* y, int nthreads) {
  b1_ctx c = {x, codes, scales, m, in, out, y};
  run_pool(b1_slice, &c, out, nthreads);
}

/* ---------------- B2: x8 dpbusd stream GEMV ---------------- */
typedef struct {
  const float* x;
  int8_t* xq;
  float* xs;
  int32_t* xsum;
} act_ctx;

static void act_slice(void* p, int64_t lo, int64_t hi) {
  act_ctx* c = (act_ctx*)p;
  for (int64_t r = lo; r < hi; r++) {
    const float* xb = c->x + r * 32;
    float a = 0.0f;
    for (int j = 0; j < 32; j++) a = fmaxf(a, fabsf(xb[j]));
    double d = (double)a / 127.0;
    double id = d == 0.0 ? 0.0 : 1.0 / d;
    c->xs[r] = (float)d;
    int32_t s = 0;
    for (int k = 0; k < 32; k++) {
      double v = floor((double)xb[k] * id + 0.5);
      int32_t q = (int32_t)(v > 127 ? 127 : v < -127 ? -127 : v);
      c->xq[r * 32 + k] = (int8_t)q;
      s += q;
    }
    c->xsum[r] = s;
  }
}

void rqb_quantize_act_i8(const float* x, int64_t M, int64_t in, int8_t* xq, float* xs, int32_t* xsum,
                         int nthreads) {
  act_ctx c = {x, xq, xs, xsum};
  run_pool(act_slice, &c, M * (in / 32), nthreads);
}

typedef struct {
  const int8_t* xq;
  const float* xs;
  const int32_t* xsum;
  const uint8_t* wqi;
  const float* wsi;
  float* y;
  int64_t in;
} x8_ctx;

__attribute__((target("avx2,fma"))) static inline __m256i tile_q8_avx2(const uint8_t* wb, const int8_t* xb) {
  __m256i ia = _mm256_setzero_si256();
  const __m256i ones = _mm256_set1_epi16(1);
  for (int ig = 0; ig < 8; ig++) {
    __m256i wv = _mm256_loadu_si256((const __m256i*)(wb + ig * 32));
    int32_t a4;
    memcpy(&a4, xb + ig * 4, 4);
    __m256i ab = _mm256_set1_epi32(a4);
    ia = _mm256_add_epi32(ia, _mm256_madd_epi16(_mm256_maddubs_epi16(wv, ab), ones));
  }
  return ia;
}

__attribute__((target("avx2,fma,avx512f,avx512vl,avx512vnni"))) static inline __m256i tile_q8_vnni(
    const uint8_t* wb, const int8_t* xb) {
  __m256i ia = _mm256_setzero_si256();
  for (int ig = 0; ig < 8; ig++) {
    __m256i wv = _mm256_loadu_si256((const __m256i*)(wb + ig * 32));
    int32_t a4;
    memcpy(&a4, xb + ig * 4, 4);
    ia = _mm256_dpbusd_epi32(ia, wv, _mm256_set1_epi32(a4));
  }
  return ia;
}

#define X8_BODY(TILE)                                                                 \
  x8_ctx* c = (x8_ctx*)p;                                                             \
  int64_t nb = c->in / 32;                                                            \
  for (int64_t g = lo; g < hi; g++) {                                                 \
    const uint8_t* wg = c->wqi + g * nb * 256;                                        \
    const float* sg = c->wsi + g * nb * 8;                                            \
    __m256 acc = _mm256_setzero_ps();                                                 \
    for (int64_t b = 0; b < nb; b++) {                                                \
      __m256i dots = TILE(wg + b * 256, c->xq + b * 32);                              \
      __m256i folded = _mm256_sub_epi32(dots, _mm256_set1_epi32(128 * c->xsum[b]));   \
      __m256 scale = _mm256_mul_ps(_mm256_set1_ps(c->xs[b]), _mm256_loadu_ps(sg + b * 8)); \
      acc = _mm256_fmadd_ps(scale, _mm256_cvtepi32_ps(folded), acc);                  \
    }                                                                                 \
    _mm256_storeu_ps(c->y + g * 8, acc);                                              \
  }

__attribute__((target("avx2,fma"))) static void x8_slice_avx2(void* p, int64_t lo, int64_t hi) {
  X8_BODY(tile_q8_avx2)
}
__attribute__((target("avx2,fma,avx512f,avx512vl,avx512vnni"))) static void x8_slice_vnni(void* p, int64_t lo,
                                                                                         int64_t hi) {
  X8_BODY(tile_q8_vnni)
}

/* Q4_0 tile: the 16 bytes of input group ig hold column j/4's element
 * ig*4 + j%4 in the low nibble of byte j and column 4 + j/4's in the high
 * nibble; low nibbles go to the low 128-bit lane, high nibbles to the high. */
__attribute__((target("avx2,fma"))) static inline __m256i tile_q4_avx2(const uint8_t* wb, const int8_t* xb) {
  __m256i ia = _mm256_setzero_si256();
  const __m256i ones = _mm256_set1_epi16(1), m4 = _mm256_set1_epi8(0x0F);
  for (int ig = 0; ig < 8; ig++) {
    __m128i raw = _mm_loadu_si128((const __m128i*)(wb + ig * 16));
    __m256i nib = _mm256_and_si256(_mm256_set_m128i(_mm_srli_epi16(raw, 4), raw), m4);
    int32_t a4;
    memcpy(&a4, xb + ig * 4, 4);
    ia = _mm256_add_epi32(ia, _mm256_madd_epi16(_mm256_maddubs_epi16(nib, _mm256_set1_epi32(a4)), ones));
  }
  return ia;
}

__attribute__((target("avx2,fma,avx512f,avx512vl,avx512vnni"))) static inline __m256i tile_q4_vnni(
    const uint8_t* wb, const int8_t* xb) {
  __m256i ia = _mm256_setzero_si256();
  const __m256i m4 = _mm256_set1_epi8(0x0F);
  for (int ig = 0; ig < 8; ig++) {
    __m128i raw = _mm_loadu_si128((const __m128i*)(wb + ig * 16));
    __m256i nib = _mm256_and_si256(_mm256_set_m128i(_mm_srli_epi16(raw, 4), raw), m4);
    int32_t a4;
    memcpy(&a4, xb + ig * 4, 4);
    ia = _mm256_dpbusd_epi32(ia, nib, _mm256_set1_epi32(a4));
  }
  return ia;
}

#define X8Q4_BODY(TILE)                                                               \
  x8_ctx* c = (x8_ctx*)p;                                                             \
  int64_t nb = c->in / 32;                                                            \
  for (int64_t g = lo; g < hi; g++) {                                                 \
    const uint8_t* wg = c->wqi + g * nb * 128;                                        \
    const float* sg = c->wsi + g * nb * 8;                                            \
    __m256 acc = _mm256_setzero_ps();                                                 \
    for (int64_t b = 0; b < nb; b++) {                                                \
      __m256i dots = TILE(wg + b * 128, c->xq + b * 32);                              \
      __m256i folded = _mm256_sub_epi32(dots, _mm256_set1_epi32(8 * c->xsum[b]));     \
      __m256 scale = _mm256_mul_ps(_mm256_set1_ps(c->xs[b]), _mm256_loadu_ps(sg + b * 8)); \
      acc = _mm256_fmadd_ps(scale, _mm256_cvtepi32_ps(folded), acc);                  \
    }                                                                                 \
    _mm256_storeu_ps(c->y + g * 8, acc);                                              \
  }

__attribute__((target("avx2,fma"))) static void x8q4_slice_avx2(void* p, int64_t lo, int64_t hi) {
  X8Q4_BODY(tile_q4_avx2)
}
__attribute__((target("avx2,fma,avx512f,avx512vl,avx512vnni"))) static void x8q4_slice_vnni(void* p, int64_t lo,
                                                                                           int64_t hi) {
  X8Q4_BODY(tile_q4_vnni)
}

int rqb_have_vnni(void) {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512vl") ? 1 : 0;
}

/* One M=1 qlinear-i8-q8! call on the x8 byte-direct layout (zero-point 128). */
void rqb_qmatmul_q8_x8(const int8_t* xq, const float* xs, const int32_t* xsum, const uint8_t* wqi,
                       const float* wsi, float* y, int64_t in, int64_t out, int nthreads) {
  x8_ctx c = {xq, xs, xsum, wqi, wsi, y, in};
  run_pool(rqb_have_vnni() ? x8_slice_vnni : x8_slice_avx2, &c, out / 8, nthreads);
}

/* One M=1 qlinear-i8! call on the x8 nibble layout (Q4_0, zero-point 8). */
void rqb_qmatmul_q4_x8(const int8_t* xq, const float* xs, const int32_t* xsum, const uint8_t* wqi,
                       const float* wsi, float* y, int64_t in, int64_t out, int nthreads) {
  x8_ctx c = {xq, xs, xsum, wqi, wsi, y, in};
  run_pool(rqb_have_vnni() ? x8q4_slice_vnni : x8q4_slice_avx2, &c, out / 8, nthreads);
}
