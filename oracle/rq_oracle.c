/*
 * rq_oracle.c — CPU restatement of Raster's block-quantized matmul path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker the HIP kernels are compared against.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Reference citations are paths inside replikativ/raster. Each function keeps
 * the reference's loop order and rounding points (JVM semantics: float operands
 * widen to double in Clojure arithmetic, Math/round = ties toward +infinity,
 * (float d) = one RNE narrowing). Compile with -ffp-contract=off.
 */
#include "rq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* java.util.Random                                                           */
/* ------------------------------------------------------------------------- */
#define JR_MULT 0x5DEECE66DLL
#define JR_ADD 0xBLL
#define JR_MASK ((1LL << 48) - 1)

void rqo_jrandom_init(rqo_jrandom* r, int64_t seed) {
  r->seed = (seed ^ JR_MULT) & JR_MASK;
  r->have_next_next_gaussian = 0;
  r->next_next_gaussian = 0.0;
}

int32_t rqo_jrandom_next(rqo_jrandom* r, int bits) {
  r->seed = (int64_t)(((uint64_t)r->seed * (uint64_t)JR_MULT + (uint64_t)JR_ADD) & (uint64_t)JR_MASK);
  return (int32_t)((uint64_t)r->seed >> (48 - bits));
}

int32_t rqo_jrandom_next_int(rqo_jrandom* r) { return rqo_jrandom_next(r, 32); }

double rqo_jrandom_next_double(rqo_jrandom* r) {
  int64_t hi = (int64_t)rqo_jrandom_next(r, 26);
  int64_t lo = (int64_t)rqo_jrandom_next(r, 27);
  return (double)((hi << 27) + lo) * 0x1.0p-53;
}

double rqo_jrandom_next_gaussian(rqo_jrandom* r) {
  if (r->have_next_next_gaussian) {
    r->have_next_next_gaussian = 0;
    return r->next_next_gaussian;
  }
  double v1, v2, s;
  do {
    v1 = 2 * rqo_jrandom_next_double(r) - 1;
    v2 = 2 * rqo_jrandom_next_double(r) - 1;
    s = v1 * v1 + v2 * v2;
  } while (s >= 1 || s == 0);
  double multiplier = sqrt(-2 * log(s) / s);
  r->next_next_gaussian = v2 * multiplier;
  r->have_next_next_gaussian = 1;
  return v1 * multiplier;
}

void rqo_jrandom_next_bytes(rqo_jrandom* r, int8_t* out, int64_t n) {
  int64_t i = 0;
  while (i < n) {
    int32_t rnd = rqo_jrandom_next_int(r);
    int64_t k = n - i < 4 ? n - i : 4;
    while (k-- > 0) {
      out[i++] = (int8_t)rnd;
      rnd >>= 8;
    }
  }
}

/* train_test.clj:14-16: (float (* mult (.nextGaussian r))) */
void rqo_jfill_gauss(int64_t seed, double mult, float* out, int64_t n) {
  rqo_jrandom r;
  rqo_jrandom_init(&r, seed);
  for (int64_t i = 0; i < n; i++) out[i] = (float)(mult * rqo_jrandom_next_gaussian(&r));
}

/* pack_test.clj:9-12: (float (- (.nextDouble r) 0.5)) */
void rqo_jfill_uniform_centered(int64_t seed, float* out, int64_t n) {
  rqo_jrandom r;
  rqo_jrandom_init(&r, seed);
  for (int64_t i = 0; i < n; i++) out[i] = (float)(rqo_jrandom_next_double(&r) - 0.5);
}

/* tile_test.clj:10-11: (.nextBytes (java.util.Random. seed) a) */
void rqo_jfill_bytes(int64_t seed, int8_t* out, int64_t n) {
  rqo_jrandom r;
  rqo_jrandom_init(&r, seed);
  rqo_jrandom_next_bytes(&r, out, n);
}

int64_t rqo_java_round(double x) {
  if (isnan(x)) return 0;
  if (x >= 9.2233720368547758e18) return INT64_MAX;
  if (x <= -9.2233720368547758e18) return INT64_MIN;
  double f = floor(x);
  double diff = x - f; /* exact: f and x share the binade or x is integral */
  int64_t r = (int64_t)f;
  return diff >= 0.5 ? r + 1 : r;
}

/* ------------------------------------------------------------------------- */
/* scalar conversions                                                         */
/* ------------------------------------------------------------------------- */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float rqo_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1F;
  uint32_t man = h & 0x3FF;
  if (exp == 0) {
    if (man == 0) return u2f(sign);
    /* subnormal: man * 2^-24, exact in f32 */
    float v = (float)man * 0x1.0p-24f;
    return sign ? -v : v;
  }
  if (exp == 31) return u2f(sign | 0x7F800000u | (man << 13));
  return u2f(sign | ((exp + 112) << 23) | (man << 13));
}

uint16_t rqo_f32_to_f16(float f) {
  uint32_t u = f2u(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
  uint32_t absu = u & 0x7FFFFFFFu;
  if (absu >= 0x7F800000u) /* inf / nan */
    return sign | 0x7C00 | (absu > 0x7F800000u ? 0x200 | ((absu >> 13) & 0x3FF) : 0);
  if (absu >= 0x477FF000u) return sign | 0x7C00; /* rounds to >= 65520 -> inf */
  if (absu < 0x38800000u) {                       /* below f16 min normal 2^-14 */
    /* subnormal f16: value / 2^-24 rounded to nearest even */
    float a = u2f(absu);
    double q = (double)a * 16777216.0; /* exact */
    double fl = floor(q);
    double diff = q - fl;
    uint32_t m = (uint32_t)fl;
    if (diff > 0.5 || (diff == 0.5 && (m & 1))) m++;
    return sign | (uint16_t)m; /* m == 0x400 becomes the min normal, still right */
  }
  uint32_t exp = ((absu >> 23) - 112);
  uint32_t man = absu & 0x7FFFFF;
  uint32_t h = (exp << 10) | (man >> 13);
  uint32_t rest = man & 0x1FFF;
  if (rest > 0x1000 || (rest == 0x1000 && (h & 1))) h++;
  return sign | (uint16_t)h;
}

float rqo_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

uint16_t rqo_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40);
  uint32_t lsb = (u >> 16) & 1;
  u += 0x7FFF + lsb;
  return (uint16_t)(u >> 16);
}

/* ------------------------------------------------------------------------- */
/* int8 MAC seam                                                              */
/* ------------------------------------------------------------------------- */
static inline int64_t sx8(uint32_t x, int sh) {
  int64_t v = (x >> sh) & 0xFF;
  return v >= 128 ? v - 256 : v;
}

int64_t rqo_dp4a(int32_t a, int32_t b, int64_t acc) {
  uint32_t ua = (uint32_t)a, ub = (uint32_t)b;
  return acc + sx8(ua, 0) * sx8(ub, 0) + sx8(ua, 8) * sx8(ub, 8) + sx8(ua, 16) * sx8(ub, 16) +
         sx8(ua, 24) * sx8(ub, 24);
}

int64_t rqo_wi8_dot_q4(const uint8_t* wq, int64_t woff, const int8_t* xq, int64_t xoff) {
  int64_t s = 0;
  for (int k = 0; k < 16; k++) {
    int64_t bv = wq[woff + k];
    s += (int64_t)xq[xoff + k] * (bv & 0xF) + (int64_t)xq[xoff + k + 16] * (bv >> 4);
  }
  return s;
}

int64_t rqo_wi8_dot(const uint8_t* wq, int64_t woff, const int8_t* xq, int64_t xoff, int64_t len) {
  int64_t s = 0;
  for (int64_t k = 0; k < len; k++) s += (int64_t)wq[woff + k] * (int64_t)xq[xoff + k];
  return s;
}

/* ------------------------------------------------------------------------- */
/* Q8_0 row-major                                                             */
/* ------------------------------------------------------------------------- */
int rqo_q8_quantize(const float* W, int64_t out, int64_t in, int8_t* codes, float* scales) {
  if (in % 32 != 0) return -1;
  int64_t nb = in / 32;
  for (int64_t o = 0; o < out; o++) {
    for (int64_t b = 0; b < nb; b++) {
      int64_t base = o * in + b * 32;
      double mm = 0.0;
      for (int k = 0; k < 32; k++) {
        double a = fabs((double)W[base + k]);
        if (a > mm) mm = a;
      }
      double d = mm / 127.0;
      double id = d > 0 ? 1.0 / d : 0.0;
      scales[o * nb + b] = (float)d;
      for (int k = 0; k < 32; k++) {
        int64_t q = rqo_java_round((double)W[base + k] * id);
        if (q > 127) q = 127;
        if (q < -127) q = -127;
        codes[base + k] = (int8_t)q;
      }
    }
  }
  return 0;
}

void rqo_dequant_q8_dense(const int8_t* codes, const float* scales, int64_t in, int64_t out, float* W) {
  int64_t nb = in / 32;
  for (int64_t o = 0; o < out; o++)
    for (int64_t i = 0; i < in; i++)
      W[o * in + i] = (float)((double)scales[o * nb + i / 32] * (double)codes[o * in + i]);
}

void rqo_qlinear_q8(const float* x, const int8_t* codes, const float* scales, int64_t m, int64_t in,
                    int64_t out, float* y) {
  int64_t nb = in / 32;
  for (int64_t p = 0; p < m * out; p++) {
    int64_t mi = p / out, o = p % out;
    const float* xr = x + mi * in;
    const int8_t* wr = codes + o * in;
    const float* sr = scales + o * nb;
    double acc = 0.0;
    for (int64_t i = 0; i < in; i++) {
      float w = sr[i / 32] * (float)wr[i]; /* f32 multiply */
      float t = w * xr[i];                 /* f32 multiply */
      acc += (double)t;
    }
    y[p] = (float)acc;
  }
}

void rqo_qlinear_q8_dx(const float* dy, const int8_t* codes, const float* scales, int64_t m,
                       int64_t in, int64_t out, float* dx) {
  int64_t nb = in / 32;
  for (int64_t p = 0; p < m * in; p++) {
    int64_t mi = p / in, i = p % in;
    double acc = 0.0;
    for (int64_t o = 0; o < out; o++) {
      float w = scales[o * nb + i / 32] * (float)codes[o * in + i];
      float t = w * dy[mi * out + o];
      acc += (double)t;
    }
    dx[p] = (float)acc;
  }
}

/* ------------------------------------------------------------------------- */
/* parametric quantizer (Q4_0 / unsigned Q8_0)                               */
/* ------------------------------------------------------------------------- */
void rqo_quantize_weight(const float* w, int64_t len, int weight_bits, int zero_point, int nibble,
                         uint8_t* wq, float* ws) {
  const int64_t blk = 32, half = 16, nb = len / blk;
  const int64_t zp = zero_point, qmax = (1LL << weight_bits) - 1;
  for (int64_t b = 0; b < nb; b++) {
    int64_t base = b * blk;
    /* the element of largest |x| (first one on ties), cpu/quant.clj:55-59 */
    double a = 0.0, v = 0.0;
    for (int64_t j = 0; j < blk; j++) {
      float x = w[base + j];
      float ax = fabsf(x);
      if ((double)ax > a) { a = ax; v = x; }
    }
    double d = v / (double)(-zp);
    double id = d == 0.0 ? 0.0 : 1.0 / d;
    ws[b] = (float)d;
#define RQO_Q(xv)                                                   \
  ({                                                                \
    int64_t q_ = rqo_java_round((double)(xv) * id) + zp;           \
    q_ = q_ > qmax ? qmax : q_;                                     \
    q_ < 0 ? 0 : q_;                                                \
  })
    if (nibble) {
      for (int64_t k = 0; k < half; k++)
        wq[b * half + k] = (uint8_t)(RQO_Q(w[base + k]) | (RQO_Q(w[base + k + half]) << 4));
    } else {
      for (int64_t k = 0; k < blk; k++) wq[base + k] = (uint8_t)RQO_Q(w[base + k]);
    }
#undef RQO_Q
  }
}

void rqo_dequant_weight(const uint8_t* wq, const float* ws, int64_t len, int zero_point, int nibble,
                        float* out) {
  const int64_t blk = 32, half = 16, zp = zero_point;
  for (int64_t b = 0; b < len / blk; b++) {
    double d = ws[b];
    int64_t base = b * blk;
    if (nibble) {
      for (int64_t k = 0; k < half; k++) {
        int64_t bv = wq[b * half + k];
        out[base + k] = (float)(d * (double)((bv & 0xF) - zp));
        out[base + k + half] = (float)(d * (double)((bv >> 4) - zp));
      }
    } else {
      for (int64_t k = 0; k < blk; k++) out[base + k] = (float)(d * (double)((int64_t)wq[base + k] - zp));
    }
  }
}

static void dequant_q4_rows(const uint8_t* wq, const uint16_t* ws_f16, const float* ws_f32, int64_t in,
                            int64_t out, float* W) {
  int64_t nb = in / 32, half = in / 2;
  for (int64_t o = 0; o < out; o++)
    for (int64_t b = 0; b < nb; b++) {
      double d = ws_f16 ? (double)rqo_f16_to_f32(ws_f16[o * nb + b]) : (double)ws_f32[o * nb + b];
      for (int k = 0; k < 16; k++) {
        int64_t bv = wq[o * half + b * 16 + k];
        W[o * in + b * 32 + k] = (float)(d * (double)((bv & 0xF) - 8));
        W[o * in + b * 32 + k + 16] = (float)(d * (double)((bv >> 4) - 8));
      }
    }
}

void rqo_dequant_q4_f16(const uint8_t* wq, const uint16_t* ws_f16, int64_t in, int64_t out, float* W) {
  dequant_q4_rows(wq, ws_f16, 0, in, out, W);
}

void rqo_dequant_q4_f32(const uint8_t* wq, const float* ws, int64_t in, int64_t out, float* W) {
  dequant_q4_rows(wq, 0, ws, in, out, W);
}

void rqo_qlinear_q4(const float* x, const uint8_t* wq, const uint16_t* ws_f16, const float* ws_f32,
                    int64_t m, int64_t in, int64_t out, float* y) {
  int64_t nb = in / 32, half = in / 2;
  for (int64_t p = 0; p < m * out; p++) {
    int64_t mi = p / out, o = p % out;
    const float* xr = x + mi * in;
    double acc = 0.0;
    for (int64_t i = 0; i < in; i++) {
      int64_t b = i / 32, e = i % 32;
      float d = ws_f16 ? rqo_f16_to_f32(ws_f16[o * nb + b]) : ws_f32[o * nb + b];
      int64_t bv = wq[o * half + b * 16 + (e < 16 ? e : e - 16)];
      int64_t q = e < 16 ? (bv & 0xF) : (bv >> 4);
      float w = d * (float)(q - 8);
      float t = w * xr[i];
      acc += (double)t;
    }
    y[p] = (float)acc;
  }
}

/* ------------------------------------------------------------------------- */
/* activation quantizer + int-activation GEMVs                               */
/* ------------------------------------------------------------------------- */
void rqo_quantize_act_i8(const float* x, int64_t M, int64_t in, int8_t* xq, float* xs, int32_t* xsum) {
  int64_t nblk = M * (in / 32);
  for (int64_t r = 0; r < nblk; r++) {
    int64_t base = r * 32;
    double a = 0.0;
    for (int j = 0; j < 32; j++) {
      double ax = fabsf(x[base + j]);
      if (ax > a) a = ax;
    }
    double d = a / 127.0;
    double id = d == 0.0 ? 0.0 : 1.0 / d;
    xs[r] = (float)d;
    int64_t s = 0;
    for (int k = 0; k < 32; k++) {
      int64_t q = rqo_java_round((double)x[base + k] * id);
      if (q > 127) q = 127;
      if (q < -127) q = -127;
      xq[base + k] = (int8_t)q;
      s += q;
    }
    xsum[r] = (int32_t)s;
  }
}

void rqo_qmatmul_q4_composable(const int8_t* xq, const float* xs, const int32_t* xsum,
                               const uint8_t* wq, const float* ws, float* y, int64_t in, int64_t out,
                               int64_t o_start, int64_t o_count) {
  (void)out;
  int64_t nb = in / 32, half = in / 2;
  for (int64_t oi = 0; oi < o_count; oi++) {
    int64_t o = o_start + oi;
    double a = 0.0;
    for (int64_t b = 0; b < nb; b++) {
      int64_t dot = rqo_wi8_dot_q4(wq, o * half + b * 16, xq, b * 32);
      int64_t folded = dot - 8 * (int64_t)xsum[b];
      double scale = (double)xs[b] * (double)ws[o * nb + b];
      a += scale * (double)folded;
    }
    y[o] = (float)a;
  }
}

/* ------------------------------------------------------------------------- */
/* x8 column-interleaved layout                                               */
/* ------------------------------------------------------------------------- */
int rqo_repack_x8(const uint8_t* wq, const float* ws, int64_t out, int64_t in, int nibble, uint8_t* wqi,
                  float* wsi) {
  const int64_t tile = 8, kgroup = 4, half = 4, igroups = 8;
  const int64_t bpi = nibble ? half * kgroup : tile * kgroup;
  if (out % tile != 0 || in % 32 != 0) return -1;
  int64_t nb = in / 32, ng = out / tile, halfw = in / 2;
  for (int64_t gi = 0; gi < ng; gi++) {
    for (int64_t b = 0; b < nb; b++) {
      for (int64_t ig = 0; ig < igroups; ig++) {
        for (int64_t j = 0; j < bpi; j++) {
          int64_t idx = gi * nb * bpi * igroups + b * bpi * igroups + ig * bpi + j;
          int64_t e = ig * kgroup + j % kgroup;
          if (!nibble) {
            int64_t row = gi * tile + j / kgroup;
            wqi[idx] = wq[row * in + b * 32 + e];
          } else {
            int64_t base = gi * tile + j / kgroup;
#define SRC_NIB(row)                                                                   \
  ({                                                                                   \
    int64_t bv_ = wq[(row) * halfw + b * 16 + (e < 16 ? e : e - 16)];                 \
    e < 16 ? (bv_ & 0xF) : (bv_ >> 4);                                                 \
  })
            int64_t nlo = SRC_NIB(base);
            int64_t nhi = SRC_NIB(base + half);
#undef SRC_NIB
            wqi[idx] = (uint8_t)(nlo | (nhi << 4));
          }
        }
      }
      for (int64_t r = 0; r < tile; r++) wsi[gi * nb * tile + b * tile + r] = ws[(gi * tile + r) * nb + b];
    }
  }
  return 0;
}

void rqo_wi8_dot_q4_x8(const uint8_t* wqi, int64_t woff, const int8_t* xq, int64_t xoff, int32_t* out8) {
  for (int L = 0; L < 8; L++) {
    int64_t acc = 0;
    for (int ig = 0; ig < 8; ig++)
      for (int k = 0; k < 4; k++) {
        int nib_idx = L * 4 + k;
        int64_t bidx = woff + ig * 16 + (nib_idx < 16 ? nib_idx : nib_idx - 16);
        int64_t bv = wqi[bidx];
        int64_t nib = nib_idx < 16 ? (bv & 0xF) : (bv >> 4);
        acc += (int64_t)xq[xoff + ig * 4 + k] * nib;
      }
    out8[L] = (int32_t)acc;
  }
}

void rqo_wi8_dot_q8_x8(const uint8_t* wqi, int64_t woff, const int8_t* xq, int64_t xoff, int32_t* out8) {
  for (int L = 0; L < 8; L++) {
    int64_t acc = 0;
    for (int ig = 0; ig < 8; ig++)
      for (int k = 0; k < 4; k++)
        acc += (int64_t)xq[xoff + ig * 4 + k] * (int64_t)wqi[woff + ig * 32 + L * 4 + k];
    out8[L] = (int32_t)acc;
  }
}

static void qmatmul_x8(const int8_t* xq, const float* xs, const int32_t* xsum, const uint8_t* wqi,
                       const float* wsi, float* y, int64_t in, int64_t g_start, int64_t g_count, int q8) {
  int64_t nb = in / 32;
  int64_t gstride = q8 ? 256 : 128;
  int64_t zp = q8 ? 128 : 8;
  int32_t out8[8];
  float acc8[8];
  for (int64_t gi = 0; gi < g_count; gi++) {
    int64_t g = g_start + gi;
    int64_t wbase = g * nb * gstride, sbase = g * nb * 8;
    for (int L = 0; L < 8; L++) acc8[L] = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
      if (q8)
        rqo_wi8_dot_q8_x8(wqi, wbase + b * 256, xq, b * 32, out8);
      else
        rqo_wi8_dot_q4_x8(wqi, wbase + b * 128, xq, b * 32, out8);
      double xsb = xs[b];
      int64_t fold = zp * (int64_t)xsum[b];
      int64_t wbaseL = sbase + b * 8;
      for (int L = 0; L < 8; L++) {
        int64_t folded = (int64_t)out8[L] - fold;
        double scale = xsb * (double)wsi[wbaseL + L];
        acc8[L] = (float)((double)acc8[L] + scale * (double)folded);
      }
    }
    for (int L = 0; L < 8; L++) y[g * 8 + L] = acc8[L];
  }
}

void rqo_qmatmul_q4_x8(const int8_t* xq, const float* xs, const int32_t* xsum, const uint8_t* wqi,
                       const float* wsi, float* y, int64_t in, int64_t out, int64_t g_start, int64_t g_count) {
  (void)out;
  qmatmul_x8(xq, xs, xsum, wqi, wsi, y, in, g_start, g_count, 0);
}

void rqo_qmatmul_q8_x8(const int8_t* xq, const float* xs, const int32_t* xsum, const uint8_t* wqi,
                       const float* wsi, float* y, int64_t in, int64_t out, int64_t g_start, int64_t g_count) {
  (void)out;
  qmatmul_x8(xq, xs, xsum, wqi, wsi, y, in, g_start, g_count, 1);
}

/* ------------------------------------------------------------------------- */
/* signed q8_0 x q8_0 prefill                                                 */
/* ------------------------------------------------------------------------- */
int rqo_quantize_one_q8(const float* W, int64_t in, int64_t out, int32_t* wp, float* ws) {
  if (in % 32 != 0) return -1;
  int64_t nb = in / 32, in4 = in / 4;
  for (int64_t o = 0; o < out; o++)
    for (int64_t b = 0; b < nb; b++) {
      int64_t base = o * in + b * 32;
      double mm = 0.0;
      for (int k = 0; k < 32; k++) {
        double a = fabs((double)W[base + k]);
        if (a > mm) mm = a;
      }
      double d = mm / 127.0;
      double id = d > 0 ? 1.0 / d : 0.0;
      ws[o * nb + b] = (float)d;
      for (int w = 0; w < 8; w++) {
        int64_t e = base + w * 4;
        uint32_t word = 0;
        for (int i = 0; i < 4; i++)
          word |= (uint32_t)(rqo_java_round((double)W[e + i] * id) & 0xFF) << (8 * i);
        wp[o * in4 + b * 8 + w] = (int32_t)word;
      }
    }
  return 0;
}

void rqo_quant_act_i8_rows(const float* x, int32_t* xp, float* xs, int64_t in, int64_t nrows) {
  int64_t nb = in / 32;
  for (int64_t rb = 0; rb < nrows * nb; rb++) {
    int64_t b = rb % nb, r = rb / nb;
    int64_t base = r * in + b * 32;
    double m = 0.0;
    for (int k = 0; k < 32; k++) {
      float v = x[base + k];
      float av = v > -v ? v : -v;
      if ((double)av > m) m = av;
    }
    double d = m / 127.0;
    double id = d > 0.0 ? 1.0 / d : 0.0;
    xs[rb] = (float)d;
    for (int w = 0; w < 8; w++) {
      int64_t e = base + w * 4;
      uint32_t word = 0;
      for (int i = 0; i < 4; i++)
        word |= (uint32_t)(rqo_java_round((double)x[e + i] * id) & 0xFF) << (8 * i);
      xp[rb * 8 + w] = (int32_t)word;
    }
  }
}

void rqo_qmatmul_i8_gemm(const int32_t* xp, const float* xs, const int32_t* wp, const float* ws, float* y,
                         int64_t in, int64_t out, int64_t nrows) {
  int64_t nb = in / 32, ni4 = in / 4;
  for (int64_t ot = 0; ot < nrows * out; ot++) {
    int64_t o = ot % out, t = ot / out;
    double a = 0.0;
    for (int64_t b = 0; b < nb; b++) {
      int64_t dp = 0;
      for (int k = 0; k < 8; k++) dp = rqo_dp4a(wp[o * ni4 + b * 8 + k], xp[t * ni4 + b * 8 + k], dp);
      a += ((double)ws[o * nb + b] * (double)xs[t * nb + b]) * (double)dp;
    }
    y[t * out + o] = (float)a;
  }
}

void rqo_i8gemv_dp4a(const int32_t* wp, const int32_t* xp, float* y, int64_t kw, int64_t out) {
  for (int64_t o = 0; o < out; o++) {
    int64_t a = 0;
    for (int64_t k = 0; k < kw; k++) a = rqo_dp4a(wp[o * kw + k], xp[k], a);
    y[o] = (float)a;
  }
}

/* ------------------------------------------------------------------------- */
/* K-quants                                                                   */
/* ------------------------------------------------------------------------- */
static inline int64_t clamp64(int64_t v, int64_t lo, int64_t hi) { return v < lo ? lo : v > hi ? hi : v; }

/* quantize-weight-q4k: raster/compiler/backend/cpu/quant.clj:92-137. Clojure
 * arithmetic on floats widens to double; min/max of floats are exact. */
void rqo_quantize_weight_q4k(const float* w, int64_t len, uint8_t* wq, float* da, float* db, uint8_t* aq,
                             int8_t* bq) {
  const int64_t sbk = 256, sub = 32, subs = 8, half = 16, nsb = len / sbk;
  for (int64_t sb = 0; sb < nsb; sb++) {
    const int64_t sbase = sb * sbk;
    double as[8], bs[8];
    for (int64_t j = 0; j < subs; j++) { /* 1. sub-block scale (max-min)/15 and min */
      const int64_t base = sbase + j * sub;
      float lo = w[base], hi = w[base];
      for (int64_t i = 1; i < sub; i++) {
        if (w[base + i] < lo) lo = w[base + i];
        if (w[base + i] > hi) hi = w[base + i];
      }
      as[j] = ((double)hi - (double)lo) / 15.0;
      bs[j] = (double)lo;
    }
    double amax = 0.0, bmax = 0.0; /* 2. super-block scales of scales / mins */
    for (int64_t j = 0; j < subs; j++) {
      if (as[j] > amax) amax = as[j];
      if (fabs(bs[j]) > bmax) bmax = fabs(bs[j]);
    }
    const double dav = amax / 63.0, dbv = bmax / 31.0;
    const double ida = dav == 0.0 ? 0.0 : 1.0 / dav, idb = dbv == 0.0 ? 0.0 : 1.0 / dbv;
    da[sb] = (float)dav;
    db[sb] = (float)dbv;
    for (int64_t j = 0; j < subs; j++) {
      const int64_t aqj = clamp64(rqo_java_round(as[j] * ida), 0, 63);
      const int64_t bqj = clamp64(rqo_java_round(bs[j] * idb), -32, 31);
      const double a1 = dav * (double)aqj, b1 = dbv * (double)bqj;
      const double ia1 = a1 == 0.0 ? 0.0 : 1.0 / a1;
      const int64_t base = sbase + j * sub, sidx = sb * subs + j;
      aq[sidx] = (uint8_t)aqj;
      bq[sidx] = (int8_t)bqj;
      /* 3. weights against the quantized sub scale / min */
      for (int64_t k = 0; k < half; k++) {
        const int64_t q0 = clamp64(rqo_java_round(((double)w[base + k] - b1) * ia1), 0, 15);
        const int64_t q1 = clamp64(rqo_java_round(((double)w[base + k + half] - b1) * ia1), 0, 15);
        wq[base / 2 + k] = (uint8_t)(q0 | (q1 << 4));
      }
    }
  }
}

/* nextpad: raster/quant/pack.clj:30-33, 256 * ceil(in / 256.0) in double. */
int64_t rqo_nextpad(int64_t in) { return (int64_t)(256.0 * ceil((double)in / 256.0)); }

/* q4k-of: raster/quant/pack.clj:35-53. Each row of the row-major [out x in] W
 * is copied into a zero row of inp = nextpad(in) (padw, pack.clj:35-43), and the
 * padded matrix is quantized by quantize-weight-q4k as one array. The outputs
 * are sized for out * inp; wq holds the nibble bytes that q4k-of reinterprets
 * as little-endian int32 words (pack.clj:20-28), which are the same bytes. */
int64_t rqo_q4k_of(const float* W, int64_t out, int64_t in, uint8_t* wq, float* da, float* db, uint8_t* aq,
                   int8_t* bq) {
  const int64_t inp = rqo_nextpad(in);
  float* Wp = (float*)calloc((size_t)(out * inp), sizeof(float));
  if (!Wp) return -1;
  for (int64_t o = 0; o < out; o++) memcpy(Wp + o * inp, W + o * in, (size_t)in * sizeof(float));
  rqo_quantize_weight_q4k(Wp, out * inp, wq, da, db, aq, bq);
  free(Wp);
  return inp;
}

/* dequant-q4k: quant.clj:139-156 */
void rqo_dequant_q4k(const uint8_t* wq, const float* da, const float* db, const uint8_t* aq, const int8_t* bq,
                     int64_t len, float* out) {
  const int64_t sbk = 256, sub = 32, subs = 8, half = 16, nsb = len / sbk;
  for (int64_t sb = 0; sb < nsb; sb++) {
    const double dav = da[sb], dbv = db[sb];
    for (int64_t j = 0; j < subs; j++) {
      const int64_t base = sb * sbk + j * sub, sidx = sb * subs + j;
      const double a1 = dav * (double)(int8_t)aq[sidx], b1 = dbv * (double)bq[sidx];
      for (int64_t k = 0; k < half; k++) {
        const int64_t bv = wq[base / 2 + k];
        out[base + k] = (float)(a1 * (double)(bv & 0xF) + b1);
        out[base + k + half] = (float)(a1 * (double)(bv >> 4) + b1);
      }
    }
  }
}

/* quantize-weight-q6k: quant.clj:214-239 */
void rqo_quantize_weight_q6k(const float* w, int64_t len, uint8_t* wq, int8_t* sc, float* ds) {
  const int64_t sbk = 256, sub = 16, subs = 16, zp = 32, nsb = len / sbk;
  for (int64_t sb = 0; sb < nsb; sb++) {
    const int64_t sbase = sb * sbk;
    double as[16];
    for (int64_t j = 0; j < subs; j++) {
      double mx = 0.0;
      for (int64_t i = 0; i < sub; i++) {
        const double a = fabsf(w[sbase + j * sub + i]);
        if (a > mx) mx = a;
      }
      as[j] = mx / 32.0;
    }
    double amax = 0.0;
    for (int64_t j = 0; j < subs; j++)
      if (as[j] > amax) amax = as[j];
    const double dv = amax / 127.0, idv = dv == 0.0 ? 0.0 : 1.0 / dv;
    ds[sb] = (float)dv;
    for (int64_t j = 0; j < subs; j++) {
      const int64_t scj = clamp64(rqo_java_round(as[j] * idv), 0, 127);
      const double a1 = dv * (double)scj, ia1 = a1 == 0.0 ? 0.0 : 1.0 / a1;
      const int64_t base = sbase + j * sub;
      sc[sb * subs + j] = (int8_t)scj;
      for (int64_t k = 0; k < sub; k++)
        wq[base + k] = (uint8_t)clamp64(rqo_java_round((double)w[base + k] * ia1) + zp, 0, 63);
    }
  }
}

/* dequant-q6k: quant.clj:241-252 */
void rqo_dequant_q6k(const uint8_t* wq, const int8_t* sc, const float* ds, int64_t len, float* out) {
  const int64_t sbk = 256, sub = 16, subs = 16, zp = 32, nsb = len / sbk;
  for (int64_t sb = 0; sb < nsb; sb++) {
    const double dv = ds[sb];
    for (int64_t j = 0; j < subs; j++) {
      const double a1 = dv * (double)sc[sb * subs + j];
      const int64_t base = sb * sbk + j * sub;
      for (int64_t k = 0; k < sub; k++) out[base + k] = (float)(a1 * (double)((int64_t)wq[base + k] - zp));
    }
  }
}

/* quantize-act-q8k: quant.clj:158-176, per row */
void rqo_quantize_act_q8k(const float* x, int64_t m, int64_t in, int64_t sub, int8_t* xq, float* xs,
                          int32_t* bsums) {
  const int64_t sbk = 256, nsb = in / sbk, subs = sbk / sub;
  for (int64_t t = 0; t < m; t++)
    for (int64_t sb = 0; sb < nsb; sb++) {
      const int64_t sbase = t * in + sb * sbk;
      double mx = 0.0;
      for (int64_t i = 0; i < sbk; i++) {
        const double a = fabsf(x[sbase + i]);
        if (a > mx) mx = a;
      }
      const double d = mx / 127.0, id = d == 0.0 ? 0.0 : 1.0 / d;
      xs[t * nsb + sb] = (float)d;
      for (int64_t j = 0; j < subs; j++) {
        int64_t s = 0;
        for (int64_t k = 0; k < sub; k++) {
          const int64_t e = sbase + j * sub + k;
          const int64_t q = clamp64(rqo_java_round((double)x[e] * id), -127, 127);
          xq[e] = (int8_t)q;
          s += q;
        }
        bsums[t * (in / sub) + sb * subs + j] = (int32_t)s;
      }
    }
}

/* qmatmul-q4k-composable!: raster/quant/kernels_k.clj:15-46 */
void rqo_qmatmul_q4k(const int8_t* xq, const float* xs, const int32_t* bsums, const uint8_t* wq, const float* da,
                     const float* db, const uint8_t* aq, const int8_t* bq, int64_t m, int64_t in, int64_t out,
                     float* y) {
  const int64_t nsb = in / 256, nsub = in / 32, wrow = in / 2;
  for (int64_t t = 0; t < m; t++)
    for (int64_t o = 0; o < out; o++) {
      const int8_t* x = xq + t * in;
      double a = 0.0;
      for (int64_t sb = 0; sb < nsb; sb++) {
        const double dav = da[o * nsb + sb], dbv = db[o * nsb + sb], dact = xs[t * nsb + sb];
        double s = 0.0;
        for (int64_t j = 0; j < 8; j++) {
          const int64_t base = sb * 256 + j * 32, sidx = sb * 8 + j;
          const double aj = dav * (double)(int8_t)aq[o * nsub + sidx], bj = dbv * (double)bq[o * nsub + sidx];
          const int64_t dp = rqo_wi8_dot_q4(wq, o * wrow + base / 2, x, base);
          s = s + aj * (double)dp + bj * (double)bsums[t * nsub + sidx];
        }
        a += dact * s;
      }
      y[t * out + o] = (float)a;
    }
}

/* qmatmul-q6k-composable!: raster/quant/kernels_k.clj:48-79 */
void rqo_qmatmul_q6k(const int8_t* xq, const float* xs, const int32_t* bsums, const uint8_t* wq, const int8_t* sc,
                     const float* ds, int64_t m, int64_t in, int64_t out, float* y) {
  const int64_t nsb = in / 256, nsub = in / 16;
  for (int64_t t = 0; t < m; t++)
    for (int64_t o = 0; o < out; o++) {
      const int8_t* x = xq + t * in;
      double a = 0.0;
      for (int64_t sb = 0; sb < nsb; sb++) {
        const double dv = ds[o * nsb + sb], dact = xs[t * nsb + sb];
        double s = 0.0;
        for (int64_t j = 0; j < 16; j++) {
          const int64_t base = sb * 256 + j * 16, sidx = sb * 16 + j;
          const int64_t scj = sc[o * nsub + sidx];
          const int64_t dp = rqo_wi8_dot(wq, o * in + base, x, base, 16);
          const int64_t folded = dp - 32 * (int64_t)bsums[t * nsub + sidx];
          s += (double)scj * (double)folded;
        }
        a += dv * dact * s;
      }
      y[t * out + o] = (float)a;
    }
}

void rqo_dense_matmul_nt_f64(const float* X, const float* W, int64_t m, int64_t in, int64_t out, double* y) {
  for (int64_t p = 0; p < m; p++)
    for (int64_t o = 0; o < out; o++) {
      double s = 0.0;
      for (int64_t i = 0; i < in; i++) s += (double)X[p * in + i] * (double)W[o * in + i];
      y[p * out + o] = s;
    }
}

/* ------------------------------------------------------------------------- */
/* dense f32 GEMM surface: the float arms of raster/linalg/blas.clj, nn/linear */
/* ------------------------------------------------------------------------- */
/* dgemm! / dgemm-tn! / dgemm-nt! (raster/linalg/blas.clj:287-337): the
 * cblas_sgemm call C = alpha op(A) op(B) + beta C, row-major; op(A) = A^T
 * (A stored [k x m]) when trans_a, op(B) = B^T (B stored [n x k]) when
 * trans_b. The products are summed in double and each element rounded to f32
 * once (a BLAS sums in f32 in an order of its own; this is the value its
 * error is measured from). m, n or k not positive: nothing (blas.clj:301,
 * 318, 334). */
void rqo_sgemm(int trans_a, int trans_b, int64_t m, int64_t k, int64_t n, float alpha, const float* A,
               const float* B, float beta, float* C) {
  if (m <= 0 || n <= 0 || k <= 0) return;
  for (int64_t i = 0; i < m; i++)
    for (int64_t j = 0; j < n; j++) {
      double s = 0.0;
      for (int64_t p = 0; p < k; p++) {
        const double a = trans_a ? A[p * m + i] : A[i * k + p];
        const double b = trans_b ? B[j * k + p] : B[p * n + j];
        s += a * b;
      }
      C[i * n + j] = (float)((double)alpha * s + (double)beta * (double)C[i * n + j]);
    }
}

/* linear! (raster/dl/nn.clj:161-183): every row of y set to b, then
 * dgemm-nt! x W y with alpha = beta = 1. */
void rqo_linear(const float* x, const float* W, const float* b, float* y, int64_t batch, int64_t in, int64_t out) {
  if (batch <= 0 || out <= 0) return;
  for (int64_t r = 0; r < batch; r++)
    for (int64_t o = 0; o < out; o++) y[r * out + o] = b[o];
  rqo_sgemm(0, 1, batch, in, out, 1.0f, x, W, 1.0f, y);
}

/* ------------------------------------------------------------------------- */
/* decoder-step glue (the host ops around the quantized linears)             */
/* ------------------------------------------------------------------------- */
/* rms-norm!: raster/dl/nn.clj:497-516. Row mean of squares in double, one
 * f32 store of x * inv * (gain_offset + w). */
void rqo_rms_norm(const float* x, const float* w, float* out, int64_t rows, int64_t features, double eps,
                  double gain_offset) {
  for (int64_t r = 0; r < rows; r++) {
    const float* xr = x + r * features;
    double s = 0.0;
    for (int64_t i = 0; i < features; i++) s += (double)xr[i] * (double)xr[i];
    const double ms = s / (double)features;
    const double inv = 1.0 / sqrt(ms + eps);
    for (int64_t i = 0; i < features; i++)
      out[r * features + i] = (float)((double)xr[i] * inv * (gain_offset + (double)w[i]));
  }
}

/* rope-pos: raster/dl/attention.clj:197-214 (NeoX half split, positions
 * pos_offset .. pos_offset + seq_len - 1). */
void rqo_rope_pos(const float* x, float* out, int64_t seq_len, int64_t heads, int64_t head_dim, double theta,
                  int64_t pos_offset) {
  const int64_t half = head_dim / 2;
  const double ln_theta = log(theta);
  for (int64_t p = 0; p < seq_len; p++)
    for (int64_t h = 0; h < heads; h++) {
      const int64_t base = p * heads * head_dim + h * head_dim;
      const double pos = (double)(pos_offset + p);
      for (int64_t i = 0; i < half; i++) {
        const double freq = exp((-2.0 * (double)i / (double)head_dim) * ln_theta);
        const double ang = pos * freq;
        const double c = cos(ang), s = sin(ang);
        const double x0 = x[base + i], x1 = x[base + i + half];
        out[base + i] = (float)(x0 * c - x1 * s);
        out[base + i + half] = (float)(x1 * c + x0 * s);
      }
    }
}

/* gqa-decode-attention: raster/dl/attention.clj:248-287. Scores and the
 * softmax numerators are stored as f32 (the `sc` scratch is an array like q);
 * dot products, the sum and the output accumulation run in double. */
void rqo_gqa_decode_attention(const float* q, const float* k, const float* v, int64_t cache_len, int64_t n_q,
                              int64_t n_kv, int64_t head_dim, double scale, float* out, float* sc) {
  const int64_t group = n_q / n_kv;
  for (int64_t hq = 0; hq < n_q; hq++) {
    const int64_t hkv = hq / group, qb = hq * head_dim;
    for (int64_t j = 0; j < cache_len; j++) {
      const int64_t kb = j * n_kv * head_dim + hkv * head_dim;
      double dot = 0.0;
      for (int64_t d = 0; d < head_dim; d++) dot += (double)q[qb + d] * (double)k[kb + d];
      sc[j] = (float)(dot * scale);
    }
    float mx = -INFINITY;
    for (int64_t j = 0; j < cache_len; j++) mx = sc[j] > mx ? sc[j] : mx;
    double sum = 0.0;
    for (int64_t j = 0; j < cache_len; j++) {
      const double e = exp((double)sc[j] - (double)mx);
      sc[j] = (float)e;
      sum += e;
    }
    const double inv = 1.0 / sum;
    for (int64_t d = 0; d < head_dim; d++) {
      double a = 0.0;
      for (int64_t j = 0; j < cache_len; j++) {
        const int64_t kvb = j * n_kv * head_dim + hkv * head_dim;
        a += ((double)sc[j] * inv) * (double)v[kvb + d];
      }
      out[qb + d] = (float)a;
    }
  }
}

/* silu-mul!: raster/dl/nn.clj:200-203. */
void rqo_silu_mul(const float* gate, const float* up, float* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    const double g = gate[i];
    out[i] = (float)((g * (1.0 / (1.0 + exp(-g)))) * (double)up[i]);
  }
}

/* residual-add!: raster/dl/nn.clj:217-219 (the double sum of two floats is
 * exact, so this is the correctly rounded f32 sum). */
void rqo_residual_add(const float* a, const float* b, float* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = (float)((double)a[i] + (double)b[i]);
}

/* kv-append!: raster/dl/attention.clj:413-416. */
void rqo_kv_append(const float* src, float* cache, int64_t kvrow, int64_t pos) {
  memcpy(cache + pos * kvrow, src, (size_t)kvrow * sizeof(float));
}

/* One pre-norm decoder layer for one token (Llama form of the step the
 * reference chains in test/raster/dl/decoder_layer_gpu_test.clj:25-83, with
 * RMSNorm, NeoX RoPE, SwiGLU and no q/k norms): the seven linears are
 * rqo_qlinear_q8 over Q8_0 weights w[0..6] = q, k, v, o, gate, up, down
 * (codes) with scales s[0..6]. kcache / vcache hold cache_len - 1 earlier
 * positions of n_kv * head_dim floats and receive the new one at position
 * cache_len - 1; x (d floats) is updated in place. gain1 / gain2 are the two
 * RMSNorm weights (gain offset 0). scratch needs 3 * d + 5 * n_q * head_dim +
 * 3 * ffn + cache_len floats. */
void rqo_decoder_layer(float* x, const int8_t* const* w, const float* const* s, const float* gain1,
                       const float* gain2, float* kcache, float* vcache, int64_t d, int64_t n_q, int64_t n_kv,
                       int64_t head_dim, int64_t ffn, int64_t cache_len, double eps, double theta,
                       float* scratch) {
  const int64_t qd = n_q * head_dim, kvd = n_kv * head_dim, pos = cache_len - 1;
  float* xn = scratch;
  float* q = xn + d;
  float* kk = q + qd;
  float* vv = kk + qd;
  float* qr = vv + qd;
  float* at = qr + qd;
  float* o = at + qd;
  float* gate = o + d;
  float* up = gate + ffn;
  float* h = up + ffn;
  float* dn = h + ffn;
  float* sc = dn + d;
  rqo_rms_norm(x, gain1, xn, 1, d, eps, 0.0);
  rqo_qlinear_q8(xn, w[0], s[0], 1, d, qd, q);
  rqo_qlinear_q8(xn, w[1], s[1], 1, d, kvd, kk);
  rqo_qlinear_q8(xn, w[2], s[2], 1, d, kvd, vv);
  rqo_rope_pos(q, qr, 1, n_q, head_dim, theta, pos);
  rqo_rope_pos(kk, kcache + pos * kvd, 1, n_kv, head_dim, theta, pos); /* rotate straight into the cache */
  rqo_kv_append(vv, vcache, kvd, pos);
  rqo_gqa_decode_attention(qr, kcache, vcache, cache_len, n_q, n_kv, head_dim, 1.0 / sqrt((double)head_dim), at,
                           sc);
  rqo_qlinear_q8(at, w[3], s[3], 1, qd, d, o);
  rqo_residual_add(x, o, x, d);
  rqo_rms_norm(x, gain2, xn, 1, d, eps, 0.0);
  rqo_qlinear_q8(xn, w[4], s[4], 1, d, ffn, gate);
  rqo_qlinear_q8(xn, w[5], s[5], 1, d, ffn, up);
  rqo_silu_mul(gate, up, h, ffn);
  rqo_qlinear_q8(h, w[6], s[6], 1, ffn, d, dn);
  rqo_residual_add(x, dn, x, d);
}
