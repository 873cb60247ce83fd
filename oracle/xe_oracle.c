/*
 * xe_oracle.c -- CPU restatement of atassis/xdna-engine's decode arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (see xe_oracle.h).  Nothing in the product
 * library calls this file; it is the checker the HIP path is compared with.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off).  OpenMP only
 * splits independent output rows / streams across threads; the arithmetic of
 * every output element is the sequential order cited below.
 */
#include "xe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

void xo_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

static inline uint32_t f2u(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

/* ------------------------------------------------------------------------ */
/* bf16                                                                     */
/* ------------------------------------------------------------------------ */

/* f32_to_bf16_bits (npu-xrt/src/lib.rs:809-817): RNE by integer bias; NaN
 * stays a quiet NaN (OR 0x0040).  Pins: tests/golden bf16 special values +
 * 200k LCG sweep (npu-xrt/src/lib.rs:1096-1122), exhaustive unpack. */
uint16_t xo_f32_to_bf16_bits(float x) {
  uint32_t bits = f2u(x);
  if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x0040u);
  uint32_t bias = 0x00007fffu + ((bits >> 16) & 1u);
  return (uint16_t)((bits + bias) >> 16);
}

/* bf16_bits_to_f32 (npu-xrt/src/lib.rs:820-822). */
float xo_bf16_bits_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* bf16_round (npu-asr-host/src/lib.rs:12-19).  Pins: test_bf16_round values
 * (npu-asr-host/src/lib.rs:876-887). */
float xo_bf16_round(float x) {
  uint32_t bits = f2u(x);
  if ((bits & 0x7fffffffu) > 0x7f800000u) return u2f(((bits >> 16) | 0x0040u) << 16);
  uint32_t bias = 0x00007fffu + ((bits >> 16) & 1u);
  return u2f((bits + bias) & 0xffff0000u);
}

void xo_pack_bf16(const float *src, uint16_t *dst, size_t n) {
  for (size_t i = 0; i < n; i++) dst[i] = xo_f32_to_bf16_bits(src[i]);
}

/* unpack_bf16_to_f32 (npu-xrt/src/lib.rs:879-900 array form): <<16. */
void xo_unpack_bf16(const uint16_t *src, float *dst, size_t n) {
  for (size_t i = 0; i < n; i++) dst[i] = xo_bf16_bits_to_f32(src[i]);
}

/* ------------------------------------------------------------------------ */
/* norms / activations                                                      */
/* ------------------------------------------------------------------------ */

/* layer_norm (npu-asr-host/src/lib.rs:79-109), also ln_row
 * (whisper_decoder.rs:1894-1900): sequential f32 sum, two-pass population
 * variance, inv = 1/sqrt(var + eps), out = (x - mean) * inv * g + b.
 * Pins: test_layer_norm expected vectors (npu-asr-host/src/lib.rs:889-900). */
void xo_layer_norm(const float *x, int rows, int d, const float *gamma,
                   const float *beta, float eps, float *out) {
  for (int r = 0; r < rows; r++) {
    const float *row = x + (size_t)r * d;
    float *o = out + (size_t)r * d;
    float sum = 0.f;
    for (int j = 0; j < d; j++) sum += row[j];
    float mean = sum / (float)d;
    float vs = 0.f;
    for (int j = 0; j < d; j++) {
      float c = row[j] - mean;
      vs += c * c;
    }
    float inv = 1.0f / sqrtf(vs / (float)d + eps);
    for (int j = 0; j < d; j++) o[j] = (row[j] - mean) * inv * gamma[j] + beta[j];
  }
}

/* layer_norm_normalize (npu-asr-host/src/lib.rs:112-141).  Pins:
 * test_layer_norm_normalize expected vectors (lib.rs:902-911). */
void xo_layer_norm_normalize(const float *x, int rows, int d, float eps,
                             float *out) {
  for (int r = 0; r < rows; r++) {
    const float *row = x + (size_t)r * d;
    float *o = out + (size_t)r * d;
    float sum = 0.f;
    for (int j = 0; j < d; j++) sum += row[j];
    float mean = sum / (float)d;
    float vs = 0.f;
    for (int j = 0; j < d; j++) {
      float c = row[j] - mean;
      vs += c * c;
    }
    float inv = 1.0f / sqrtf(vs / (float)d + eps);
    for (int j = 0; j < d; j++) o[j] = (row[j] - mean) * inv;
  }
}

/* rmsnorm_ref (npu-gemma/src/lib.rs:55-64): ms = sum(v*v)/n, inv =
 * 1/sqrt(ms+eps), out = v * inv * (1 + w).  Pins: rmsnorm_unit
 * (lib.rs:83-91) + closed form for constant |x| (RMS of +-c is c). */
void xo_rmsnorm(const float *x, int n, const float *w, float eps, float *out) {
  float ms = 0.f;
  for (int i = 0; i < n; i++) ms += x[i] * x[i];
  ms = ms / (float)n;
  float inv = 1.0f / sqrtf(ms + eps);
  for (int i = 0; i < n; i++) out[i] = x[i] * inv * (1.0f + w[i]);
}

/* erf_scalar (npu-asr-host/src/lib.rs:464-475), Abramowitz & Stegun 7.1.26.
 * Pins: |erf_as - erf| < 1.5e-7 (the published A&S bound), odd symmetry. */
float xo_erf_as(float x) {
  float sign = x < 0.0f ? -1.0f : 1.0f;
  x = fabsf(x);
  float t = 1.0f / (1.0f + 0.3275911f * x);
  float y = 1.0f - (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t -
                     0.284496736f) * t + 0.254829592f) * t * expf(-x * x);
  return sign * y;
}

/* gelu (npu-asr-host/src/lib.rs:477-489): 0.5 x (1 + erf(x / sqrt 2)).
 * Pins: gelu(0)=0, gelu(x) - gelu(-x) = x, libm-erf GELU within 2e-7|x|. */
float xo_gelu_erf(float x) {
  const float inv_sqrt2 = 0.70710678118654752f;
  return 0.5f * x * (1.0f + xo_erf_as(x * inv_sqrt2));
}

/* gelu_tanh (npu-gemma/src/lib.rs:74-77).  Pins: geglu_shapes (gelu(0)=0,
 * lib.rs:93-99) and |gelu_tanh - gelu_erf| < 1e-3 (published bound). */
float xo_gelu_tanh(float x) {
  const float c = 0.79788456f;
  return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

/* fast_exp_nonpos (npu-asr-host/src/lib.rs:38-58).  Pins:
 * test_fast_exp_accuracy bound 5e-4 (lib.rs:847-859). */
float xo_fast_exp_nonpos(float x) {
  if (x < -87.0f) x = -87.0f;
  const float log2e = 1.442695040888963f;
  float y = x * log2e;
  float yf = floorf(y);
  float f = y - yf;
  float p = 1.0f + f * (0.6931471805599453f +
                        f * (0.2402265069591007f +
                             f * (0.05550410866482158f +
                                  f * (0.009618129107628477f + f * 0.0013333558146428443f))));
  uint32_t e = (uint32_t)((int)yf + 127);
  return p * u2f(e << 23);
}

/* ------------------------------------------------------------------------ */
/* int8 quantisation                                                        */
/* ------------------------------------------------------------------------ */

/* quant_i8 (ctx2.rs:1352-1354): (x / scale).round().clamp(-127, 127); Rust
 * round() is half away from zero = C roundf.  Pins: exact ties (0.5 -> 1,
 * -0.5 -> -1, 2.5 -> 3), clamp. */
int8_t xo_quant_i8(float x, float scale) {
  float v = roundf(x / scale);
  if (v != v) return 0; /* Rust's saturating `as i8` maps NaN to 0 */
  if (v < -127.0f) v = -127.0f;
  if (v > 127.0f) v = 127.0f;
  return (int8_t)v;
}

/* quant_scale (ctx2.rs:1361-1377): max|a| / 127, 1.0 for all-zero. */
float xo_quant_scale(const float *a, size_t n) {
  float amax = 0.f;
  for (size_t i = 0; i < n; i++) {
    float v = fabsf(a[i]);
    amax = v > amax ? v : amax;
  }
  return amax > 0.0f ? amax / 127.0f : 1.0f;
}

/* Per-output-channel weight quant (opt125m_decode.rs:45-62, ctx2.rs:564-580)
 * for an [M,K] matrix: s[r] = max_k |w[r,k]| / 127 (1.0 if 0). */
void xo_quant_rows_i8(const float *w, int m, int k, int8_t *q, float *s) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < m; r++) {
    const float *row = w + (size_t)r * k;
    float amax = 0.f;
    for (int j = 0; j < k; j++) {
      float v = fabsf(row[j]);
      amax = v > amax ? v : amax;
    }
    float sc = amax > 0.0f ? amax / 127.0f : 1.0f;
    s[r] = sc;
    for (int j = 0; j < k; j++) q[(size_t)r * k + j] = xo_quant_i8(row[j], sc);
  }
}

/* qrow of the fused-decode generator (route_b_kernels/decode_fused/
 * gen_decode.py:158-165) and w_or_i8 (:291-298): s = max|row| / 127 in fp32
 * (1.0 for an all-zero row), q = numpy round (half to even) of w / s,
 * clamped to +-127; the scale the GEMV output is multiplied by is stored as
 * bf16 (`weights_to_write[...] = bf16(s)`), so s_out = bf16(s) while q uses
 * the fp32 s. */
void xo_quant_rows_i8_elf(const float *w, int m, int k, int8_t *q, float *s_out) {
  for (int r = 0; r < m; r++) {
    const float *row = w + (size_t)r * k;
    float amax = 0.f;
    for (int j = 0; j < k; j++) {
      float v = fabsf(row[j]);
      amax = v > amax ? v : amax;
    }
    float sc = amax / 127.0f;
    if (!(sc > 0.0f)) sc = 1.0f;
    for (int j = 0; j < k; j++) {
      float v = rintf(row[j] / sc); /* round half to even (default mode) */
      if (v != v) v = 0.0f;
      if (v < -127.0f) v = -127.0f;
      if (v > 127.0f) v = 127.0f;
      q[(size_t)r * k + j] = (int8_t)v;
    }
    s_out[r] = xo_bf16_round(sc);
  }
}

/* The reference's own layout: W [K,N], per-column scale
 * (opt125m_decode.rs:45-62 verbatim shape). */
void xo_quant_cols_i8(const float *w_kn, int k, int n, int8_t *q_kn, float *s) {
  for (int c = 0; c < n; c++) {
    float amax = 0.f;
    for (int r = 0; r < k; r++) {
      float v = fabsf(w_kn[(size_t)r * n + c]);
      amax = v > amax ? v : amax;
    }
    s[c] = amax > 0.0f ? amax / 127.0f : 1.0f;
  }
  for (int r = 0; r < k; r++)
    for (int c = 0; c < n; c++)
      q_kn[(size_t)r * n + c] = xo_quant_i8(w_kn[(size_t)r * n + c], s[c]);
}

/* dequant_epi Epi::None / Epi::Bias (ctx2.rs:1386-1435): the exact order
 * (acc as f32 * scale_a) * ws[c] (+ bias[c]). */
void xo_dequant_epi(const int32_t *acc, int mp, int n, float scale_a,
                    const float *ws, const float *bias, float *out) {
  for (int r = 0; r < mp; r++)
    for (int c = 0; c < n; c++) {
      float v = (float)acc[(size_t)r * n + c] * scale_a * ws[c];
      out[(size_t)r * n + c] = bias ? v + bias[c] : v;
    }
}

/* ------------------------------------------------------------------------ */
/* GEMV                                                                     */
/* ------------------------------------------------------------------------ */

/* Lin::fwd int8 (opt125m_decode.rs:106-125) in [M,K] layout: y[r] = sum over
 * k = 0..K-1 in order of x[k] * (float)q[r,k], then y * s[r] + b[r].
 * Pins: integer x gives an exact integer dot (brute force), all-zero weight
 * scale 1.0, and the [K,N] restatement xo_lin_fwd_i8_kn agrees bit for bit. */
void xo_gemv_i8(const float *x, int b, int k, int m, const int8_t *q,
                const float *s, const float *bias, float *y) {
  for (int bi = 0; bi < b; bi++) {
    const float *xb = x + (size_t)bi * k;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < m; r++) {
      const int8_t *row = q + (size_t)r * k;
      float acc = 0.f;
      for (int j = 0; j < k; j++) acc += xb[j] * (float)row[j];
      float v = acc * s[r];
      y[(size_t)bi * m + r] = bias ? v + bias[r] : v;
    }
  }
}

/* xo_gemv_i8 over a copy of q stored in blocks of eight rows, k-major
 * (qb[(blk * K + j) * 8 + i] = q[blk * 8 + i, j]; rows past M are zero).
 * Each output still accumulates x[j] * q[r, j] for j = 0..K-1 in order in
 * its own fp32 accumulator (a separate multiply and add, as in the scalar
 * loop): the eight lanes of a block, and the blocks, are independent sums,
 * so the AVX2 form computes exactly what the scalar form does. */
static void xo_dot8_i8_scalar(const float *xb, int k, const int8_t *tq, int nb, float *out) {
  for (int bl = 0; bl < nb; bl++) {
    const int8_t *t = tq + (size_t)bl * k * 8;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j = 0; j < k; j++) {
      float xj = xb[j];
      for (int i = 0; i < 8; i++) acc[i] += xj * (float)t[(size_t)j * 8 + i];
    }
    for (int i = 0; i < 8; i++) out[bl * 8 + i] = acc[i];
  }
}

#if defined(__x86_64__)
#include <immintrin.h>
/* Four blocks (32 rows) per pass: four independent accumulator vectors. */
__attribute__((target("avx2")))
static void xo_dot8_i8_avx2(const float *xb, int k, const int8_t *tq, int nb, float *out) {
  int bl = 0;
  for (; bl + 4 <= nb; bl += 4) {
    const int8_t *t0 = tq + (size_t)bl * k * 8;
    const int8_t *t1 = t0 + (size_t)k * 8, *t2 = t1 + (size_t)k * 8, *t3 = t2 + (size_t)k * 8;
    __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
    __m256 a2 = _mm256_setzero_ps(), a3 = _mm256_setzero_ps();
    for (int j = 0; j < k; j++) {
      __m256 xj = _mm256_broadcast_ss(xb + j);
      __m256 w0 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)(t0 + (size_t)j * 8))));
      __m256 w1 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)(t1 + (size_t)j * 8))));
      __m256 w2 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)(t2 + (size_t)j * 8))));
      __m256 w3 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)(t3 + (size_t)j * 8))));
      a0 = _mm256_add_ps(a0, _mm256_mul_ps(xj, w0));
      a1 = _mm256_add_ps(a1, _mm256_mul_ps(xj, w1));
      a2 = _mm256_add_ps(a2, _mm256_mul_ps(xj, w2));
      a3 = _mm256_add_ps(a3, _mm256_mul_ps(xj, w3));
    }
    _mm256_storeu_ps(out + bl * 8, a0);
    _mm256_storeu_ps(out + bl * 8 + 8, a1);
    _mm256_storeu_ps(out + bl * 8 + 16, a2);
    _mm256_storeu_ps(out + bl * 8 + 24, a3);
  }
  if (bl < nb) xo_dot8_i8_scalar(xb, k, tq + (size_t)bl * k * 8, nb - bl, out + bl * 8);
}
#endif

static void xo_dot8_i8(const float *xb, int k, const int8_t *tq, int nb, float *out) {
#if defined(__x86_64__)
  if (__builtin_cpu_supports("avx2")) {
    xo_dot8_i8_avx2(xb, k, tq, nb, out);
    return;
  }
#endif
  xo_dot8_i8_scalar(xb, k, tq, nb, out);
}

static int8_t *xo_block8_i8(const int8_t *q, int m, int k) {
  int nblk = (m + 7) / 8;
  int8_t *qb = (int8_t *)calloc((size_t)nblk * k * 8, 1);
#pragma omp parallel for schedule(static)
  for (int blk = 0; blk < nblk; blk++)
    for (int i = 0; i < 8 && blk * 8 + i < m; i++) {
      const int8_t *row = q + (size_t)(blk * 8 + i) * k;
      int8_t *dst = qb + (size_t)blk * k * 8 + i;
      for (int j = 0; j < k; j++) dst[(size_t)j * 8] = row[j];
    }
  return qb;
}

static void xo_gemv_i8_blocked(const float *xb, int k, int m, const int8_t *qb,
                               const float *s, const float *bias, float *y) {
  int nblk = (m + 7) / 8, ngrp = (nblk + 3) / 4;
#pragma omp parallel for schedule(static)
  for (int g = 0; g < ngrp; g++) {
    int b0 = g * 4, nb = nblk - b0 < 4 ? nblk - b0 : 4;
    float acc[32];
    xo_dot8_i8(xb, k, qb + (size_t)b0 * k * 8, nb, acc);
    for (int i = 0; i < nb * 8 && b0 * 8 + i < m; i++) {
      int r = b0 * 8 + i;
      float v = acc[i] * s[r];
      y[r] = bias ? v + bias[r] : v;
    }
  }
}

/* xo_gemv_i8 through the row-blocked copy the decoder models use
 * (xo_block8_i8 + xo_gemv_i8_blocked).  Pins: equal to xo_gemv_i8 bit for
 * bit on ragged shapes (tests/test_oracle.py). */
void xo_gemv_i8_rowblocked(const float *x, int b, int k, int m, const int8_t *q,
                           const float *s, const float *bias, float *y) {
  int8_t *qb = xo_block8_i8(q, m, k);
  for (int bi = 0; bi < b; bi++)
    xo_gemv_i8_blocked(x + (size_t)bi * k, k, m, qb, s, bias, y + (size_t)bi * m);
  free(qb);
}

/* Lin::fwd int8 verbatim loop shape: W [K,N], k-outer (opt125m_decode.rs:
 * 106-125).  Kept to pin xo_gemv_i8 against the reference's own layout. */
void xo_lin_fwd_i8_kn(const float *x, int b, int k, int n, const int8_t *q_kn,
                      const float *s, const float *bias, float *y) {
  for (int mi = 0; mi < b; mi++) {
    float *yr = y + (size_t)mi * n;
    for (int ni = 0; ni < n; ni++) yr[ni] = 0.f;
    for (int ki = 0; ki < k; ki++) {
      float a = x[(size_t)mi * k + ki];
      const int8_t *wrow = q_kn + (size_t)ki * n;
      for (int ni = 0; ni < n; ni++) yr[ni] += a * (float)wrow[ni];
    }
    for (int ni = 0; ni < n; ni++) yr[ni] = yr[ni] * s[ni] + (bias ? bias[ni] : 0.0f);
  }
}

/* ------------------------------------------------------------------------ */
/* int4 weights (OPT_INT4, opt125m_decode.rs:63-105)                        */
/* ------------------------------------------------------------------------ */

/* Nibble sign extension `((v as i32) ^ 0x8) - 0x8` (opt125m_decode.rs:87). */
static inline int xo_sext4(unsigned v) { return (int)((v & 0xFu) ^ 0x8u) - 0x8; }

/* Lin::load int4 branch (opt125m_decode.rs:63-79) in the reference's own
 * layout: W [K,N]; s[c] = max_r |W[r,c]| / 7 (1.0 if 0); q = round(W/s)
 * (half away from zero) clamped to +-7; packed [K, N/2], the even column in
 * the low nibble, the odd one in the high nibble.  N even. */
void xo_quant_cols_i4(const float *w_kn, int k, int n, uint8_t *packed_kn, float *s) {
  for (int c = 0; c < n; c++) {
    float amax = 0.f;
    for (int r = 0; r < k; r++) {
      float v = fabsf(w_kn[(size_t)r * n + c]);
      amax = v > amax ? v : amax;
    }
    s[c] = amax > 0.0f ? amax / 7.0f : 1.0f;
  }
  for (int r = 0; r < k; r++)
    for (int c2 = 0; c2 < n / 2; c2++) {
      unsigned nib[2];
      for (int h = 0; h < 2; h++) {
        int c = 2 * c2 + h;
        float v = roundf(w_kn[(size_t)r * n + c] / s[c]);
        if (v != v) v = 0.0f; /* saturating `as i32` maps NaN to 0 */
        if (v < -7.0f) v = -7.0f;
        if (v > 7.0f) v = 7.0f;
        nib[h] = (unsigned)((int)v & 0x0F);
      }
      packed_kn[(size_t)r * (n / 2) + c2] = (uint8_t)(nib[0] | (nib[1] << 4));
    }
}

/* Lin::fwd int4 branch verbatim loop shape (opt125m_decode.rs:83-105): k
 * outer, y[2j] += a * sext(lo), y[2j+1] += a * sext(hi) in k order (f32),
 * then y * s + b. */
void xo_lin_fwd_i4_kn(const float *x, int b, int k, int n, const uint8_t *packed_kn,
                      const float *s, const float *bias, float *y) {
  const int nh = n / 2;
  for (int mi = 0; mi < b; mi++) {
    float *yr = y + (size_t)mi * n;
    for (int ni = 0; ni < n; ni++) yr[ni] = 0.f;
    for (int ki = 0; ki < k; ki++) {
      float a = x[(size_t)mi * k + ki];
      const uint8_t *row = packed_kn + (size_t)ki * nh;
      for (int nj = 0; nj < nh; nj++) {
        uint8_t byte = row[nj];
        yr[2 * nj] += a * (float)xo_sext4(byte & 0x0F);
        yr[2 * nj + 1] += a * (float)xo_sext4(byte >> 4);
      }
    }
    for (int ni = 0; ni < n; ni++) yr[ni] = yr[ni] * s[ni] + (bias ? bias[ni] : 0.0f);
  }
}

/* The same quantisation in the build's [M,K] layout (out-major rows): row r
 * is output channel r, s[r] = max_k |W[r,k]| / 7, and the row's K values are
 * packed along K: byte j holds k = 2j (low nibble) and k = 2j+1 (high).  K
 * even.  Same q and s as xo_quant_cols_i4 on the transpose. */
void xo_quant_rows_i4(const float *w, int m, int k, uint8_t *packed, float *s) {
  for (int r = 0; r < m; r++) {
    const float *row = w + (size_t)r * k;
    float amax = 0.f;
    for (int j = 0; j < k; j++) {
      float v = fabsf(row[j]);
      amax = v > amax ? v : amax;
    }
    float sc = amax > 0.0f ? amax / 7.0f : 1.0f;
    s[r] = sc;
    for (int j2 = 0; j2 < k / 2; j2++) {
      unsigned nib[2];
      for (int h = 0; h < 2; h++) {
        float v = roundf(row[2 * j2 + h] / sc);
        if (v != v) v = 0.0f;
        if (v < -7.0f) v = -7.0f;
        if (v > 7.0f) v = 7.0f;
        nib[h] = (unsigned)((int)v & 0x0F);
      }
      packed[(size_t)r * (k / 2) + j2] = (uint8_t)(nib[0] | (nib[1] << 4));
    }
  }
}

/* Lin::fwd int4 in [M,K] layout: y[r] = sum over k in order of
 * x[k] * sext(q[r,k]), then y * s[r] + b[r] (the per-output sum of
 * xo_lin_fwd_i4_kn, in the same k order, so the two agree bit for bit). */
void xo_gemv_i4(const float *x, int b, int k, int m, const uint8_t *packed,
                const float *s, const float *bias, float *y) {
  for (int bi = 0; bi < b; bi++) {
    const float *xb = x + (size_t)bi * k;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < m; r++) {
      const uint8_t *row = packed + (size_t)r * (k / 2);
      float acc = 0.f;
      for (int j = 0; j < k; j++) {
        uint8_t byte = row[j / 2];
        acc += xb[j] * (float)xo_sext4((j & 1) ? (unsigned)(byte >> 4) : (unsigned)byte);
      }
      float v = acc * s[r];
      y[(size_t)bi * m + r] = bias ? v + bias[r] : v;
    }
  }
}

/* linear_row (whisper_decoder.rs:215-230) semantics with an [M,K] f32
 * weight: bias first, then += x[k] * w in k order. */
void xo_gemv_f32(const float *x, int b, int k, int m, const float *w,
                 const float *bias, float *y) {
  for (int bi = 0; bi < b; bi++)
    for (int r = 0; r < m; r++) {
      float acc = bias ? bias[r] : 0.f;
      for (int j = 0; j < k; j++) acc += x[(size_t)bi * k + j] * w[(size_t)r * k + j];
      y[(size_t)bi * m + r] = acc;
    }
}

/* bf16-weight GEMV (ctx_decode.rs:269-366: W packed to bf16 RNE, fp32
 * accumulate), host bias added after the sum.  Parity: tolerance. */
void xo_gemv_bf16w(const float *x, int b, int k, int m, const uint16_t *w,
                   const float *bias, float *y) {
  for (int bi = 0; bi < b; bi++) {
    const float *xb = x + (size_t)bi * k;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < m; r++) {
      const uint16_t *row = w + (size_t)r * k;
      float acc = 0.f;
      for (int j = 0; j < k; j++) acc += xb[j] * xo_bf16_bits_to_f32(row[j]);
      y[(size_t)bi * m + r] = bias ? acc + bias[r] : acc;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* bfp16ebs8                                                                */
/* ------------------------------------------------------------------------ */

/* to_bfp16_blocks after to_bf16 (ffn_bfp16/golden_ffn_gemm.py:21-49, 56-60):
 * blocks of 8 along K; e = floor(log2(max|x|)) (max 0 -> 1.0 -> e = 0);
 * quantum 2^(e-6); q = round-half-even(x / quantum).  Storage decision for
 * the sim's gap (q can round to +128, outside int8): saturate to 127; -128
 * is representable and kept.  Exponent byte = e + 127, clamped to [0, 254].
 * Pins: decode(encode(x)) == the sim's q*quantum whenever no saturation
 * occurs (power-of-two quanta make it exact), block max within 1 quantum. */
void xo_bfp16_encode(const float *w, int m, int k, int8_t *mant, uint8_t *exps) {
  int nb = k / 8;
  for (int r = 0; r < m; r++)
    for (int bk = 0; bk < nb; bk++) {
      float v[8];
      float maxabs = 0.f;
      for (int i = 0; i < 8; i++) {
        v[i] = xo_bf16_round(w[(size_t)r * k + bk * 8 + i]);
        float a = fabsf(v[i]);
        maxabs = a > maxabs ? a : maxabs;
      }
      if (maxabs == 0.0f) maxabs = 1.0f;
      int e2;
      (void)frexpf(maxabs, &e2); /* maxabs = f * 2^e2, f in [0.5, 1): exact */
      int e = e2 - 1;            /* floor(log2(maxabs)) */
      if (e < -127) e = -127;
      if (e > 127) e = 127;
      float quantum = ldexpf(1.0f, e - 6);
      for (int i = 0; i < 8; i++) {
        float qv = rintf(v[i] / quantum);
        if (qv > 127.0f) qv = 127.0f;
        if (qv < -128.0f) qv = -128.0f;
        mant[(size_t)r * k + bk * 8 + i] = (int8_t)qv;
      }
      exps[(size_t)r * nb + bk] = (uint8_t)(e + 127);
    }
}

void xo_bfp16_decode(const int8_t *mant, const uint8_t *exps, int m, int k, float *w) {
  int nb = k / 8;
  for (int r = 0; r < m; r++)
    for (int j = 0; j < k; j++) {
      int e = (int)exps[(size_t)r * nb + j / 8] - 127;
      w[(size_t)r * k + j] = ldexpf((float)mant[(size_t)r * k + j], e - 6);
    }
}

/* gemm_bfp16 (golden_ffn_gemm.py:56-60) with the activation kept fp32 (the
 * decode path's x is not block-quantised): decoded weight, fp32 accumulate in
 * k order, bias after.  Parity: tolerance. */
void xo_gemv_bfp16(const float *x, int b, int k, int m, const int8_t *mant,
                   const uint8_t *exps, const float *bias, float *y) {
  int nb = k / 8;
  for (int bi = 0; bi < b; bi++) {
    const float *xb = x + (size_t)bi * k;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < m; r++) {
      float acc = 0.f;
      for (int j = 0; j < k; j++) {
        int e = (int)exps[(size_t)r * nb + j / 8] - 127;
        acc += xb[j] * ldexpf((float)mant[(size_t)r * k + j], e - 6);
      }
      y[(size_t)bi * m + r] = bias ? acc + bias[r] : acc;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* W8A8                                                                     */
/* ------------------------------------------------------------------------ */

/* int8 x int8 -> int32 (the device part of forward_view_int8,
 * ctx2.rs:771-830): acc[p, r] = sum_k a[p,k] * w[r,k].  Exact integers.
 * Pins: brute-force identity with int64 accumulation on small shapes. */
void xo_gemm_i8i8_i32(const int8_t *a, int mp, int k, const int8_t *w, int m,
                      int32_t *acc) {
  for (int p = 0; p < mp; p++)
    for (int r = 0; r < m; r++) {
      int32_t s = 0;
      for (int j = 0; j < k; j++) s += (int32_t)a[(size_t)p * k + j] * (int32_t)w[(size_t)r * k + j];
      acc[(size_t)p * m + r] = s;
    }
}

/* forward_view_int8 (ctx2.rs:771-830): scale_a = quant_scale(A) per tensor,
 * A_i8 = quant_i8(A, scale_a), i32 GEMM, dequant_epi(Bias). */
void xo_w8a8_linear(const float *a, int mp, int k, const int8_t *wq,
                    const float *ws, int m, const float *bias, float *out,
                    float *scale_a_out) {
  xo_w8a8_linear_epi(a, mp, k, wq, ws, m, bias, bias ? XO_EPI_BIAS : XO_EPI_NONE, out,
                     scale_a_out);
}

/* fast_sigmoid (ctx2.rs:1338-1348): stable sigmoid on fast_exp_nonpos. */
float xo_fast_sigmoid(float x) {
  if (x >= 0.0f) return 1.0f / (1.0f + xo_fast_exp_nonpos(-x));
  float e = xo_fast_exp_nonpos(x);
  return e / (1.0f + e);
}

/* forward_view_int8 with the op's epilogue (dequant_epi, ctx2.rs:1386-1435):
 * v = (acc as f32 * scale_a) * ws[c]; Epi::None -> v; Epi::Bias -> v + b[c];
 * Epi::SiluBias -> z = v + b[c], z * fast_sigmoid(z). */
void xo_w8a8_linear_epi(const float *a, int mp, int k, const int8_t *wq,
                        const float *ws, int m, const float *bias, int epi, float *out,
                        float *scale_a_out) {
  float scale_a = xo_quant_scale(a, (size_t)mp * k);
  int8_t *aq = (int8_t *)malloc((size_t)mp * k);
  int32_t *acc = (int32_t *)malloc((size_t)mp * m * 4);
  for (size_t i = 0; i < (size_t)mp * k; i++) aq[i] = xo_quant_i8(a[i], scale_a);
  xo_gemm_i8i8_i32(aq, mp, k, wq, m, acc);
  for (int r = 0; r < mp; r++)
    for (int c = 0; c < m; c++) {
      float v = (float)acc[(size_t)r * m + c] * scale_a * ws[c];
      if (epi == XO_EPI_BIAS) {
        v = v + bias[c];
      } else if (epi == XO_EPI_SILU_BIAS) {
        float z = v + bias[c];
        v = z * xo_fast_sigmoid(z);
      }
      out[(size_t)r * m + c] = v;
    }
  if (scale_a_out) *scale_a_out = scale_a;
  free(aq);
  free(acc);
}

/* ------------------------------------------------------------------------ */
/* fused norm + GEMV                                                        */
/* ------------------------------------------------------------------------ */

/* The norm half of fused_norm_gemv (ctx_decode.rs:617-643), applied to x
 * before the projection; the reference folds gamma into W (register_fused,
 * :566-612) which is the same linear map (fold identity pinned by
 * xo_fold_weight vs norm_gemv_probe.rs:76-94).  Stats follow the host norm
 * (layer_norm lib.rs:79-109 / rmsnorm_ref) in f32. */
void xo_norm_row(const float *x, int k, int norm, const float *gamma,
                 const float *beta, float eps, float *out) {
  if (norm == XO_NORM_NONE) {
    memcpy(out, x, (size_t)k * 4);
  } else if (norm == XO_NORM_LN) {
    xo_layer_norm(x, 1, k, gamma, beta, eps, out);
  } else if (norm == XO_NORM_RMS1P) {
    xo_rmsnorm(x, k, gamma, eps, out);
  } else { /* plain RMS: x * inv * gamma */
    float ms = 0.f;
    for (int i = 0; i < k; i++) ms += x[i] * x[i];
    ms = ms / (float)k;
    float inv = 1.0f / sqrtf(ms + eps);
    for (int i = 0; i < k; i++) out[i] = x[i] * inv * gamma[i];
  }
}

/* register_fused fold (ctx_decode.rs:566-612) for an [M,K] weight:
 * W''[r,k] = gamma[k] W[r,k]; bias'[r] = sum_k beta[k] W[r,k] + bias[r]
 * (beta NULL -> RMS: bias' = bias). */
void xo_fold_weight(const float *w, int m, int k, const float *gamma,
                    const float *beta, const float *bias, float *w_fold,
                    float *bias_fold) {
  for (int r = 0; r < m; r++) {
    float s = 0.f;
    for (int j = 0; j < k; j++) {
      w_fold[(size_t)r * k + j] = gamma[j] * w[(size_t)r * k + j];
      if (beta) s += beta[j] * w[(size_t)r * k + j];
    }
    bias_fold[r] = s + (bias ? bias[r] : 0.0f);
  }
}

/* ------------------------------------------------------------------------ */
/* attention                                                                */
/* ------------------------------------------------------------------------ */

/* attend_one (whisper_decoder.rs:242-278): q [H*hd], K/V [s, H*hd] f32;
 * scores = (q.k) * (1/sqrt hd); 3-pass softmax (max, exp/sum, * 1/sum);
 * ctx += p * v.  Pins: test_mha_no_round vectors (npu-asr-host/src/lib.rs:
 * 990-1001, unmasked mha rows are attend_one per query), s = 1 -> ctx = v,
 * identical keys -> ctx = mean of values. */
void xo_attend_one(const float *q, const float *k_flat, const float *v_flat,
                   int s, int n_heads, int head_dim, float *ctx) {
  int d = n_heads * head_dim;
  float scale = 1.0f / sqrtf((float)head_dim);
  float *scores = (float *)malloc((size_t)s * 4);
  for (int i = 0; i < d; i++) ctx[i] = 0.f;
  for (int h = 0; h < n_heads; h++) {
    int base = h * head_dim;
    for (int j = 0; j < s; j++) {
      const float *krow = k_flat + (size_t)j * d + base;
      float dot = 0.f;
      for (int t = 0; t < head_dim; t++) dot += q[base + t] * krow[t];
      scores[j] = dot * scale;
    }
    float maxv = -INFINITY;
    for (int j = 0; j < s; j++) maxv = fmaxf(maxv, scores[j]);
    float sum = 0.f;
    for (int j = 0; j < s; j++) {
      scores[j] = expf(scores[j] - maxv);
      sum += scores[j];
    }
    float inv = 1.0f / sum;
    for (int j = 0; j < s; j++) {
      float p = scores[j] * inv;
      const float *vrow = v_flat + (size_t)j * d + base;
      for (int t = 0; t < head_dim; t++) ctx[base + t] += p * vrow[t];
    }
  }
  free(scores);
}

/* attend_one generalised to the build's cache: bf16 K/V [b, hkv, max_ctx,
 * hd], GQA (query head h reads kv head h / (hq/hkv)), per-stream lengths and
 * a given scale.  Same 3-pass arithmetic as attend_one. */
void xo_attn_decode(const float *q, const uint16_t *kc, const uint16_t *vc,
                    const int *lens, int batch, int hq, int hkv, int hd,
                    int max_ctx, float scale, float *out) {
  int group = hq / hkv;
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < batch; b++)
    for (int h = 0; h < hq; h++) {
      int len = lens[b];
      int kvh = h / group;
      const float *qh = q + ((size_t)b * hq + h) * hd;
      const uint16_t *kh = kc + ((size_t)b * hkv + kvh) * (size_t)max_ctx * hd;
      const uint16_t *vh = vc + ((size_t)b * hkv + kvh) * (size_t)max_ctx * hd;
      float *o = out + ((size_t)b * hq + h) * hd;
      float *sc = (float *)malloc((size_t)len * 4);
      for (int j = 0; j < len; j++) {
        float dot = 0.f;
        for (int t = 0; t < hd; t++) dot += qh[t] * xo_bf16_bits_to_f32(kh[(size_t)j * hd + t]);
        sc[j] = dot * scale;
      }
      float maxv = -INFINITY;
      for (int j = 0; j < len; j++) maxv = fmaxf(maxv, sc[j]);
      float sum = 0.f;
      for (int j = 0; j < len; j++) {
        sc[j] = expf(sc[j] - maxv);
        sum += sc[j];
      }
      float inv = 1.0f / sum;
      for (int t = 0; t < hd; t++) o[t] = 0.f;
      for (int j = 0; j < len; j++) {
        float p = sc[j] * inv;
        for (int t = 0; t < hd; t++) o[t] += p * xo_bf16_bits_to_f32(vh[(size_t)j * hd + t]);
      }
      free(sc);
    }
}

/* mha_tile online softmax (mha_decode.cc:126-165) for one head: per key
 * m_new = max(m, s); corr = exp(m - m_new); p = exp(s - m_new);
 * l = l*corr + p; acc = acc*corr + p*v; finalize acc / l.  exp in f32 (the
 * AIE's bf16 exp2 is a datapath limit, mha_decode.cc:83-88).  Pins: agrees
 * with the 3-pass attend_one within 1e-5 relative (same mathematics). */
void xo_attn_online(const float *q, const uint16_t *kc, const uint16_t *vc,
                    int len, int hd, float scale, float *out) {
  float m = -3.0e38f, l = 0.f;
  float *acc = (float *)calloc((size_t)hd, 4);
  for (int s = 0; s < len; s++) {
    float dot = 0.f;
    for (int t = 0; t < hd; t++) dot += q[t] * xo_bf16_bits_to_f32(kc[(size_t)s * hd + t]);
    float score = dot * scale;
    float m_new = score > m ? score : m;
    float corr = expf(m - m_new);
    float p = expf(score - m_new);
    l = l * corr + p;
    m = m_new;
    for (int t = 0; t < hd; t++)
      acc[t] = acc[t] * corr + p * xo_bf16_bits_to_f32(vc[(size_t)s * hd + t]);
  }
  float inv = 1.0f / l;
  for (int t = 0; t < hd; t++) out[t] = acc[t] * inv;
  free(acc);
}

/* rope (npu-asr-host/src/lib.rs:143-185): per head, rotate_half pairing
 * out[d] = x[d]*cos[d] + rot[d]*sin[d], rot[d] = -x[d+half] (d < half) else
 * x[d-half]; cos/sin are [rows, head_dim].  Pins: test_rope expected vectors
 * (npu-asr-host/src/lib.rs:913-948). */
void xo_rope(const float *x, int rows, int n_heads, int head_dim,
             const float *cos_t, const float *sin_t, float *out) {
  int d = n_heads * head_dim, half = head_dim / 2;
  for (int t = 0; t < rows; t++) {
    const float *ir = x + (size_t)t * d;
    const float *cr = cos_t + (size_t)t * head_dim;
    const float *sr = sin_t + (size_t)t * head_dim;
    float *orow = out + (size_t)t * d;
    for (int h = 0; h < n_heads; h++) {
      int base = h * head_dim;
      for (int j = 0; j < head_dim; j++) {
        float xr = ir[base + j];
        float rot = j < half ? -ir[base + j + half] : ir[base + j - half];
        orow[base + j] = xr * cr[j] + rot * sr[j];
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* argmax                                                                   */
/* ------------------------------------------------------------------------ */

/* whisper.rs:749-757 and argmax_slice.cc:19-24: strict >, first max wins. */
int xo_argmax_first(const float *v, int n) {
  int best = 0;
  for (int i = 1; i < n; i++)
    if (v[i] > v[best]) best = i;
  return best;
}

/* opt125m_decode.rs:303: Iterator::max_by(partial_cmp) returns the LAST of
 * equal maxima. */
int xo_argmax_last(const float *v, int n) {
  int best = 0;
  for (int i = 1; i < n; i++)
    if (v[i] >= v[best]) best = i;
  return best;
}

/* ------------------------------------------------------------------------ */
/* synthetic weights                                                        */
/* ------------------------------------------------------------------------ */
/* Counter-based generator (no reference counterpart: the reference loads real
 * weights; BASELINE fixes seeded random init).  Element idx of tensor id
 * under seed: h = mix64(base + idx), base = mix64(seed * C1 + id); the four
 * 16-bit fields of h are summed (Irwin-Hall n = 4, an approximately normal
 * integer with variance (65536^2 - 1)/3) and scaled:
 *   value = mean + (float)(sum - 131070) * (stdv * XO_IH4_INV_STD)
 * Integer work is exact and the float ops are single correctly rounded
 * operations, so the GPU generator reproduces every bit.  The reference's
 * mha probe uses the same sum-of-uniforms idea (mha_decode_probe.rs:119-124).
 */
#define XO_IH4_INV_STD 2.6428997e-05f /* 1 / sqrt((65536^2 - 1) / 3) */

static inline uint64_t xo_mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t xo_synth_base(uint64_t seed, uint32_t tensor) {
  return xo_mix64(seed * 0xD1B54A32D192ED03ull + (uint64_t)tensor);
}

float xo_synth_value(uint64_t base, uint64_t idx, float mean, float stdv) {
  uint64_t h = xo_mix64(base + idx);
  int32_t sum = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) +
                (int32_t)((h >> 32) & 0xffff) + (int32_t)(h >> 48);
  float k = stdv * XO_IH4_INV_STD;
  float v = (float)(sum - 131070) * k;
  return v + mean;
}

/* Elements [start, start + n) of a synthetic stream (the product's
 * xe_buf_fill_synthetic, before its storage rounding). */
void xo_synth_fill_range(uint64_t seed, uint32_t tensor, float mean, float stdv,
                         uint64_t start, float *out, size_t n) {
  uint64_t base = xo_synth_base(seed, tensor);
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; i++) out[i] = xo_synth_value(base, start + i, mean, stdv);
}

void xo_synth_fill(uint64_t seed, uint32_t tensor, float mean, float stdv,
                   float *out, size_t n) {
  uint64_t base = xo_synth_base(seed, tensor);
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; i++) out[i] = xo_synth_value(base, i, mean, stdv);
}

/* ------------------------------------------------------------------------ */
/* decoder models                                                           */
/* ------------------------------------------------------------------------ */

typedef struct {
  int present;
  int rows, cols;   /* matrices: [rows=out, cols=in]; vectors: rows = 1 */
  int quant;        /* stored in the model's wdtype (linears + embedding) */
  float mean, stdv;
  float *f32;       /* unquantised tensors */
  int8_t *q;        /* XE_I8 */
  int8_t *qb;       /* XE_I8 copy in blocks of 8 rows, k-major (xo_block8_i8) */
  int8_t *qkn;      /* XE_I8 copy in the reference's [K, N] layout (k-outer mode) */
  float *s;
  uint16_t *bf;     /* XE_BF16 */
  int8_t *mant;     /* XE_BFP16 */
  uint8_t *exps;
} xo_tensor;

struct xo_model {
  xe_model_config c;
  uint64_t seed;
  int batch;
  xo_tensor t[XE_T_COUNT][65]; /* [kind][layer + 1] (index 0 = global) */
  uint16_t *kc, *vc;           /* [L][batch][hkv][max_ctx][hd] bf16 */
  uint16_t *xk, *xv;           /* Whisper cross K/V [L][h][n_cross][hd] */
  float *rope_cos, *rope_sin;  /* [max_ctx][hd/2] */
  /* fp32 K/V caches (self and cross), used instead of the bf16 ones when
   * kv_f32 is set: the reference CPU paths keep their caches in f32
   * (opt125m_decode.rs:263-268, whisper_decoder.rs:458, 472). */
  int kv_f32;
  float *kcf, *vcf, *xkf, *xvf;
  /* int8 cross K/V [L][h][n_cross][hd] + channel scales [L][h * hd] */
  int cross_i8k, cross_i8v;
  int8_t *xk8, *xv8;
  float *xks, *xvs;
  int mutation; /* XO_MUT_*: a planted composition mistake (tests only) */
  int kouter;   /* int8 linears through the reference's k-outer [K, N] loop */
};

/* Shape + init law of every tensor a family has.  Linear weights, biases and
 * embeddings ~ N(0, 0.02) (BASELINE configs 1/4/5).  LayerNorm gammas are
 * 1 + N(0, 0.02); Gemma's (1 + w) norms store w ~ N(0, 0.02).  Whisper has
 * no k_proj bias (HF WhisperAttention k_proj bias=False). */
static int xo_tensor_spec(const xe_model_config *c, int kind, int layer, int *rows,
                          int *cols, int *quant, float *mean, float *stdv) {
  int D = c->d_model, hq = c->n_heads * c->head_dim, hk = c->n_kv_heads * c->head_dim;
  int F = c->ffn, fam = c->family;
  int gem = fam == XE_GEMMA3, wh = fam == XE_WHISPER, opt = fam == XE_OPT;
  int R = 0, C = 0, Q = 0;
  float mu = 0.f, sd = 0.02f;
  if (layer < 0) {
    switch (kind) {
      case XE_T_TOK_EMB: R = c->vocab; C = D; Q = 1; break;
      case XE_T_POS_EMB:
        if (gem) return 0;
        R = opt ? c->max_pos + 2 : c->max_pos; C = D; break;
      case XE_T_LNF_W: R = 1; C = D; mu = gem ? 0.f : 1.f; break;
      case XE_T_LNF_B: if (gem) return 0; R = 1; C = D; break;
      case XE_T_ENC_OUT: if (!wh) return 0; R = c->n_cross; C = D; sd = 1.0f; break;
      default: return 0;
    }
  } else {
    switch (kind) {
      case XE_T_LN1_W: case XE_T_LN2_W: R = 1; C = D; mu = gem ? 0.f : 1.f; break;
      case XE_T_LN1_B: case XE_T_LN2_B: if (gem) return 0; R = 1; C = D; break;
      case XE_T_Q_W: R = hq; C = D; Q = 1; break;
      case XE_T_K_W: case XE_T_V_W: R = hk; C = D; Q = 1; break;
      case XE_T_Q_B: if (gem) return 0; R = 1; C = hq; break;
      case XE_T_K_B: if (!opt) return 0; R = 1; C = hk; break;
      case XE_T_V_B: if (gem) return 0; R = 1; C = hk; break;
      case XE_T_O_W: R = D; C = hq; Q = 1; break;
      case XE_T_O_B: if (gem) return 0; R = 1; C = D; break;
      case XE_T_FC1_W: R = F; C = D; Q = 1; break;
      case XE_T_FC1_B: if (gem) return 0; R = 1; C = F; break;
      case XE_T_UP_W: if (!gem) return 0; R = F; C = D; Q = 1; break;
      case XE_T_FC2_W: R = D; C = F; Q = 1; break;
      case XE_T_FC2_B: if (gem) return 0; R = 1; C = D; break;
      case XE_T_QNORM_W: case XE_T_KNORM_W:
        if (!gem) return 0;
        R = 1; C = c->head_dim; break;
      case XE_T_POST_ATTN_W: case XE_T_POST_FFN_W: if (!gem) return 0; R = 1; C = D; break;
      case XE_T_LNX_W: if (!wh) return 0; R = 1; C = D; mu = 1.f; break;
      case XE_T_LNX_B: case XE_T_XQ_B: case XE_T_XV_B: case XE_T_XO_B:
        if (!wh) return 0;
        R = 1; C = D; break;
      case XE_T_XQ_W: case XE_T_XK_W: case XE_T_XV_W: case XE_T_XO_W:
        if (!wh) return 0;
        R = D; C = D; Q = 1; break;
      default: return 0;
    }
  }
  *rows = R; *cols = C; *quant = Q; *mean = mu; *stdv = sd;
  return 1;
}

static void xo_tensor_build(xo_model *m, int kind, int layer) {
  xo_tensor *t = &m->t[kind][layer + 1];
  int R, C, Q;
  float mu, sd;
  if (!xo_tensor_spec(&m->c, kind, layer, &R, &C, &Q, &mu, &sd)) return;
  t->present = 1; t->rows = R; t->cols = C; t->quant = Q; t->mean = mu; t->stdv = sd;
  size_t n = (size_t)R * C;
  float *w = (float *)malloc(n * 4);
  xo_synth_fill(m->seed, XE_SYNTH_ID(kind, layer), mu, sd, w, n);
  if (!Q) { t->f32 = w; return; }
  if (m->c.wdtype == XE_I8) {
    t->q = (int8_t *)malloc(n);
    t->s = (float *)malloc((size_t)R * 4);
    xo_quant_rows_i8(w, R, C, t->q, t->s);
    t->qb = xo_block8_i8(t->q, R, C);
  } else if (m->c.wdtype == XE_BF16) {
    t->bf = (uint16_t *)malloc(n * 2);
    xo_pack_bf16(w, t->bf, n);
  } else {
    t->mant = (int8_t *)malloc(n);
    t->exps = (uint8_t *)malloc(n / 8);
    xo_bfp16_encode(w, R, C, t->mant, t->exps);
  }
  free(w);
}

static void xo_rope_table(xo_model *m) {
  int hd = m->c.head_dim, half = hd / 2, T = m->c.max_ctx;
  m->rope_cos = (float *)malloc((size_t)T * hd * 4);
  m->rope_sin = (float *)malloc((size_t)T * hd * 4);
  /* HF rotary embedding: inv_freq = 1 / theta^(2i/d) in f32; angle =
   * pos * inv_freq in f32; cos/sin in f32, duplicated over both halves
   * (emb = cat(freqs, freqs)). */
  for (int p = 0; p < T; p++)
    for (int i = 0; i < half; i++) {
      float e = (float)(2 * i) / (float)hd;
      float theta = m->mutation == XO_MUT_ROPE_THETA ? 10000.0f : m->c.rope_theta;
      float inv = 1.0f / powf(theta, e);
      float ang = (float)p * inv;
      float cv = cosf(ang), sv = sinf(ang);
      m->rope_cos[(size_t)p * hd + i] = cv;
      m->rope_cos[(size_t)p * hd + i + half] = cv;
      m->rope_sin[(size_t)p * hd + i] = sv;
      m->rope_sin[(size_t)p * hd + i + half] = sv;
    }
}

xo_model *xo_model_create(const xe_model_config *cfg, uint64_t seed, int batch) {
  xo_model *m = (xo_model *)calloc(1, sizeof(xo_model));
  m->c = *cfg;
  m->seed = seed;
  m->batch = batch;
  if (cfg->n_layers > 64) { free(m); return NULL; }
  for (int kind = 0; kind < XE_T_COUNT; kind++) {
    xo_tensor_build(m, kind, -1);
    for (int l = 0; l < cfg->n_layers; l++) xo_tensor_build(m, kind, l);
  }
  size_t kv = (size_t)cfg->n_layers * batch * cfg->n_kv_heads * cfg->max_ctx * cfg->head_dim;
  m->kc = (uint16_t *)calloc(kv, 2);
  m->vc = (uint16_t *)calloc(kv, 2);
  if (cfg->family == XE_GEMMA3) xo_rope_table(m);
  return m;
}

void xo_model_free(xo_model *m) {
  if (!m) return;
  for (int k = 0; k < XE_T_COUNT; k++)
    for (int l = 0; l < 65; l++) {
      xo_tensor *t = &m->t[k][l];
      free(t->f32); free(t->q); free(t->qb); free(t->qkn); free(t->s); free(t->bf); free(t->mant); free(t->exps);
    }
  free(m->kc); free(m->vc); free(m->xk); free(m->xv);
  free(m->kcf); free(m->vcf); free(m->xkf); free(m->xvf);
  free(m->xk8); free(m->xv8); free(m->xks); free(m->xvs);
  free(m->rope_cos); free(m->rope_sin);
  free(m);
}

void xo_model_reset(xo_model *m) {
  size_t kv = (size_t)m->c.n_layers * m->batch * m->c.n_kv_heads * m->c.max_ctx * m->c.head_dim;
  memset(m->kc, 0, kv * 2);
  memset(m->vc, 0, kv * 2);
  if (m->kcf) {
    memset(m->kcf, 0, kv * 4);
    memset(m->vcf, 0, kv * 4);
  }
}

/* Keep the K/V caches (self and, after the next set_cross, cross) in fp32
 * instead of rounding them to bf16: the reference CPU decoders' own choice
 * (opt125m_decode.rs:263-268, whisper_decoder.rs:458, 472).  The product
 * rounds K/V to bf16, so the bf16 caches are the
 * default; the fp32 mode exists to compare the oracle's decoder composition
 * with independent fp32 implementations.  Clears the caches. */
int xo_model_set_kv_f32(xo_model *m, int on) {
  size_t kv = (size_t)m->c.n_layers * m->batch * m->c.n_kv_heads * m->c.max_ctx * m->c.head_dim;
  free(m->kcf); free(m->vcf); free(m->xkf); free(m->xvf);
  m->kcf = m->vcf = m->xkf = m->xvf = NULL;
  m->kv_f32 = on ? 1 : 0;
  if (on) {
    m->kcf = (float *)calloc(kv, 4);
    m->vcf = (float *)calloc(kv, 4);
    if (!m->kcf || !m->vcf) return -1;
  }
  xo_model_reset(m);
  return 0;
}

static const xo_tensor *T(const xo_model *m, int kind, int layer) {
  const xo_tensor *t = &m->t[kind][layer + 1];
  return t->present ? t : NULL;
}

/* y[rows] = W x (+ bias) for a stored linear (one stream). */
static void xo_lin(const xo_model *m, int kind, int layer, int bias_kind,
                   const float *x, float *y) {
  const xo_tensor *w = T(m, kind, layer);
  const xo_tensor *b = bias_kind >= 0 ? T(m, bias_kind, layer) : NULL;
  const float *bias = b ? b->f32 : NULL;
  if (m->c.wdtype == XE_I8 && m->kouter)
    xo_lin_fwd_i8_kn(x, 1, w->cols, w->rows, w->qkn, w->s, bias, y);
  else if (m->c.wdtype == XE_I8)
    xo_gemv_i8_blocked(x, w->cols, w->rows, w->qb, w->s, bias, y);
  else if (m->c.wdtype == XE_BF16)
    xo_gemv_bf16w(x, 1, w->cols, w->rows, w->bf, bias, y);
  else
    xo_gemv_bfp16(x, 1, w->cols, w->rows, w->mant, w->exps, bias, y);
}

/* Embedding row (tied table) dequantised to f32. */
static void xo_embed_row(const xo_model *m, int tok, float *x) {
  const xo_tensor *e = T(m, XE_T_TOK_EMB, -1);
  int D = e->cols;
  for (int d = 0; d < D; d++) {
    size_t i = (size_t)tok * D + d;
    if (m->c.wdtype == XE_I8)
      x[d] = (float)e->q[i] * e->s[tok];
    else if (m->c.wdtype == XE_BF16)
      x[d] = xo_bf16_bits_to_f32(e->bf[i]);
    else
      x[d] = ldexpf((float)e->mant[i], (int)e->exps[i / 8] - 127 - 6);
  }
}

/* Plant one composition mistake (XO_MUT_*; 0 restores the faithful step).
 * Test infrastructure: the HF cross-check fixtures must catch every one of
 * them, which shows the fixtures pin the composition. */
int xo_model_set_mutation(xo_model *m, int code) {
  m->mutation = code;
  if (m->c.family == XE_GEMMA3) {
    free(m->rope_cos);
    free(m->rope_sin);
    xo_rope_table(m);
  }
  return 0;
}

/* int8 linears through the reference's own loop shape: W in [K, N], k
 * outer, one f32 accumulator per output updated in k order
 * (opt125m_decode.rs:106-125, xo_lin_fwd_i8_kn) -- the same values as the
 * default row-blocked form, with the reference's memory traffic.  For the
 * reference-shaped CPU timing. */
int xo_model_set_kouter(xo_model *m, int on) {
  m->kouter = 0;
  if (!on) return 0;
  if (m->c.wdtype != XE_I8) return -1;
  for (int kind = 0; kind < XE_T_COUNT; kind++)
    for (int l = 0; l < 65; l++) {
      xo_tensor *t = &m->t[kind][l];
      if (!t->present || !t->q || t->qkn) continue;
      t->qkn = (int8_t *)malloc((size_t)t->rows * t->cols);
      if (!t->qkn) return -1;
#pragma omp parallel for schedule(static)
      for (int r = 0; r < t->rows; r++)
        for (int c = 0; c < t->cols; c++) t->qkn[(size_t)c * t->rows + r] = t->q[(size_t)r * t->cols + c];
    }
  m->kouter = 1;
  return 0;
}

/* Fill stream b's K/V rows [0, n_pos) of every layer with synthetic bf16
 * values (N(0,1) from the counter generator): a cache of a given length
 * without feeding a prompt, for timing steps at long contexts. */
int xo_model_prime_kv(xo_model *m, int b, int n_pos, uint64_t seed) {
  if (b < 0 || b >= m->batch || n_pos < 0 || n_pos > m->c.max_ctx) return -1;
  int Hk = m->c.n_kv_heads, hd = m->c.head_dim, MC = m->c.max_ctx;
  for (int l = 0; l < m->c.n_layers; l++)
    for (int h = 0; h < Hk; h++) {
      size_t base = ((((size_t)l * m->batch + b) * Hk + h) * MC) * hd;
      uint64_t kb = xo_synth_base(seed, (uint32_t)(2 * (l * Hk + h)));
      uint64_t vb = xo_synth_base(seed, (uint32_t)(2 * (l * Hk + h) + 1));
#pragma omp parallel for schedule(static)
      for (size_t i = 0; i < (size_t)n_pos * hd; i++) {
        float kv = xo_synth_value(kb, i, 0.0f, 1.0f), vv = xo_synth_value(vb, i, 0.0f, 1.0f);
        if (m->kv_f32) {
          m->kcf[base + i] = xo_bf16_round(kv);
          m->vcf[base + i] = xo_bf16_round(vv);
        } else {
          m->kc[base + i] = xo_f32_to_bf16_bits(kv);
          m->vc[base + i] = xo_f32_to_bf16_bits(vv);
        }
      }
    }
  return 0;
}

void xo_quant_cross_i8(const float *x, int T, int H, int hd, int8_t *q, float *s) {
  int D = H * hd;
  for (int c = 0; c < D; c++) s[c] = 0.0f;
  for (int t = 0; t < T; t++)
    for (int c = 0; c < D; c++) {
      float a = fabsf(x[(size_t)t * D + c]);
      if (a > s[c]) s[c] = a;
    }
  /* headroom 1.0 (the default of INT8_CK_HEADROOM / INT8_CV_HEADROOM) */
  for (int c = 0; c < D; c++) s[c] = s[c] > 0.0f ? s[c] * 1.0f / 127.0f : 1.0f;
  for (int t = 0; t < T; t++)
    for (int h = 0; h < H; h++)
      for (int d = 0; d < hd; d++) {
        int c = h * hd + d;
        float inv = s[c] != 0.0f ? 1.0f / s[c] : 0.0f;
        float r = roundf(x[(size_t)t * D + c] * inv); /* Rust round(): half away from zero */
        r = r != r ? 0.0f : r < -127.0f ? -127.0f : r > 127.0f ? 127.0f : r; /* NaN -> 0 (`as i8`) */
        q[((size_t)h * T + t) * hd + d] = (int8_t)r;
      }
}

int xo_model_set_cross_i8(xo_model *m, int k_int8, int v_int8) {
  if (m->c.family != XE_WHISPER) return -1;
  m->cross_i8k = k_int8 ? 1 : 0;
  m->cross_i8v = v_int8 ? 1 : 0;
  return 0;
}

int xo_model_set_cross(xo_model *m, const float *enc) {
  if (m->c.family != XE_WHISPER) return -1;
  int Tn = m->c.n_cross, D = m->c.d_model, H = m->c.n_heads, hd = m->c.head_dim, L = m->c.n_layers;
  const float *src = enc ? enc : T(m, XE_T_ENC_OUT, -1)->f32;
  float *e = (float *)malloc((size_t)Tn * D * 4);
  for (size_t i = 0; i < (size_t)Tn * D; i++) e[i] = xo_bf16_round(src[i]);
  free(m->xk); free(m->xv); free(m->xkf); free(m->xvf);
  m->xkf = m->xvf = NULL;
  m->xk = (uint16_t *)malloc((size_t)L * Tn * D * 2);
  m->xv = (uint16_t *)malloc((size_t)L * Tn * D * 2);
  if (m->kv_f32) {
    m->xkf = (float *)malloc((size_t)L * Tn * D * 4);
    m->xvf = (float *)malloc((size_t)L * Tn * D * 4);
  }
  /* precompute_cross (whisper_decoder.rs:1143-1232 / host path :388-397):
   * K = enc . cross_k (no bias), V = enc . cross_v + b, stored bf16 in the
   * head-major [h][t][hd] layout of the fused path (:1167-1186). */
  for (int l = 0; l < L; l++) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < Tn; t++) {
      float kr[4096], vr[4096];
      xo_lin(m, XE_T_XK_W, l, -1, e + (size_t)t * D, kr);
      xo_lin(m, XE_T_XV_W, l, XE_T_XV_B, e + (size_t)t * D, vr);
      for (int h = 0; h < H; h++)
        for (int j = 0; j < hd; j++) {
          size_t o = (((size_t)l * H + h) * Tn + t) * hd + j;
          m->xk[o] = xo_f32_to_bf16_bits(kr[h * hd + j]);
          if (m->xkf) {
            m->xkf[o] = kr[h * hd + j];
            m->xvf[o] = vr[h * hd + j];
          }
          m->xv[o] = xo_f32_to_bf16_bits(vr[h * hd + j]);
        }
    }
  }
  /* per-utterance int8 (whisper_decoder.rs:1186-1219): from the fp32
   * projections, not from the bf16 copies */
  free(m->xk8); free(m->xv8); free(m->xks); free(m->xvs);
  m->xk8 = m->xv8 = NULL;
  m->xks = m->xvs = NULL;
  if (m->cross_i8k || m->cross_i8v) {
    float *kf = (float *)malloc((size_t)Tn * D * 4), *vf = (float *)malloc((size_t)Tn * D * 4);
    if (m->cross_i8k) {
      m->xk8 = (int8_t *)malloc((size_t)L * Tn * D);
      m->xks = (float *)malloc((size_t)L * D * 4);
    }
    if (m->cross_i8v) {
      m->xv8 = (int8_t *)malloc((size_t)L * Tn * D);
      m->xvs = (float *)malloc((size_t)L * D * 4);
    }
    for (int l = 0; l < L; l++) {
#pragma omp parallel for schedule(static)
      for (int t = 0; t < Tn; t++) {
        xo_lin(m, XE_T_XK_W, l, -1, e + (size_t)t * D, kf + (size_t)t * D);
        xo_lin(m, XE_T_XV_W, l, XE_T_XV_B, e + (size_t)t * D, vf + (size_t)t * D);
      }
      if (m->xk8) xo_quant_cross_i8(kf, Tn, H, hd, m->xk8 + (size_t)l * Tn * D, m->xks + (size_t)l * D);
      if (m->xv8) xo_quant_cross_i8(vf, Tn, H, hd, m->xv8 + (size_t)l * Tn * D, m->xvs + (size_t)l * D);
    }
    free(kf);
    free(vf);
  }
  free(e);
  return 0;
}

void xo_head_attend_x8(const float *qh, const int8_t *k8, const float *sk, const uint16_t *kb,
                       const int8_t *v8, const float *sv, const uint16_t *vb, int len, int hd,
                       float scale, float *sc, float *oh) {
  float qs[1024];
  for (int d = 0; d < hd; d++) qs[d] = k8 ? qh[d] * sk[d] : qh[d];
  for (int j = 0; j < len; j++) {
    float dot = 0.f;
    for (int d = 0; d < hd; d++)
      dot += qs[d] * (k8 ? (float)k8[(size_t)j * hd + d] : xo_bf16_bits_to_f32(kb[(size_t)j * hd + d]));
    sc[j] = dot * scale;
  }
  float mx = -INFINITY;
  for (int j = 0; j < len; j++) mx = fmaxf(mx, sc[j]);
  float sum = 0.f;
  for (int j = 0; j < len; j++) {
    sc[j] = expf(sc[j] - mx);
    sum += sc[j];
  }
  float inv = 1.0f / sum;
  for (int j = 0; j < len; j++) sc[j] = sc[j] * inv;
  for (int d = 0; d < hd; d++) {
    float acc = 0.f;
    for (int j = 0; j < len; j++)
      acc += sc[j] * (v8 ? (float)v8[(size_t)j * hd + d] : xo_bf16_bits_to_f32(vb[(size_t)j * hd + d]));
    oh[d] = v8 ? acc * sv[d] : acc;
  }
}

static void xo_rope_apply(const xo_model *m, float *v, int pos) {
  int hd = m->c.head_dim;
  float tmp[1024];
  xo_rope(v, 1, 1, hd, m->rope_cos + (size_t)pos * hd, m->rope_sin + (size_t)pos * hd, tmp);
  memcpy(v, tmp, (size_t)hd * 4);
}

/* Scores of keys [j0, min(j0 + 8, len)): sc[j] = (sum over t = 0..hd-1 in
 * order of q[t] * k[j][t]) * scale, each key its own sequential f32 sum.
 * The AVX2 form runs the eight keys in the eight lanes (gathering k[j][t]
 * across keys), which leaves every key's arithmetic the scalar loop's. */
static void xo_scores8_scalar(const float *qh, const uint16_t *kb, const float *kf, int j0,
                              int len, int hd, float scale, float *sc) {
  for (int j = j0; j < len && j < j0 + 8; j++) {
    float dot = 0.f;
    if (kf)
      for (int t = 0; t < hd; t++) dot += qh[t] * kf[(size_t)j * hd + t];
    else
      for (int t = 0; t < hd; t++) dot += qh[t] * xo_bf16_bits_to_f32(kb[(size_t)j * hd + t]);
    sc[j] = dot * scale;
  }
}

#if defined(__x86_64__)
__attribute__((target("avx2")))
static void xo_scores8_avx2(const float *qh, const uint16_t *kb, const float *kf, int j0,
                            int hd, float scale, float *sc) {
  __m256 acc = _mm256_setzero_ps();
  if (kf) {
    const __m256i idx = _mm256_mullo_epi32(_mm256_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7),
                                           _mm256_set1_epi32(hd));
    const float *base = kf + (size_t)j0 * hd;
    for (int t = 0; t < hd; t++) {
      __m256 kv = _mm256_i32gather_ps(base + t, idx, 4);
      acc = _mm256_add_ps(acc, _mm256_mul_ps(_mm256_set1_ps(qh[t]), kv));
    }
  } else {
    /* 32-bit words holding elements t (low half) and t + 1 (high half) */
    const __m256i idx = _mm256_mullo_epi32(_mm256_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7),
                                           _mm256_set1_epi32(hd * 2));
    const char *base = (const char *)(kb + (size_t)j0 * hd);
    const __m256i hi_mask = _mm256_set1_epi32((int)0xffff0000u);
    for (int t = 0; t < hd; t += 2) {
      __m256i w = _mm256_i32gather_epi32((const int *)(base + 2 * t), idx, 1);
      __m256 k0 = _mm256_castsi256_ps(_mm256_slli_epi32(w, 16));
      __m256 k1 = _mm256_castsi256_ps(_mm256_and_si256(w, hi_mask));
      acc = _mm256_add_ps(acc, _mm256_mul_ps(_mm256_set1_ps(qh[t]), k0));
      acc = _mm256_add_ps(acc, _mm256_mul_ps(_mm256_set1_ps(qh[t + 1]), k1));
    }
  }
  _mm256_storeu_ps(sc + j0, _mm256_mul_ps(acc, _mm256_set1_ps(scale)));
}
#endif

static void xo_scores8(const float *qh, const uint16_t *kb, const float *kf, int j0, int len,
                       int hd, float scale, float *sc) {
#if defined(__x86_64__)
  if (j0 + 8 <= len && hd % 2 == 0 && __builtin_cpu_supports("avx2")) {
    xo_scores8_avx2(qh, kb, kf, j0, hd, scale, sc);
    return;
  }
#endif
  xo_scores8_scalar(qh, kb, kf, j0, len, hd, scale, sc);
}

/* One query head against `len` cached rows: attend_one per head
 * (whisper_decoder.rs:242-278): scores (q . k) * scale in f32, max, exp and
 * a sequential sum, then ctx += p * v over the keys in order.  OPT divides
 * each probability by the sum (opt125m_decode.rs:277-280, div_by_sum);
 * attend_one multiplies by 1/sum (:266-270).  Rows come from the bf16 cache
 * (kb, vb) or the fp32 one (kf, vf).  The OpenMP splits are over keys (each
 * score is its own dot product) and over output dimensions (each keeps the
 * key order), so every value is the sequential computation. */
static void xo_head_attend(const float *qh, const uint16_t *kb, const uint16_t *vb,
                           const float *kf, const float *vf, int len, int hd, float scale,
                           int div_by_sum, float *sc, float *oh) {
  int nk8 = (len + 7) / 8;
#pragma omp parallel for schedule(static) if (len >= 256)
  for (int j8 = 0; j8 < nk8; j8++) xo_scores8(qh, kb, kf, j8 * 8, len, hd, scale, sc);
  float mx = -INFINITY;
  for (int j = 0; j < len; j++) mx = fmaxf(mx, sc[j]);
  float sum = 0.f;
  for (int j = 0; j < len; j++) {
    sc[j] = expf(sc[j] - mx);
    sum += sc[j];
  }
  float inv = 1.0f / sum;
  for (int j = 0; j < len; j++) sc[j] = div_by_sum ? sc[j] / sum : sc[j] * inv;
  int nblk = (hd + 15) / 16;
#pragma omp parallel for schedule(static) if (len >= 256)
  for (int tb = 0; tb < nblk; tb++) {
    int t0 = tb * 16, t1 = t0 + 16 < hd ? t0 + 16 : hd;
    float acc[16];
    for (int t = t0; t < t1; t++) acc[t - t0] = 0.f;
    for (int j = 0; j < len; j++) {
      float p = sc[j];
      if (vf)
        for (int t = t0; t < t1; t++) acc[t - t0] += p * vf[(size_t)j * hd + t];
      else
        for (int t = t0; t < t1; t++) acc[t - t0] += p * xo_bf16_bits_to_f32(vb[(size_t)j * hd + t]);
    }
    for (int t = t0; t < t1; t++) oh[t] = acc[t - t0];
  }
}

/* One stream's decode step.  OPT: Opt::step (opt125m_decode.rs:252-293).
 * Whisper: HostDecoder::step host path (whisper_decoder.rs:401-535).
 * Gemma-3: HF Gemma3DecoderLayer built from rmsnorm_ref / geglu_ref
 * (npu-gemma/src/lib.rs:55-77) and GEMMA3_1B (config.rs:156-170) with the
 * BASELINE simplification of one RoPE theta and global attention (the
 * reference has no Gemma decode loop, npu-gemma/src/lib.rs:9-15; the
 * composition is checked against Hugging Face's Gemma3ForCausalLM).
 * Numerics of the build, applied identically on the GPU: fp32 activations,
 * weights as stored (int8 per-row scale / bf16 / bfp16), K/V rounded to
 * bf16 when written to the cache, tied quantised embedding for the lm-head. */
static void xo_step_one(xo_model *m, int b, int tok, int pos, float *logits) {
  const xe_model_config *c = &m->c;
  int D = c->d_model, H = c->n_heads, Hk = c->n_kv_heads, hd = c->head_dim, F = c->ffn;
  int fam = c->family, L = c->n_layers, MC = c->max_ctx;
  int hq = H * hd, hk = Hk * hd, group = H / Hk;
  float *x = (float *)malloc((size_t)D * 4), *h = (float *)malloc((size_t)D * 4);
  float *q = (float *)malloc((size_t)hq * 4), *k = (float *)malloc((size_t)hk * 4);
  float *v = (float *)malloc((size_t)hk * 4), *ctx = (float *)malloc((size_t)hq * 4);
  float *o = (float *)malloc((size_t)D * 4), *f1 = (float *)malloc((size_t)F * 4);
  float *f2 = (float *)malloc((size_t)F * 4), *sc = (float *)malloc((size_t)(MC > c->n_cross ? MC : c->n_cross) * 4);
  const float eps = c->eps;

  xo_embed_row(m, tok, x);
  if (fam == XE_OPT || fam == XE_WHISPER) {
    const xo_tensor *pe = T(m, XE_T_POS_EMB, -1);
    int prow = fam == XE_OPT ? pos + (m->mutation == XO_MUT_OPT_POS_OFFSET ? 1 : 2) : pos;
    for (int d = 0; d < D; d++) x[d] = x[d] + pe->f32[(size_t)prow * D + d];
  } else {
    float nrm = m->mutation == XO_MUT_GEMMA_NO_EMB_SCALE ? 1.0f : sqrtf((float)D);
    for (int d = 0; d < D; d++) x[d] = x[d] * nrm;
  }

  for (int l = 0; l < L; l++) {
    /* --- self attention --- */
    if (fam == XE_GEMMA3)
      xo_rmsnorm(x, D, T(m, XE_T_LN1_W, l)->f32, eps, h);
    else
      xo_layer_norm(x, 1, D, T(m, XE_T_LN1_W, l)->f32, T(m, XE_T_LN1_B, l)->f32, eps, h);
    xo_lin(m, XE_T_Q_W, l, XE_T_Q_B, h, q);
    xo_lin(m, XE_T_K_W, l, XE_T_K_B, h, k);
    xo_lin(m, XE_T_V_W, l, XE_T_V_B, h, v);
    float scale;
    if (fam == XE_OPT) {
      float s = m->mutation == XO_MUT_OPT_NO_Q_SCALE ? 1.0f : powf((float)hd, -0.5f);
      for (int i = 0; i < hq; i++) q[i] = q[i] * s;
      scale = 1.0f;
    } else if (fam == XE_WHISPER) {
      scale = 1.0f / sqrtf((float)hd);
    } else {
      for (int hh = 0; hh < H; hh++) {
        xo_rmsnorm(q + hh * hd, hd, T(m, XE_T_QNORM_W, l)->f32, eps, ctx);
        memcpy(q + hh * hd, ctx, (size_t)hd * 4);
        xo_rope_apply(m, q + hh * hd, pos);
      }
      for (int hh = 0; hh < Hk; hh++) {
        xo_rmsnorm(k + hh * hd, hd, T(m, XE_T_KNORM_W, l)->f32, eps, ctx);
        memcpy(k + hh * hd, ctx, (size_t)hd * 4);
        xo_rope_apply(m, k + hh * hd, pos);
      }
      scale = 1.0f / sqrtf((float)hd); /* query_pre_attn_scalar = head_dim */
    }
    size_t lb = ((size_t)l * m->batch + b) * Hk;
    for (int hh = 0; hh < Hk; hh++)
      for (int j = 0; j < hd; j++) {
        size_t off = ((lb + hh) * MC + pos) * hd + j;
        if (m->kv_f32) {
          m->kcf[off] = k[hh * hd + j];
          m->vcf[off] = v[hh * hd + j];
        } else {
          m->kc[off] = xo_f32_to_bf16_bits(k[hh * hd + j]);
          m->vc[off] = xo_f32_to_bf16_bits(v[hh * hd + j]);
        }
      }
    int len = pos + 1;
    for (int hh = 0; hh < H; hh++) {
      size_t base = (lb + hh / group) * MC * hd;
      if (m->kv_f32)
        xo_head_attend(q + hh * hd, NULL, NULL, m->kcf + base, m->vcf + base, len, hd, scale,
                       fam == XE_OPT, sc, ctx + hh * hd);
      else
        xo_head_attend(q + hh * hd, m->kc + base, m->vc + base, NULL, NULL, len, hd, scale,
                       fam == XE_OPT, sc, ctx + hh * hd);
    }
    xo_lin(m, XE_T_O_W, l, XE_T_O_B, ctx, o);
    if (fam == XE_GEMMA3) {
      xo_rmsnorm(o, D, T(m, m->mutation == XO_MUT_GEMMA_SWAP_POST_NORMS ? XE_T_POST_FFN_W : XE_T_POST_ATTN_W, l)->f32,
                 eps, h);
      for (int d = 0; d < D; d++) x[d] = x[d] + h[d];
    } else {
      for (int d = 0; d < D; d++) x[d] = x[d] + o[d];
    }

    /* --- Whisper cross attention (whisper_decoder.rs:484-500) --- */
    if (fam == XE_WHISPER) {
      int Tn = c->n_cross;
      xo_layer_norm(x, 1, D, T(m, XE_T_LNX_W, l)->f32, T(m, XE_T_LNX_B, l)->f32, eps, h);
      xo_lin(m, XE_T_XQ_W, l, XE_T_XQ_B, h, q);
      float xscale = m->mutation == XO_MUT_WHISPER_CROSS_SCALE ? 1.0f : scale;
      for (int hh = 0; hh < H; hh++) {
        size_t base = ((size_t)l * H + hh) * Tn * hd;
        if (m->xk8 || m->xv8)
          xo_head_attend_x8(q + hh * hd, m->xk8 ? m->xk8 + base : NULL,
                            m->xks ? m->xks + (size_t)l * D + hh * hd : NULL, m->xk + base,
                            m->xv8 ? m->xv8 + base : NULL, m->xvs ? m->xvs + (size_t)l * D + hh * hd : NULL,
                            m->xv + base, Tn, hd, xscale, sc, ctx + hh * hd);
        else if (m->kv_f32)
          xo_head_attend(q + hh * hd, NULL, NULL, m->xkf + base, m->xvf + base, Tn, hd, xscale, 0,
                         sc, ctx + hh * hd);
        else
          xo_head_attend(q + hh * hd, m->xk + base, m->xv + base, NULL, NULL, Tn, hd, xscale, 0,
                         sc, ctx + hh * hd);
      }
      xo_lin(m, XE_T_XO_W, l, XE_T_XO_B, ctx, o);
      for (int d = 0; d < D; d++) x[d] = x[d] + o[d];
    }

    /* --- feed-forward --- */
    if (fam == XE_GEMMA3) {
      xo_rmsnorm(x, D, T(m, XE_T_LN2_W, l)->f32, eps, h);
      xo_lin(m, XE_T_FC1_W, l, -1, h, f1);
      xo_lin(m, XE_T_UP_W, l, -1, h, f2);
      /* geglu_ref (npu-gemma/src/lib.rs:68-71) */
      for (int i = 0; i < F; i++) f1[i] = xo_gelu_tanh(f1[i]) * f2[i];
      xo_lin(m, XE_T_FC2_W, l, -1, f1, o);
      xo_rmsnorm(o, D, T(m, XE_T_POST_FFN_W, l)->f32, eps, h);
      for (int d = 0; d < D; d++) x[d] = x[d] + h[d];
    } else {
      xo_layer_norm(x, 1, D, T(m, XE_T_LN2_W, l)->f32, T(m, XE_T_LN2_B, l)->f32, eps, h);
      xo_lin(m, XE_T_FC1_W, l, XE_T_FC1_B, h, f1);
      if (fam == XE_OPT)
        for (int i = 0; i < F; i++) f1[i] = f1[i] > 0.0f ? f1[i] : 0.0f; /* relu :287 */
      else
        for (int i = 0; i < F; i++) f1[i] = xo_gelu_erf(f1[i]); /* gelu_row :1903 */
      xo_lin(m, XE_T_FC2_W, l, XE_T_FC2_B, f1, o);
      for (int d = 0; d < D; d++) x[d] = x[d] + o[d];
    }
  }

  /* final norm + tied lm-head */
  if (fam == XE_GEMMA3)
    xo_rmsnorm(x, D, T(m, XE_T_LNF_W, -1)->f32, eps, h);
  else
    xo_layer_norm(x, 1, D, T(m, XE_T_LNF_W, -1)->f32, T(m, XE_T_LNF_B, -1)->f32, eps, h);
  xo_lin(m, XE_T_TOK_EMB, -1, -1, h, logits);

  free(x); free(h); free(q); free(k); free(v); free(ctx); free(o); free(f1); free(f2); free(sc);
}

/* Streams are independent (own K/V rows, own outputs, read-only weights):
 * with more than one, each thread takes whole streams and the OpenMP regions
 * inside a step run on that thread alone (nested regions are inactive). */
void xo_model_step(xo_model *m, const int *tokens, const int *pos, int batch, float *logits) {
  if (batch == 1) { /* no enclosing region: the step's own regions use every thread */
    xo_step_one(m, 0, tokens[0], pos[0], logits);
    return;
  }
#pragma omp parallel for schedule(dynamic, 1)
  for (int b = 0; b < batch; b++)
    xo_step_one(m, b, tokens[b], pos[b], logits + (size_t)b * m->c.vocab);
}

int xo_model_argmax(const xo_model *m, const float *logits) {
  return m->c.family == XE_OPT ? xo_argmax_last(logits, m->c.vocab)
                               : xo_argmax_first(logits, m->c.vocab);
}

static float xo_margin(const float *v, int n, int best) {
  float second = -INFINITY;
  for (int i = 0; i < n; i++)
    if (i != best && v[i] > second) second = v[i];
  return v[best] - second;
}

/* One stream of Opt::generate (opt125m_decode.rs:296-315): the prompt fed
 * from position 0, then greedy steps; the argmax after the last prompt token
 * is the first emitted token.  With stop >= 0 the stream ends at the first
 * emitted token equal to stop (the EOT rule of whisper.rs:371-380): that
 * token and every later slot of out hold stop, *n_out is the number of
 * tokens before it.  (The reference's batched loop keeps feeding EOT to a
 * finished stream, whisper.rs:651; streams are independent, so nothing
 * emitted depends on those steps and this stream simply ends.) */
static void xo_generate_one(xo_model *m, int b, const int *prompt, int n_prompt, int n_new,
                            int stop, int *out, float *margins, int *n_out) {
  int V = m->c.vocab;
  float *logits = (float *)malloc((size_t)V * 4);
  for (int p = 0; p < n_prompt; p++) xo_step_one(m, b, prompt[p], p, logits);
  int pos = n_prompt, n = n_new;
  for (int i = 0; i < n_new; i++) {
    int next = xo_model_argmax(m, logits);
    out[i] = next;
    if (margins) margins[i] = xo_margin(logits, V, next);
    if (stop >= 0 && next == stop) {
      n = i;
      for (int j = i + 1; j < n_new; j++) {
        out[j] = stop;
        if (margins) margins[j] = INFINITY;
      }
      break;
    }
    if (i + 1 == n_new) break;
    xo_step_one(m, b, next, pos, logits);
    pos++;
  }
  if (n_out) *n_out = n;
  free(logits);
}

int xo_model_generate_until(xo_model *m, const int *prompt, int n_prompt, int batch, int n_new,
                            int stop, int *out, int *n_out, float *margins) {
  if (batch > m->batch || n_prompt < 1 || n_new < 1 || n_prompt + n_new > m->c.max_ctx + 1) return -1;
  if (batch == 1) {
    xo_generate_one(m, 0, prompt, n_prompt, n_new, stop, out, margins, n_out);
    return 0;
  }
#pragma omp parallel for schedule(dynamic, 1)
  for (int b = 0; b < batch; b++)
    xo_generate_one(m, b, prompt + (size_t)b * n_prompt, n_prompt, n_new, stop, out + (size_t)b * n_new,
                    margins ? margins + (size_t)b * n_new : NULL, n_out ? n_out + b : NULL);
  return 0;
}

int xo_model_generate(xo_model *m, const int *prompt, int n_prompt, int batch,
                      int n_new, int *out, float *margins) {
  return xo_model_generate_until(m, prompt, n_prompt, batch, n_new, -1, out, NULL, margins);
}

size_t xo_model_tensor_numel(const xo_model *m, int kind, int layer) {
  if (kind < 0 || kind >= XE_T_COUNT || layer < -1 || layer >= m->c.n_layers) return 0;
  const xo_tensor *t = T(m, kind, layer);
  return t ? (size_t)t->rows * t->cols : 0;
}

/* The fp32 tensor as generated (quantised tensors are regenerated). */
int xo_model_tensor_f32(const xo_model *m, int kind, int layer, float *out) {
  size_t n = xo_model_tensor_numel(m, kind, layer);
  if (!n) return -1;
  const xo_tensor *t = T(m, kind, layer);
  if (t->f32)
    memcpy(out, t->f32, n * 4);
  else
    xo_synth_fill(m->seed, XE_SYNTH_ID(kind, layer), t->mean, t->stdv, out, n);
  return 0;
}

int xo_model_tensor_q8(const xo_model *m, int kind, int layer, int8_t *q, float *s) {
  size_t n = xo_model_tensor_numel(m, kind, layer);
  if (!n) return -1;
  const xo_tensor *t = T(m, kind, layer);
  if (!t->q) return -1;
  memcpy(q, t->q, n);
  memcpy(s, t->s, (size_t)t->rows * 4);
  return 0;
}
