/*
 * gemv_ref.c — TEST INFRASTRUCTURE ONLY (the oracle).  Never part of the product.
 *
 * A plain-C restatement of the reference's CPU GEMV, helm/kernels/fp16_gemv.cpp:
 *   hsum256        :32-39   horizontal sum: (v[i] + v[i+4]) then two pairwise adds
 *   dot_fp16_row   :45-86   four independent 8-lane fp32 FMA accumulators over 32
 *                           elements per step, an 8-wide tail into acc0, combine
 *                           (acc0+acc1)+(acc2+acc3), hsum, then a scalar tail
 *   gemv_fp16      :92-100  rows split statically over OpenMP threads
 *   helm_fp16_linear :139-151  fp32 result (+ bias in fp32) rounded once to fp16
 * The same summation order is kept, so oracle_fp16_gemv reproduces the
 * reference's fp16 GEMV bit for bit on AVX2/F16C/FMA hosts.
 *
 * oracle_int8_gemv applies the identical loop structure to an int8 weight row
 * (each int8 converted exactly to fp32) and multiplies the dot product by the
 * row's fp16 scale before the bias: y = fp16(scale[n] * dot + bias[n]).  It is
 * the CPU baseline for the INT8 GEMV and a second implementation of the
 * closed form the GPU kernel is checked against.
 */
#include <immintrin.h>
#include <stdint.h>

static inline float hsum8(__m256 v) {
  __m128 hi = _mm256_extractf128_ps(v, 1);
  __m128 lo = _mm256_castps256_ps128(v);
  lo = _mm_add_ps(lo, hi);
  lo = _mm_hadd_ps(lo, lo);
  lo = _mm_hadd_ps(lo, lo);
  return _mm_cvtss_f32(lo);
}

static inline float half_to_float(uint16_t h) { return _cvtsh_ss(h); }
static inline uint16_t float_to_half(float f) { return _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }

static inline __m256 load8_h(const uint16_t* p) {
  return _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)p));
}
static inline __m256 load8_i8(const int8_t* p) {
  return _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)p)));
}

/* One row, fp16 weights: the accumulation order of dot_fp16_row. */
static float dot_row_f16(const uint16_t* w, const uint16_t* x, int64_t n) {
  __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
  __m256 a2 = _mm256_setzero_ps(), a3 = _mm256_setzero_ps();
  int64_t j = 0;
  for (; j <= n - 32; j += 32) {
    a0 = _mm256_fmadd_ps(load8_h(w + j), load8_h(x + j), a0);
    a1 = _mm256_fmadd_ps(load8_h(w + j + 8), load8_h(x + j + 8), a1);
    a2 = _mm256_fmadd_ps(load8_h(w + j + 16), load8_h(x + j + 16), a2);
    a3 = _mm256_fmadd_ps(load8_h(w + j + 24), load8_h(x + j + 24), a3);
  }
  for (; j <= n - 8; j += 8) a0 = _mm256_fmadd_ps(load8_h(w + j), load8_h(x + j), a0);
  a0 = _mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3));
  float r = hsum8(a0);
  for (; j < n; ++j) r += half_to_float(w[j]) * half_to_float(x[j]);
  return r;
}

/* One row, int8 weights, same order. */
static float dot_row_i8(const int8_t* w, const uint16_t* x, int64_t n) {
  __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
  __m256 a2 = _mm256_setzero_ps(), a3 = _mm256_setzero_ps();
  int64_t j = 0;
  for (; j <= n - 32; j += 32) {
    a0 = _mm256_fmadd_ps(load8_i8(w + j), load8_h(x + j), a0);
    a1 = _mm256_fmadd_ps(load8_i8(w + j + 8), load8_h(x + j + 8), a1);
    a2 = _mm256_fmadd_ps(load8_i8(w + j + 16), load8_h(x + j + 16), a2);
    a3 = _mm256_fmadd_ps(load8_i8(w + j + 24), load8_h(x + j + 24), a3);
  }
  for (; j <= n - 8; j += 8) a0 = _mm256_fmadd_ps(load8_i8(w + j), load8_h(x + j), a0);
  a0 = _mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3));
  float r = hsum8(a0);
  for (; j < n; ++j) r += (float)w[j] * half_to_float(x[j]);
  return r;
}

/* y[m, n] = fp16(dot(W[n], x[m]) + bias[n]) for m < M; bias may be NULL.
 * x [M, K] fp16 rows, W [N, K] fp16 rows, y [M, N] fp16.  Each token row is a
 * separate GEMV, as the reference runs one GEMV per decode token. */
void oracle_fp16_gemv(const uint16_t* x, const uint16_t* w, const uint16_t* bias, uint16_t* y,
                      int64_t M, int64_t N, int64_t K) {
  for (int64_t m = 0; m < M; ++m) {
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      float r = dot_row_f16(w + n * K, x + m * K, K);
      if (bias) r += half_to_float(bias[n]);
      y[m * N + n] = float_to_half(r);
    }
  }
}

/* y[m, n] = fp16(scale[n] * dot(q[n], x[m]) + bias[n]); bias may be NULL. */
void oracle_int8_gemv(const uint16_t* x, const int8_t* q, const uint16_t* scale,
                      const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int64_t K) {
  for (int64_t m = 0; m < M; ++m) {
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      float r = dot_row_i8(q + n * K, x + m * K, K) * half_to_float(scale[n]);
      if (bias) r += half_to_float(bias[n]);
      y[m * N + n] = float_to_half(r);
    }
  }
}

/* fp32 variant without the final rounding (used to measure accumulation error). */
void oracle_int8_gemv_f32(const uint16_t* x, const int8_t* q, const uint16_t* scale, float* y,
                          int64_t M, int64_t N, int64_t K) {
  for (int64_t m = 0; m < M; ++m) {
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) y[m * N + n] = dot_row_i8(q + n * K, x + m * K, K) * half_to_float(scale[n]);
  }
}
