/*
 * qk_oracle.c -- C port of the reference's quantized matvecs.
 * TEST INFRASTRUCTURE ONLY: linked by tests/ and timed by bench.py's
 * cpu_baseline leg; never part of the product library.
 *
 * Restates, in float32 as the reference computes it:
 *   _matvec_int4 (examples/llm/qwen3.py:243-267): per group,
 *     s * sum_j x_j q_j + b * sum_j x_j, summed over groups;
 *   the affine int8 config (w = s*q + b) in the same factoring;
 * for bf16 activations and bf16 scale/offset, given as raw uint16 bits.
 * Rows are split over OpenMP threads.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf16f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

int qo_num_threads(int requested) {
#ifdef _OPENMP
  return requested > 0 ? requested : omp_get_max_threads();
#else
  (void)requested;
  return 1;
#endif
}

/* bf16 rows of x as float32, and each row's per-group sums of x. */
static void prepare_x(const uint16_t* x, float* xf, float* xsum, int64_t M,
                      int64_t K, int g) {
  const int64_t G = K / g;
  for (int64_t i = 0; i < M * K; ++i) xf[i] = bf16f(x[i]);
  for (int64_t m = 0; m < M; ++m)
    for (int64_t gi = 0; gi < G; ++gi) {
      float t = 0.f;
      for (int j = 0; j < g; ++j) t += xf[m * K + gi * g + j];
      xsum[m * G + gi] = t;
    }
}

/* x [M,K] bf16 bits; words [N, K/8] (element 8i+j in bits 4j..4j+3);
 * s, b [N, K/g] bf16 bits; y [M,N] float32. When mag is not NULL it
 * receives sum_k |x[m,k]| * |s*q + b| (in double), the scale of the
 * rounding error a float32 product can make, for elementwise tolerances.
 * Output rows are split over threads; each weight row is decoded once for
 * all M rows of x (the per-element arithmetic is that of one row). */
void qo_matvec_int4_u32x8(const uint16_t* x, const uint32_t* words,
                          const uint16_t* s, const uint16_t* b, float* y,
                          double* mag, int64_t M, int64_t N, int64_t K, int g,
                          int threads) {
  const int64_t G = K / g;
  const int nt = qo_num_threads(threads);
  float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K));
  float* xsum = (float*)malloc(sizeof(float) * (size_t)(M * G));
  prepare_x(x, xf, xsum, M, K, g);
#pragma omp parallel num_threads(nt)
  {
    float* q = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int64_t o = 0; o < N; ++o) {
      const uint32_t* wr = words + o * (K / 8);
      for (int64_t i = 0; i < K / 8; ++i)
        for (int j = 0; j < 8; ++j) q[8 * i + j] = (float)((wr[i] >> (4 * j)) & 15u);
      for (int64_t m = 0; m < M; ++m) {
        const float* xm = xf + m * K;
        float acc = 0.f;
        double am = 0.0;
        for (int64_t gi = 0; gi < G; ++gi) {
          float d = 0.f;
          const float* xg = xm + gi * g;
          const float* qg = q + gi * g;
          for (int j = 0; j < g; ++j) d += xg[j] * qg[j];
          const float sc = bf16f(s[o * G + gi]), of = bf16f(b[o * G + gi]);
          acc += sc * d + of * xsum[m * G + gi];
          if (mag) {
            for (int j = 0; j < g; ++j)
              am += fabs((double)xg[j]) * fabs((double)sc * qg[j] + of);
          }
        }
        y[m * N + o] = acc;
        if (mag) mag[m * N + o] = am;
      }
    }
    free(q);
  }
  free(xf);
  free(xsum);
}

/* Affine uint8 codes [N, K]; as above. */
void qo_matvec_u8(const uint16_t* x, const uint8_t* codes, const uint16_t* s,
                  const uint16_t* b, float* y, double* mag, int64_t M,
                  int64_t N, int64_t K, int g, int threads) {
  const int64_t G = K / g;
  const int nt = qo_num_threads(threads);
  float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K));
  float* xsum = (float*)malloc(sizeof(float) * (size_t)(M * G));
  prepare_x(x, xf, xsum, M, K, g);
#pragma omp parallel num_threads(nt)
  {
    float* q = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int64_t o = 0; o < N; ++o) {
      const uint8_t* cr = codes + o * K;
      for (int64_t k = 0; k < K; ++k) q[k] = (float)cr[k];
      for (int64_t m = 0; m < M; ++m) {
        const float* xm = xf + m * K;
        float acc = 0.f;
        double am = 0.0;
        for (int64_t gi = 0; gi < G; ++gi) {
          float d = 0.f;
          const float* xg = xm + gi * g;
          const float* qg = q + gi * g;
          for (int j = 0; j < g; ++j) d += xg[j] * qg[j];
          const float sc = bf16f(s[o * G + gi]), of = bf16f(b[o * G + gi]);
          acc += sc * d + of * xsum[m * G + gi];
          if (mag) {
            for (int j = 0; j < g; ++j)
              am += fabs((double)xg[j]) * fabs((double)sc * qg[j] + of);
          }
        }
        y[m * N + o] = acc;
        if (mag) mag[m * N + o] = am;
      }
    }
    free(q);
  }
  free(xf);
  free(xsum);
}
