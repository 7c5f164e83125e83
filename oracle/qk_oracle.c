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
#include <stdint.h>
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

/* x [M,K] bf16 bits; words [N, K/8] (element 8i+j in bits 4j..4j+3);
 * s, b [N, K/g] bf16 bits; y [M,N] float32. */
void qo_matvec_int4_u32x8(const uint16_t* x, const uint32_t* words,
                          const uint16_t* s, const uint16_t* b, float* y,
                          int64_t M, int64_t N, int64_t K, int g,
                          int threads) {
  const int64_t G = K / g;
  const int nt = qo_num_threads(threads);
  for (int64_t m = 0; m < M; ++m) {
    float* xf = (float*)__builtin_alloca(sizeof(float) * (size_t)K);
    float* xsum = (float*)__builtin_alloca(sizeof(float) * (size_t)G);
    for (int64_t k = 0; k < K; ++k) xf[k] = bf16f(x[m * K + k]);
    for (int64_t gi = 0; gi < G; ++gi) {
      float t = 0.f;
      for (int j = 0; j < g; ++j) t += xf[gi * g + j];
      xsum[gi] = t;
    }
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t o = 0; o < N; ++o) {
      const uint32_t* wr = words + o * (K / 8);
      float acc = 0.f;
      for (int64_t gi = 0; gi < G; ++gi) {
        float d = 0.f;
        const float* xg = xf + gi * g;
        const uint32_t* wg = wr + gi * (g / 8);
        for (int i = 0; i < g / 8; ++i) {
          const uint32_t w = wg[i];
          for (int j = 0; j < 8; ++j)
            d += xg[8 * i + j] * (float)((w >> (4 * j)) & 15u);
        }
        acc += bf16f(s[o * G + gi]) * d + bf16f(b[o * G + gi]) * xsum[gi];
      }
      y[m * N + o] = acc;
    }
  }
}

/* Affine uint8 codes [N, K]. */
void qo_matvec_u8(const uint16_t* x, const uint8_t* codes, const uint16_t* s,
                  const uint16_t* b, float* y, int64_t M, int64_t N,
                  int64_t K, int g, int threads) {
  const int64_t G = K / g;
  const int nt = qo_num_threads(threads);
  for (int64_t m = 0; m < M; ++m) {
    float* xf = (float*)__builtin_alloca(sizeof(float) * (size_t)K);
    float* xsum = (float*)__builtin_alloca(sizeof(float) * (size_t)G);
    for (int64_t k = 0; k < K; ++k) xf[k] = bf16f(x[m * K + k]);
    for (int64_t gi = 0; gi < G; ++gi) {
      float t = 0.f;
      for (int j = 0; j < g; ++j) t += xf[gi * g + j];
      xsum[gi] = t;
    }
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t o = 0; o < N; ++o) {
      const uint8_t* cr = codes + o * K;
      float acc = 0.f;
      for (int64_t gi = 0; gi < G; ++gi) {
        float d = 0.f;
        for (int j = 0; j < g; ++j) d += xf[gi * g + j] * (float)cr[gi * g + j];
        acc += bf16f(s[o * G + gi]) * d + bf16f(b[o * G + gi]) * xsum[gi];
      }
      y[m * N + o] = acc;
    }
  }
}
