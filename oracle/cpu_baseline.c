/*
 * cpu_baseline.c -- multi-threaded CPU W4A16 GEMV, the CPU leg that bench.py
 * times next to the GPU kernel (the reference's MLX CPU backend cannot run
 * here). Same semantics as sq_w4a16_matmul in sparkq_oracle.c: dequantize
 * each group to fp32 (q*s+b, exact), then an fp32 dot with x; OpenMP over
 * output rows; the inner loops are written for the compiler's vectorizer.
 *
 * TEST INFRASTRUCTURE ONLY (bench.py cpu_baseline leg); not product code.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <omp.h>

static inline float bf16f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* y[m,n] (fp32) for x [M,K] bf16, w [N,K/8], scales/biases [N,K/G] bf16,
 * G <= 128. Returns the number of threads used, or -1 on a bad argument. */
int sq_cpu_w4a16_gemv(const uint16_t* x, const uint32_t* w,
                      const uint16_t* scales, const uint16_t* biases,
                      int64_t M, int64_t N, int64_t K, int G, float* y,
                      int threads) {
  if (G > 128 || G % 8 || K % G) return -1;
  if (threads > 0) omp_set_num_threads(threads);
  float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K));
  if (!xf) return -1;
  for (int64_t i = 0; i < M * K; ++i) xf[i] = bf16f(x[i]);
  int used = 1;
  const int64_t ng = K / G;
#pragma omp parallel
  {
#pragma omp single
    used = omp_get_num_threads();
    float wbuf[128];
#pragma omp for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      float acc[16];
      for (int64_t m0 = 0; m0 < M; m0 += 16) {
        const int64_t mc = M - m0 < 16 ? M - m0 : 16;
        for (int64_t m = 0; m < mc; ++m) acc[m] = 0.0f;
        for (int64_t g = 0; g < ng; ++g) {
          const float s = bf16f(scales[n * ng + g]);
          const float b = bf16f(biases[n * ng + g]);
          const uint32_t* wg = w + n * (K / 8) + g * (G / 8);
          for (int i = 0; i < G / 8; ++i) {
            const uint32_t word = wg[i];
            for (int j = 0; j < 8; ++j)
              wbuf[8 * i + j] = (float)((word >> (4 * j)) & 15u) * s + b;
          }
          for (int64_t m = 0; m < mc; ++m) {
            const float* xr = xf + (m0 + m) * K + g * G;
            float part = 0.0f;
            for (int i = 0; i < G; ++i) part += xr[i] * wbuf[i];
            acc[m] += part;
          }
        }
        for (int64_t m = 0; m < mc; ++m) y[(m0 + m) * N + n] = acc[m];
      }
    }
  }
  free(xf);
  return used;
}
