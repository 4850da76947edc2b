/*
 * cpu_baseline.c -- multi-threaded CPU legs that bench.py times next to the
 * GPU kernels (the reference's MLX CPU backend cannot run here). Each leg has
 * the semantics of the matching oracle function in sparkq_oracle.c, with the
 * summation order left to the vectorizer:
 *
 *   sq_cpu_w4a16_matmul  W4A16 affine linear: dequantize to fp32 (q*s+b,
 *                        exact), fp32 products and sums. Up to 8 activation
 *                        rows: each weight row decoded once per group and
 *                        dotted as s*sum(q*x) + b*sum(x). More rows: 16 weight
 *                        columns are dequantized once into a k-major panel
 *                        and multiplied against 8 activation rows at a time
 *                        (8 independent 16-lane accumulators per k step), k
 *                        blocked so the panel stays in L2.
 *   sq_cpu_w8a8_linear   W8A8: per-token int8 quantization (absmax/127,
 *                        rint, clamp to +-127), int8 x int8 dots into int32,
 *                        then acc * sa[m] * sw[n].
 *   sq_cpu_int8kv_sdpa   INT8-KV GQA decode attention (one query token per
 *                        head): s8 codes with one fp16 scale per (token, KV
 *                        head), fp32 online softmax; the work is split over
 *                        (sequence, KV head, token range) and merged by LSE.
 *
 * Built twice by the Makefile: for AVX2+FMA and for AVX-512 (BW/VL/VNNI);
 * oracle.py loads the AVX-512 build when the host CPU has those features.
 *
 * TEST INFRASTRUCTURE ONLY (bench.py cpu_baseline legs); not product code.
 */
#include <math.h>
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

static inline float f16f(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15) << 31;
  uint32_t e = (h >> 10) & 31u, m = h & 1023u, u;
  if (e == 31) {
    u = s | 0x7F800000u | (m << 13);
  } else if (e == 0) {
    if (m == 0) {
      u = s;
    } else { /* subnormal: normalise */
      int sh = 0;
      while (!(m & 1024u)) {
        m <<= 1;
        ++sh;
      }
      u = s | ((uint32_t)(113 - sh) << 23) | ((m & 1023u) << 13);
    }
  } else {
    u = s | ((e + 112) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static int set_threads(int threads) {
  if (threads > 0) omp_set_num_threads(threads);
  int used = 1;
#pragma omp parallel
  {
#pragma omp single
    used = omp_get_num_threads();
  }
  return used;
}

/* ---------------------------------------------------------------------- */
/* W4A16                                                                   */
/* ---------------------------------------------------------------------- */

#define NB 16  /* weight columns per panel (one 16-lane vector) */
#define MB 8   /* activation rows per micro-tile */
#define KC 512 /* k per panel block */

/* Few activation rows (M <= GEMV_MAXM): each weight row is decoded once and
 * dotted with every activation row. Inside a group of W = G/8 words the
 * activations are stored transposed (xp[8*W*g + W*j + i] = x[8*W*g + 8*i + j])
 * so that nibble j of words 0..W-1 meets W consecutive activations, and the
 * group's dot is s*sum(q*x) + b*sum(x). */
#define GEMV_MAXM 8

static inline __attribute__((always_inline)) void w4_gemv_rows(
    const float* xp, const float* xs, const uint32_t* w, const uint16_t* scales,
    const uint16_t* biases, int64_t M, int64_t N, int64_t K, const int W, float* y) {
  const int64_t G = 8 * W, ng = K / G, kw = K / 8;
#pragma omp for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    float acc[GEMV_MAXM] = {0};
    const uint32_t* wr = w + n * kw;
    for (int64_t g = 0; g < ng; ++g) {
      float cf[8][16];
      for (int j = 0; j < 8; ++j)
        for (int i = 0; i < W; ++i) cf[j][i] = (float)((wr[g * W + i] >> (4 * j)) & 15u);
      const float sc = bf16f(scales[n * ng + g]), bi = bf16f(biases[n * ng + g]);
      for (int64_t m = 0; m < M; ++m) {
        const float* xg = xp + m * K + g * G;
        float part[16] = {0};
        for (int j = 0; j < 8; ++j)
          for (int i = 0; i < W; ++i) part[i] += cf[j][i] * xg[W * j + i];
        float dot = 0.0f;
        for (int i = 0; i < W; ++i) dot += part[i];
        acc[m] += sc * dot + bi * xs[m * ng + g];
      }
    }
    for (int64_t m = 0; m < M; ++m) y[m * N + n] = acc[m];
  }
}

static int w4_gemv(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                   const uint16_t* biases, int64_t M, int64_t N, int64_t K, int G, float* y,
                   int used) {
  const int64_t ng = K / G, W = G / 8;
  float* xp = (float*)malloc(sizeof(float) * (size_t)(M * K));
  float* xs = (float*)malloc(sizeof(float) * (size_t)(M * ng));
  if (!xp || !xs) {
    free(xp);
    free(xs);
    return -1;
  }
  for (int64_t m = 0; m < M; ++m)
    for (int64_t g = 0; g < ng; ++g) {
      float sum = 0.0f;
      for (int64_t i = 0; i < W; ++i)
        for (int j = 0; j < 8; ++j) {
          const float v = bf16f(x[m * K + g * G + 8 * i + j]);
          xp[m * K + g * G + W * j + i] = v;
          sum += v;
        }
      xs[m * ng + g] = sum;
    }
#pragma omp parallel
  {
    if (W == 4) w4_gemv_rows(xp, xs, w, scales, biases, M, N, K, 4, y);
    else if (W == 8) w4_gemv_rows(xp, xs, w, scales, biases, M, N, K, 8, y);
    else w4_gemv_rows(xp, xs, w, scales, biases, M, N, K, 16, y);
  }
  free(xp);
  free(xs);
  return used;
}

/* y[m,n] (fp32) for x [M,K] bf16, w [N,K/8], scales/biases [N,K/G] bf16.
 * Returns the number of threads used, or -1 on a bad argument. */
int sq_cpu_w4a16_matmul(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                        const uint16_t* biases, int64_t M, int64_t N, int64_t K, int G,
                        float* y, int threads) {
  if (G % 8 || K % G || K % 8 || M < 1 || N < 1) return -1;
  const int used = set_threads(threads);
  if (M <= GEMV_MAXM && (G == 32 || G == 64 || G == 128))
    return w4_gemv(x, w, scales, biases, M, N, K, G, y, used);
  float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K));
  if (!xf) return -1;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M * K; ++i) xf[i] = bf16f(x[i]);
  const int64_t ng = K / G, kw = K / 8;
  const int64_t nblk = (N + NB - 1) / NB;
  int fail = 0;
#pragma omp parallel
  {
    float* panel = (float*)aligned_alloc(64, sizeof(float) * KC * NB);
    float* acc = (float*)aligned_alloc(64, sizeof(float) * (size_t)M * NB);
    if (!panel || !acc) {
#pragma omp atomic write
      fail = 1;
    }
#pragma omp for schedule(dynamic, 1)
    for (int64_t nb = 0; nb < nblk; ++nb) {
      if (!panel || !acc) continue;
      const int64_t n0 = nb * NB;
      memset(acc, 0, sizeof(float) * (size_t)M * NB);
      for (int64_t k0 = 0; k0 < K; k0 += KC) {
        const int64_t kc = K - k0 < KC ? K - k0 : KC;
        /* dequantize the panel: panel[k][r] = w[n0 + r][k0 + k] */
        for (int64_t c = 0; c < kc / 8; ++c) {
          const int64_t word = k0 / 8 + c, g = (8 * word) / G;
          uint32_t wv[NB];
          float sv[NB], bv[NB];
          for (int r = 0; r < NB; ++r) {
            const int64_t n = n0 + r < N ? n0 + r : N - 1;
            wv[r] = w[n * kw + word];
            sv[r] = bf16f(scales[n * ng + g]);
            bv[r] = bf16f(biases[n * ng + g]);
          }
          for (int j = 0; j < 8; ++j) {
            float* p = panel + (8 * c + j) * NB;
            for (int r = 0; r < NB; ++r) p[r] = (float)((wv[r] >> (4 * j)) & 15u) * sv[r] + bv[r];
          }
        }
        /* acc[m][r] += x[m][k0 + k] * panel[k][r], MB rows at a time (MB
         * independent 16-lane accumulators per k step) */
        for (int64_t m0 = 0; m0 < M; m0 += MB) {
          const int64_t mc = M - m0 < MB ? M - m0 : MB;
          if (mc == 1) {
            /* one row: four chains over interleaved k keep the FMA unit busy */
            float a[4][NB];
            const float* x0 = xf + m0 * K + k0;
            for (int r = 0; r < NB; ++r) {
              a[0][r] = acc[m0 * NB + r];
              a[1][r] = a[2][r] = a[3][r] = 0.0f;
            }
            for (int64_t k = 0; k < kc; k += 4)
              for (int i = 0; i < 4; ++i) {
                const float xv = x0[k + i];
                const float* p = panel + (k + i) * NB;
                for (int r = 0; r < NB; ++r) a[i][r] += xv * p[r];
              }
            for (int r = 0; r < NB; ++r) acc[m0 * NB + r] = (a[0][r] + a[1][r]) + (a[2][r] + a[3][r]);
            continue;
          }
          float a[MB][NB];
          const float* xr[MB];
          for (int i = 0; i < MB; ++i) {
            const int64_t m = m0 + (i < mc ? i : 0);
            xr[i] = xf + m * K + k0;
            for (int r = 0; r < NB; ++r) a[i][r] = i < mc ? acc[(m0 + i) * NB + r] : 0.0f;
          }
          for (int64_t k = 0; k < kc; ++k) {
            const float* p = panel + k * NB;
            for (int i = 0; i < MB; ++i) {
              const float xv = xr[i][k];
              for (int r = 0; r < NB; ++r) a[i][r] += xv * p[r];
            }
          }
          for (int i = 0; i < mc; ++i)
            for (int r = 0; r < NB; ++r) acc[(m0 + i) * NB + r] = a[i][r];
        }
      }
      const int64_t nc = N - n0 < NB ? N - n0 : NB;
      for (int64_t m = 0; m < M; ++m)
        for (int64_t r = 0; r < nc; ++r) y[m * N + n0 + r] = acc[m * NB + r];
    }
    free(panel);
    free(acc);
  }
  free(xf);
  return fail ? -1 : used;
}

/* The previous name, kept for callers that time the GEMV. */
int sq_cpu_w4a16_gemv(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                      const uint16_t* biases, int64_t M, int64_t N, int64_t K, int G, float* y,
                      int threads) {
  return sq_cpu_w4a16_matmul(x, w, scales, biases, M, N, K, G, y, threads);
}

/* ---------------------------------------------------------------------- */
/* W8A8                                                                    */
/* ---------------------------------------------------------------------- */

/* y[m,n] = (float(sum_k qa[m,k] * wq[n,k]) * sa[m]) * sw[n], with qa, sa
 * the per-token int8 quantization of x (bf16; scale 1 for an all-zero row).
 * The integer dots vectorize without reassociation; the fp32 epilogue keeps
 * the oracle's multiply order. Returns threads used or -1. */
__attribute__((optimize("no-associative-math")))
int sq_cpu_w8a8_linear(const uint16_t* x, const int8_t* wq, const float* sw, int64_t M,
                       int64_t N, int64_t K, float* y, int threads) {
  if (M < 1 || N < 1 || K < 1) return -1;
  const int used = set_threads(threads);
  int8_t* qa = (int8_t*)malloc((size_t)(M * K));
  float* sa = (float*)malloc(sizeof(float) * (size_t)M);
  if (!qa || !sa) {
    free(qa);
    free(sa);
    return -1;
  }
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) amax = fmaxf(amax, fabsf(bf16f(x[m * K + k])));
    const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
    sa[m] = s;
    for (int64_t k = 0; k < K; ++k) {
      float v = rintf(bf16f(x[m * K + k]) / s);
      v = v > 127.0f ? 127.0f : (v < -127.0f ? -127.0f : v);
      qa[m * K + k] = (int8_t)v;
    }
  }
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const int8_t* wr = wq + n * K;
    for (int64_t m = 0; m < M; ++m) {
      const int8_t* ar = qa + m * K;
      int32_t acc = 0;
      for (int64_t k = 0; k < K; ++k) acc += (int32_t)ar[k] * (int32_t)wr[k];
      y[m * N + n] = (float)acc * sa[m] * sw[n];
    }
  }
  free(qa);
  free(sa);
  return used;
}

/* ---------------------------------------------------------------------- */
/* INT8-KV decode attention                                                */
/* ---------------------------------------------------------------------- */

#define SDPA_MAXG 16   /* query heads per KV head */
#define SDPA_MAXD 256

/* q [B,Hq,D] bf16; kc/vc [B,Hkv,N,D] int8; ks/vs [B,Hkv,N] fp16 bits;
 * out [B,Hq,D] fp32. Returns threads used or -1. */
int sq_cpu_int8kv_sdpa(const uint16_t* q, const int8_t* kc, const uint16_t* ks,
                       const int8_t* vc, const uint16_t* vs, int64_t B, int64_t Hq,
                       int64_t Hkv, int64_t N, int64_t D, float scale, float* out,
                       int threads) {
  if (B < 1 || Hkv < 1 || Hq % Hkv || Hq / Hkv > SDPA_MAXG || D > SDPA_MAXD || D % 16 || N < 1)
    return -1;
  const int used = set_threads(threads);
  const int64_t gq = Hq / Hkv, units = B * Hkv;
  int64_t splits = (2 * used + units - 1) / units;
  if (splits > N) splits = N;
  const int64_t per = (N + splits - 1) / splits;
  /* partials: (max, sum, acc[D]) per (unit, split, query head) */
  const int64_t stride = 2 + D;
  float* part = (float*)malloc(sizeof(float) * (size_t)(units * splits * gq * stride));
  if (!part) return -1;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t job = 0; job < units * splits; ++job) {
    const int64_t u = job / splits, sp = job % splits;
    const int64_t b = u / Hkv, h = u % Hkv;
    const int64_t t0 = sp * per, t1 = t0 + per < N ? t0 + per : N;
    float qf[SDPA_MAXG][SDPA_MAXD], acc[SDPA_MAXG][SDPA_MAXD], kf[SDPA_MAXD];
    float mx[SDPA_MAXG], sm[SDPA_MAXG];
    for (int64_t g = 0; g < gq; ++g) {
      const uint16_t* qr = q + (b * Hq + h * gq + g) * D;
      for (int64_t d = 0; d < D; ++d) {
        qf[g][d] = bf16f(qr[d]) * scale;
        acc[g][d] = 0.0f;
      }
      mx[g] = -INFINITY;
      sm[g] = 0.0f;
    }
    const int8_t* kb = kc + (b * Hkv + h) * N * D;
    const int8_t* vb = vc + (b * Hkv + h) * N * D;
    const uint16_t* ksb = ks + (b * Hkv + h) * N;
    const uint16_t* vsb = vs + (b * Hkv + h) * N;
    for (int64_t t = t0; t < t1; ++t) {
      const float kscale = f16f(ksb[t]), vscale = f16f(vsb[t]);
      for (int64_t d = 0; d < D; ++d) kf[d] = (float)kb[t * D + d] * kscale;
      for (int64_t g = 0; g < gq; ++g) {
        float s = 0.0f;
        for (int64_t d = 0; d < D; ++d) s += qf[g][d] * kf[d];
        if (s > mx[g]) {
          const float c = expf(mx[g] - s);
          sm[g] *= c;
          for (int64_t d = 0; d < D; ++d) acc[g][d] *= c;
          mx[g] = s;
        }
        const float p = expf(s - mx[g]);
        sm[g] += p;
        const float pv = p * vscale;
        for (int64_t d = 0; d < D; ++d) acc[g][d] += pv * (float)vb[t * D + d];
      }
    }
    for (int64_t g = 0; g < gq; ++g) {
      float* o = part + ((u * splits + sp) * gq + g) * stride;
      o[0] = mx[g];
      o[1] = sm[g];
      for (int64_t d = 0; d < D; ++d) o[2 + d] = acc[g][d];
    }
  }
  /* merge the splits by log-sum-exp */
#pragma omp parallel for schedule(static)
  for (int64_t ug = 0; ug < units * gq; ++ug) {
    const int64_t u = ug / gq, g = ug % gq;
    float m = -INFINITY;
    for (int64_t sp = 0; sp < splits; ++sp) m = fmaxf(m, part[((u * splits + sp) * gq + g) * stride]);
    float den = 0.0f, o[SDPA_MAXD];
    for (int64_t d = 0; d < D; ++d) o[d] = 0.0f;
    for (int64_t sp = 0; sp < splits; ++sp) {
      const float* p = part + ((u * splits + sp) * gq + g) * stride;
      if (p[1] == 0.0f) continue;
      const float c = expf(p[0] - m);
      den += p[1] * c;
      for (int64_t d = 0; d < D; ++d) o[d] += p[2 + d] * c;
    }
    const int64_t b = u / Hkv, h = u % Hkv;
    float* dst = out + (b * Hq + h * gq + g) * D;
    for (int64_t d = 0; d < D; ++d) dst[d] = o[d] / den;
  }
  free(part);
  return used;
}
