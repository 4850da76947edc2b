/*
 * sparkq_oracle.c -- CPU restatement of the quantized-linear hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg. The product library (libsparkq.so) never
 * links, loads or calls this file.
 *
 * Built with -ffp-contract=off so that every a*b+c below rounds twice unless
 * fmaf() is written explicitly; see oracle/Makefile.
 */
#include "sparkq_oracle.h"

#include <math.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* scalar conversions                                                        */
/* ------------------------------------------------------------------------ */

static uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* spark_mlx_llm/conversion.py:154-159: (w + 0x7FFF + ((w >> 16) & 1)) >> 16 */
uint16_t sq_f32_to_bf16(float f) {
  uint32_t w = f2u(f);
  if ((w & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((w >> 16) | 0x0040u);
  return (uint16_t)((w + 0x7FFFu + ((w >> 16) & 1u)) >> 16);
}

float sq_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t sq_f32_to_f16(float f) {
  uint32_t x = f2u(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t a = x & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);      /* NaN */
  if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);     /* >= 65520 */
  if (a < 0x38800000u) {                                       /* < 2^-14 */
    float r = rintf(u2f(a) * 16777216.0f); /* exact scale by 2^24, RNE */
    return (uint16_t)(sign | (uint32_t)r);
  }
  uint32_t rounded = a + 0xFFFu + ((a >> 13) & 1u);
  return (uint16_t)(sign | ((rounded - 0x38000000u) >> 13));
}

float sq_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  if (e == 0) {
    float v = (float)m * (1.0f / 16777216.0f); /* m * 2^-24, exact */
    return sign ? -v : v;
  }
  if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t sq_round16(float f, int dtype) {
  return dtype == SQ_F16 ? sq_f32_to_f16(f) : sq_f32_to_bf16(f);
}

float sq_widen16(uint16_t h, int dtype) {
  return dtype == SQ_F16 ? sq_f16_to_f32(h) : sq_bf16_to_f32(h);
}

/* ------------------------------------------------------------------------ */
/* generator: splitmix64 -> Box-Muller                                       */
/* ------------------------------------------------------------------------ */

static uint64_t splitmix64(uint64_t* s) {
  uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void sq_randn(uint64_t seed, uint64_t stream, float std, float* out,
              int64_t n) {
  uint64_t s = seed ^ (stream * 0xD1B54A32D192ED03ull);
  (void)splitmix64(&s);
  for (int64_t i = 0; i < n; i += 2) {
    uint64_t a = splitmix64(&s), b = splitmix64(&s);
    double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
    double r = sqrt(-2.0 * log(u1));
    double t = 6.283185307179586476925 * u2;
    out[i] = (float)(std * r * cos(t));
    if (i + 1 < n) out[i + 1] = (float)(std * r * sin(t));
  }
}

void sq_randn16(uint64_t seed, uint64_t stream, float std, int dtype,
                uint16_t* out, int64_t n) {
  const int64_t chunk = 4096;
  float buf[4096];
  /* generate in one stream, converting chunk by chunk */
  uint64_t s = seed ^ (stream * 0xD1B54A32D192ED03ull);
  (void)splitmix64(&s);
  for (int64_t base = 0; base < n; base += chunk) {
    int64_t cnt = n - base < chunk ? n - base : chunk;
    for (int64_t i = 0; i < cnt; i += 2) {
      uint64_t a = splitmix64(&s), b = splitmix64(&s);
      double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
      double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
      double r = sqrt(-2.0 * log(u1));
      double t = 6.283185307179586476925 * u2;
      buf[i] = (float)(std * r * cos(t));
      if (i + 1 < cnt) buf[i + 1] = (float)(std * r * sin(t));
    }
    for (int64_t i = 0; i < cnt; ++i) out[base + i] = sq_round16(buf[i], dtype);
  }
}

/* ------------------------------------------------------------------------ */
/* W4 affine                                                                 */
/* ------------------------------------------------------------------------ */

/* spark_mlx_llm/conversion.py:429-433 */
void sq_pack4(const uint8_t* codes, uint32_t* words, int64_t N, int64_t K) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t w = 0; w < K / 8; ++w) {
      uint32_t v = 0;
      for (int j = 0; j < 8; ++j)
        v |= (uint32_t)(codes[n * K + 8 * w + j] & 15u) << (4 * j);
      words[n * (K / 8) + w] = v;
    }
}

void sq_unpack4(const uint32_t* words, uint8_t* codes, int64_t N, int64_t K) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k)
      codes[n * K + k] =
          (uint8_t)((words[n * (K / 8) + k / 8] >> (4 * (k % 8))) & 15u);
}

void sq_w4_quantize(const float* w, int64_t N, int64_t K, int G, int dtype,
                    uint32_t* wq, uint16_t* scales, uint16_t* biases) {
  const int64_t ng = K / G;
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t g = 0; g < ng; ++g) {
      const float* v = w + n * K + g * G;
      float mn = v[0], mx = v[0];
      for (int i = 1; i < G; ++i) {
        mn = v[i] < mn ? v[i] : mn;
        mx = v[i] > mx ? v[i] : mx;
      }
      uint16_t s16 = sq_round16((mx - mn) / 15.0f, dtype);
      uint16_t b16 = sq_round16(mn, dtype);
      float s = sq_widen16(s16, dtype), b = sq_widen16(b16, dtype);
      scales[n * ng + g] = s16;
      biases[n * ng + g] = b16;
      for (int i = 0; i < G; ++i) {
        float q = 0.0f;
        if (s != 0.0f) {
          q = rintf((v[i] - b) / s);
          q = q < 0.0f ? 0.0f : (q > 15.0f ? 15.0f : q);
        }
        int64_t k = g * G + i;
        uint32_t* word = &wq[n * (K / 8) + k / 8];
        if (k % 8 == 0) *word = 0;
        *word |= (uint32_t)q << (4 * (k % 8));
      }
    }
  }
}

/* spark_mlx_llm/conversion.py:564-583 (kind "bf16-int4") */
void sq_w4_quantize_converter(const float* w, int64_t N, int64_t K, int G,
                              uint32_t* wq, uint16_t* scales,
                              uint16_t* biases) {
  const int64_t ng = K / G;
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t g = 0; g < ng; ++g) {
      const float* v = w + n * K + g * G;
      float lower = v[0], upper = v[0];
      for (int i = 1; i < G; ++i) {
        lower = v[i] < lower ? v[i] : lower;
        upper = v[i] > upper ? v[i] : upper;
      }
      lower = lower < 0.0f ? lower : 0.0f;
      upper = upper > 0.0f ? upper : 0.0f;
      float s = (upper - lower) / 15.0f;
      if (s == 0.0f) s = 1.0f;
      uint16_t s16 = sq_f32_to_bf16(s);
      float rs = sq_bf16_to_f32(s16);
      float zero = rintf(-lower / rs);
      zero = zero < 0.0f ? 0.0f : (zero > 15.0f ? 15.0f : zero);
      scales[n * ng + g] = s16;
      biases[n * ng + g] = sq_f32_to_bf16(-zero * rs);
      for (int i = 0; i < G; ++i) {
        float q = rintf(v[i] / rs) + zero;
        q = q < 0.0f ? 0.0f : (q > 15.0f ? 15.0f : q);
        int64_t k = g * G + i;
        uint32_t* word = &wq[n * (K / 8) + k / 8];
        if (k % 8 == 0) *word = 0;
        *word |= (uint32_t)q << (4 * (k % 8));
      }
    }
  }
}

void sq_w4_dequantize(const uint32_t* wq, const uint16_t* scales,
                      const uint16_t* biases, int64_t N, int64_t K, int G,
                      int sdtype, float* out) {
  const int64_t ng = K / G;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      float q = (float)((wq[n * (K / 8) + k / 8] >> (4 * (k % 8))) & 15u);
      float s = sq_widen16(scales[n * ng + k / G], sdtype);
      float b = sq_widen16(biases[n * ng + k / G], sdtype);
      out[n * K + k] = fmaf(q, s, b); /* one rounding, also at overflow */
    }
}

void sq_w4a16_matmul(const uint16_t* x, int xdtype, const uint32_t* wq,
                     const uint16_t* scales, const uint16_t* biases,
                     int64_t M, int64_t N, int64_t K, int G, double* y) {
  const int64_t ng = K / G;
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t m = 0; m < M; ++m) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        float q = (float)((wq[n * (K / 8) + k / 8] >> (4 * (k % 8))) & 15u);
        float s = sq_widen16(scales[n * ng + k / G], xdtype);
        float b = sq_widen16(biases[n * ng + k / G], xdtype);
        float wv = fmaf(q, s, b);
        acc += (double)sq_widen16(x[m * K + k], xdtype) * (double)wv;
      }
      y[m * N + n] = acc;
    }
  }
}

/* X/src/kernels/w8a16_matvec.metal:12-31 (sum, then times the scale) */
void sq_w8a16_matmul(const uint16_t* x, int xdtype, const int8_t* w,
                     const float* scales, int64_t M, int64_t N, int64_t K,
                     double* y) {
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t m = 0; m < M; ++m) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k)
        acc += (double)sq_widen16(x[m * K + k], xdtype) * (double)w[n * K + k];
      y[m * N + n] = acc * (double)scales[n];
    }
  }
}

/* ------------------------------------------------------------------------ */
/* W8A8                                                                      */
/* ------------------------------------------------------------------------ */

/* X/src/kernels/w8a8_quantize.metal:11-27 */
void sq_a8_quantize(const float* x, int64_t M, int64_t K, int8_t* q,
                    float* scales) {
  for (int64_t m = 0; m < M; ++m) {
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      float a = fabsf(x[m * K + k]);
      amax = a > amax ? a : amax;
    }
    float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    scales[m] = scale;
    for (int64_t k = 0; k < K; ++k) {
      float v = rintf(x[m * K + k] / scale);
      v = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
      q[m * K + k] = (int8_t)v;
    }
  }
}

/* spark_mlx_llm/conversion.py:570,586 with the fp32 scale kept */
void sq_w8_quantize_channel(const float* w, int64_t N, int64_t K, int8_t* q,
                            float* scales) {
  for (int64_t n = 0; n < N; ++n) {
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      float a = fabsf(w[n * K + k]);
      amax = a > amax ? a : amax;
    }
    float scale = amax / 127.0f;
    if (scale == 0.0f) scale = 1.0f;
    scales[n] = scale;
    for (int64_t k = 0; k < K; ++k) {
      float v = rintf(w[n * K + k] / scale);
      v = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
      q[n * K + k] = (int8_t)v;
    }
  }
}

/* spark_mlx_llm/ops/linear.py:323,365 */
void sq_w8_unpack_affine(const uint32_t* words, int64_t N, int64_t K,
                         int8_t* out) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      uint32_t byte = (words[n * (K / 4) + k / 4] >> (8 * (k % 4))) & 255u;
      out[n * K + k] = (int8_t)(uint8_t)(byte ^ 0x80u);
    }
}

int sq_int8_matmul(const int8_t* a, const int8_t* b, int64_t M, int64_t N,
                   int64_t K, int32_t* c) {
  int ok = 0;
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      int64_t acc = 0;
      for (int64_t k = 0; k < K; ++k)
        acc += (int64_t)a[m * K + k] * (int64_t)b[n * K + k];
      if (acc > 2147483647LL || acc < -2147483648LL) ok = -1;
      c[m * N + n] = (int32_t)acc;
    }
  return ok;
}

/* X/src/kernels/w8a8_tensor.metal:63 */
void sq_w8a8_epilogue(const int32_t* acc, const float* sa, const float* sw,
                      const float* bias, int64_t M, int64_t N, float* y) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      float t = (float)acc[m * N + n] * sa[m];
      y[m * N + n] = fmaf(t, sw[n], bias ? bias[n] : 0.0f);
    }
}

/* ------------------------------------------------------------------------ */
/* INT8 KV                                                                   */
/* ------------------------------------------------------------------------ */

void sq_kv_quantize_s8(const float* x, int64_t R, int64_t D, int8_t* codes,
                       uint16_t* scales_f16) {
  for (int64_t r = 0; r < R; ++r) {
    float amax = 0.0f;
    for (int64_t d = 0; d < D; ++d) {
      float a = fabsf(x[r * D + d]);
      amax = a > amax ? a : amax;
    }
    uint16_t s16 = sq_f32_to_f16(amax / 127.0f);
    if (sq_f16_to_f32(s16) == 0.0f) s16 = 0x3C00u; /* 1.0 */
    float s = sq_f16_to_f32(s16);
    scales_f16[r] = s16;
    for (int64_t d = 0; d < D; ++d) {
      float v = rintf(x[r * D + d] / s);
      v = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
      codes[r * D + d] = (int8_t)v;
    }
  }
}

void sq_kv_quantize_affine_u8(const float* x, int64_t R, int64_t D, int G,
                              int dtype, uint32_t* packed, uint16_t* scales,
                              uint16_t* biases) {
  const int64_t ng = D / G;
  for (int64_t r = 0; r < R; ++r)
    for (int64_t g = 0; g < ng; ++g) {
      const float* v = x + r * D + g * G;
      float mn = v[0], mx = v[0];
      for (int i = 1; i < G; ++i) {
        mn = v[i] < mn ? v[i] : mn;
        mx = v[i] > mx ? v[i] : mx;
      }
      uint16_t s16 = sq_round16((mx - mn) / 255.0f, dtype);
      uint16_t b16 = sq_round16(mn, dtype);
      float s = sq_widen16(s16, dtype), b = sq_widen16(b16, dtype);
      scales[r * ng + g] = s16;
      biases[r * ng + g] = b16;
      for (int i = 0; i < G; ++i) {
        float q = 0.0f;
        if (s != 0.0f) {
          q = rintf((v[i] - b) / s);
          q = q < 0.0f ? 0.0f : (q > 255.0f ? 255.0f : q);
        }
        int64_t d = g * G + i;
        uint32_t* word = &packed[r * (D / 4) + d / 4];
        if (d % 4 == 0) *word = 0;
        *word |= (uint32_t)q << (8 * (d % 4));
      }
    }
}

void sq_kv_dequantize_s8(const int8_t* codes, const uint16_t* scales_f16,
                         int64_t R, int64_t D, float* out) {
  for (int64_t r = 0; r < R; ++r) {
    float s = sq_f16_to_f32(scales_f16[r]);
    for (int64_t d = 0; d < D; ++d) out[r * D + d] = (float)codes[r * D + d] * s;
  }
}

/* value = u8 * scale + bias, X/spark_mlx_ext/_int8_sdpa_sources.py:105-111 */
void sq_kv_dequantize_affine_u8(const uint32_t* packed, const uint16_t* scales,
                                const uint16_t* biases, int64_t R, int64_t D,
                                int G, int dtype, float* out) {
  const int64_t ng = D / G;
  for (int64_t r = 0; r < R; ++r)
    for (int64_t d = 0; d < D; ++d) {
      float u = (float)((packed[r * (D / 4) + d / 4] >> (8 * (d % 4))) & 255u);
      float s = sq_widen16(scales[r * ng + d / G], dtype);
      float b = sq_widen16(biases[r * ng + d / G], dtype);
      out[r * D + d] = u * s + b; /* u*s exact (8+8 bits): one rounding */
    }
}

/* X/spark_mlx_ext/int8_quantized_sdpa.py:122-153 with L = 1 */
void sq_sdpa_decode(const float* q, const float* kdq, const float* vdq,
                    int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                    double scale, double* out) {
  const int64_t rep = Hq / Hkv;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < Hq; ++h) {
      const int64_t kh = h / rep;
      const float* qq = q + (b * Hq + h) * D;
      const float* kk = kdq + (b * Hkv + kh) * N * D;
      const float* vv = vdq + (b * Hkv + kh) * N * D;
      double* o = out + (b * Hq + h) * D;
      double mx = -INFINITY;
      /* two passes: max, then exp-sum and weighted values */
      for (int64_t t = 0; t < N; ++t) {
        double s = 0.0;
        for (int64_t d = 0; d < D; ++d) s += (double)qq[d] * kk[t * D + d];
        s *= scale;
        mx = s > mx ? s : mx;
      }
      double z = 0.0;
      for (int64_t d = 0; d < D; ++d) o[d] = 0.0;
      for (int64_t t = 0; t < N; ++t) {
        double s = 0.0;
        for (int64_t d = 0; d < D; ++d) s += (double)qq[d] * kk[t * D + d];
        double p = exp(s * scale - mx);
        z += p;
        for (int64_t d = 0; d < D; ++d) o[d] += p * vv[t * D + d];
      }
      for (int64_t d = 0; d < D; ++d) o[d] /= z;
    }
}
