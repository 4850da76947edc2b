/*
 * sparkq_oracle.h -- CPU restatement of Spark-MLX-LLM's quantized-linear hot
 * path, used ONLY as the checker: by tests/, by __graft_entry__.smoke() and by
 * bench.py's cpu_baseline leg. No product code links or calls it.
 *
 * Each function cites the reference file:line whose algorithm it restates
 * (paths relative to the reference repository; X/ = extensions/spark-mlx-ext/).
 *
 * Pinning (how each function is checked independently of its own formula) is
 * listed in tests/test_oracle.py; functions that only an import of MLX could
 * pin are marked "parity unpinned" below.
 */
#ifndef SPARKQ_ORACLE_H_
#define SPARKQ_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes shared with include/sparkq.h */
#define SQ_F32 0
#define SQ_F16 1
#define SQ_BF16 2

/* --- scalar conversions ------------------------------------------------ */
/* bf16 round-to-nearest-even, spark_mlx_llm/conversion.py:154-159
 * (NaN kept quiet instead of the converter's finite-only requirement). */
uint16_t sq_f32_to_bf16(float f);
float sq_bf16_to_f32(uint16_t h);
/* IEEE binary16 round-to-nearest-even (subnormals, overflow to inf). */
uint16_t sq_f32_to_f16(float f);
float sq_f16_to_f32(uint16_t h);
/* 16-bit storage of dtype (SQ_F16 or SQ_BF16) */
uint16_t sq_round16(float f, int dtype);
float sq_widen16(uint16_t h, int dtype);

/* --- deterministic generator ------------------------------------------- */
/* splitmix64 -> Box-Muller normal samples, std * N(0,1) rounded to fp32.
 * stream selects an independent sub-stream (e.g. hash of config/layer/tensor).
 * The reference's mx.random.normal stream is not reproducible here
 * (parity unpinned; inputs are the build's own documented generator). */
void sq_randn(uint64_t seed, uint64_t stream, float std, float* out,
              int64_t n);
/* same, rounded to a 16-bit dtype (values stored as uint16) */
void sq_randn16(uint64_t seed, uint64_t stream, float std, int dtype,
                uint16_t* out, int64_t n);

/* --- W4 affine format -------------------------------------------------- */
/* _packed (spark_mlx_llm/conversion.py:429-433): word k/8 of row n holds
 * code k at bits 4*(k%8). codes [N,K] (0..15) -> words [N,K/8]. */
void sq_pack4(const uint8_t* codes, uint32_t* words, int64_t N, int64_t K);
void sq_unpack4(const uint32_t* words, uint8_t* codes, int64_t N, int64_t K);

/* Affine 4-bit quantizer with the formula the benchmark states for
 * mx.quantize(bits=4, group_size=G): per group scale = (max-min)/15,
 * bias = min, both rounded to dtype; codes = clamp(rint((w-b)/s), 0, 15)
 * from the rounded scale/bias; a zero scale gives code 0.
 * Bit-identity with MLX's own mx.quantize is parity unpinned (MLX absent).
 * w holds values already representable in dtype. */
void sq_w4_quantize(const float* w, int64_t N, int64_t K, int G, int dtype,
                    uint32_t* wq, uint16_t* scales, uint16_t* biases);

/* The converter's BF16 -> W4 quantizer (spark_mlx_llm/conversion.py:564-583):
 * groups of G; lower = min(min,0), upper = max(max,0); scale = (upper-lower)/15
 * (1 if 0) rounded to bf16; zero = clip(rint(-lower/s), 0, 15);
 * code = clip(rint(w/s) + zero, 0, 15); bias = bf16(-zero*s).
 * Pinned at G32 against vectors the converter itself wrote
 * (tests/golden/converter_vectors.npz, tests/golden/make_converter_vectors.py). */
void sq_w4_quantize_converter(const float* w, int64_t N, int64_t K, int G,
                              uint32_t* wq, uint16_t* scales,
                              uint16_t* biases);

/* fp32 dequantization fmaf(q, s, b): the exact q*s+b rounded once. (q*s is
 * exact unless it overflows, so mul-then-add agrees except there.)
 * Per-element decode of X/spark_mlx_ext/_w4a16_multirow_sources.py:31-39. */
void sq_w4_dequantize(const uint32_t* wq, const uint16_t* scales,
                      const uint16_t* biases, int64_t N, int64_t K, int G,
                      int sdtype, float* out);

/* y[m,n] = sum_k x[m,k] * deq[n,k] accumulated in fp64 (the float32
 * dequantize-then-matmul reference of mx.quantized_matmul, transpose=True,
 * spark_mlx_llm/ops/linear.py:181-191). x is [M,K] 16-bit in xdtype. */
void sq_w4a16_matmul(const uint16_t* x, int xdtype, const uint32_t* wq,
                     const uint16_t* scales, const uint16_t* biases,
                     int64_t M, int64_t N, int64_t K, int G, double* y);

/* --- W8A16 ------------------------------------------------------------- */
/* y[m,n] = scale[n] * sum_k x[m,k] * w[n,k] in fp64: the fp32 dot times the
 * channel scale of w8a16_per_channel (X/src/kernels/w8a16_matvec.metal:
 * 12-31), computed exactly enough to serve as its reference. x is [M,K]
 * 16-bit in xdtype, w [N,K] int8, scales [N] fp32. */
void sq_w8a16_matmul(const uint16_t* x, int xdtype, const int8_t* w,
                     const float* scales, int64_t M, int64_t N, int64_t K,
                     double* y);

/* --- W8A8 -------------------------------------------------------------- */
/* Per-token quantizer, X/src/kernels/w8a8_quantize.metal:11-27:
 * amax = max|x|; scale = amax > 0 ? amax/127 : 1; q = clamp(rint(x/scale),
 * -127, 127). x [M,K] fp32 values (exact widening of the 16-bit inputs). */
void sq_a8_quantize(const float* x, int64_t M, int64_t K, int8_t* q,
                    float* scales);

/* Per-output-channel symmetric weights for the benchmark's W8A8 workload:
 * scale = max|w[n,:]|/127 (1 if 0), q = clamp(rint(w/scale), -127, 127);
 * the converter's channel formula (spark_mlx_llm/conversion.py:570,586). */
void sq_w8_quantize_channel(const float* w, int64_t N, int64_t K, int8_t* q,
                            float* scales);

/* Unpack of MLX affine W8 storage to signed int8 (byte XOR 0x80),
 * spark_mlx_llm/ops/linear.py:323,365. words [N,K/4]. */
void sq_w8_unpack_affine(const uint32_t* words, int64_t N, int64_t K,
                         int8_t* out);

/* C = A . B^T with exact integer accumulation (int64, range-checked);
 * returns 0 on success, -1 if any sum leaves int32. */
int sq_int8_matmul(const int8_t* a, const int8_t* b, int64_t M, int64_t N,
                   int64_t K, int32_t* c);

/* Epilogue T(float(acc)*sa[m]*sw[n] + bias[n]) of
 * X/src/kernels/w8a8_tensor.metal:63, evaluated as
 * fmaf(float(acc) * sa[m], sw[n], bias[n]) in fp32 (bias NULL = 0). */
void sq_w8a8_epilogue(const int32_t* acc, const float* sa, const float* sw,
                      const float* bias, int64_t M, int64_t N, float* y);

/* --- INT8 KV ----------------------------------------------------------- */
/* Symmetric per-row KV quantizer for the s8 + fp16-scale format:
 * scale = fp16(amax/127) (1 if that is 0); code = clamp(rint(x/scale),
 * -127, 127) with the fp16-rounded scale. x [R,D] fp32 values. */
void sq_kv_quantize_s8(const float* x, int64_t R, int64_t D, int8_t* codes,
                       uint16_t* scales_f16);

/* MLX affine 8-bit KV quantizer for the (packed, scales, biases) tuple
 * (the QuantizedKVCache format consumed at
 * X/spark_mlx_ext/int8_quantized_sdpa.py:207-222): per group of G dims
 * scale = (max-min)/255, bias = min, rounded to dtype; code = clamp(rint((x-b)
 * /s), 0, 255). Bit-identity with mlx-lm's quantizer is parity unpinned. */
void sq_kv_quantize_affine_u8(const float* x, int64_t R, int64_t D, int G,
                              int dtype, uint32_t* packed, uint16_t* scales,
                              uint16_t* biases);

/* Decode attention reference in fp64: dequantize K/V, scores =
 * scale * q.K^T, softmax, out = p.V (the staged arithmetic of _fallback,
 * X/spark_mlx_ext/int8_quantized_sdpa.py:122-153, with all N tokens visible).
 * q [B,Hq,D] fp32 values; K/V given as already-dequantized fp32 [B,Hkv,N,D].
 * out [B,Hq,D] fp64. */
void sq_sdpa_decode(const float* q, const float* kdq, const float* vdq,
                    int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                    double scale, double* out);

/* dequantizers feeding sq_sdpa_decode */
void sq_kv_dequantize_s8(const int8_t* codes, const uint16_t* scales_f16,
                         int64_t R, int64_t D, float* out);
void sq_kv_dequantize_affine_u8(const uint32_t* packed, const uint16_t* scales,
                                const uint16_t* biases, int64_t R, int64_t D,
                                int G, int dtype, float* out);

#ifdef __cplusplus
}
#endif

#endif /* SPARKQ_ORACLE_H_ */
