/*
 * sparkq.h -- C-ABI of the MI355X (gfx950) quantized-linear hot path.
 *
 * One shared library, libsparkq.so, exports these entry points. Every entry
 * point:
 *   - takes caller-owned device pointers and a hipStream_t (passed as void*,
 *     NULL means the default stream), enqueues its kernels on that stream and
 *     returns without synchronising;
 *   - never allocates device memory: scratch space, where an operation needs
 *     it, is a caller-provided workspace sized by the matching
 *     *_workspace_bytes() query;
 *   - returns SPARKQ_OK (0) or a negative status, with a thread-local message
 *     available from sparkq_last_error().
 * Tensors are row-major and densely packed unless a stride argument says
 * otherwise. Element types are given by the sparkq_dtype codes below.
 *
 * Reference interfaces (paths relative to the Spark-MLX-LLM repository; X/ is
 * extensions/spark-mlx-ext/) are cited at each entry point.
 */
#ifndef SPARKQ_H_
#define SPARKQ_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types. */
enum sparkq_dtype {
  SPARKQ_F32 = 0,
  SPARKQ_F16 = 1,
  SPARKQ_BF16 = 2,
};

/* KV-cache storage formats for the INT8-KV decode attention. */
enum sparkq_kv_format {
  /* Symmetric signed int8 codes [B,Hkv,Ncap,D] plus one fp16 scale per
   * (batch, KV head, token) [B,Hkv,Ncap]; value = code * scale. */
  SPARKQ_KV_S8_F16SCALE = 0,
  /* MLX affine 8-bit tuple (packed, scales, biases): packed uint32
   * [B,Hkv,Ncap,D/4] with byte j of word w holding dim 4w+j, scales and
   * biases [B,Hkv,Ncap,D/G] in the query dtype; value = u8 * scale + bias. */
  SPARKQ_KV_AFFINE_U8 = 1,
  /* MLX affine 4-bit and 2-bit tuples: packed uint32 [B,Hkv,Ncap,D*bits/32],
   * code of dim cpw*w+j at bits (bits*j) of word w (cpw = 32/bits), scales
   * and biases [B,Hkv,Ncap,D/G]. Appended by sparkq_kv_append and read by
   * sparkq_quantized_sdpa and, at one query token, sparkq_int8kv_sdpa_decode. */
  SPARKQ_KV_AFFINE_U4 = 2,
  SPARKQ_KV_AFFINE_U2 = 3,
};

/* Status codes. */
#define SPARKQ_OK 0
#define SPARKQ_ERR_INVALID (-1)     /* bad shape, dtype, pointer or size */
#define SPARKQ_ERR_UNSUPPORTED (-2) /* valid request the library does not run */
#define SPARKQ_ERR_DEVICE (-3)      /* HIP runtime or launch failure */
#define SPARKQ_ERR_WORKSPACE (-4)   /* workspace missing or too small */

/* Thread-local description of the last failing call on this thread. */
const char* sparkq_last_error(void);

/* ABI version, bumped on any signature change. */
int sparkq_abi_version(void);

/* 1 when the current HIP device is a gfx950 (MI355X) that runs every kernel
 * of this library, 0 otherwise. Replaces the capability probe
 * is_w8a8_available (X/src/spark_w8a8.cpp:204-216), which answers the same
 * question for Apple M5+ GPUs. */
int sparkq_is_available(void);

/* ------------------------------------------------------------------------
 * W4A16 affine quantized linear (MLX layout)
 * y[m,n] = sum_k x[m,k] * (q[n,k] * s[n,k/G] + b[n,k/G])
 *   x       [M,K]   x_dtype (BF16 or F16)
 *   w       [N,K/8] uint32, nibble k%8 of word k/8 at bits 4*(k%8)
 *   scales  [N,K/G] x_dtype
 *   biases  [N,K/G] x_dtype
 *   y       [M,N]   y_dtype (x_dtype, or F32 for the unrounded epilogue)
 * group_size in {32, 64, 128}; bits must be 4; K % 64 == 0; K % G == 0.
 * Dispatches internally (sparkq_w4a16_workspace_bytes gives the size each
 * shape needs; the decode GEMVs need none):
 *   - 1 <= M <= 4 with rows of whole 512-k spans (at most 8) and N % 4 == 0:
 *     the one-round GEMV (one row quad per wave, every quad resident at once);
 *   - M = 1, rows longer than that: the streaming GEMV (one workgroup per
 *     CU, 4x4x4 MFMA blocks, activations staged once per CU);
 *   - 5 <= M <= 16 with K % 128 == 0, at most one 16-row tile per CU and
 *     rows of at most 32 128-k segments: the segment-major 16x16x32 MFMA
 *     decode (16 weight rows x 16 activation rows per MFMA, activations
 *     loaded straight into registers);
 *   - 9 <= M <= 16 with K % 128 == 0 otherwise: the tile-major 16x16x32 MFMA
 *     decode; rows whose activations exceed its staging split K into ranges
 *     combined in the same launch (workspace);
 *   - 2 <= M <= 16 with K % 512 == 0 and N % 4 == 0 (except M <= 4 with
 *     K <= 2560), when the M activation rows fit LDS: the multi-row
 *     streaming GEMV (one decode shared by all row quartets);
 *   - otherwise M <= 4 within the LDS budget: the whole-row decode GEMV;
 *   - other M <= 32: the weight-streaming skinny kernel (MFMA 32x32x16; when
 *     the shape splits K across workgroups the last workgroup of each 32-row
 *     tile combines the partials in the same launch);
 *   - larger M: the MFMA GEMM behind a prologue (bf16: exact fp16 operands
 *     under power-of-two row shifts, with the bias term as extra MFMA slots,
 *     and an in-launch split-K for long rows; fp16: a group-sum prologue and
 *     a per-group fp32 epilogue).
 * Workspace: the first 16384 bytes hold per-tile counters and must be zero
 * before the first call; every call leaves them zero again. Give each entry
 * point its own workspace buffer, and do not share one buffer between
 * streams.
 *
 * Replaces mx.quantized_matmul(x, w, scales, biases, transpose=True,
 * group_size, bits, mode="affine") as called by AffineParameters.native
 * (spark_mlx_llm/ops/linear.py:181-191), the split-K GEMV w4a16_qmv
 * (X/spark_mlx_ext/w4a16_qmv.py:37-98) and the M=2..8 verify kernels
 * w4a16_multirow (X/spark_mlx_ext/w4a16_multirow.py:238-437).
 * ---------------------------------------------------------------------- */
size_t sparkq_w4a16_workspace_bytes(int64_t M, int64_t N, int64_t K,
                                    int group_size);
int sparkq_w4a16_linear(const void* x, const uint32_t* w, const void* scales,
                        const void* biases, void* y, int64_t M, int64_t N,
                        int64_t K, int group_size, int bits, int x_dtype,
                        int y_dtype, void* workspace, size_t workspace_bytes,
                        void* stream);

/* Derived weight buffer of one W4 projection, made once per weight set and
 * kept beside it (outside the checkpoint tensors), like the reference's
 * prepared W4 buffers that are derived lazily and rebuilt when the source
 * arrays change (spark_mlx_llm/ops/linear.py:260-268, built by
 * prepare_w4a16_nax4, X/spark_mlx_ext/w4a16_multirow.py:169-222). It holds
 * the weight half of the bf16 GEMM prologue: per-row power-of-two shifted
 * fp16 scales [N,K/G], the row shifts [N] and the bias slots [N,3K/G
 * padded to 16] (b + 8s split into bf16 pairs). Only bfloat16 scales and
 * biases have a prepared form. sparkq_w4a16_prepared_bytes gives its size
 * (0 for an unsupported group size); the buffer must be 256-byte aligned.
 * Reads scales and biases only; never allocates. */
size_t sparkq_w4a16_prepared_bytes(int64_t N, int64_t K, int group_size);
int sparkq_w4a16_prepare(const void* scales, const void* biases,
                         void* prepared, size_t prepared_bytes, int64_t N,
                         int64_t K, int group_size, int dtype, void* stream);

/* sparkq_w4a16_linear with the prepared buffer of (scales, biases): the same
 * dispatch and the same results bit for bit; when the MFMA GEMM serves the
 * call (bf16 x, more than 32 rows) its prologue converts the activation
 * rows only and the GEMM reads the prepared weight half. prepared may be
 * NULL (then identical to sparkq_w4a16_linear); a non-NULL prepared needs
 * bfloat16 x and must come from sparkq_w4a16_prepare of these very scales
 * and biases with the same N, K and group_size (not checked). Same
 * workspace as sparkq_w4a16_linear. Replaces the prepared-parameter call of
 * the multirow_packed projection (spark_mlx_llm/ops/linear.py:223-244). */
int sparkq_w4a16_linear_prepared(const void* x, const uint32_t* w,
                                 const void* scales, const void* biases,
                                 const void* prepared, void* y, int64_t M,
                                 int64_t N, int64_t K, int group_size,
                                 int bits, int x_dtype, int y_dtype,
                                 void* workspace, size_t workspace_bytes,
                                 void* stream);

/* Dequantization to fp32: out[n,k] = fmaf(q[n,k], s[n,k/G], b[n,k/G]), the
 * exact q*s+b rounded once. (The product of a 4-bit code and a 16-bit float
 * is exact in fp32 unless it overflows, so mul-then-add agrees except there.)
 * Debug entry; the reference's equivalent is the per-element decode of the
 * affine kernels (X/spark_mlx_ext/_w4a16_multirow_sources.py:31-39). */
int sparkq_w4a16_dequantize(const uint32_t* w, const void* scales,
                            const void* biases, float* out, int64_t N,
                            int64_t K, int group_size, int scale_dtype,
                            void* stream);

/* Affine 4-bit quantizer on the device, writing the layout above with the
 * benchmark's formula: per group of G values, scale = to_dtype((max-min)/15),
 * bias = to_dtype(min), code = clamp(rint((w - bias) / scale), 0, 15) with
 * the rounded scale and bias (a zero scale gives code 0). w is [N,K] in dtype
 * (BF16 or F16). The reference fills this layout with mx.quantize(bits=4)
 * (spark_mlx_llm/dspark/draft_quantization.py:119), whose rule differs: it
 * makes the larger-magnitude edge of the group exact (negative scale when
 * that edge is the minimum, bias = edge), so its tuples are not these. */
int sparkq_w4_quantize(const void* w, uint32_t* wq, void* scales, void* biases,
                       int64_t N, int64_t K, int group_size, int dtype,
                       void* stream);

/* ------------------------------------------------------------------------
 * W8A8: per-token int8 activations, per-channel int8 weights, int32 MACs
 * ---------------------------------------------------------------------- */

/* Per-token symmetric quantizer, bit-exact with
 * X/src/kernels/w8a8_quantize.metal:11-27: amax = max|x[m,:]|,
 * scale = amax > 0 ? amax / 127 : 1 (IEEE fp32 division),
 * q = (int8) clamp(rint(x / scale), -127, 127). x is [M,K] in x_dtype. */
int sparkq_a8_quantize_per_token(const void* x, int8_t* q, float* scales,
                                 int64_t M, int64_t K, int x_dtype,
                                 void* stream);

/* Raw int32 C[M,N] = A[M,K] . B[N,K]^T, exact. Replaces int8_matmul_int32
 * (X/src/spark_w8a8.cpp:218-228, X/src/bindings.cpp:33-35).
 * K % 32 == 0 and K <= 131040 so that no int32 sum can overflow. The
 * workspace holds split-K tile counters (first 16384 bytes, zero before the
 * first call and left zero by every call) and int32 partials. */
size_t sparkq_int8_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K);
int sparkq_int8_matmul_i32(const int8_t* a, const int8_t* b, int32_t* c,
                           int64_t M, int64_t N, int64_t K, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Workspace for sparkq_w8a8_linear: counters (first 16384 bytes, zero
 * before the first call and left zero by every call: split-K tile counters,
 * or the rows-ready and workgroups-done counts of the one-launch quantizer
 * for 3..16 rows with K > 4096), the int8 activations, their fp32 scales and
 * any split-K int32 partials. Calls that share a workspace must be ordered
 * (one stream). */
size_t sparkq_w8a8_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* y[m,n] = to_dtype(fmaf(float(acc[m,n]) * sa[m], sw[n], bias[n])) with acc
 * the exact int32 dot of the per-token int8 activations and the int8 weights.
 * x [M,K] and y [M,N] in x_dtype; w [N,K] int8; w_scales [N] fp32; bias [N]
 * in bias_dtype or NULL (zero). Replaces w8a8_linear
 * (X/src/spark_w8a8.cpp:230-257; epilogue X/src/kernels/w8a8_tensor.metal:63).
 * y_dtype may be F32 to read the unrounded epilogue. */
int sparkq_w8a8_linear(const void* x, const int8_t* w, const float* w_scales,
                       const void* bias, int bias_dtype, void* y, int64_t M,
                       int64_t N, int64_t K, int x_dtype, int y_dtype,
                       void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * W8A16: per-channel int8 weights, 16-bit activations (decode, M <= 4)
 * y[m,n] = to_dtype(scale[n] * sum_k x[m,k] * w[n,k]), the dot in fp32.
 *   x       [M,K]  x_dtype (BF16 or F16)
 *   w       [N,K]  int8
 *   scales  [N]    fp32
 *   y       [M,N]  y_dtype (x_dtype, or F32 for the unrounded epilogue)
 * K % 16 == 0 and M*K <= 32768. Replaces w8a16_per_channel
 * (X/src/spark_w8a16.cpp:80-110, bindings X/src/bindings.cpp:17; kernel
 * X/src/kernels/w8a16_matvec.metal:12-31), which takes one activation row;
 * rows 2..4 extend it for short verify batches.
 * ---------------------------------------------------------------------- */
int sparkq_w8a16_linear(const void* x, const int8_t* w, const float* scales,
                        void* y, int64_t M, int64_t N, int64_t K, int x_dtype,
                        int y_dtype, void* stream);

/* ------------------------------------------------------------------------
 * W8 affine quantized linear (MLX layout, groupwise)
 * y[m,n] = sum_k x[m,k] * (u[n,k] * s[n,k/G] + b[n,k/G]), u the unsigned
 * byte k%4 of word k/4 of row n:
 *   x       [M,K]   x_dtype (BF16 or F16)
 *   w       [N,K/4] uint32
 *   scales  [N,K/G] scale_dtype (F32, F16 or BF16; biases alike)
 *   y       [M,N]   y_dtype (x_dtype, or F32)
 * group_size in {32, 64, 128}; K % group_size == 0; any M. The codes are
 * exact 16-bit MFMA operands and each group adds s*D + b*X in fp32, with D
 * the group's dot of x and the codes and X the group's sum of x. No
 * workspace.
 * Replaces mx.quantized_matmul(x, w, scales, biases, transpose=True,
 * group_size, bits=8, mode="affine") behind the affine W8 nn.QuantizedLinear
 * that the W8 adapters keep as their fallback (spark_mlx_llm/ops/linear.py:
 * 413-476, 531-562) and that 'native' and 'auto' W8 checkpoints run
 * directly (spark_mlx_llm/ops/linear.py:651-711).
 * ---------------------------------------------------------------------- */
int sparkq_w8_affine_linear(const void* x, const uint32_t* w, const void* scales,
                            const void* biases, void* y, int64_t M, int64_t N, int64_t K,
                            int group_size, int x_dtype, int scale_dtype, int y_dtype,
                            void* stream);

/* ------------------------------------------------------------------------
 * INT8-KV GQA decode attention (one query token per sequence)
 *   q    [B,Hq,D] (the L=1 axis of [B,Hq,1,D] dropped), q_dtype
 *   out  [B,Hq,D], out_dtype (q_dtype, or F32 for the unrounded epilogue)
 *   K/V codes, scales and biases per kv_format (see enum above), each a view
 *   whose innermost axis is contiguous: element strides (batch, head, token)
 *   are given in strides[] in this order:
 *     strides[0..2]  key codes    (bytes)
 *     strides[3..5]  key scales   (elements; biases share them)
 *     strides[6..8]  value codes  (bytes)
 *     strides[9..11] value scales (elements; biases share them)
 *   All N tokens are visible (bottom-right causal decode with L=1).
 * out = softmax(scale * q . K^T) . V in fp32 with an online softmax, split
 * over the context and merged by log-sum-exp (in the same launch, by the
 * last split to finish, for 16-bit queries; for the affine formats when
 * every scale and bias vector of a token is aligned to its byte width and
 * the code rows and q are 16-byte aligned, as in a contiguous cache). A
 * split decode needs the workspace: per-(batch, KV head) counters in its
 * first 16384 bytes (zero before the first call, left zero), then partials.
 * Replaces int8_quantized_sdpa (X/spark_mlx_ext/int8_quantized_sdpa.py:
 * 156-287) and its kernels spark_affine_u8_sdpa_{decode,merge,short}
 * (X/spark_mlx_ext/_int8_sdpa_sources.py:8-376). D in {64,128,256};
 * Hq/Hkv in {1,2,4,8}; for the affine formats group_size in {32,64,128}.
 * kv_format may also be SPARKQ_KV_AFFINE_U4 or SPARKQ_KV_AFFINE_U2 (the
 * 4- and 2-bit MLX tuples of mlx-lm's QuantizedKVCache, which the reference
 * attends through its staged _fallback, X/spark_mlx_ext/
 * int8_quantized_sdpa.py:122-153): the same one-pass decode on their codes.
 * ---------------------------------------------------------------------- */
size_t sparkq_int8kv_sdpa_workspace_bytes(int64_t B, int64_t Hq, int64_t N,
                                          int64_t D);
int sparkq_int8kv_sdpa_decode(const void* q, const void* k_codes,
                              const void* k_scales, const void* k_biases,
                              const void* v_codes, const void* v_scales,
                              const void* v_biases, void* out, int64_t B,
                              int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                              int group_size, int kv_format, int q_dtype,
                              int out_dtype, float scale,
                              const int64_t* strides, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Allocation-free variant of sparkq_int8kv_sdpa_decode, with the same
 * arguments, checks, kernels and results, minus the workspace. No
 * counterpart in the reference: it is for callers that cannot allocate or
 * hold a workspace (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Its scratch space (split counters and
 * partials) is a fixed 8 MiB array of device memory per GPU, held until the
 * process ends; a call whose split decode needs more (the size
 * sparkq_int8kv_sdpa_workspace_bytes reports: at most 64 splits per batch,
 * so B=8, Hq=32, N=32768 needs 1.1 MB at D=128, and up to 64 query heads
 * at D=256 fit for any B and N) returns SPARKQ_ERR_UNSUPPORTED. The first call on a device resolves the array's
 * address and clears its counters with a kernel on `stream`; every call
 * leaves the counters zero. All calls on one GPU share the array: calls that
 * overlap in time on one GPU (different streams or threads) race and give
 * wrong results; serialise them on one stream. */
int sparkq_int8kv_sdpa_decode_noalloc(const void* q, const void* k_codes,
                                      const void* k_scales, const void* k_biases,
                                      const void* v_codes, const void* v_scales,
                                      const void* v_biases, void* out, int64_t B,
                                      int64_t Hq, int64_t Hkv, int64_t N,
                                      int64_t D, int group_size, int kv_format,
                                      int q_dtype, int out_dtype, float scale,
                                      const int64_t* strides, void* stream);

/* Symmetric int8 KV quantizer for the S8_F16SCALE format (the quantize-on-
 * append producer, mlx-lm QuantizedKVCache as configured by
 * spark_mlx_llm/generation.py:316-329,339-384): per row of D values,
 * scale = fp16(amax / 127) (1 when that is zero), code =
 * clamp(rint(x / float(scale)), -127, 127). x [R,D] in x_dtype; codes [R,D]
 * int8; scales [R] fp16. */
int sparkq_kv_quantize_s8(const void* x, int8_t* codes, void* scales,
                          int64_t R, int64_t D, int x_dtype, void* stream);

/* INT8-KV GQA prefill attention (L > 1 query tokens per sequence) over the
 * symmetric S8_F16SCALE cache: q [B,Hq,L,D] contiguous in q_dtype (BF16 or
 * F16), out [B,Hq,L,D] in out_dtype (q_dtype or F32); K/V codes and scales
 * and strides[0..11] as for sparkq_int8kv_sdpa_decode. causal = 1 applies
 * the bottom-right causal mask (query position i of L sees tokens
 * 0 .. N-L+i, L <= N); 0 lets every query see all N tokens. fp32 online
 * softmax; QK and PV on the fp16 MFMA with exact operands.
 * Replaces the L > 1 branch of int8_quantized_sdpa
 * (X/spark_mlx_ext/int8_quantized_sdpa.py:236-245) and its kernel
 * spark_affine_u8_sdpa_prefill (X/spark_mlx_ext/int8_quantized_sdpa_prefill.py:
 * 44-57, X/spark_mlx_ext/_int8_prefill_sources.py:7-154), which serves the
 * MLX affine u8/G32 cache at D=256 (served here by
 * sparkq_int8kv_sdpa_prefill_affine); this entry point serves the symmetric
 * s8 format at D in {64,128,256}. */
int sparkq_int8kv_sdpa_prefill(const void* q, const void* k_codes,
                               const void* k_scales, const void* v_codes,
                               const void* v_scales, void* out, int64_t B,
                               int64_t Hq, int64_t Hkv, int64_t L, int64_t N,
                               int64_t D, int causal, int q_dtype,
                               int out_dtype, float scale,
                               const int64_t* strides, void* stream);

/* INT8-KV GQA prefill attention (L > 1 query tokens per sequence) over the
 * MLX affine 8-bit cache: q [B,Hq,L,D] contiguous in q_dtype (BF16 or F16),
 * out [B,Hq,L,D] in out_dtype (q_dtype or F32); packed uint32 codes
 * [B,Hkv,N,D/4] (dim 4w+j in byte j of word w), scales and biases
 * [B,Hkv,N,D/group_size] in q_dtype, strides[0..11] as for
 * sparkq_int8kv_sdpa_decode (packed strides in bytes, multiples of 16).
 * causal as for sparkq_int8kv_sdpa_prefill. K and V dequantize to q_dtype
 * as code * scale + bias (one rounding), the softmax weights are rounded to
 * q_dtype for the PV product; scores, normalizer and output accumulate in
 * fp32 (the numerics of the reference kernel, except that q is not
 * pre-multiplied by scale and rounded). Any Hq/Hkv; D in {64,128,256};
 * group_size in {32,64,128}. When the grid of 128-row tiles is short of the
 * chip, each tile's context is split over several workgroups merged in the
 * same launch: that needs the workspace of
 * sparkq_int8kv_sdpa_prefill_affine_workspace_bytes (0 when no split; tile
 * counters in its first 16384 bytes, zero before the first call and left
 * zero, then partials). Calls that share a workspace must not overlap.
 * Replaces the L > 1 branch of int8_quantized_sdpa
 * (X/spark_mlx_ext/int8_quantized_sdpa.py:236-245) and its kernel
 * spark_affine_u8_sdpa_prefill (X/spark_mlx_ext/int8_quantized_sdpa_prefill.py:
 * 44-57, X/spark_mlx_ext/_int8_prefill_sources.py:7-154), which the
 * reference serves at D=256, group size 32 and Hq/Hkv in {1,2,4,8}. */
int sparkq_int8kv_sdpa_prefill_affine(const void* q, const void* k_packed,
                                      const void* k_scales,
                                      const void* k_biases,
                                      const void* v_packed,
                                      const void* v_scales,
                                      const void* v_biases, void* out,
                                      int64_t B, int64_t Hq, int64_t Hkv,
                                      int64_t L, int64_t N, int64_t D,
                                      int group_size, int causal,
                                      int q_dtype, int out_dtype, float scale,
                                      const int64_t* strides, void* workspace,
                                      size_t workspace_bytes, void* stream);
size_t sparkq_int8kv_sdpa_prefill_affine_workspace_bytes(int64_t B, int64_t Hq,
                                                         int64_t Hkv, int64_t L,
                                                         int64_t N, int64_t D,
                                                         int causal);

/* Quantize-on-append into a preallocated INT8 KV cache (mlx-lm
 * QuantizedKVCache.update_and_fetch as used by spark_mlx_llm/generation.py:
 * 13,316-329,339-384): row (b, h, l) of x [B,H,L,D] (contiguous, x_dtype) is
 * quantized and written to token offset+l of the cache.
 *   S8_F16SCALE: codes int8 [B,H,Ncap,D], scales fp16 [B,H,Ncap]; the
 *     sparkq_kv_quantize_s8 formula. biases unused (may be NULL).
 *   AFFINE_U8: packed uint32 [B,H,Ncap,D/4] (dim 4w+j in byte j of word w),
 *     scales and biases [B,H,Ncap,D/G] in x_dtype (BF16 or F16); per group of
 *     G dims scale = to_dtype((max-min)/255), bias = to_dtype(min), code =
 *     clamp(rint((x - bias)/scale), 0, 255) with the rounded scale and bias
 *     (code 0 when the scale is 0). This is the min/max formula of the 4-bit
 *     quantizer with 255 bins, not mlx-lm's mx.quantize(bits=8) rule (which
 *     makes the larger-magnitude edge exact), so a cache written here holds
 *     different codes, scales and biases than mlx-lm's for the same keys.
 * strides[0..2] codes (batch, head, token) in bytes; strides[3..5] scales and
 * biases (batch, head, token) in elements. The cache is written in place;
 * tokens outside [offset, offset+L) are untouched. */
/* (kv_format AFFINE_U4 / AFFINE_U2 store the same formula with 15 / 3 bins
 * and 8 / 16 codes per uint32.) */
int sparkq_kv_append(const void* x, void* codes, void* scales, void* biases,
                     int64_t B, int64_t H, int64_t L, int64_t D,
                     int64_t offset, int group_size, int kv_format,
                     int x_dtype, const int64_t* strides, void* stream);

/* ------------------------------------------------------------------------
 * Decoder-layer steps around the W4 projections (16-bit graph semantics:
 * every operation computes in fp32 and rounds to dtype, BF16 or F16; all
 * tensors contiguous, weights in the W4 affine layout of
 * sparkq_w4a16_linear, group_size in {32,64,128}).
 * ---------------------------------------------------------------------- */

/* FFN block of the decoder layer: compiled_ffn (spark_mlx_llm/ops/ffn.py:
 * 83-105, dispatched by dispatch_ffn :17-80):
 *   hidden = x + attn
 *   normed = rms_norm(hidden, norm_w, eps) = w * to_dtype(hidden * rsqrt(
 *            mean(hidden^2) + eps))                    (mx.fast.rms_norm)
 *   act    = gelu(gate(normed)) * up(normed),  gelu(v) = v * (1 +
 *            erf(v / sqrt(2))) / 2                     (mlx.nn.gelu)
 *   out    = hidden + down(act)
 *   x, attn, out [M,K]; norm_w [K]; gate, up: weights [I,K/8] and scales,
 *   biases [I,K/G]; down: [K,I/8] and [K,I/G]. K and I multiples of 64.
 * One launch does the residual, the norm, both projections and the
 * activation for M <= 4 rows, and the down projection adds the residual in
 * its epilogue. The workspace (sparkq_ffn_workspace_bytes) holds the
 * projections' split-K counters first (zero before the first call, left
 * zero) and then hidden, the normed rows and act. */
size_t sparkq_ffn_workspace_bytes(int64_t M, int64_t K, int64_t I, int group_size);
int sparkq_ffn(const void* x, const void* attn, const void* norm_w, float eps,
               const uint32_t* gate_w, const void* gate_scales, const void* gate_biases,
               const uint32_t* up_w, const void* up_scales, const void* up_biases,
               const uint32_t* down_w, const void* down_scales, const void* down_biases,
               void* out, int64_t M, int64_t K, int64_t I, int group_size, int dtype,
               void* workspace, size_t workspace_bytes, void* stream);

/* Fused QKV projection + RoPE of one token: spark_qkv_rope
 * (X/src/spark_qkv_rope.cpp:14-102; bindings X/src/bindings.cpp:73-74;
 * caller spark_mlx_llm/ops/qkv.py:41-53,110-137):
 *   qkv = quantized_matmul(x, w, scales, biases) [N], N = q_size + 2*kv_size
 *   q [n_heads,head_dim], k [n_kv_heads,head_dim] = mx.fast.rope(.,
 *     rope_dims, traditional=false, rope_base, scale=1, offset); v as is.
 * x [hidden] (the [1,1,hidden] token). q, k, v are contiguous [heads,
 * head_dim], i.e. [1,heads,1,head_dim]. One launch when head_dim and
 * rope_dims are multiples of 8 and hidden >= 1536; otherwise the projection
 * and a rope pass through the workspace (sparkq_qkv_rope_workspace_bytes;
 * counters first, as above). Only bits == 4 is run. */
size_t sparkq_qkv_rope_workspace_bytes(int64_t hidden, int num_heads, int num_kv_heads,
                                       int head_dim, int group_size);
int sparkq_qkv_rope(const void* x, const uint32_t* w, const void* scales, const void* biases,
                    void* q, void* k, void* v, int64_t hidden, int q_size, int kv_size,
                    int num_heads, int num_kv_heads, int head_dim, int rope_dims,
                    float rope_base, int64_t offset, int group_size, int bits, int dtype,
                    void* workspace, size_t workspace_bytes, void* stream);

/* mx.fast.rms_norm with an optional residual (spark_mlx_llm/ops/ffn.py:98-99
 * and the decoder's input_layernorm, spark_mlx_llm/model.py:240-254): per row
 * of x [M,K], hidden = x (+ residual), out = weight * to_dtype(hidden *
 * rsqrt(mean(hidden^2) + eps)); hidden is also written to hidden_out when
 * that is not NULL. residual may be NULL. */
int sparkq_rms_norm(const void* x, const void* residual, const void* weight, float eps,
                    void* hidden_out, void* out, int64_t M, int64_t K, int dtype, void* stream);

/* mx.fast.rope over x [rows,D] (rows = B*H*L, token l = row % L at position
 * offset + l), as applied by _apply_rope (spark_mlx_llm/ops/qkv.py:176-177)
 * and spark_qkv_rope (X/src/spark_qkv_rope.cpp:99-100): pairs (i, i+dims/2)
 * (or (2i, 2i+1) when traditional) for i < dims/2 rotated by theta =
 * (scale * position) * base^(-2i/dims); dims past `dims` copied. out may
 * equal x. */
int sparkq_rope(const void* x, void* out, int64_t rows, int64_t L, int64_t D, int dims,
                int traditional, float base, float scale, int64_t offset, int dtype,
                void* stream);

/* ------------------------------------------------------------------------
 * Attention over an MLX affine quantized KV cache of any width: the
 * reference's staged _fallback (X/spark_mlx_ext/int8_quantized_sdpa.py:
 * 122-153, validation :188-224), which serves every bits/group/head-dim/mask
 * combination its fused kernels do not:
 *   q        [B,Hq,L,D] contiguous, q_dtype (F32, F16 or BF16)
 *   K        packed uint32 [B,Hkv,N,D*bits/32], scales and biases
 *            [B,Hkv,N,D/G] in q_dtype; V alike with head dim Dv
 *   out      [B,Hq,L,Dv] in out_dtype (q_dtype or F32)
 *   strides  as for sparkq_int8kv_sdpa_decode (packed strides in bytes,
 *            multiples of 4; token strides positive)
 *   mask_kind 0: none; 1: "causal", bottom-right (row i of L sees tokens
 *            0 .. N-L+i); 2: boolean array (uint8, nonzero = visible);
 *            3: additive array of mask_dtype. mask_strides[0..3] are the
 *            element strides of the mask over (batch, query head, row,
 *            token), 0 for broadcast axes.
 * bits in {2,4,8}; group_size in {32,64,128}; D and Dv multiples of the
 * group size up to 512; any Hq divisible by Hkv. Masked scores take the
 * lowest finite value of q_dtype, as mx.where does, so a row that sees
 * nothing averages all values. Scores, softmax and output run in fp32 (the
 * reference's staged form rounds q*scale, the scores and the weights to the
 * query dtype). A long context is split over several workgroups and merged
 * by a second launch; the workspace (sparkq_quantized_sdpa_workspace_bytes,
 * 0 without a split) holds the partials.
 * ---------------------------------------------------------------------- */
size_t sparkq_quantized_sdpa_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv,
                                             int64_t L, int64_t N, int64_t Dv);
int sparkq_quantized_sdpa(const void* q, const void* k_packed, const void* k_scales,
                          const void* k_biases, const void* v_packed,
                          const void* v_scales, const void* v_biases,
                          const void* mask, int mask_kind, int mask_dtype,
                          const int64_t* mask_strides, void* out, int64_t B,
                          int64_t Hq, int64_t Hkv, int64_t L, int64_t N, int64_t D,
                          int64_t Dv, int group_size, int bits, int q_dtype,
                          int out_dtype, float scale, const int64_t* strides,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Head-wise sigmoid gate of the attention output, the step between the
 * attention and the output projection in _compiled_affine_output,
 * _compiled_w8a16_output and _module_output (spark_mlx_llm/ops/
 * attention_output.py:69-95, called from spark_mlx_llm/model.py:205):
 *   gate[b,l,h] = T(sigmoid(float(T(x[b,l,:] . gate_w[h,:]))))
 *   out[b,l,h*D+d] = T(attn[b,h,l,d] * gate[b,l,h])
 * x [B,L,hidden], attn [B,H,L,D] and gate_w [H,hidden] (the bias-free
 * g_proj) contiguous in dtype (BF16 or F16); out [B,L,H*D], the transposed
 * and gated output ready for the output projection; gate_out [B,L,H] or
 * NULL. hidden % 8 == 0. The sigmoid is that of the rounded
 * dot, computed so that its rounding to T is the exact sigmoid's. */
int sparkq_attention_gate(const void* x, const void* attn, const void* gate_w,
                          void* out, void* gate_out, int64_t B, int64_t L,
                          int64_t H, int64_t D, int64_t hidden, int dtype,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPARKQ_H_ */
