// abi.cpp -- the extern "C" entry points of libsparkq.so: argument
// validation with the reference's error categories, device capability check,
// and dispatch to the kernel launchers. No entry point allocates device
// memory or synchronises the stream.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <mutex>

#include "common.h"
#include "sparkq.h"

namespace sparkq {

// launchers (w4a16.hip, w8a8.hip, sdpa.hip)
size_t w4a16_workspace(int64_t M, int64_t N, int64_t K, int G);
int w4a16_linear(const void* x, const uint32_t* w, const void* s, const void* b, void* y,
                 int64_t M, int64_t N, int64_t K, int G, int xdt, int ydt, void* ws,
                 size_t wsb, hipStream_t st, const void* res = nullptr,
                 bool* res_done = nullptr, const void* prep = nullptr);
size_t w4a16_prepared_bytes(int64_t N, int64_t K, int G);
int w4a16_prepare(const void* s, const void* b, void* prep, int64_t N, int64_t K, int G,
                  hipStream_t st);
int w4a16_dequantize(const uint32_t* w, const void* s, const void* b, float* out, int64_t N,
                     int64_t K, int G, int sdt, hipStream_t st);
int w4_quantize(const void* w, uint32_t* wq, void* s, void* b, int64_t N, int64_t K, int G,
                int dt, hipStream_t st);
int a8_quantize(const void* x, int8_t* q, float* scales, int64_t M, int64_t K, int xdt,
                hipStream_t st);
size_t i8_matmul_workspace(int64_t M, int64_t N, int64_t K);
int int8_matmul_i32(const int8_t* a, const int8_t* b, int32_t* c, int64_t M, int64_t N,
                    int64_t K, void* ws, size_t wsb, hipStream_t st);
size_t w8a8_workspace(int64_t M, int64_t N, int64_t K);
int w8a8_linear(const void* x, const int8_t* w, const float* wsc, const void* bias,
                int bias_dtype, void* y, int64_t M, int64_t N, int64_t K, int xdt, int ydt,
                void* ws, size_t wsb, hipStream_t st);
size_t sdpa_workspace(int64_t B, int64_t Hq, int64_t N, int64_t D);
int int8kv_sdpa_decode(const void* q, const void* kc, const void* ks, const void* kb,
                       const void* vc, const void* vs, const void* vb, void* out, int64_t B,
                       int64_t Hq, int64_t Hkv, int64_t N, int64_t D, int G, int fmt,
                       int qdt, int odt, float scale, const int64_t* strides, void* ws,
                       size_t wsb, hipStream_t st);
int int8kv_sdpa_decode_noalloc(const void* q, const void* kc, const void* ks, const void* kb,
                               const void* vc, const void* vs, const void* vb, void* out,
                               int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D, int G,
                               int fmt, int qdt, int odt, float scale, const int64_t* strides,
                               hipStream_t st);
size_t decode_scratch_bytes();
int kv_quantize_s8(const void* x, int8_t* codes, void* scales, int64_t R, int64_t D, int xdt,
                   hipStream_t st);
int kv_append(const void* x, void* codes, void* scales, void* biases, int64_t B, int64_t H,
              int64_t L, int64_t D, int64_t offset, int G, int fmt, int xdt,
              const int64_t* strides, hipStream_t st);
int int8kv_sdpa_prefill(const void* q, const void* kc, const void* ks, const void* vc,
                        const void* vs, void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                        int64_t N, int64_t D, int causal, int qdt, int odt, float scale,
                        const int64_t* strides, hipStream_t st);
size_t int8kv_sdpa_prefill_affine_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                                            int64_t D, int causal);
int int8kv_sdpa_prefill_affine(const void* q, const void* kc, const void* ks, const void* kb,
                               const void* vc, const void* vs, const void* vb, void* out,
                               int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t N,
                               int64_t D, int G, int causal, int qdt, int odt, float scale,
                               const int64_t* strides, void* ws, size_t wsb, hipStream_t st);
int w8a16_linear(const void* x, const int8_t* w, const float* scales, void* y, int64_t M,
                 int64_t N, int64_t K, int xdt, int ydt, hipStream_t st);
int w8_affine_linear(const void* x, const uint32_t* w, const void* s, const void* b, void* y,
                     int64_t M, int64_t N, int64_t K, int G, int xdt, int sdt, int ydt,
                     hipStream_t st);
// launchers (layer.hip)
size_t ffn_workspace(int64_t M, int64_t K, int64_t I, int G);
int ffn(const void* x, const void* attn, const void* nw, float eps, const uint32_t* wg,
        const void* sg, const void* bg, const uint32_t* wu, const void* su, const void* bu,
        const uint32_t* wd, const void* sd, const void* bd, void* out, int64_t M, int64_t K,
        int64_t I, int G, int dt, void* ws, size_t wsb, hipStream_t st);
size_t qkv_rope_workspace(int64_t K, int nh, int nkv, int hd, int G);
int qkv_rope(const void* x, const uint32_t* w, const void* s, const void* b, void* q, void* k,
             void* v, int64_t K, int nh, int nkv, int hd, int rd, float base, int64_t offset,
             int G, int dt, void* ws, size_t wsb, hipStream_t st);
int rope(const void* x, void* out, int64_t rows, int64_t L, int64_t D, int dims, int traditional,
         float base, float scale, int64_t offset, int dt, hipStream_t st);
int rms_norm(const void* x, const void* xres, const void* w, float eps, void* hid, void* out,
             int64_t M, int64_t K, int dt, hipStream_t st);
int attention_gate(const void* x, const void* attn, const void* gw, void* out, void* gate_out,
                   int64_t B, int64_t L, int64_t H, int64_t D, int64_t K, int dt,
                   hipStream_t st);
size_t sdpa_gen_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t N,
                          int64_t Dv);
int sdpa_generic(const void* q, const void* kp, const void* ks, const void* kb, const void* vp,
                 const void* vs, const void* vb, const void* mask, int mask_kind,
                 int mask_dtype, const int64_t* mask_strides, void* out, int64_t B, int64_t Hq,
                 int64_t Hkv, int64_t L, int64_t N, int64_t D, int64_t Dv, int G, int bits,
                 int qdt, int odt, float scale, const int64_t* strides, void* ws, size_t wsb,
                 hipStream_t st);

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(SPARKQ_ERR_DEVICE, "%s: launch failed: %s", what, hipGetErrorString(e));
  return SPARKQ_OK;
}

// Per-device capability cache: 0 unknown, 1 gfx950, -1 other.
static int g_device_ok[64];
static std::mutex g_device_mu;

int device_check() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(SPARKQ_ERR_DEVICE, "no HIP device: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return set_error(SPARKQ_ERR_DEVICE, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_device_mu);
  if (g_device_ok[dev] == 0) {
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess)
      return set_error(SPARKQ_ERR_DEVICE, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    g_device_ok[dev] = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : -1;
    if (g_device_ok[dev] < 0)
      return set_error(SPARKQ_ERR_UNSUPPORTED,
                       "sparkq kernels require an MI355X (gfx950) device, found %s",
                       prop.gcnArchName);
  }
  if (g_device_ok[dev] < 0)
    return set_error(SPARKQ_ERR_UNSUPPORTED, "sparkq kernels require an MI355X (gfx950) device");
  return SPARKQ_OK;
}

static int g_device_cus[64];

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(g_device_mu);
  if (g_device_cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return 256;
    g_device_cus[dev] = n;
  }
  return g_device_cus[dev];
}

}  // namespace sparkq

using namespace sparkq;

#define REQUIRE(cond, ...)                                 \
  do {                                                     \
    if (!(cond)) return set_error(SPARKQ_ERR_INVALID, __VA_ARGS__); \
  } while (0)
#define REQUIRE_SUPPORTED(cond, ...)                       \
  do {                                                     \
    if (!(cond)) return set_error(SPARKQ_ERR_UNSUPPORTED, __VA_ARGS__); \
  } while (0)
#define DEVICE_OK()                          \
  do {                                       \
    if (int rc_ = device_check()) return rc_; \
  } while (0)

static bool is_float_dtype(int dt) { return dt == SPARKQ_F32 || dt == SPARKQ_F16 || dt == SPARKQ_BF16; }
static bool is_half_dtype(int dt) { return dt == SPARKQ_F16 || dt == SPARKQ_BF16; }
static constexpr int64_t kI32Max = 2147483647LL;

// Kernels address each tensor (or each sequence's slice of a KV cache) through
// a buffer descriptor with 32-bit offsets, and lanes with nothing to read use
// the offset kOob = 2^31, which must lie outside every range. A range is a
// product of shape terms in bytes; a negative value marks an overflow.
static int64_t range_bytes(std::initializer_list<int64_t> terms) {
  int64_t r = 1;
  for (int64_t t : terms) {
    if (t < 0) return -1;
    if (t != 0 && r > (int64_t)kOob / t + 1) return -1;
    r *= t;
  }
  return r;
}
static bool fits_range(std::initializer_list<int64_t> terms) {
  const int64_t r = range_bytes(terms);
  return r >= 0 && r <= (int64_t)kOob;
}

extern "C" {

const char* sparkq_last_error(void) { return g_last_error; }

int sparkq_abi_version(void) { return 1; }

int sparkq_is_available(void) { return device_check() == SPARKQ_OK ? 1 : 0; }

size_t sparkq_w4a16_workspace_bytes(int64_t M, int64_t N, int64_t K, int group_size) {
  return w4a16_workspace(M, N, K, group_size);
}

static int w4a16_linear_checked(const void* x, const uint32_t* w, const void* scales,
                                const void* biases, const void* prepared, void* y, int64_t M,
                                int64_t N, int64_t K, int group_size, int bits, int x_dtype,
                                int y_dtype, void* workspace, size_t workspace_bytes,
                                void* stream) {
  REQUIRE(x && w && scales && biases && y, "w4a16_linear: null tensor pointer");
  REQUIRE(M > 0 && N > 0 && K > 0, "w4a16_linear: M, N and K must be positive");
  REQUIRE(M <= kI32Max && N <= kI32Max && K <= kI32Max, "w4a16_linear: dimension too large");
  REQUIRE_SUPPORTED(bits == 4, "w4a16_linear: only bits=4 is supported (got %d)", bits);
  REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
          "w4a16_linear: group_size must be 32, 64 or 128 (got %d)", group_size);
  REQUIRE(K % group_size == 0, "w4a16_linear: K=%lld is not a multiple of group_size=%d",
          (long long)K, group_size);
  REQUIRE_SUPPORTED(K % 64 == 0, "w4a16_linear: K must be a multiple of 64 (got %lld)",
                    (long long)K);
  REQUIRE_SUPPORTED(is_half_dtype(x_dtype), "w4a16_linear: x must be bfloat16 or float16");
  REQUIRE(y_dtype == x_dtype || y_dtype == SPARKQ_F32,
          "w4a16_linear: y dtype must equal x dtype or be float32");
  REQUIRE_SUPPORTED(fits_range({N, K / 2}) && fits_range({N, K / group_size, 2}) &&
                        (M > 32 || fits_range({M, K, 2})),
                    "w4a16_linear: weights, scales or activations exceed the 2 GiB range of "
                    "one buffer descriptor");
  REQUIRE(aligned(x, 16) && aligned(w, 16), "w4a16_linear: x and w must be 16-byte aligned");
  REQUIRE(aligned(scales, 4) && aligned(biases, 4) && aligned(y, 4),
          "w4a16_linear: scales, biases and y must be 4-byte aligned");
  REQUIRE(aligned(prepared, 256), "w4a16_linear: the prepared buffer must be 256-byte aligned");
  DEVICE_OK();
  return w4a16_linear(x, w, scales, biases, y, M, N, K, group_size, x_dtype, y_dtype, workspace,
                      workspace_bytes, (hipStream_t)stream, nullptr, nullptr, prepared);
}

int sparkq_w4a16_linear(const void* x, const uint32_t* w, const void* scales,
                        const void* biases, void* y, int64_t M, int64_t N, int64_t K,
                        int group_size, int bits, int x_dtype, int y_dtype, void* workspace,
                        size_t workspace_bytes, void* stream) {
  return w4a16_linear_checked(x, w, scales, biases, nullptr, y, M, N, K, group_size, bits,
                              x_dtype, y_dtype, workspace, workspace_bytes, stream);
}

size_t sparkq_w4a16_prepared_bytes(int64_t N, int64_t K, int group_size) {
  if (group_size != 32 && group_size != 64 && group_size != 128) return 0;
  return w4a16_prepared_bytes(N, K, group_size);
}

int sparkq_w4a16_prepare(const void* scales, const void* biases, void* prepared,
                         size_t prepared_bytes, int64_t N, int64_t K, int group_size,
                         int dtype, void* stream) {
  REQUIRE(scales && biases && prepared, "w4a16_prepare: null tensor pointer");
  REQUIRE(N > 0 && K > 0 && N <= kI32Max && K <= kI32Max,
          "w4a16_prepare: N and K must be positive 32-bit sizes");
  REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
          "w4a16_prepare: group_size must be 32, 64 or 128 (got %d)", group_size);
  REQUIRE(K % group_size == 0 && K % 64 == 0,
          "w4a16_prepare: K=%lld must be a multiple of 64 and of group_size=%d", (long long)K,
          group_size);
  REQUIRE_SUPPORTED(dtype == SPARKQ_BF16,
                    "w4a16_prepare: only bfloat16 scales have a prepared form");
  REQUIRE_SUPPORTED(fits_range({N, K / group_size, 2}) && fits_range({N, 3 * K / group_size + 16, 2}),
                    "w4a16_prepare: scales or bias slots exceed the 2 GiB range of one buffer "
                    "descriptor");
  REQUIRE(aligned(scales, 4) && aligned(biases, 4) && aligned(prepared, 256),
          "w4a16_prepare: scales and biases must be 4-byte and prepared 256-byte aligned");
  const size_t need = w4a16_prepared_bytes(N, K, group_size);
  if (prepared_bytes < need)
    return set_error(SPARKQ_ERR_WORKSPACE, "w4a16_prepare needs %zu bytes (got %zu)", need,
                     prepared_bytes);
  DEVICE_OK();
  return w4a16_prepare(scales, biases, prepared, N, K, group_size, (hipStream_t)stream);
}

int sparkq_w4a16_linear_prepared(const void* x, const uint32_t* w, const void* scales,
                                 const void* biases, const void* prepared, void* y, int64_t M,
                                 int64_t N, int64_t K, int group_size, int bits, int x_dtype,
                                 int y_dtype, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  REQUIRE(prepared == nullptr || x_dtype == SPARKQ_BF16,
          "w4a16_linear_prepared: a prepared buffer serves bfloat16 activations only");
  return w4a16_linear_checked(x, w, scales, biases, prepared, y, M, N, K, group_size, bits,
                              x_dtype, y_dtype, workspace, workspace_bytes, stream);
}

int sparkq_w4a16_dequantize(const uint32_t* w, const void* scales, const void* biases, float* out,
                            int64_t N, int64_t K, int group_size, int scale_dtype, void* stream) {
  REQUIRE(w && scales && biases && out, "w4a16_dequantize: null tensor pointer");
  REQUIRE(N > 0 && K > 0 && N * K / 8 <= kI32Max * 64LL, "w4a16_dequantize: bad shape");
  REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
          "w4a16_dequantize: group_size must be 32, 64 or 128");
  REQUIRE(K % group_size == 0, "w4a16_dequantize: K not a multiple of group_size");
  REQUIRE_SUPPORTED(is_half_dtype(scale_dtype), "w4a16_dequantize: scales must be bf16 or f16");
  REQUIRE(aligned(out, 16) && aligned(w, 4), "w4a16_dequantize: misaligned pointer");
  DEVICE_OK();
  return w4a16_dequantize(w, scales, biases, out, N, K, group_size, scale_dtype,
                          (hipStream_t)stream);
}

int sparkq_w4_quantize(const void* w, uint32_t* wq, void* scales, void* biases, int64_t N,
                       int64_t K, int group_size, int dtype, void* stream) {
  REQUIRE(w && wq && scales && biases, "w4_quantize: null tensor pointer");
  REQUIRE(N > 0 && K > 0, "w4_quantize: N and K must be positive");
  REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
          "w4_quantize: group_size must be 32, 64 or 128");
  REQUIRE(K % group_size == 0, "w4_quantize: K not a multiple of group_size");
  REQUIRE_SUPPORTED(is_half_dtype(dtype), "w4_quantize: weights must be bf16 or f16");
  DEVICE_OK();
  return w4_quantize(w, wq, scales, biases, N, K, group_size, dtype, (hipStream_t)stream);
}

int sparkq_a8_quantize_per_token(const void* x, int8_t* q, float* scales, int64_t M, int64_t K,
                                 int x_dtype, void* stream) {
  REQUIRE(x && q && scales, "a8_quantize_per_token: null tensor pointer");
  REQUIRE(M > 0 && K > 0 && M <= kI32Max, "a8_quantize_per_token: bad shape");
  REQUIRE(is_float_dtype(x_dtype), "x must have dtype float16, bfloat16, or float32.");
  DEVICE_OK();
  return a8_quantize(x, q, scales, M, K, x_dtype, (hipStream_t)stream);
}

size_t sparkq_int8_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return i8_matmul_workspace(M, N, K);
}

// Mirrors validate_dimensions, X/src/spark_w8a8.cpp:51-65
static int validate_i8_dims(const char* op, int64_t M, int64_t N, int64_t K) {
  REQUIRE(M > 0 && N > 0 && K > 0, "%s: Expected nonempty x[..., K] and weight[N, K] with matching K.", op);
  REQUIRE(K % 32 == 0 && K <= 131040, "%s: K must be a multiple of 32 in [32, 131040].", op);
  REQUIRE(M <= kI32Max && N <= kI32Max, "%s: dimension too large", op);
  REQUIRE_SUPPORTED(fits_range({N, K}) && (M > 16 || fits_range({M, K, 4})),
                    "%s: weights or activations exceed the 2 GiB range of one buffer descriptor",
                    op);
  return SPARKQ_OK;
}

int sparkq_int8_matmul_i32(const int8_t* a, const int8_t* b, int32_t* c, int64_t M, int64_t N,
                           int64_t K, void* workspace, size_t workspace_bytes, void* stream) {
  REQUIRE(a && b && c, "int8_matmul_i32: null tensor pointer");
  if (int rc = validate_i8_dims("int8_matmul_i32", M, N, K)) return rc;
  REQUIRE(aligned(a, 16) && aligned(b, 16) && aligned(c, 4),
          "int8_matmul_i32: a and b must be 16-byte aligned");
  DEVICE_OK();
  return int8_matmul_i32(a, b, c, M, N, K, workspace, workspace_bytes, (hipStream_t)stream);
}

size_t sparkq_w8a8_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  return w8a8_workspace(M, N, K);
}

int sparkq_w8a8_linear(const void* x, const int8_t* w, const float* w_scales, const void* bias,
                       int bias_dtype, void* y, int64_t M, int64_t N, int64_t K, int x_dtype,
                       int y_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  REQUIRE(x && w && w_scales && y, "w8a8_linear: null tensor pointer");
  if (int rc = validate_i8_dims("w8a8_linear", M, N, K)) return rc;
  REQUIRE(is_float_dtype(x_dtype), "x must have dtype float16, bfloat16, or float32.");
  REQUIRE(y_dtype == x_dtype || y_dtype == SPARKQ_F32,
          "w8a8_linear: y dtype must equal x dtype or be float32");
  REQUIRE(bias == nullptr || is_float_dtype(bias_dtype),
          "bias must have shape [N] and a real floating dtype.");
  REQUIRE(aligned(w, 16) && aligned(w_scales, 4), "w8a8_linear: misaligned weight pointer");
  REQUIRE(aligned(workspace, 256), "w8a8_linear: workspace must be 256-byte aligned");
  DEVICE_OK();
  return w8a8_linear(x, w, w_scales, bias, bias_dtype, y, M, N, K, x_dtype, y_dtype, workspace,
                     workspace_bytes, (hipStream_t)stream);
}

size_t sparkq_int8kv_sdpa_workspace_bytes(int64_t B, int64_t Hq, int64_t N, int64_t D) {
  return sdpa_workspace(B, Hq, N, D);
}

// Argument checks of the decode entry points (the reference's messages where
// it has them, X/spark_mlx_ext/int8_quantized_sdpa.py:188-224).
static int check_sdpa_decode(const void* q, const void* k_codes, const void* k_scales,
                             const void* k_biases, const void* v_codes, const void* v_scales,
                             const void* v_biases, const void* out, int64_t B, int64_t Hq,
                             int64_t Hkv, int64_t N, int64_t D, int group_size, int kv_format,
                             int q_dtype, int out_dtype, float scale, const int64_t* strides) {
  REQUIRE(q && k_codes && k_scales && v_codes && v_scales && out && strides,
          "int8kv_sdpa_decode: null tensor pointer");
  REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && N > 0 && D > 0,
          "Nonempty inputs and query heads divisible by KV heads required");
  REQUIRE(Hq % Hkv == 0, "Nonempty inputs and query heads divisible by KV heads required");
  REQUIRE(B * Hkv <= 65535 && N <= kI32Max && B * Hq <= kI32Max, "int8kv_sdpa_decode: shape too large");
  const int64_t gqa = Hq / Hkv;
  REQUIRE_SUPPORTED(gqa == 1 || gqa == 2 || gqa == 4 || gqa == 8,
                    "int8kv_sdpa_decode: query heads per KV head must be 1, 2, 4 or 8");
  REQUIRE_SUPPORTED(D == 64 || D == 128 || D == 256,
                    "int8kv_sdpa_decode: head dim must be 64, 128 or 256");
  REQUIRE(std::isfinite(scale), "scale must be a finite Python number");
  REQUIRE(is_float_dtype(q_dtype), "Q and metadata must be float16, bfloat16 or float32");
  REQUIRE(out_dtype == q_dtype || out_dtype == SPARKQ_F32,
          "int8kv_sdpa_decode: out dtype must equal q dtype or be float32");
  REQUIRE(kv_format == SPARKQ_KV_S8_F16SCALE || kv_format == SPARKQ_KV_AFFINE_U8 ||
              kv_format == SPARKQ_KV_AFFINE_U4 || kv_format == SPARKQ_KV_AFFINE_U2,
          "int8kv_sdpa_decode: unknown kv_format %d", kv_format);
  if (kv_format != SPARKQ_KV_S8_F16SCALE) {
    REQUIRE(k_biases && v_biases, "int8kv_sdpa_decode: affine format needs biases");
    REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
            "Supported affine formats: bits 2/4/8, group size 32/64/128");
    REQUIRE(D % group_size == 0, "Incompatible key packed shape, affine metadata or dtype");
  }
  for (int i : {0, 1, 2, 6, 7, 8})
    REQUIRE(strides[i] % 8 == 0 && strides[i] >= 0,
            "int8kv_sdpa_decode: code strides must be non-negative multiples of 8 bytes");
  for (int i : {3, 4, 5, 9, 10, 11})
    REQUIRE(strides[i] >= 0, "int8kv_sdpa_decode: negative scale stride");
  for (int i : {2, 5, 8, 11})
    REQUIRE(strides[i] > 0, "int8kv_sdpa_decode: token strides must be positive (materialise "
                            "broadcast views)");
  REQUIRE_SUPPORTED(fits_range({N, std::max(strides[2], strides[8])}) &&
                        fits_range({N, std::max(strides[5], strides[11]), 2}),
                    "int8kv_sdpa_decode: cache too long for 32-bit offsets");
  REQUIRE(aligned(k_codes, 8) && aligned(v_codes, 8), "int8kv_sdpa_decode: codes must be 8-byte aligned");
  return SPARKQ_OK;
}

int sparkq_int8kv_sdpa_decode(const void* q, const void* k_codes, const void* k_scales,
                              const void* k_biases, const void* v_codes, const void* v_scales,
                              const void* v_biases, void* out, int64_t B, int64_t Hq,
                              int64_t Hkv, int64_t N, int64_t D, int group_size, int kv_format,
                              int q_dtype, int out_dtype, float scale, const int64_t* strides,
                              void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_sdpa_decode(q, k_codes, k_scales, k_biases, v_codes, v_scales, v_biases,
                                 out, B, Hq, Hkv, N, D, group_size, kv_format, q_dtype,
                                 out_dtype, scale, strides))
    return rc;
  DEVICE_OK();
  return int8kv_sdpa_decode(q, k_codes, k_scales, k_biases, v_codes, v_scales, v_biases, out, B,
                            Hq, Hkv, N, D, group_size, kv_format, q_dtype, out_dtype, scale,
                            strides, workspace, workspace_bytes, (hipStream_t)stream);
}

int sparkq_int8kv_sdpa_decode_noalloc(const void* q, const void* k_codes, const void* k_scales,
                                      const void* k_biases, const void* v_codes,
                                      const void* v_scales, const void* v_biases, void* out,
                                      int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                                      int group_size, int kv_format, int q_dtype, int out_dtype,
                                      float scale, const int64_t* strides, void* stream) {
  if (int rc = check_sdpa_decode(q, k_codes, k_scales, k_biases, v_codes, v_scales, v_biases,
                                 out, B, Hq, Hkv, N, D, group_size, kv_format, q_dtype,
                                 out_dtype, scale, strides))
    return rc;
  REQUIRE_SUPPORTED(sdpa_workspace(B, Hq, N, D) <= decode_scratch_bytes(),
                    "int8kv_sdpa_decode_noalloc: B=%lld Hq=%lld N=%lld D=%lld needs %zu bytes of "
                    "scratch, above the fixed %zu",
                    (long long)B, (long long)Hq, (long long)N, (long long)D,
                    sdpa_workspace(B, Hq, N, D), decode_scratch_bytes());
  DEVICE_OK();
  return int8kv_sdpa_decode_noalloc(q, k_codes, k_scales, k_biases, v_codes, v_scales, v_biases,
                                    out, B, Hq, Hkv, N, D, group_size, kv_format, q_dtype,
                                    out_dtype, scale, strides, (hipStream_t)stream);
}

int sparkq_kv_quantize_s8(const void* x, int8_t* codes, void* scales, int64_t R, int64_t D,
                          int x_dtype, void* stream) {
  REQUIRE(x && codes && scales, "kv_quantize_s8: null tensor pointer");
  REQUIRE(R > 0 && D > 0, "kv_quantize_s8: R and D must be positive");
  REQUIRE(is_float_dtype(x_dtype), "kv_quantize_s8: x must be float16, bfloat16 or float32");
  DEVICE_OK();
  return kv_quantize_s8(x, codes, scales, R, D, x_dtype, (hipStream_t)stream);
}

int sparkq_int8kv_sdpa_prefill(const void* q, const void* k_codes, const void* k_scales,
                               const void* v_codes, const void* v_scales, void* out, int64_t B,
                               int64_t Hq, int64_t Hkv, int64_t L, int64_t N, int64_t D,
                               int causal, int q_dtype, int out_dtype, float scale,
                               const int64_t* strides, void* stream) {
  REQUIRE(q && k_codes && k_scales && v_codes && v_scales && out && strides,
          "int8kv_sdpa_prefill: null tensor pointer");
  REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && L > 0 && N > 0 && D > 0 && Hq % Hkv == 0,
          "Nonempty inputs and query heads divisible by KV heads required");
  REQUIRE(B * Hkv <= 65535 && N <= kI32Max && L * Hq <= kI32Max,
          "int8kv_sdpa_prefill: shape too large");
  REQUIRE(!causal || L <= N, "int8kv_sdpa_prefill: a causal mask needs L <= N");
  const int64_t gqa = Hq / Hkv;
  REQUIRE_SUPPORTED(gqa == 1 || gqa == 2 || gqa == 4 || gqa == 8,
                    "int8kv_sdpa_prefill: query heads per KV head must be 1, 2, 4 or 8");
  REQUIRE_SUPPORTED(D == 64 || D == 128 || D == 256,
                    "int8kv_sdpa_prefill: head dim must be 64, 128 or 256");
  REQUIRE(std::isfinite(scale), "scale must be a finite Python number");
  REQUIRE_SUPPORTED(is_half_dtype(q_dtype),
                    "int8kv_sdpa_prefill: queries must be float16 or bfloat16");
  REQUIRE(out_dtype == q_dtype || out_dtype == SPARKQ_F32,
          "int8kv_sdpa_prefill: out dtype must equal q dtype or be float32");
  for (int i : {0, 1, 2, 6, 7, 8})
    REQUIRE(strides[i] % 16 == 0 && strides[i] >= 0,
            "int8kv_sdpa_prefill: code strides must be non-negative multiples of 16 bytes");
  for (int i : {3, 4, 5, 9, 10, 11})
    REQUIRE(strides[i] >= 0, "int8kv_sdpa_prefill: negative scale stride");
  for (int i : {2, 5, 8, 11})
    REQUIRE(strides[i] > 0, "int8kv_sdpa_prefill: token strides must be positive (materialise "
                            "broadcast views)");
  REQUIRE_SUPPORTED(fits_range({N, std::max(strides[2], strides[8])}) &&
                        fits_range({N, std::max(strides[5], strides[11]), 2}),
                    "int8kv_sdpa_prefill: cache too long for 32-bit offsets");
  REQUIRE(aligned(q, 16) && aligned(k_codes, 16) && aligned(v_codes, 16),
          "int8kv_sdpa_prefill: q and codes must be 16-byte aligned");
  DEVICE_OK();
  return int8kv_sdpa_prefill(q, k_codes, k_scales, v_codes, v_scales, out, B, Hq, Hkv, L, N, D,
                             causal, q_dtype, out_dtype, scale, strides, (hipStream_t)stream);
}

int sparkq_int8kv_sdpa_prefill_affine(const void* q, const void* k_packed, const void* k_scales,
                                      const void* k_biases, const void* v_packed,
                                      const void* v_scales, const void* v_biases, void* out,
                                      int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t N,
                                      int64_t D, int group_size, int causal, int q_dtype,
                                      int out_dtype, float scale, const int64_t* strides,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  REQUIRE(q && k_packed && k_scales && k_biases && v_packed && v_scales && v_biases && out &&
              strides,
          "int8kv_sdpa_prefill_affine: null tensor pointer");
  REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && L > 0 && N > 0 && D > 0 && Hq % Hkv == 0,
          "Nonempty inputs and query heads divisible by KV heads required");
  REQUIRE(B * Hkv <= 65535 && N <= kI32Max && L * Hq <= kI32Max,
          "int8kv_sdpa_prefill_affine: shape too large");
  REQUIRE(!causal || L <= N, "int8kv_sdpa_prefill_affine: a causal mask needs L <= N");
  REQUIRE_SUPPORTED(D == 64 || D == 128 || D == 256,
                    "int8kv_sdpa_prefill_affine: head dim must be 64, 128 or 256");
  REQUIRE_SUPPORTED(group_size == 32 || group_size == 64 || group_size == 128,
                    "Supported affine formats: bits 8, group size 32/64/128");
  REQUIRE(D % group_size == 0, "int8kv_sdpa_prefill_affine: head dim must be a multiple of group_size");
  REQUIRE(std::isfinite(scale), "scale must be a finite Python number");
  REQUIRE_SUPPORTED(is_half_dtype(q_dtype),
                    "int8kv_sdpa_prefill_affine: queries must be float16 or bfloat16");
  REQUIRE(out_dtype == q_dtype || out_dtype == SPARKQ_F32,
          "int8kv_sdpa_prefill_affine: out dtype must equal q dtype or be float32");
  for (int i : {0, 1, 2, 6, 7, 8})
    REQUIRE(strides[i] % 16 == 0 && strides[i] >= 0,
            "int8kv_sdpa_prefill_affine: packed strides must be non-negative multiples of 16 bytes");
  for (int i : {3, 4, 5, 9, 10, 11})
    REQUIRE(strides[i] >= 0, "int8kv_sdpa_prefill_affine: negative scale stride");
  for (int i : {2, 5, 8, 11})
    REQUIRE(strides[i] > 0, "int8kv_sdpa_prefill_affine: token strides must be positive "
                            "(materialise broadcast views)");
  // the per-(sequence, head) token range is addressed with 32-bit offsets
  REQUIRE_SUPPORTED(fits_range({N, std::max(strides[2], strides[8])}) &&
                        fits_range({N, std::max(strides[5], strides[11]), 2}),
                    "int8kv_sdpa_prefill_affine: cache too long for 32-bit offsets");
  REQUIRE(aligned(q, 16) && aligned(k_packed, 16) && aligned(v_packed, 16),
          "int8kv_sdpa_prefill_affine: q and packed codes must be 16-byte aligned");
  DEVICE_OK();
  return int8kv_sdpa_prefill_affine(q, k_packed, k_scales, k_biases, v_packed, v_scales, v_biases,
                                    out, B, Hq, Hkv, L, N, D, group_size, causal, q_dtype,
                                    out_dtype, scale, strides, workspace, workspace_bytes,
                                    (hipStream_t)stream);
}

size_t sparkq_int8kv_sdpa_prefill_affine_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv,
                                                         int64_t L, int64_t N, int64_t D,
                                                         int causal) {
  (void)N;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || L <= 0 || D <= 0 || Hq % Hkv) return 0;
  return int8kv_sdpa_prefill_affine_workspace(B, Hq, Hkv, L, D, causal);
}

int sparkq_kv_append(const void* x, void* codes, void* scales, void* biases, int64_t B,
                     int64_t H, int64_t L, int64_t D, int64_t offset, int group_size,
                     int kv_format, int x_dtype, const int64_t* strides, void* stream) {
  REQUIRE(x && codes && scales && strides, "kv_append: null tensor pointer");
  REQUIRE(B > 0 && H > 0 && L > 0 && D > 0 && offset >= 0, "kv_append: bad shape or offset");
  REQUIRE(B * H * L * D <= kI32Max * 4LL && offset + L <= kI32Max, "kv_append: shape too large");
  REQUIRE(kv_format == SPARKQ_KV_S8_F16SCALE || kv_format == SPARKQ_KV_AFFINE_U8 ||
              kv_format == SPARKQ_KV_AFFINE_U4 || kv_format == SPARKQ_KV_AFFINE_U2,
          "kv_append: unknown kv_format %d", kv_format);
  for (int i = 0; i < 6; ++i) REQUIRE(strides[i] >= 0, "kv_append: negative stride");
  if (kv_format == SPARKQ_KV_S8_F16SCALE) {
    REQUIRE(is_float_dtype(x_dtype), "kv_append: x must be float16, bfloat16 or float32");
  } else {
    REQUIRE(biases, "kv_append: affine format needs biases");
    REQUIRE(is_half_dtype(x_dtype), "kv_append: affine KV needs float16 or bfloat16 x");
    REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
            "Supported affine formats: bits 2/4/8, group size 32/64/128");
    REQUIRE(D % group_size == 0, "kv_append: head dim not a multiple of group_size");
    REQUIRE(strides[0] % 4 == 0 && strides[1] % 4 == 0 && strides[2] % 4 == 0,
            "kv_append: packed code strides must be multiples of 4 bytes");
    REQUIRE(aligned(codes, 4), "kv_append: packed codes must be 4-byte aligned");
  }
  DEVICE_OK();
  return kv_append(x, codes, scales, biases, B, H, L, D, offset, group_size, kv_format, x_dtype,
                   strides, (hipStream_t)stream);
}

// Mirrors the checks of w8a16_per_channel (X/src/spark_w8a16.cpp:80-104).
int sparkq_w8a16_linear(const void* x, const int8_t* w, const float* scales, void* y, int64_t M,
                        int64_t N, int64_t K, int x_dtype, int y_dtype, void* stream) {
  REQUIRE(x && w && scales && y, "w8a16_linear: null tensor pointer");
  REQUIRE(M > 0 && N > 0 && K > 0,
          "w8a16_per_channel requires one activation row x[..., K] with singleton leading "
          "dimensions and nonempty weight[N, K].");
  REQUIRE(N <= kI32Max && K <= kI32Max, "w8a16_linear: dimension too large");
  REQUIRE(is_half_dtype(x_dtype), "w8a16_per_channel x must have dtype bfloat16 or float16.");
  REQUIRE(y_dtype == x_dtype || y_dtype == SPARKQ_F32,
          "w8a16_linear: y dtype must equal x dtype or be float32");
  REQUIRE_SUPPORTED(M <= 4, "w8a16_linear: at most 4 activation rows (got %lld)", (long long)M);
  REQUIRE_SUPPORTED(K % 16 == 0, "w8a16_linear: K must be a multiple of 16 (got %lld)",
                    (long long)K);
  REQUIRE_SUPPORTED(fits_range({N, K}),
                    "w8a16_linear: weights exceed the 2 GiB range of one buffer descriptor");
  REQUIRE(aligned(x, 16) && aligned(w, 16) && aligned(scales, 4) && aligned(y, 4),
          "w8a16_linear: x and w must be 16-byte aligned");
  DEVICE_OK();
  return w8a16_linear(x, w, scales, y, M, N, K, x_dtype, y_dtype, (hipStream_t)stream);
}

int sparkq_w8_affine_linear(const void* x, const uint32_t* w, const void* scales,
                            const void* biases, void* y, int64_t M, int64_t N, int64_t K,
                            int group_size, int x_dtype, int scale_dtype, int y_dtype,
                            void* stream) {
  REQUIRE(x && w && scales && biases && y, "w8_affine_linear: null tensor pointer");
  REQUIRE(M > 0 && N > 0 && K > 0, "w8_affine_linear: M, N and K must be positive");
  REQUIRE(M <= kI32Max && N <= kI32Max && K <= kI32Max, "w8_affine_linear: dimension too large");
  REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
          "w8_affine_linear: group_size must be 32, 64 or 128 (got %d)", group_size);
  REQUIRE(K % group_size == 0, "w8_affine_linear: K=%lld is not a multiple of group_size=%d",
          (long long)K, group_size);
  REQUIRE_SUPPORTED(is_half_dtype(x_dtype), "w8_affine_linear: x must be bfloat16 or float16");
  REQUIRE(is_float_dtype(scale_dtype), "w8_affine_linear: scales must be a floating dtype");
  REQUIRE(y_dtype == x_dtype || y_dtype == SPARKQ_F32,
          "w8_affine_linear: y dtype must equal x dtype or be float32");
  REQUIRE_SUPPORTED(fits_range({N, K}) && fits_range({M, K, 2}),
                    "w8_affine_linear: weights or activations exceed the 2 GiB range of one "
                    "buffer descriptor");
  REQUIRE(aligned(x, 16) && aligned(w, 16), "w8_affine_linear: x and w must be 16-byte aligned");
  REQUIRE(aligned(scales, 2) && aligned(biases, 2) && aligned(y, 4),
          "w8_affine_linear: scales, biases and y must be aligned to their element size");
  DEVICE_OK();
  return w8_affine_linear(x, w, scales, biases, y, M, N, K, group_size, x_dtype, scale_dtype,
                          y_dtype, (hipStream_t)stream);
}

size_t sparkq_ffn_workspace_bytes(int64_t M, int64_t K, int64_t I, int group_size) {
  if (M <= 0 || K <= 0 || I <= 0 || group_size <= 0) return 0;
  return ffn_workspace(M, K, I, group_size);
}

int sparkq_ffn(const void* x, const void* attn, const void* norm_w, float eps,
               const uint32_t* gate_w, const void* gate_scales, const void* gate_biases,
               const uint32_t* up_w, const void* up_scales, const void* up_biases,
               const uint32_t* down_w, const void* down_scales, const void* down_biases,
               void* out, int64_t M, int64_t K, int64_t I, int group_size, int dtype,
               void* workspace, size_t workspace_bytes, void* stream) {
  REQUIRE(x && attn && norm_w && gate_w && gate_scales && gate_biases && up_w && up_scales &&
              up_biases && down_w && down_scales && down_biases && out,
          "ffn: null tensor pointer");
  REQUIRE(M > 0 && K > 0 && I > 0, "ffn: M, K and I must be positive");
  REQUIRE(M <= kI32Max && K <= kI32Max && I <= kI32Max && M * K <= kI32Max && M * I <= kI32Max,
          "ffn: dimension too large");
  REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
          "ffn: group_size must be 32, 64 or 128 (got %d)", group_size);
  REQUIRE_SUPPORTED(K % 64 == 0 && I % 64 == 0,
                    "ffn: hidden and intermediate sizes must be multiples of 64 (got %lld, %lld)",
                    (long long)K, (long long)I);
  REQUIRE(K % group_size == 0 && I % group_size == 0,
          "ffn: hidden and intermediate sizes must be multiples of group_size=%d", group_size);
  REQUIRE_SUPPORTED(is_half_dtype(dtype), "ffn: dtype must be bfloat16 or float16");
  REQUIRE(std::isfinite(eps) && eps >= 0.0f, "ffn: eps must be finite and non-negative");
  REQUIRE(aligned(x, 16) && aligned(attn, 16) && aligned(norm_w, 16) && aligned(out, 4) &&
              aligned(gate_w, 16) && aligned(up_w, 16) && aligned(down_w, 16),
          "ffn: x, attn, norm_w and the weights must be 16-byte aligned");
  REQUIRE(aligned(gate_scales, 4) && aligned(gate_biases, 4) && aligned(up_scales, 4) &&
              aligned(up_biases, 4) && aligned(down_scales, 4) && aligned(down_biases, 4),
          "ffn: scales and biases must be 4-byte aligned");
  REQUIRE_SUPPORTED(fits_range({I, K / 2}) && fits_range({I, K / group_size, 2}) &&
                        fits_range({K, I / 2}) && fits_range({K, I / group_size, 2}) &&
                        (M > 32 || fits_range({M, I, 2})),
                    "ffn: weights exceed the 2 GiB range of one buffer descriptor");
  REQUIRE(aligned(workspace, 256), "ffn: workspace must be 256-byte aligned");
  DEVICE_OK();
  return ffn(x, attn, norm_w, eps, gate_w, gate_scales, gate_biases, up_w, up_scales, up_biases,
             down_w, down_scales, down_biases, out, M, K, I, group_size, dtype, workspace,
             workspace_bytes, (hipStream_t)stream);
}

size_t sparkq_qkv_rope_workspace_bytes(int64_t hidden, int num_heads, int num_kv_heads,
                                       int head_dim, int group_size) {
  if (hidden <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || group_size <= 0)
    return 0;
  return qkv_rope_workspace(hidden, num_heads, num_kv_heads, head_dim, group_size);
}

int sparkq_qkv_rope(const void* x, const uint32_t* w, const void* scales, const void* biases,
                    void* q, void* k, void* v, int64_t hidden, int q_size, int kv_size,
                    int num_heads, int num_kv_heads, int head_dim, int rope_dims,
                    float rope_base, int64_t offset, int group_size, int bits, int dtype,
                    void* workspace, size_t workspace_bytes, void* stream) {
  // the checks and messages of X/src/spark_qkv_rope.cpp:29-81
  REQUIRE(x && w && scales && biases && q && k && v, "[spark_qkv_rope] null tensor pointer.");
  REQUIRE(hidden > 0 && hidden <= kI32Max,
          "[spark_qkv_rope] x must have shape [1, 1, hidden] with hidden > 0.");
  REQUIRE(num_heads > 0 && num_kv_heads > 0 && head_dim > 0 &&
              num_heads % num_kv_heads == 0 &&
              (int64_t)q_size == (int64_t)num_heads * head_dim &&
              (int64_t)kv_size == (int64_t)num_kv_heads * head_dim,
          "[spark_qkv_rope] Invalid head counts, head_dim, q_size, or kv_size.");
  REQUIRE(rope_dims > 0 && rope_dims % 2 == 0 && rope_dims <= head_dim &&
              std::isfinite(rope_base) && rope_base > 0.0f,
          "[spark_qkv_rope] rope_dims must be positive, even, and no larger than head_dim; "
          "rope_base must be positive and finite.");
  REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
          "[spark_qkv_rope] group_size must be 32, 64, or 128.");
  REQUIRE(bits == 1 || bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8,
          "[spark_qkv_rope] bits must be 1, 2, 3, 4, 5, 6, or 8.");
  REQUIRE_SUPPORTED(bits == 4, "[spark_qkv_rope] only bits=4 is supported here (got %d)", bits);
  REQUIRE(hidden % group_size == 0,
          "[spark_qkv_rope] Packed weight and quantization metadata shapes do not match x, "
          "q_size, kv_size, group_size, and bits.");
  REQUIRE((int64_t)q_size + 2LL * kv_size <= kI32Max, "[spark_qkv_rope] q_size + 2*kv_size too large");
  REQUIRE_SUPPORTED(hidden % 64 == 0, "[spark_qkv_rope] hidden must be a multiple of 64 (got %lld)",
                    (long long)hidden);
  REQUIRE_SUPPORTED(fits_range({(int64_t)q_size + 2LL * kv_size, hidden / 2}) &&
                        fits_range({(int64_t)q_size + 2LL * kv_size, hidden / group_size, 2}),
                    "[spark_qkv_rope] weights exceed the 2 GiB range of one buffer descriptor");
  REQUIRE_SUPPORTED(is_half_dtype(dtype), "[spark_qkv_rope] x must be bfloat16 or float16");
  REQUIRE(offset >= 0 && offset < (1LL << 24), "[spark_qkv_rope] offset must be in [0, 2^24)");
  REQUIRE(aligned(x, 16) && aligned(w, 16) && aligned(scales, 4) && aligned(biases, 4) &&
              aligned(q, 2) && aligned(k, 2) && aligned(v, 2) && aligned(workspace, 256),
          "[spark_qkv_rope] x and w must be 16-byte aligned");
  DEVICE_OK();
  return qkv_rope(x, w, scales, biases, q, k, v, hidden, num_heads, num_kv_heads, head_dim,
                  rope_dims, rope_base, offset, group_size, dtype, workspace, workspace_bytes,
                  (hipStream_t)stream);
}

int sparkq_rope(const void* x, void* out, int64_t rows, int64_t L, int64_t D, int dims,
                int traditional, float base, float scale, int64_t offset, int dtype,
                void* stream) {
  REQUIRE(x && out, "rope: null tensor pointer");
  REQUIRE(rows >= 0 && L > 0 && D > 0 && rows % L == 0, "rope: rows must be a multiple of L > 0");
  REQUIRE(rows * D <= (1LL << 40) && D <= kI32Max && L <= kI32Max, "rope: dimension too large");
  REQUIRE(dims > 0 && dims % 2 == 0 && dims <= D,
          "rope: dims must be positive, even and no larger than the last axis");
  REQUIRE(std::isfinite(base) && base > 0.0f && std::isfinite(scale),
          "rope: base must be positive and finite");
  REQUIRE(offset >= 0 && offset + L <= (1LL << 24), "rope: positions must lie in [0, 2^24)");
  REQUIRE_SUPPORTED(is_half_dtype(dtype), "rope: dtype must be bfloat16 or float16");
  REQUIRE(aligned(x, 2) && aligned(out, 2), "rope: tensors must be 2-byte aligned");
  DEVICE_OK();
  return rope(x, out, rows, L, D, dims, traditional ? 1 : 0, base, scale, offset, dtype,
              (hipStream_t)stream);
}

int sparkq_rms_norm(const void* x, const void* residual, const void* weight, float eps,
                    void* hidden_out, void* out, int64_t M, int64_t K, int dtype, void* stream) {
  REQUIRE(x && weight && out, "rms_norm: null tensor pointer");
  REQUIRE(M >= 0 && K > 0 && M <= kI32Max && K <= kI32Max && M * K <= (1LL << 40),
          "rms_norm: bad shape");
  REQUIRE(std::isfinite(eps) && eps >= 0.0f, "rms_norm: eps must be finite and non-negative");
  REQUIRE_SUPPORTED(is_half_dtype(dtype), "rms_norm: dtype must be bfloat16 or float16");
  REQUIRE(aligned(x, 2) && aligned(weight, 2) && aligned(out, 2) && aligned(residual, 2) &&
              aligned(hidden_out, 2),
          "rms_norm: tensors must be 2-byte aligned");
  if (M == 0) return 0;
  DEVICE_OK();
  return rms_norm(x, residual, weight, eps, hidden_out, out, M, K, dtype, (hipStream_t)stream);
}

int sparkq_attention_gate(const void* x, const void* attn, const void* gate_w, void* out,
                          void* gate_out, int64_t B, int64_t L, int64_t H, int64_t D,
                          int64_t hidden, int dtype, void* stream) {
  REQUIRE(x && attn && gate_w && out, "attention_gate: null tensor pointer");
  REQUIRE(B > 0 && L > 0 && H > 0 && D > 0 && hidden > 0, "attention_gate: empty shape");
  REQUIRE(B * L <= kI32Max && H <= 4LL * 65535 && D <= kI32Max && hidden <= kI32Max &&
              B * L * H * D <= (1LL << 40) && B * L * hidden <= (1LL << 40),
          "attention_gate: shape too large");
  REQUIRE_SUPPORTED(hidden % 8 == 0, "attention_gate: hidden size must be a multiple of 8");
  REQUIRE_SUPPORTED(is_half_dtype(dtype), "attention_gate: dtype must be bfloat16 or float16");
  REQUIRE(aligned(x, 16) && aligned(gate_w, 16) && aligned(attn, 2) && aligned(out, 2) &&
              aligned(gate_out, 2),
          "attention_gate: x and the gate weight must be 16-byte aligned");
  DEVICE_OK();
  return attention_gate(x, attn, gate_w, out, gate_out, B, L, H, D, hidden, dtype,
                        (hipStream_t)stream);
}

size_t sparkq_quantized_sdpa_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                                             int64_t N, int64_t Dv) {
  return sdpa_gen_workspace(B, Hq, Hkv, L, N, Dv);
}

int sparkq_quantized_sdpa(const void* q, const void* k_packed, const void* k_scales,
                          const void* k_biases, const void* v_packed, const void* v_scales,
                          const void* v_biases, const void* mask, int mask_kind, int mask_dtype,
                          const int64_t* mask_strides, void* out, int64_t B, int64_t Hq,
                          int64_t Hkv, int64_t L, int64_t N, int64_t D, int64_t Dv,
                          int group_size, int bits, int q_dtype, int out_dtype, float scale,
                          const int64_t* strides, void* workspace, size_t workspace_bytes,
                          void* stream) {
  // the validation of X/spark_mlx_ext/int8_quantized_sdpa.py:188-224
  REQUIRE(q && k_packed && k_scales && k_biases && v_packed && v_scales && v_biases && out &&
              strides,
          "quantized_sdpa: null tensor pointer");
  REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && L > 0 && N > 0 && D > 0 && Dv > 0 && Hq % Hkv == 0,
          "Nonempty inputs and query heads divisible by KV heads required");
  REQUIRE(bits == 2 || bits == 4 || bits == 8,
          "Supported affine formats: bits 2/4/8, group size 32/64/128");
  REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
          "Supported affine formats: bits 2/4/8, group size 32/64/128");
  REQUIRE(D % group_size == 0 && Dv % group_size == 0,
          "Incompatible key packed shape, affine metadata or dtype");
  REQUIRE_SUPPORTED(D <= 512 && Dv <= 512, "quantized_sdpa: head dims above 512 are not served");
  REQUIRE(std::isfinite(scale), "scale must be a finite Python number");
  REQUIRE(is_float_dtype(q_dtype), "Q and metadata must be float16, bfloat16 or float32");
  REQUIRE(out_dtype == q_dtype || out_dtype == SPARKQ_F32,
          "quantized_sdpa: out dtype must equal q dtype or be float32");
  REQUIRE(mask_kind >= 0 && mask_kind <= 3, "quantized_sdpa: unknown mask kind %d", mask_kind);
  REQUIRE(mask_kind < 2 || (mask && mask_strides), "quantized_sdpa: mask array missing");
  REQUIRE(mask_kind != 3 || is_float_dtype(mask_dtype),
          "quantized_sdpa: additive masks must be floating");
  if (mask_kind >= 2)
    for (int i = 0; i < 4; ++i)
      REQUIRE(mask_strides[i] >= 0, "quantized_sdpa: negative mask stride");
  for (int i : {0, 1, 2, 6, 7, 8})
    REQUIRE(strides[i] % 4 == 0 && strides[i] >= 0,
            "quantized_sdpa: packed strides must be non-negative multiples of 4 bytes");
  for (int i : {3, 4, 5, 9, 10, 11})
    REQUIRE(strides[i] >= 0, "quantized_sdpa: negative scale stride");
  for (int i : {2, 5, 8, 11})
    REQUIRE(strides[i] > 0, "quantized_sdpa: token strides must be positive");
  REQUIRE(N <= kI32Max && L <= kI32Max && B * Hq * L <= kI32Max,
          "quantized_sdpa: shape too large");
  REQUIRE_SUPPORTED(B * Hkv * cdiv(Hq / Hkv, 8) <= 65535 && L * 64 <= kI32Max,
                    "quantized_sdpa: too many sequences and heads for one launch");
  REQUIRE(aligned(k_packed, 4) && aligned(v_packed, 4), "quantized_sdpa: packed codes misaligned");
  DEVICE_OK();
  return sdpa_generic(q, k_packed, k_scales, k_biases, v_packed, v_scales, v_biases, mask,
                      mask_kind, mask_dtype, mask_strides, out, B, Hq, Hkv, L, N, D, Dv,
                      group_size, bits, q_dtype, out_dtype, scale, strides, workspace,
                      workspace_bytes, (hipStream_t)stream);
}

}  // extern "C"
