// layer.hip -- the decoder-layer steps around the W4 projections: the FFN
// (residual add, RMSNorm, gate/up, gelu(gate) * up, down, residual add) and
// the QKV projection with rotary embedding, as single fused launches where
// the decode GEMV serves the shape, and otherwise composed from the
// projections and the elementwise kernels below. Every step keeps the
// rounding points of the reference's 16-bit graph (spark_mlx_llm/ops/ffn.py:
// 83-105; X/src/spark_qkv_rope.cpp:83-101): each operation computes in fp32
// and rounds to the 16-bit type.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "common.h"

namespace sparkq {

// launchers of w4a16.hip
size_t w4a16_workspace(int64_t M, int64_t N, int64_t K, int G);
int w4a16_linear(const void* x, const uint32_t* w, const void* s, const void* b, void* y,
                 int64_t M, int64_t N, int64_t K, int G, int xdt, int ydt, void* ws,
                 size_t wsb, hipStream_t st, const void* res, bool* res_done,
                 const void* prep = nullptr);
int w4_ffn_gate_up(const void* x, const void* xres, const void* nw, float eps,
                   const uint32_t* wg, const void* sg, const void* bg, const uint32_t* wu,
                   const void* su, const void* bu, void* act, void* hid, void* nrm, int64_t M,
                   int64_t K, int64_t I, int G, int dt, hipStream_t st);
int w4_qkv_rope(const void* x, const uint32_t* w, const void* s, const void* b, void* q,
                void* k, void* v, int64_t K, int nh, int nkv, int hd, int rd, float log2_base,
                int64_t pos, int G, int dt, hipStream_t st);

namespace {

// ---------------------------------------------------------------------------
// hidden = x + xres and its RMSNorm, one workgroup per row (mx.fast.rms_norm:
// w * T(hidden * rsqrt(mean(hidden^2) + eps)), spark_mlx_llm/ops/ffn.py:98-99).
// The sum of squares runs in a fixed order: each thread's elements in order,
// a butterfly over the wave, the four waves in order.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void rms_residual_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ xres,
                                                           const uint16_t* __restrict__ nw,
                                                           float eps, uint16_t* __restrict__ hid,
                                                           uint16_t* __restrict__ nrm, int K) {
  __shared__ float red[4];
  const int64_t base = (int64_t)blockIdx.x * K;
  auto h_at = [&](int k) {
    float h = T::to_f32(x[base + k]);
    if (xres) h = T::to_f32(T::from_f32(h + T::to_f32(xres[base + k])));
    return h;
  };
  float ss = 0.0f;
  for (int k = threadIdx.x; k < K; k += 256) {
    const float h = h_at(k);
    if (hid) hid[base + k] = T::from_f32(h);
    ss = fmaf(h, h, ss);
  }
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float t = ((red[0] + red[1]) + red[2]) + red[3];
  const float inv = (float)(1.0 / sqrt((double)(t / (float)K + eps)));
  for (int k = threadIdx.x; k < K; k += 256) {
    const float n = T::to_f32(T::from_f32(h_at(k) * inv));
    nrm[base + k] = T::from_f32(T::to_f32(nw[k]) * n);
  }
}

// act = gelu(gate) * up over n elements of 16-bit gate and up
template <typename T>
__global__ __launch_bounds__(256) void gelu_mul_kernel(const uint16_t* __restrict__ g,
                                                       const uint16_t* __restrict__ u,
                                                       uint16_t* __restrict__ act, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    act[i] = T::from_f32(gelu_mul<T>(T::to_f32(g[i]), T::to_f32(u[i])));
}

// y = y + res over n elements (hidden + mlp_output, spark_mlx_llm/ops/ffn.py:105)
template <typename T>
__global__ __launch_bounds__(256) void residual_add_kernel(uint16_t* __restrict__ y,
                                                           const uint16_t* __restrict__ res,
                                                           int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    y[i] = T::from_f32(add_rounded<T>(T::to_f32(y[i]), res[i]));
}

// mx.fast.rope over rows of D elements, row r at position offset + r % L
// (X/src/spark_qkv_rope.cpp:99-100; spark_mlx_llm/ops/qkv.py:176-177): pair i
// < dims/2 is (i, i + dims/2), or (2i, 2i + 1) when traditional, rotated by
// theta = (scale * position) * inv_freq(i); dims past `dims` are copied. One
// thread per pair reads both elements before writing, so out may be x.
template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(const uint16_t* x, uint16_t* out,
                                                   int64_t rows, int L, int D, int dims,
                                                   int traditional, float log2_base, float scale,
                                                   int64_t offset) {
  const int half = dims >> 1, per_row = half + (D - dims);
  const int64_t total = rows * per_row;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * 256) {
    const int64_t r = t / per_row;
    const int i = (int)(t - r * per_row);
    const int64_t base = r * D;
    if (i >= half) {  // a dim past the rotated ones
      const int d = dims + (i - half);
      out[base + d] = x[base + d];
      continue;
    }
    const int d1 = traditional ? 2 * i : i, d2 = traditional ? 2 * i + 1 : i + half;
    const float pos = scale * (float)(offset + r % L);
    float sn, cs;
    sincosf(pos * rope_inv_freq(i, half, log2_base), &sn, &cs);
    const float x1 = T::to_f32(x[base + d1]), x2 = T::to_f32(x[base + d2]);
    out[base + d1] = T::from_f32(x1 * cs - x2 * sn);
    out[base + d2] = T::from_f32(x1 * sn + x2 * cs);
  }
}

unsigned grid_for(int64_t n) { return (unsigned)std::max<int64_t>(1, std::min<int64_t>(cdiv(n, 256), 8192)); }

template <typename T>
void launch_rope(const void* x, void* out, int64_t rows, int L, int D, int dims, int traditional,
                 float log2_base, float scale, int64_t offset, hipStream_t st) {
  const int64_t total = rows * ((dims >> 1) + (D - dims));
  hipLaunchKernelGGL(rope_kernel<T>, dim3(grid_for(total)), dim3(256), 0, st,
                     (const uint16_t*)x, (uint16_t*)out, rows, L, D, dims, traditional, log2_base,
                     scale, offset);
}

}  // namespace

float rope_log2_base(float base) { return (float)std::log2((double)base); }

int rope(const void* x, void* out, int64_t rows, int64_t L, int64_t D, int dims, int traditional,
         float base, float scale, int64_t offset, int dt, hipStream_t st) {
  if (rows == 0) return 0;
  if (dt == SPARKQ_BF16)
    launch_rope<BF16>(x, out, rows, (int)L, (int)D, dims, traditional, rope_log2_base(base), scale,
                      offset, st);
  else
    launch_rope<F16>(x, out, rows, (int)L, (int)D, dims, traditional, rope_log2_base(base), scale,
                     offset, st);
  return check_launch("rope_kernel");
}

int rms_norm(const void* x, const void* xres, const void* w, float eps, void* hid, void* out,
             int64_t M, int64_t K, int dt, hipStream_t st) {
  if (dt == SPARKQ_BF16)
    hipLaunchKernelGGL(rms_residual_kernel<BF16>, dim3((unsigned)M), dim3(256), 0, st,
                       (const uint16_t*)x, (const uint16_t*)xres, (const uint16_t*)w, eps,
                       (uint16_t*)hid, (uint16_t*)out, (int)K);
  else
    hipLaunchKernelGGL(rms_residual_kernel<F16>, dim3((unsigned)M), dim3(256), 0, st,
                       (const uint16_t*)x, (const uint16_t*)xres, (const uint16_t*)w, eps,
                       (uint16_t*)hid, (uint16_t*)out, (int)K);
  return check_launch("rms_residual_kernel");
}

// ---------------------------------------------------------------------------
// FFN block: out = hidden + down(gelu(gate(n)) * up(n)), hidden = x + attn,
// n = rms_norm(hidden) (spark_mlx_llm/ops/ffn.py:83-105)
// ---------------------------------------------------------------------------
// Workspace: the projections' workspace (counters first), then hidden and
// the normed rows [M][K], act, gate and up [M][I].
size_t ffn_workspace(int64_t M, int64_t K, int64_t I, int G) {
  const size_t lin = std::max(w4a16_workspace(M, I, K, G), w4a16_workspace(M, K, I, G));
  return round_up(lin, 256) + 2 * round_up((size_t)(M * K * 2), 256) +
         3 * round_up((size_t)(M * I * 2), 256);
}

int ffn(const void* x, const void* attn, const void* nw, float eps, const uint32_t* wg,
        const void* sg, const void* bg, const uint32_t* wu, const void* su, const void* bu,
        const uint32_t* wd, const void* sd, const void* bd, void* out, int64_t M, int64_t K,
        int64_t I, int G, int dt, void* ws, size_t wsb, hipStream_t st) {
  const size_t need = ffn_workspace(M, K, I, G);
  if (ws == nullptr || wsb < need)
    return set_error(SPARKQ_ERR_WORKSPACE, "ffn needs a workspace of %zu bytes (got %zu)", need, wsb);
  const size_t lin = round_up(std::max(w4a16_workspace(M, I, K, G), w4a16_workspace(M, K, I, G)), 256);
  unsigned char* p = static_cast<unsigned char*>(ws);
  void* lws = lin ? p : nullptr;
  uint16_t* hid = reinterpret_cast<uint16_t*>(p + lin);
  uint16_t* nrm = hid + round_up((size_t)(M * K * 2), 256) / 2;
  uint16_t* act = nrm + round_up((size_t)(M * K * 2), 256) / 2;
  uint16_t* gate = act + round_up((size_t)(M * I * 2), 256) / 2;
  uint16_t* up = gate + round_up((size_t)(M * I * 2), 256) / 2;
  int rc = w4_ffn_gate_up(x, attn, nw, eps, wg, sg, bg, wu, su, bu, act, hid, nrm, M, K, I, G, dt, st);
  if (rc < 0) return rc;
  if (rc == 1) {
    if ((rc = rms_norm(x, attn, nw, eps, hid, nrm, M, K, dt, st)) != 0) return rc;
    if ((rc = w4a16_linear(nrm, wg, sg, bg, gate, M, I, K, G, dt, dt, lws, lin, st, nullptr,
                           nullptr)) != 0)
      return rc;
    if ((rc = w4a16_linear(nrm, wu, su, bu, up, M, I, K, G, dt, dt, lws, lin, st, nullptr,
                           nullptr)) != 0)
      return rc;
    const int64_t n = M * I;
    if (dt == SPARKQ_BF16)
      hipLaunchKernelGGL(gelu_mul_kernel<BF16>, dim3(grid_for(n)), dim3(256), 0, st, gate, up, act, n);
    else
      hipLaunchKernelGGL(gelu_mul_kernel<F16>, dim3(grid_for(n)), dim3(256), 0, st, gate, up, act, n);
    if ((rc = check_launch("gelu_mul_kernel")) != 0) return rc;
  }
  bool done = false;
  if ((rc = w4a16_linear(act, wd, sd, bd, out, M, K, I, G, dt, dt, lws, lin, st, hid, &done)) != 0)
    return rc;
  if (!done) {
    const int64_t n = M * K;
    if (dt == SPARKQ_BF16)
      hipLaunchKernelGGL(residual_add_kernel<BF16>, dim3(grid_for(n)), dim3(256), 0, st,
                         (uint16_t*)out, hid, n);
    else
      hipLaunchKernelGGL(residual_add_kernel<F16>, dim3(grid_for(n)), dim3(256), 0, st,
                         (uint16_t*)out, hid, n);
    return check_launch("residual_add_kernel");
  }
  return 0;
}

// ---------------------------------------------------------------------------
// QKV projection of one token + RoPE (X/src/spark_qkv_rope.cpp:83-101)
// ---------------------------------------------------------------------------
// Workspace (only when the fused launch does not serve the shape): the
// projection's workspace, then the [N] projection.
size_t qkv_rope_workspace(int64_t K, int nh, int nkv, int hd, int G) {
  const int64_t N = (int64_t)(nh + 2 * nkv) * hd;
  return round_up(w4a16_workspace(1, N, K, G), 256) + round_up((size_t)N * 2, 256);
}

int qkv_rope(const void* x, const uint32_t* w, const void* s, const void* b, void* q, void* k,
             void* v, int64_t K, int nh, int nkv, int hd, int rd, float base, int64_t offset,
             int G, int dt, void* ws, size_t wsb, hipStream_t st) {
  const float l2b = rope_log2_base(base);
  int rc = w4_qkv_rope(x, w, s, b, q, k, v, K, nh, nkv, hd, rd, l2b, offset, G, dt, st);
  if (rc != 1) return rc;
  const size_t need = qkv_rope_workspace(K, nh, nkv, hd, G);
  if (ws == nullptr || wsb < need)
    return set_error(SPARKQ_ERR_WORKSPACE,
                     "qkv_rope needs a workspace of %zu bytes for this shape (got %zu)", need, wsb);
  const int64_t N = (int64_t)(nh + 2 * nkv) * hd;
  const size_t lin = round_up(w4a16_workspace(1, N, K, G), 256);
  unsigned char* p = static_cast<unsigned char*>(ws);
  uint16_t* qkv = reinterpret_cast<uint16_t*>(p + lin);
  if ((rc = w4a16_linear(x, w, s, b, qkv, 1, N, K, G, dt, dt, lin ? p : nullptr, lin, st,
                         nullptr, nullptr)) != 0)
    return rc;
  if ((rc = rope(qkv, q, nh, 1, hd, rd, 0, base, 1.0f, offset, dt, st)) != 0) return rc;
  if ((rc = rope(qkv + (int64_t)nh * hd, k, nkv, 1, hd, rd, 0, base, 1.0f, offset, dt, st)) != 0)
    return rc;
  if (hipMemcpyAsync(v, qkv + (int64_t)(nh + nkv) * hd, (size_t)nkv * hd * 2,
                     hipMemcpyDeviceToDevice, st) != hipSuccess)
    return set_error(SPARKQ_ERR_DEVICE, "qkv_rope: value copy failed");
  return 0;
}

// ---------------------------------------------------------------------------
// Head-wise sigmoid gate of the attention output (the body of
// _compiled_affine_output / _compiled_w8a16_output / _module_output,
// spark_mlx_llm/ops/attention_output.py:69-95):
//   gate[m, h] = T(sigmoid(float(T(x[m, :] . g_proj[h, :]))))
//   out[m, h*D + d] = T(attn[b, h, l, d] * gate[m, h]),  m = b*L + l
// i.e. the transpose of [B,H,L,D] to [B,L,H*D] with each head scaled, ready
// for the output projection. One wave per (token, head): the dot in fp32 in a
// fixed order (lanes stride the row in 16-byte pieces, then the wave sum),
// rounded to T as the 16-bit matmul returns it; sigmoid in fp32, redone in
// double where the fp32 value lies within 16 units of a T rounding tie, so
// the gate is the rounding of the exact sigmoid; the product of two T values
// is exact in fp32 and rounds once.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float sigmoid_for16(float t) {
  float e = 1.0f / (1.0f + expf(-t));
  const uint32_t u = __float_as_uint(e);
  bool redo;
  if constexpr (T::code == SPARKQ_BF16) {
    const int low = (int)(u & 0xFFFFu) - 0x8000;
    redo = low > -16 && low < 16;
  } else {
    const int low = (int)(u & 0x1FFFu) - 0x1000;
    redo = (low > -16 && low < 16) || e < 6.2e-5f;
  }
  if (redo) e = (float)(1.0 / (1.0 + exp(-(double)t)));
  return e;
}

template <typename T>
__global__ __launch_bounds__(256) void attn_gate_kernel(const uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ attn,
                                                        const uint16_t* __restrict__ gw,
                                                        uint16_t* __restrict__ out,
                                                        uint16_t* __restrict__ gate_out, int L,
                                                        int H, int D, int K) {
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int64_t m = blockIdx.x;
  if (h >= H) return;
  const u32x4_t* xr = reinterpret_cast<const u32x4_t*>(x + m * K);
  const u32x4_t* wr = reinterpret_cast<const u32x4_t*>(gw + (int64_t)h * K);
  float acc = 0.0f;
  for (int c = lane; c < K / 8; c += 64) {
    const u32x4_t xv = xr[c], wv = wr[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc = fmaf(lo16<T>(xv[e]), lo16<T>(wv[e]), acc);
      acc = fmaf(hi16<T>(xv[e]), hi16<T>(wv[e]), acc);
    }
  }
  const float dot = wave_sum(acc);
  const uint16_t g16 = T::from_f32(sigmoid_for16<T>(T::to_f32(T::from_f32(dot))));
  const float g = T::to_f32(g16);
  if (gate_out && lane == 0) gate_out[m * H + h] = g16;
  const int64_t b = m / L, l = m - b * L;
  const uint16_t* src = attn + (((b * H + h) * L + l) * D);
  uint16_t* dst = out + (m * H + h) * D;
  for (int d = lane; d < D; d += 64) dst[d] = T::from_f32(T::to_f32(src[d]) * g);
}

int attention_gate(const void* x, const void* attn, const void* gw, void* out, void* gate_out,
                   int64_t B, int64_t L, int64_t H, int64_t D, int64_t K, int dt,
                   hipStream_t st) {
  const dim3 grid((unsigned)(B * L), (unsigned)cdiv(H, 4));
  auto* k = dt == SPARKQ_BF16 ? attn_gate_kernel<BF16> : attn_gate_kernel<F16>;
  hipLaunchKernelGGL(k, grid, dim3(256), 0, st, (const uint16_t*)x, (const uint16_t*)attn,
                     (const uint16_t*)gw, (uint16_t*)out, (uint16_t*)gate_out, (int)L, (int)H,
                     (int)D, (int)K);
  return check_launch("attn_gate_kernel");
}

}  // namespace sparkq
