// sdpa.hip -- INT8-KV GQA decode attention (one query token) on gfx950.
//
// out[b,h,:] = softmax(scale * q[b,h,:] . K[b,h/G,:,:]^T) . V[b,h/G,:,:]
// K/V are int8 (symmetric s8 + fp16 scale per token and KV head) or the MLX
// affine 8-bit tuple (packed u8, per-group scale and bias in the query dtype).
//
// Kernels
//   sdpa_decode_kernel  grid (splits, B*Hkv): a workgroup owns one KV head of
//                       one sequence and a contiguous range of tokens, and
//                       serves all GQA query heads of that KV head, so every
//                       KV byte is read once. A token is handled by D/8 lanes
//                       (8 dims each, 8-byte loads); the 64/(D/8) token slots
//                       of a wave each keep an fp32 online softmax state
//                       (log2 domain) updated once per block of 4 tokens.
//                       Slots merge by shuffles, waves through LDS, and the
//                       workgroup writes either the final output (one split)
//                       or its (max, sum, acc) partial.
//   sdpa_merge_kernel   log-sum-exp merge of the split partials.
//   kv_quantize_s8_kernel  s8 + fp16-scale quantizer (one wave per row).
#include "common.h"

namespace sparkq {

struct SdpaArgs {
  const void* q;
  const uint8_t* kc;
  const void* ks;
  const void* kb;
  const uint8_t* vc;
  const void* vs;
  const void* vb;
  void* out;
  float* pm;
  float* pz;
  float* pacc;
  int64_t kc_b, kc_h, kc_t;  // key codes (bytes)
  int64_t ks_b, ks_h, ks_t;  // key scales/biases (elements)
  int64_t vc_b, vc_h, vc_t;  // value codes (bytes)
  int64_t vs_b, vs_h, vs_t;  // value scales/biases (elements)
  int B, Hq, Hkv, N, G;
  int q_dtype, out_dtype;
  int tps, S;
  float scale_log2;  // softmax scale * log2(e)
};

constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ float exp2_guarded(float x_minus_m, bool live) {
  return live ? __builtin_amdgcn_exp2f(x_minus_m) : 0.0f;
}

template <int D, int GQA, int FMT>
__global__ __launch_bounds__(256) void sdpa_decode_kernel(SdpaArgs a) {
  constexpr int LPT = D / 8;         // lanes per token
  constexpr int TPW = 64 / LPT;      // token slots per wave
  constexpr int SLOTS = 4 * TPW;     // token slots per workgroup
  constexpr int TU = 4;              // tokens per slot per block
  __shared__ float wm[4][GQA], wz[4][GQA];
  __shared__ __attribute__((aligned(16))) float wacc[4][GQA][D];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int split = blockIdx.x;
  const int b = blockIdx.y / a.Hkv, kh = blockIdx.y - b * a.Hkv;
  const int slot = wave * TPW + lane / LPT;
  const int dl = lane % LPT, d0 = dl * 8;
  const int t_begin = split * a.tps;
  const int t_end = min(a.N, t_begin + a.tps);

  float qf[GQA][8], qsum[GQA];
#pragma unroll
  for (int h = 0; h < GQA; ++h) {
    const int64_t qo = ((int64_t)b * a.Hq + kh * GQA + h) * D + d0;
    qsum[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      qf[h][i] = load_in(a.q, qo + i, a.q_dtype) * a.scale_log2;
      qsum[h] += qf[h][i];
    }
  }

  const uint8_t* kcb = a.kc + b * a.kc_b + kh * a.kc_h + d0;
  const uint8_t* vcb = a.vc + b * a.vc_b + kh * a.vc_h + d0;
  const int64_t ksb = b * a.ks_b + kh * a.ks_h + (FMT == 1 ? d0 / a.G : 0);
  const int64_t vsb = b * a.vs_b + kh * a.vs_h + (FMT == 1 ? d0 / a.G : 0);

  float mrun[GQA], zrun[GQA], acc[GQA][8];
#pragma unroll
  for (int h = 0; h < GQA; ++h) {
    mrun[h] = kNegInf;
    zrun[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[h][i] = 0.0f;
  }

  for (int t0 = t_begin + slot; t0 < t_end; t0 += SLOTS * TU) {
    uint2 kw[TU], vw[TU];
    float ksc[TU], kbi[TU], vsc[TU], vbi[TU];
    bool valid[TU];
#pragma unroll
    for (int u = 0; u < TU; ++u) {
      const int t = t0 + u * SLOTS;
      valid[u] = t < t_end;
      const int64_t tu = valid[u] ? t : t0;
      kw[u] = *reinterpret_cast<const uint2*>(kcb + tu * a.kc_t);
      vw[u] = *reinterpret_cast<const uint2*>(vcb + tu * a.vc_t);
      if constexpr (FMT == 0) {
        ksc[u] = f16_to_f32(reinterpret_cast<const uint16_t*>(a.ks)[ksb + tu * a.ks_t]);
        vsc[u] = f16_to_f32(reinterpret_cast<const uint16_t*>(a.vs)[vsb + tu * a.vs_t]);
        kbi[u] = 0.0f;
        vbi[u] = 0.0f;
      } else {
        ksc[u] = load_in(a.ks, ksb + tu * a.ks_t, a.q_dtype);
        kbi[u] = load_in(a.kb, ksb + tu * a.ks_t, a.q_dtype);
        vsc[u] = load_in(a.vs, vsb + tu * a.vs_t, a.q_dtype);
        vbi[u] = load_in(a.vb, vsb + tu * a.vs_t, a.q_dtype);
      }
    }
    // scores (log2 units)
    float sc[TU][GQA];
#pragma unroll
    for (int u = 0; u < TU; ++u) {
      float kv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t word = i < 4 ? kw[u].x : kw[u].y;
        const uint32_t byte = (word >> (8 * (i & 3))) & 0xFFu;
        kv[i] = FMT == 0 ? (float)(int8_t)byte : (float)byte;
      }
#pragma unroll
      for (int h = 0; h < GQA; ++h) {
        float p = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) p = fmaf(qf[h][i], kv[i], p);
        if constexpr (FMT == 1) p = fmaf(ksc[u], p, kbi[u] * qsum[h]);
#pragma unroll
        for (int off = LPT / 2; off > 0; off >>= 1) p += __shfl_xor(p, off);
        if constexpr (FMT == 0) p *= ksc[u];
        sc[u][h] = valid[u] ? p : kNegInf;
      }
    }
    // one online-softmax update per block
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
      float mb = mrun[h];
#pragma unroll
      for (int u = 0; u < TU; ++u) mb = fmaxf(mb, sc[u][h]);
      const float alpha = exp2_guarded(mrun[h] - mb, mrun[h] != kNegInf);
      float p[TU];
      float zs = 0.0f;
#pragma unroll
      for (int u = 0; u < TU; ++u) {
        p[u] = exp2_guarded(sc[u][h] - mb, valid[u]);
        zs += p[u];
      }
      zrun[h] = fmaf(zrun[h], alpha, zs);
      mrun[h] = mb;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] *= alpha;
#pragma unroll
      for (int u = 0; u < TU; ++u) {
        const float pw = FMT == 0 ? p[u] * vsc[u] : p[u];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t word = i < 4 ? vw[u].x : vw[u].y;
          const uint32_t byte = (word >> (8 * (i & 3))) & 0xFFu;
          const float vv = FMT == 0 ? (float)(int8_t)byte : fmaf((float)byte, vsc[u], vbi[u]);
          acc[h][i] = fmaf(pw, vv, acc[h][i]);
        }
      }
    }
  }

  // merge the token slots of this wave (lanes l and l^off share dims)
#pragma unroll
  for (int off = LPT; off < 64; off <<= 1) {
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
      const float mo = __shfl_xor(mrun[h], off);
      const float zo = __shfl_xor(zrun[h], off);
      const float mm = fmaxf(mrun[h], mo);
      const float wa = exp2_guarded(mrun[h] - mm, mrun[h] != kNegInf);
      const float wb = exp2_guarded(mo - mm, mo != kNegInf);
      zrun[h] = zrun[h] * wa + zo * wb;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float ao = __shfl_xor(acc[h][i], off);
        acc[h][i] = acc[h][i] * wa + ao * wb;
      }
      mrun[h] = mm;
    }
  }
  if (lane < LPT) {
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
      if (lane == 0) {
        wm[wave][h] = mrun[h];
        wz[wave][h] = zrun[h];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) wacc[wave][h][d0 + i] = acc[h][i];
    }
  }
  __syncthreads();
  for (int e = tid; e < GQA * D; e += 256) {
    const int h = e / D, d = e - h * D;
    float mm = kNegInf;
#pragma unroll
    for (int w = 0; w < 4; ++w) mm = fmaxf(mm, wm[w][h]);
    float z = 0.0f, o = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float wt = exp2_guarded(wm[w][h] - mm, wm[w][h] != kNegInf);
      z = fmaf(wz[w][h], wt, z);
      o = fmaf(wacc[w][h][d], wt, o);
    }
    const int64_t bh = (int64_t)b * a.Hq + kh * GQA + h;
    if (a.S == 1) {
      store_out(a.out, bh * D + d, z > 0.0f ? o / z : 0.0f, a.out_dtype);
    } else {
      a.pacc[(bh * a.S + split) * D + d] = o;
      if (d == 0) {
        a.pm[bh * a.S + split] = mm;
        a.pz[bh * a.S + split] = z;
      }
    }
  }
}

__global__ __launch_bounds__(256) void sdpa_merge_kernel(const float* __restrict__ pm,
                                                         const float* __restrict__ pz,
                                                         const float* __restrict__ pacc,
                                                         void* __restrict__ out, int out_dtype,
                                                         int S, int D) {
  const int64_t bh = blockIdx.x;
  const int d = threadIdx.x;
  if (d >= D) return;
  float mm = kNegInf;
  for (int s = 0; s < S; ++s) mm = fmaxf(mm, pm[bh * S + s]);
  float z = 0.0f, o = 0.0f;
  for (int s = 0; s < S; ++s) {
    const float m = pm[bh * S + s];
    const float wt = exp2_guarded(m - mm, m != kNegInf);
    z = fmaf(pz[bh * S + s], wt, z);
    o = fmaf(pacc[(bh * S + s) * D + d], wt, o);
  }
  store_out(out, bh * D + d, z > 0.0f ? o / z : 0.0f, out_dtype);
}

__global__ __launch_bounds__(256) void kv_quantize_s8_kernel(const void* __restrict__ x,
                                                             int8_t* __restrict__ codes,
                                                             uint16_t* __restrict__ scales,
                                                             int64_t R, int64_t D, int xdt) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= R) return;
  float amax = 0.0f;
  for (int64_t d = lane; d < D; d += 64) amax = fmaxf(amax, fabsf(load_in(x, row * D + d, xdt)));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  uint16_t s16 = f32_to_f16(amax / 127.0f);
  if (f16_to_f32(s16) == 0.0f) s16 = 0x3C00u;
  const float s = f16_to_f32(s16);
  if (lane == 0) scales[row] = s16;
  for (int64_t d = lane; d < D; d += 64) {
    float v = __builtin_rintf(load_in(x, row * D + d, xdt) / s);
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    codes[row * D + d] = (int8_t)v;
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
// Context splits: about 128 workgroups per sequence batch-wide, at least 64
// tokens per split, and no empty split.
static int sdpa_splits(int64_t B, int64_t N, int64_t* tps_out = nullptr) {
  int64_t S = cdiv(128, B);
  const int64_t cap = cdiv(N, 64);
  if (S > cap) S = cap;
  if (S < 1) S = 1;
  const int64_t tps = cdiv(N, S);
  S = cdiv(N, tps);
  if (tps_out) *tps_out = tps;
  return (int)S;
}

size_t sdpa_workspace(int64_t B, int64_t Hq, int64_t N, int64_t D) {
  if (B <= 0 || Hq <= 0 || N <= 0 || D <= 0) return 0;
  const int S = sdpa_splits(B, N);
  if (S == 1) return 0;
  const size_t rows = (size_t)B * Hq * S;
  return round_up(rows * 4, 256) * 2 + round_up(rows * D * 4, 256);
}

template <int D, int GQA>
static void launch_decode_g(const SdpaArgs& a, int fmt, dim3 grid, hipStream_t st) {
  if (fmt == SPARKQ_KV_S8_F16SCALE)
    hipLaunchKernelGGL((sdpa_decode_kernel<D, GQA, 0>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((sdpa_decode_kernel<D, GQA, 1>), grid, dim3(256), 0, st, a);
}

template <int D>
static void launch_decode_d(const SdpaArgs& a, int gqa, int fmt, dim3 grid, hipStream_t st) {
  switch (gqa) {
    case 1: launch_decode_g<D, 1>(a, fmt, grid, st); break;
    case 2: launch_decode_g<D, 2>(a, fmt, grid, st); break;
    case 4: launch_decode_g<D, 4>(a, fmt, grid, st); break;
    default: launch_decode_g<D, 8>(a, fmt, grid, st); break;
  }
}

int int8kv_sdpa_decode(const void* q, const void* kc, const void* ks, const void* kb,
                       const void* vc, const void* vs, const void* vb, void* out, int64_t B,
                       int64_t Hq, int64_t Hkv, int64_t N, int64_t D, int G, int fmt,
                       int qdt, int odt, float scale, const int64_t* strides, void* ws,
                       size_t wsb, hipStream_t st) {
  int64_t tps = 0;
  const int S = sdpa_splits(B, N, &tps);
  const size_t need = sdpa_workspace(B, Hq, N, D);
  if (need > 0 && (ws == nullptr || wsb < need))
    return set_error(SPARKQ_ERR_WORKSPACE,
                     "int8kv_sdpa_decode needs a workspace of %zu bytes (got %zu)", need, wsb);
  SdpaArgs a{};
  a.q = q;
  a.kc = reinterpret_cast<const uint8_t*>(kc);
  a.ks = ks;
  a.kb = kb;
  a.vc = reinterpret_cast<const uint8_t*>(vc);
  a.vs = vs;
  a.vb = vb;
  a.out = out;
  a.kc_b = strides[0];
  a.kc_h = strides[1];
  a.kc_t = strides[2];
  a.ks_b = strides[3];
  a.ks_h = strides[4];
  a.ks_t = strides[5];
  a.vc_b = strides[6];
  a.vc_h = strides[7];
  a.vc_t = strides[8];
  a.vs_b = strides[9];
  a.vs_h = strides[10];
  a.vs_t = strides[11];
  a.B = (int)B;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.N = (int)N;
  a.G = G;
  a.q_dtype = qdt;
  a.out_dtype = odt;
  a.S = S;
  a.tps = (int)tps;
  a.scale_log2 = scale * 1.4426950408889634f;
  if (S > 1) {
    const size_t rows = (size_t)B * Hq * S;
    unsigned char* base = reinterpret_cast<unsigned char*>(ws);
    a.pm = reinterpret_cast<float*>(base);
    a.pz = reinterpret_cast<float*>(base + round_up(rows * 4, 256));
    a.pacc = reinterpret_cast<float*>(base + 2 * round_up(rows * 4, 256));
  }
  const int gqa = (int)(Hq / Hkv);
  dim3 grid((unsigned)S, (unsigned)(B * Hkv));
  if (D == 64)
    launch_decode_d<64>(a, gqa, fmt, grid, st);
  else if (D == 128)
    launch_decode_d<128>(a, gqa, fmt, grid, st);
  else
    launch_decode_d<256>(a, gqa, fmt, grid, st);
  if (int rc = check_launch("sdpa_decode_kernel")) return rc;
  if (S > 1) {
    hipLaunchKernelGGL(sdpa_merge_kernel, dim3((unsigned)(B * Hq)), dim3(256), 0, st, a.pm,
                       a.pz, a.pacc, out, odt, S, (int)D);
    if (int rc = check_launch("sdpa_merge_kernel")) return rc;
  }
  return SPARKQ_OK;
}

int kv_quantize_s8(const void* x, int8_t* codes, void* scales, int64_t R, int64_t D, int xdt,
                   hipStream_t st) {
  hipLaunchKernelGGL(kv_quantize_s8_kernel, dim3((unsigned)cdiv(R, 4)), dim3(256), 0, st, x,
                     codes, (uint16_t*)scales, R, D, xdt);
  return check_launch("kv_quantize_s8_kernel");
}

}  // namespace sparkq
