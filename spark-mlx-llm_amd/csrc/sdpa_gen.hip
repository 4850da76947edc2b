// sdpa_gen.hip -- attention over an MLX affine quantized KV cache of any
// width the fused kernels do not take: 2-, 4- or 8-bit codes, group size 32,
// 64 or 128, any head dims (multiples of the group size, keys and values may
// differ), any query-to-KV head ratio, L >= 1 query rows, and masks given as
// None, "causal" (bottom-right), a boolean array or an additive array. This
// is the reference's staged _fallback (X/spark_mlx_ext/int8_quantized_sdpa.py:
// 122-153): scores = (q*scale) . K^T over the dequantized keys, masked
// entries replaced by the lowest finite value of the query dtype (so a row
// with nothing visible averages every value, as mx.where + softmax do) or
// offset by the additive mask, a softmax, and the weights times V.
//
// Here everything after the inputs runs in fp32 (the reference rounds q*scale,
// the scores and the weights to the query dtype in between; those roundings
// are not restated). Kernel sdpa_gen_kernel: one workgroup per (query row,
// context split, sequence and KV head, chunk of up to 8 query heads of that
// KV head), so each key and value row is dequantized once for the chunk.
// The context goes in chunks of 256 tokens:
//  1. thread t takes token n0+t: it dequantizes the key row on the fly
//     (code * scale + bias in fp32) and forms the dot with every query head
//     of the chunk (the queries, times scale*log2(e), sit in LDS);
//  2. per head, the chunk max (LDS reduction) updates the running max, the
//     weights 2^(s - m) replace the scores in LDS and the running sum and
//     the output accumulators are rescaled;
//  3. the chunk's values are dequantized 32 tokens at a time into LDS and
//     each thread accumulates its (head, dim) outputs.
// With several context splits each workgroup stores (max, sum, outputs) and
// sdpa_gen_merge_kernel combines them in split order.
#include <algorithm>
#include <cfloat>

#include "common.h"

namespace sparkq {

struct GenSdpaArgs {
  const void* q;                  // [B,Hq,L,D] contiguous, q dtype
  const uint32_t* kp;             // packed codes, D*bits/32 words per token
  const void* ks;                 // scales [.., D/G], q dtype
  const void* kb;                 // biases, same strides as scales
  const uint32_t* vp;
  const void* vs;
  const void* vb;
  const void* mask;               // mask array or null
  void* out;                      // [B,Hq,L,Dv]
  float* pm;                      // split partials: max [rows][S]
  float* pz;                      //   sums [rows][S]
  float* pacc;                    //   outputs [rows][S][Dv]
  int64_t kp_b, kp_h, kp_t;       // strides in words
  int64_t ks_b, ks_h, ks_t;       // strides in elements (biases share them)
  int64_t vp_b, vp_h, vp_t;
  int64_t vs_b, vs_h, vs_t;
  int64_t m_b, m_h, m_l, m_n;     // mask strides in elements (0 to broadcast)
  int mask_kind;                  // kMask*
  int mask_dtype;                 // additive masks: SPARKQ_F32/F16/BF16
  int B, Hq, Hkv, L, N, D, Dv, G, bits;
  int q_dtype, out_dtype;
  int RC, nch;                    // query heads per workgroup, chunks per KV head
  int S, tps;                     // context splits, tokens per split
  int vt;                         // value tokens per LDS stage
  float scale_log2;               // softmax scale times log2(e)
  float masked;                   // score of a masked entry, in log2 units
};

[[maybe_unused]] constexpr int kMaskNone = 0, kMaskCausal = 1, kMaskBool = 2, kMaskAdd = 3;
constexpr int kGenMaxRC = 8;
constexpr int kGenMaxDim = 512;
constexpr int kGenChunk = 256;
constexpr int kGenMaxOut = (kGenMaxRC * kGenMaxDim) / 256;
constexpr int kGenLdsFloats = 16384;  // 64 KB of LDS per workgroup

// value tokens per LDS stage: what fits beside the queries and weights, a
// multiple of 8 from 8 to 64
__host__ __device__ __forceinline__ int gen_value_tokens(int RC, int D, int Dv) {
  const int room = (kGenLdsFloats - RC * D - RC * kGenChunk - 8 * RC) / Dv;
  return room >= 64 ? 64 : (room / 8 * 8 < 8 ? 8 : room / 8 * 8);
}
__host__ __device__ __forceinline__ size_t gen_lds_bytes(int RC, int D, int Dv) {
  return (size_t)(RC * D + RC * kGenChunk + gen_value_tokens(RC, D, Dv) * Dv + 8 * RC) * 4;
}

__device__ __forceinline__ float gen_load(const void* p, int64_t i, int dt) {
  return load_in(p, i, dt);
}

// block reduction over 256 threads of one value per head (max or sum)
template <bool MAX>
__device__ __forceinline__ float block_reduce(float v, float* red, int slot) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float w = __shfl_xor(v, o);
    v = MAX ? fmaxf(v, w) : v + w;
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[slot * 4 + wave] = v;
  __syncthreads();
  const float* r = red + slot * 4;
  return MAX ? fmaxf(fmaxf(r[0], r[1]), fmaxf(r[2], r[3])) : (r[0] + r[1]) + (r[2] + r[3]);
}

// Metadata (scales, biases) loads: MF32 for fp32 metadata, else 16-bit
// (bf16 or fp16 by q_dtype). A load's data is only used after every load of
// its batch has been issued, so one wait covers the batch.
template <bool MF32>
__device__ __forceinline__ float gen_meta(rsrc_t r, int64_t idx, int dt) {
  if constexpr (MF32) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)(idx * 4), 0, 0));
  } else {
    const uint32_t h = __builtin_amdgcn_raw_buffer_load_b16(r, (int)(idx * 2), 0, 0);
    const float fb = __uint_as_float(h << 16), fh = f16_to_f32((uint16_t)h);
    return dt == SPARKQ_BF16 ? fb : fh;
  }
}

template <int BITS, bool MF32>
__global__ __launch_bounds__(256) void sdpa_gen_kernel(GenSdpaArgs a) {
  constexpr int CPW = 32 / BITS;                 // codes per word
  constexpr uint32_t CMASK = (1u << BITS) - 1u;
  constexpr int WPP = 128 / CPW;                 // words per pass of 128 dims of a key row
  constexpr int VB = 8;                          // value elements per thread per load batch
  extern __shared__ float lds[];
  const int tid = threadIdx.x;
  const int l = blockIdx.x / a.S, split = blockIdx.x - (blockIdx.x / a.S) * a.S;
  const int chunk = blockIdx.y % a.nch;
  const int bk = blockIdx.y / a.nch;
  const int kvh = bk % a.Hkv, b = bk / a.Hkv;
  const int R = a.Hq / a.Hkv;
  const int h0 = kvh * R + chunk * a.RC;
  const int rc = min(a.RC, R - chunk * a.RC);
  const int D = a.D, Dv = a.Dv, G = a.G;
  const int gsh = G == 32 ? 5 : (G == 64 ? 6 : 7);  // log2 of the group size
  const int VT = a.vt;                       // value tokens per LDS stage
  float* qs = lds;                           // [RC][D]
  float* sc = qs + a.RC * D;                 // [RC][256]
  float* vt = sc + a.RC * kGenChunk;         // [VT][Dv]
  float* red = vt + VT * Dv;                 // reductions

  for (int i = tid; i < rc * D; i += 256) {
    const int r = i / D, d = i - (i / D) * D;
    const int64_t qi = (((int64_t)b * a.Hq + h0 + r) * a.L + l) * D + d;
    qs[i] = gen_load(a.q, qi, a.q_dtype) * a.scale_log2;
  }
  // outputs of this thread: e = tid + 256*j over [rc][Dv]
  const int nout = rc * Dv;
  float acc[kGenMaxOut];
#pragma unroll
  for (int j = 0; j < kGenMaxOut; ++j) acc[j] = 0.0f;
  float mrun[kGenMaxRC], zrun[kGenMaxRC];
#pragma unroll
  for (int r = 0; r < kGenMaxRC; ++r) {
    mrun[r] = -INFINITY;
    zrun[r] = 0.0f;
  }
  const int t_begin = split * a.tps;
  const int t_end = min(a.N, t_begin + a.tps);
  const int limit = a.N - a.L + l;  // causal: last visible token of this row
  // bounded descriptors over this (sequence, KV head)'s first t_end tokens;
  // every index below is clamped into them
  const int wpr = D * BITS / 32, vwpr = Dv * BITS / 32;  // words per key / value row
  const int ng = D / G, nvg = Dv / G;
  const rsrc_t rk = make_rsrc(a.kp + b * a.kp_b + kvh * a.kp_h,
                              (uint32_t)(((int64_t)(t_end - 1) * a.kp_t + wpr) * 4));
  const rsrc_t rv = make_rsrc(a.vp + b * a.vp_b + kvh * a.vp_h,
                              (uint32_t)(((int64_t)(t_end - 1) * a.vp_t + vwpr) * 4));
  const int esz = MF32 ? 4 : 2;
  const int64_t ksb = b * a.ks_b + kvh * a.ks_h, vsb = b * a.vs_b + kvh * a.vs_h;
  const rsrc_t rks = make_rsrc(reinterpret_cast<const unsigned char*>(a.ks) + ksb * esz,
                               (uint32_t)(((int64_t)(t_end - 1) * a.ks_t + ng) * esz));
  const rsrc_t rkb = make_rsrc(reinterpret_cast<const unsigned char*>(a.kb) + ksb * esz,
                               (uint32_t)(((int64_t)(t_end - 1) * a.ks_t + ng) * esz));
  const rsrc_t rvs = make_rsrc(reinterpret_cast<const unsigned char*>(a.vs) + vsb * esz,
                               (uint32_t)(((int64_t)(t_end - 1) * a.vs_t + nvg) * esz));
  const rsrc_t rvb = make_rsrc(reinterpret_cast<const unsigned char*>(a.vb) + vsb * esz,
                               (uint32_t)(((int64_t)(t_end - 1) * a.vs_t + nvg) * esz));
  const float inv_dv = 1.0f / (float)Dv;
  __syncthreads();

  for (int n0 = t_begin; n0 < t_end; n0 += kGenChunk) {
    // 1. scores of token n0+tid for every head of the chunk: the key row in
    // passes of 128 dims, each pass's words and its groups' scales and
    // biases loaded together before any is used
    const int n = n0 + tid;
    const int nl = min(n, t_end - 1);
    float s[kGenMaxRC];
#pragma unroll
    for (int r = 0; r < kGenMaxRC; ++r) s[r] = 0.0f;
    for (int w0 = 0; w0 < wpr; w0 += WPP) {
      // each word with its group's scale and bias (a group spans at least
      // one word; repeated loads of a group hit the cache)
      uint32_t kw[WPP];
      float gs[WPP], gb[WPP];
#pragma unroll
      for (int i = 0; i < WPP; ++i) {  // words past the row read zeros (out of range)
        const bool in = w0 + i < wpr;
        kw[i] = __builtin_amdgcn_raw_buffer_load_b32(
            rk, in ? (int)(((int64_t)nl * a.kp_t + w0 + i) * 4) : (int)kOob, 0, 0);
        const int64_t gi = (int64_t)nl * a.ks_t + (min(w0 + i, wpr - 1) * CPW >> gsh);
        gs[i] = gen_meta<MF32>(rks, gi, a.q_dtype);
        gb[i] = gen_meta<MF32>(rkb, gi, a.q_dtype);
      }
      const int nw = min(WPP, wpr - w0);  // words of this pass (uniform)
#pragma unroll
      for (int i = 0; i < WPP; ++i) {
        if (i < nw) {
#pragma unroll
          for (int j = 0; j < CPW; ++j) {
            const float kv = fmaf((float)((kw[i] >> (BITS * j)) & CMASK), gs[i], gb[i]);
            const int d = (w0 + i) * CPW + j;
#pragma unroll
            for (int r = 0; r < kGenMaxRC; ++r)
              if (r < rc) s[r] = fmaf(qs[r * D + d], kv, s[r]);
          }
        }
      }
    }
    if (n < t_end) {
      if (a.mask_kind == kMaskCausal) {
        if (n > limit) {
#pragma unroll
          for (int r = 0; r < kGenMaxRC; ++r) s[r] = a.masked;
        }
      } else if (a.mask_kind == kMaskBool || a.mask_kind == kMaskAdd) {
#pragma unroll
        for (int r = 0; r < kGenMaxRC; ++r) {
          if (r < rc) {
            const int64_t mi = b * a.m_b + (int64_t)(h0 + r) * a.m_h + (int64_t)l * a.m_l +
                               (int64_t)n * a.m_n;
            if (a.mask_kind == kMaskBool)
              s[r] = reinterpret_cast<const unsigned char*>(a.mask)[mi] ? s[r] : a.masked;
            else  // a dtype-minimum mask stays finite (its product would overflow)
              s[r] += fmaxf(gen_load(a.mask, mi, a.mask_dtype) * 1.4426950408889634f, -FLT_MAX);
          }
        }
      }
    }
    // 2. per head: chunk max, running max, weights, sums, rescale (rc is the
    // same for the whole workgroup, so the barriers inside are uniform)
#pragma unroll
    for (int r = 0; r < kGenMaxRC; ++r) {
      if (r < rc) {
        const float v = n < t_end ? s[r] : -INFINITY;
        const float cm = block_reduce<true>(v, red, 0);
        const float mnew = fmaxf(mrun[r], cm);
        // nothing visible yet (every score so far -inf from an additive
        // mask): no weight, no rescale, so no -inf - -inf = NaN enters the
        // sums; a -inf score weighs 0 once a finite one has been seen
        const float alpha = mrun[r] == -INFINITY ? 0.0f : exp2f(mrun[r] - mnew);
        const float p = (n < t_end && v != -INFINITY) ? exp2f(v - mnew) : 0.0f;
        sc[r * kGenChunk + tid] = p;
        const float cz = block_reduce<false>(p, red, 1);
        zrun[r] = fmaf(zrun[r], alpha, cz);
        mrun[r] = mnew;
#pragma unroll
        for (int j = 0; j < kGenMaxOut; ++j) {
          const int e = tid + 256 * j;
          if (e < nout && e / Dv == r) acc[j] *= alpha;
        }
        __syncthreads();
      }
    }
    // 3. values, VT tokens at a time through LDS, dequantized in batches of
    // VB elements per thread whose loads go out together
    const int cend = min(kGenChunk, t_end - n0);
    for (int t0 = 0; t0 < cend; t0 += VT) {
      const int nt = min(VT, cend - t0);
      for (int i0 = 0; i0 < nt * Dv; i0 += 256 * VB) {
        uint32_t vw[VB];
        float vsf[VB], vbf[VB];
        int vi[VB];
#pragma unroll
        for (int u = 0; u < VB; ++u) {
          const int i = min(i0 + tid + 256 * u, nt * Dv - 1);
          // (token, dim) of element i: a float quotient, corrected by one
          int t = (int)((float)i * inv_dv);
          int d = i - t * Dv;
          t = d < 0 ? t - 1 : (d >= Dv ? t + 1 : t);
          d = i - t * Dv;
          const int64_t tok = min(n0 + t0 + t, t_end - 1);
          vi[u] = i;
          vw[u] = __builtin_amdgcn_raw_buffer_load_b32(
              rv, (int)((tok * a.vp_t + d / CPW) * 4), 0, 0);
          const int64_t si = tok * a.vs_t + (d >> gsh);
          vsf[u] = gen_meta<MF32>(rvs, si, a.q_dtype);
          vbf[u] = gen_meta<MF32>(rvb, si, a.q_dtype);
          vw[u] = (vw[u] >> (BITS * (d % CPW))) & CMASK;
        }
#pragma unroll
        for (int u = 0; u < VB; ++u)
          if (i0 + tid + 256 * u < nt * Dv) vt[vi[u]] = fmaf((float)vw[u], vsf[u], vbf[u]);
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < kGenMaxOut; ++j) {
        const int e = tid + 256 * j;
        if (e < nout) {
          const int r = e / Dv, d = e - (e / Dv) * Dv;
          const float* pr = sc + r * kGenChunk + t0;
          float o = acc[j];
          for (int t = 0; t < nt; ++t) o = fmaf(pr[t], vt[t * Dv + d], o);
          acc[j] = o;
        }
      }
      __syncthreads();
    }
  }

  // results: the normalised output, or this split's partials
#pragma unroll
  for (int j = 0; j < kGenMaxOut; ++j) {
    const int e = tid + 256 * j;
    if (e >= nout) continue;
    const int r = e / Dv, d = e - (e / Dv) * Dv;
    const int64_t row = ((int64_t)b * a.Hq + h0 + r) * a.L + l;
    float z = 0.0f, m = -INFINITY;
#pragma unroll
    for (int rr = 0; rr < kGenMaxRC; ++rr)
      if (rr == r) {
        z = zrun[rr];
        m = mrun[rr];
      }
    if (a.S == 1) {
      store_out(a.out, row * Dv + d, acc[j] / z, a.out_dtype);
    } else {
      a.pacc[(row * a.S + split) * Dv + d] = acc[j];
      if (d == 0) {
        a.pm[row * a.S + split] = m;
        a.pz[row * a.S + split] = z;
      }
    }
  }
}

// one workgroup per output row: out = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) z_s.
// The split maxima and sums are reduced across the threads (a fixed tree, so
// the result is deterministic), the weights go to LDS, and each output sums
// its partials in split order with eight loads in flight.
__global__ __launch_bounds__(256) void sdpa_gen_merge_kernel(const float* __restrict__ pm,
                                                             const float* __restrict__ pz,
                                                             const float* __restrict__ pacc,
                                                             void* __restrict__ out,
                                                             int out_dtype, int S, int Dv) {
  __shared__ float wts[1024];
  __shared__ float red[8];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  float m = -INFINITY;
  for (int s = tid; s < S; s += 256) m = fmaxf(m, pm[row * S + s]);
  const float mm = block_reduce<true>(m, red, 0);
  float z = 0.0f;
  for (int s = tid; s < S; s += 256) {
    const float ms = pm[row * S + s];
    const float w = ms == -INFINITY ? 0.0f : exp2f(ms - mm);
    wts[s] = w;
    z = fmaf(pz[row * S + s], w, z);
  }
  z = block_reduce<false>(z, red, 1);
  __syncthreads();
  for (int d = tid; d < Dv; d += 256) {
    const float* p = pacc + row * S * Dv + d;
    float o = 0.0f;
    int s = 0;
    for (; s + 8 <= S; s += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = p[(int64_t)(s + u) * Dv];
#pragma unroll
      for (int u = 0; u < 8; ++u) o = fmaf(v[u], wts[s + u], o);
    }
    for (; s < S; ++s) o = fmaf(p[(int64_t)s * Dv], wts[s], o);
    store_out(out, row * Dv + d, o / z, out_dtype);
  }
}


// context splits: enough workgroups to cover the chip four times, at least
// 128 tokens per split, at most 128 splits
static int gen_splits(int64_t rows_grid, int64_t N, int64_t* tps) {
  int64_t S = std::max<int64_t>(1, cdiv(1024, std::max<int64_t>(rows_grid, 1)));
  S = std::min<int64_t>(S, std::min<int64_t>(128, cdiv(N, 128)));
  S = std::max<int64_t>(S, 1);
  *tps = cdiv(N, S);
  return (int)cdiv(N, *tps);
}

static void gen_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t N, int* RC,
                     int* nch, int* S, int64_t* tps) {
  const int64_t R = Hq / Hkv;
  *RC = (int)std::min<int64_t>(R, kGenMaxRC);
  *nch = (int)cdiv(R, *RC);
  *S = gen_splits(L * B * Hkv * *nch, N, tps);
}

template <int BITS>
static void launch_gen_m(const GenSdpaArgs& a, bool mf32, dim3 grid, size_t lds, hipStream_t st) {
  // (the workgroup's dynamic LDS stays within 64 KB, the default limit)
  if (mf32)
    hipLaunchKernelGGL((sdpa_gen_kernel<BITS, true>), grid, dim3(256), lds, st, a);
  else
    hipLaunchKernelGGL((sdpa_gen_kernel<BITS, false>), grid, dim3(256), lds, st, a);
}
static void launch_gen_b(const GenSdpaArgs& a, int bits, bool mf32, dim3 grid, size_t lds,
                         hipStream_t st) {
  if (bits == 2)
    launch_gen_m<2>(a, mf32, grid, lds, st);
  else if (bits == 4)
    launch_gen_m<4>(a, mf32, grid, lds, st);
  else
    launch_gen_m<8>(a, mf32, grid, lds, st);
}

size_t sdpa_gen_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t N,
                          int64_t Dv) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || L <= 0 || N <= 0 || Dv <= 0 || Hq % Hkv) return 0;
  int RC, nch, S;
  int64_t tps;
  gen_plan(B, Hq, Hkv, L, N, &RC, &nch, &S, &tps);
  if (S == 1) return 0;
  const size_t rows = (size_t)B * Hq * L;
  return round_up(rows * S * 4, 256) * 2 + round_up(rows * S * Dv * 4, 256);
}

int sdpa_generic(const void* q, const void* kp, const void* ks, const void* kb, const void* vp,
                 const void* vs, const void* vb, const void* mask, int mask_kind,
                 int mask_dtype, const int64_t* mask_strides, void* out, int64_t B, int64_t Hq,
                 int64_t Hkv, int64_t L, int64_t N, int64_t D, int64_t Dv, int G, int bits,
                 int qdt, int odt, float scale, const int64_t* strides, void* ws, size_t wsb,
                 hipStream_t st) {
  GenSdpaArgs a{};
  a.q = q;
  a.kp = (const uint32_t*)kp;
  a.ks = ks;
  a.kb = kb;
  a.vp = (const uint32_t*)vp;
  a.vs = vs;
  a.vb = vb;
  a.mask = mask;
  a.out = out;
  a.kp_b = strides[0] / 4;
  a.kp_h = strides[1] / 4;
  a.kp_t = strides[2] / 4;
  a.ks_b = strides[3];
  a.ks_h = strides[4];
  a.ks_t = strides[5];
  a.vp_b = strides[6] / 4;
  a.vp_h = strides[7] / 4;
  a.vp_t = strides[8] / 4;
  a.vs_b = strides[9];
  a.vs_h = strides[10];
  a.vs_t = strides[11];
  if (mask_strides) {
    a.m_b = mask_strides[0];
    a.m_h = mask_strides[1];
    a.m_l = mask_strides[2];
    a.m_n = mask_strides[3];
  }
  a.mask_kind = mask_kind;
  a.mask_dtype = mask_dtype;
  a.B = (int)B;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.L = (int)L;
  a.N = (int)N;
  a.D = (int)D;
  a.Dv = (int)Dv;
  a.G = G;
  a.bits = bits;
  a.q_dtype = qdt;
  a.out_dtype = odt;
  int64_t tps;
  gen_plan(B, Hq, Hkv, L, N, &a.RC, &a.nch, &a.S, &tps);
  a.tps = (int)tps;
  a.scale_log2 = scale * 1.4426950408889634f;
  // the reference fills masked scores with the lowest finite value of the
  // query dtype: any visible score outweighs it completely, and a row with
  // nothing visible weighs every token equally. The same value, used as is
  // in the kernel's log2 units (times log2(e) it would overflow to -inf and
  // turn such a row into NaN), keeps both properties.
  a.masked = qdt == SPARKQ_F16 ? -65504.0f : qdt == SPARKQ_BF16 ? -3.38953139e38f
                                                                  : -3.40282347e38f;
  if (a.S > 1) {
    const size_t need = sdpa_gen_workspace(B, Hq, Hkv, L, N, Dv);
    if (ws == nullptr || wsb < need)
      return set_error(SPARKQ_ERR_WORKSPACE,
                       "quantized_sdpa needs a workspace of %zu bytes (got %zu)", need, wsb);
    const size_t rows = (size_t)B * Hq * L;
    unsigned char* p = static_cast<unsigned char*>(ws);
    a.pm = reinterpret_cast<float*>(p);
    a.pz = reinterpret_cast<float*>(p + round_up(rows * a.S * 4, 256));
    a.pacc = reinterpret_cast<float*>(p + 2 * round_up(rows * a.S * 4, 256));
  }
  a.vt = gen_value_tokens(a.RC, (int)D, (int)Dv);
  const size_t lds = gen_lds_bytes(a.RC, (int)D, (int)Dv);
  const dim3 grid((unsigned)(L * a.S), (unsigned)(B * Hkv * a.nch));
  launch_gen_b(a, bits, qdt == SPARKQ_F32, grid, lds, st);
  if (int rc = check_launch("sdpa_gen_kernel")) return rc;
  if (a.S > 1) {
    hipLaunchKernelGGL(sdpa_gen_merge_kernel, dim3((unsigned)(B * Hq * L)), dim3(256), 0, st,
                       a.pm, a.pz, a.pacc, out, odt, a.S, (int)Dv);
    if (int rc = check_launch("sdpa_gen_merge_kernel")) return rc;
  }
  return SPARKQ_OK;
}

}  // namespace sparkq
