// sdpa_common.h -- argument block and device helpers shared by the decode
// attention kernels (sdpa.hip: the s8 and generic kernels; sdpa_affine.hip:
// the MFMA decode over the MLX affine caches).
#pragma once

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
  unsigned* counters;  // per (batch, KV head): the last split's workgroup merges (or null)
  int64_t kc_b, kc_h, kc_t;  // key codes (bytes)
  int64_t ks_b, ks_h, ks_t;  // key scales/biases (elements)
  int64_t vc_b, vc_h, vc_t;  // value codes (bytes)
  int64_t vs_b, vs_h, vs_t;  // value scales/biases (elements)
  int B, Hq, Hkv, N, G;
  int q_dtype, out_dtype;
  int tps, S;
  int L, causal;     // prefill: query length, bottom-right causal mask
  int pair;          // affine prefill: each workgroup takes row tiles T-1-x and x
  float scale_log2;  // softmax scale * log2(e)
  int xcd;           // prefill: XCD-grouped work order (xcd_grid_item)
};

// Workgroup (x, y) of a 2-D grid is dispatched as item y * gx + x and runs
// on XCD item % 8. With xcd set, the item order is regrouped so that each XCD
// takes a contiguous chunk of the (y, x) order: the row tiles of one
// (sequence, KV head) share an XCD's L2 for their K/V blocks, and within a
// chunk the items keep their relative order (the longest causal tiles still
// start first). A bijection on the grid; a grid of a size not divisible by
// 8 keeps its order.
__device__ __forceinline__ void xcd_grid_item(bool xcd, int& x, int& y) {
  x = (int)blockIdx.x;
  y = (int)blockIdx.y;
  const int gx = (int)gridDim.x, T = gx * (int)gridDim.y;
  if (!xcd || (T & 7) != 0) return;
  const int id = y * gx + x, v = (id & 7) * (T >> 3) + (id >> 3);
  y = v / gx;
  x = v - y * gx;
}

constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ float exp2_guarded(float x_minus_m, bool live) {
  return live ? __builtin_amdgcn_exp2f(x_minus_m) : 0.0f;
}

// fp16 in the low half of a register to fp32. The conversion reads only the
// low 16 bits; written as one instruction so that no masking of the loaded
// scale registers is hoisted to where their loads are still in flight.
__device__ __forceinline__ float f16lo_to_f32(int v) {
  float r;
  asm volatile("v_cvt_f32_f16 %0, %1" : "=v"(r) : "v"(v));
  return r;
}

__device__ __forceinline__ f32x4_t mfma16x16x32_f16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// The split merge done by the last workgroup of a (batch, KV head) to finish
// (the others' partials are read with coherent loads): per query head the
// maximum over the splits, the split weights and the normalizer (one wave
// per head), then each output as the weighted sum of the partial outputs in
// split order, eight loads in flight. sm holds gqa*S + gqa floats. GQA
// bounds the query heads per KV head (sizes the registers); gqa, the actual
// count, defaults to it.
template <int D, int GQA, int NT = 256>
__device__ void sdpa_fold_merge(const SdpaArgs& a, int b, int kh, float* sm, int gqa = GQA) {
  const int S = a.S, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float* wts = sm;             // [gqa][S]
  float* zs = sm + gqa * S;    // [gqa]
  // the maxima and sums of a head's splits are loaded together (one round
  // trip for up to 64 splits)
  for (int h = wave; h < gqa; h += NT / 64) {
    const int64_t bh = (int64_t)b * a.Hq + kh * gqa + h;
    float mm = kNegInf, z = 0.0f;
    if (S <= 64) {
      const bool live = lane < S;
      const float m = live ? splitk_load(a.pm + bh * S + lane) : kNegInf;
      const float zp = live ? splitk_load(a.pz + bh * S + lane) : 0.0f;
      mm = m;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) mm = fmaxf(mm, __shfl_xor(mm, o));
      const float w = exp2_guarded(m - mm, m != kNegInf);
      if (live) wts[h * S + lane] = w;
      z = zp * w;
    } else {
      for (int s = lane; s < S; s += 64) mm = fmaxf(mm, splitk_load(a.pm + bh * S + s));
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) mm = fmaxf(mm, __shfl_xor(mm, o));
      for (int s = lane; s < S; s += 64) {
        const float m = splitk_load(a.pm + bh * S + s);
        const float w = exp2_guarded(m - mm, m != kNegInf);
        wts[h * S + s] = w;
        z = fmaf(splitk_load(a.pz + bh * S + s), w, z);
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) z += __shfl_xor(z, o);
    if (lane == 0) zs[h] = z;
  }
  __syncthreads();
  // each thread's outputs (e = tid + 256 k) summed over the splits in split
  // order, the loads of all its outputs for eight splits in flight together
  constexpr int EPT = (GQA * D + NT - 1) / NT;
  const int E = gqa * D;
  float o[EPT];
  const float* p[EPT];
  const float* w[EPT];
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int e = min(tid + NT * k, E - 1), h = e / D, d = e - h * D;
    const int64_t bh = (int64_t)b * a.Hq + kh * gqa + h;
    o[k] = 0.0f;
    p[k] = a.pacc + bh * S * D + d;
    w[k] = wts + h * S;
  }
  int s = 0;
  for (; s + 8 <= S; s += 8) {
    float v[EPT][8];
#pragma unroll
    for (int k = 0; k < EPT; ++k)
#pragma unroll
      for (int u = 0; u < 8; ++u) v[k][u] = splitk_load(p[k] + (int64_t)(s + u) * D);
#pragma unroll
    for (int k = 0; k < EPT; ++k)
#pragma unroll
      for (int u = 0; u < 8; ++u) o[k] = fmaf(v[k][u], w[k][s + u], o[k]);
  }
  for (; s < S; ++s)
#pragma unroll
    for (int k = 0; k < EPT; ++k) o[k] = fmaf(splitk_load(p[k] + (int64_t)s * D), w[k][s], o[k]);
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int e = tid + NT * k;
    if (e < E) {
      const int h = e / D, d = e - h * D;
      const int64_t bh = (int64_t)b * a.Hq + kh * gqa + h;
      store_out(a.out, bh * D + d, zs[h] > 0.0f ? o[k] / zs[h] : 0.0f, a.out_dtype);
    }
  }
}

}  // namespace sparkq
