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
//   sdpa_mfma_kernel    the s8 + fp16-scale format with a 16-bit query: both
//                       products on the fp16 MFMA (see its comment)
//   sdpa_merge_kernel   log-sum-exp merge of the split partials.
//   kv_quantize_s8_kernel  s8 + fp16-scale quantizer (one wave per row).
//   sdpa_prefill_kernel    L > 1 queries, s8 + fp16 scale: the MFMA block step
//                          with (position, head) rows, bottom-right causal.
//   sdpa_prefill_affine_kernel  L > 1 queries over the MLX affine u8 cache:
//                          blocks dequantized once per workgroup into LDS.
//   kv_append_s8_kernel, kv_append_u8_kernel  quantize-on-append into a
//                          strided cache (s8 + fp16 scale; MLX affine u8).
#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "sdpa_common.h"

namespace sparkq {

// Code width of the decode formats: FMT 0 symmetric s8, 1 affine u8, 2
// affine u4, 3 affine u2 (the MLX packing, code j of a word at bits*j).
template <int FMT>
struct KvCodes {
  static constexpr int BITS = FMT <= 1 ? 8 : (FMT == 2 ? 4 : 2);
};

// the lane's CB bytes of codes of one token (8, 4 or 2)
template <int CB>
__device__ __forceinline__ uint2 load_codes(const uint8_t* p) {
  if constexpr (CB == 8) return *reinterpret_cast<const uint2*>(p);
  if constexpr (CB == 4) return uint2{*reinterpret_cast<const uint32_t*>(p), 0u};
  return uint2{(uint32_t)*reinterpret_cast<const uint16_t*>(p), 0u};
}

// code i of the lane's codes (little-endian bytes, BITS per code)
template <int BITS>
__device__ __forceinline__ uint32_t code_at(uint2 w, int i) {
  constexpr int PW = 32 / BITS;  // codes per word
  const uint32_t word = i < PW ? w.x : w.y;
  return (word >> (BITS * (i % PW))) & ((1u << BITS) - 1u);
}

// DPL dims per lane: 8 for 8-bit codes; 16 for 4- and 2-bit codes (8 or 4
// bytes a lane and token) up to four query heads per KV head, 8 above (the
// query and accumulator registers grow with DPL * GQA). DPL divides every
// group size, so a lane's dims share one (scale, bias).
template <int FMT, int GQA>
__host__ __device__ constexpr int decode_dpl() {
  return FMT <= 1 || GQA > 4 ? 8 : 16;
}

template <int D, int GQA, int FMT>
__global__ __launch_bounds__(256) void sdpa_decode_kernel(SdpaArgs a) {
  constexpr int BITS = KvCodes<FMT>::BITS;
  constexpr int DPL = decode_dpl<FMT, GQA>();  // dims per lane
  constexpr int CB = DPL * BITS / 8;           // code bytes per lane and token
  constexpr int LPT = D / DPL;       // lanes per token
  constexpr int TPW = 64 / LPT;      // token slots per wave
  constexpr int SLOTS = 4 * TPW;     // token slots per workgroup
  constexpr int TU = 4;              // tokens per slot per block
  constexpr bool AFF = FMT >= 1;     // affine (scale, bias per group)
  __shared__ float wm[4][GQA], wz[4][GQA];
  __shared__ __attribute__((aligned(16))) float wacc[4][GQA][D];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int split = blockIdx.x;
  const int b = blockIdx.y / a.Hkv, kh = blockIdx.y - b * a.Hkv;
  const int slot = wave * TPW + lane / LPT;
  const int dl = lane % LPT, d0 = dl * DPL;
  const int t_begin = split * a.tps;
  const int t_end = min(a.N, t_begin + a.tps);

  float qf[GQA][DPL], qsum[GQA];
#pragma unroll
  for (int h = 0; h < GQA; ++h) {
    const int64_t qo = ((int64_t)b * a.Hq + kh * GQA + h) * D + d0;
    qsum[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      qf[h][i] = load_in(a.q, qo + i, a.q_dtype) * a.scale_log2;
      qsum[h] += qf[h][i];
    }
  }

  const uint8_t* kcb = a.kc + b * a.kc_b + kh * a.kc_h + d0 * BITS / 8;
  const uint8_t* vcb = a.vc + b * a.vc_b + kh * a.vc_h + d0 * BITS / 8;
  const int64_t ksb = b * a.ks_b + kh * a.ks_h + (AFF ? d0 / a.G : 0);
  const int64_t vsb = b * a.vs_b + kh * a.vs_h + (AFF ? d0 / a.G : 0);

  float mrun[GQA], zrun[GQA], acc[GQA][DPL];
#pragma unroll
  for (int h = 0; h < GQA; ++h) {
    mrun[h] = kNegInf;
    zrun[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[h][i] = 0.0f;
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
      kw[u] = load_codes<CB>(kcb + tu * a.kc_t);
      vw[u] = load_codes<CB>(vcb + tu * a.vc_t);
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
      float kv[DPL];
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        const uint32_t c = code_at<BITS>(kw[u], i);
        kv[i] = FMT == 0 ? (float)(int8_t)c : (float)c;
      }
#pragma unroll
      for (int h = 0; h < GQA; ++h) {
        float p = 0.0f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) p = fmaf(qf[h][i], kv[i], p);
        if constexpr (AFF) p = fmaf(ksc[u], p, kbi[u] * qsum[h]);
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
      for (int i = 0; i < DPL; ++i) acc[h][i] *= alpha;
#pragma unroll
      for (int u = 0; u < TU; ++u) {
        const float pw = FMT == 0 ? p[u] * vsc[u] : p[u];
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
          const uint32_t c = code_at<BITS>(vw[u], i);
          const float vv = FMT == 0 ? (float)(int8_t)c : fmaf((float)c, vsc[u], vbi[u]);
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
      for (int i = 0; i < DPL; ++i) {
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
      for (int i = 0; i < DPL; ++i) wacc[wave][h][d0 + i] = acc[h][i];
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

// ---------------------------------------------------------------------------
// MFMA decode attention for the symmetric s8 + fp16-scale format
// ---------------------------------------------------------------------------
// A workgroup (4 waves) owns one (sequence, KV head) and one split of the
// context; each wave walks blocks of 32 tokens with 16-byte loads. Both
// products run on v_mfma_f32_16x16x32_f16, with the GQA query heads as the
// (zero-padded) 16-row side:
//  * QK: A = the query heads, B = 16 tokens x 32 dims of K. The int8 codes
//    become exact fp16 values 1152 + k with one byte permute and one xor
//    under the fp16 1024 pattern (code ^ 0x80 = k + 128); the 1152 * sum(q)
//    the offset adds is subtracted in fp32. The query is shifted per head by
//    a power of two so that it is an exact fp16 operand.
//  * PV: A = p * v_scale over 32 tokens as an fp16 hi/lo pair (two MFMAs,
//    ~22 significant bits), transposed to head-major through per-wave LDS
//    strips; B = 16 dims x 32 tokens of V, read from an
//    LDS copy of the block with ds_read_b64_tr_b8 (the 8 bytes of a lane are
//    one dim of 8 consecutive tokens) and decoded like K; the 1152 offset is
//    removed with the running sum of the fp16 weights.
// Online softmax in the log2 domain: a block max across the 16 token lanes,
// per-lane partial sums reduced once at the end. Waves combine through LDS;
// the workgroup writes the output (one split) or its (max, sum, acc) partial.
__device__ __forceinline__ u32x4_t s8x8_to_f16(uint32_t lo, uint32_t hi) {
  // bytes b0..b7 -> fp16 pairs (1152 + b0, 1152 + b1), ... in byte order
  const uint32_t m = 0x64806480u;
  return u32x4_t{__builtin_amdgcn_perm(0u, lo, 0x0C010C00u) ^ m,
                 __builtin_amdgcn_perm(0u, lo, 0x0C030C02u) ^ m,
                 __builtin_amdgcn_perm(0u, hi, 0x0C010C00u) ^ m,
                 __builtin_amdgcn_perm(0u, hi, 0x0C030C02u) ^ m};
}

template <int D, int NW = 4>  // NW waves per workgroup
struct SdpaMfmaLds {
  static constexpr int VROW = D + 16;                 // padded token row of the V copy
  static constexpr int VT = 32 * VROW;                // one wave's V block
  static constexpr int PT = 2 * 16 * 32 * 2;          // one wave's P strips (hi, lo) [16 heads][32 tokens] fp16
  static constexpr int LOOP = NW * (VT + PT);
  static constexpr int MERGE = NW * 8 * 4 * 2 + NW * 8 * D * 4;
  static constexpr int BYTES = LOOP > MERGE ? LOOP : MERGE;
};

// NW waves per workgroup: 4, or 8 for grids of at most one workgroup per CU
template <int D, int GQA, int NW = 4>
__global__ __launch_bounds__(64 * NW, (D == 256 || NW == 8) ? 1 : 2) void sdpa_mfma_kernel(SdpaArgs a) {
  constexpr int NC = D / 32;   // k chunks of QK
  constexpr int PL = D / 64;   // 16-byte K pieces per lane per 16-token group
  constexpr int NJ = D / 16;   // 16-dim column groups of PV
  constexpr int VL = D / 32;   // 16-byte V pieces per lane per block
  using L = SdpaMfmaLds<D, NW>;
  __shared__ __attribute__((aligned(16))) unsigned char smem[L::BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15, grp = lane >> 4;
  const int split = blockIdx.x;
  const int b = blockIdx.y / a.Hkv, kh = blockIdx.y - b * a.Hkv;
  const int t_begin = split * a.tps;
  const int t_end = min(a.N, t_begin + a.tps);
  unsigned char* vtile = smem + wave * L::VT;
  uint16_t* pstrip = reinterpret_cast<uint16_t*>(smem + NW * L::VT + wave * L::PT);

  // query operand: lane (head n16, k quarter grp); chunk c covers dims
  // 16*(grp + 4*(c/2)) + 8*(c%2) .. +8, matching the K piece order below
  u32x4_t qa[NC];
  float qmax = 0.0f, qs = 0.0f;
  {
    const int h = n16;
    float qv[NC][8];
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) +
                           ((int64_t)b * a.Hq + kh * GQA + min(h, GQA - 1)) * D;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d0 = 16 * (grp + 4 * (c >> 1)) + 8 * (c & 1);
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(qrow + d0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint16_t bits = (uint16_t)(w[i >> 1] >> (16 * (i & 1)));
        const float v = a.q_dtype == SPARKQ_BF16 ? bf16_to_f32(bits) : f16_to_f32(bits);
        qv[c][i] = h < GQA ? v : 0.0f;
        qmax = fmaxf(qmax, fabsf(qv[c][i]));
      }
    }
    qmax = fmaxf(qmax, __shfl_xor(qmax, 16));
    qmax = fmaxf(qmax, __shfl_xor(qmax, 32));
    const int e = (qmax > 0.0f && qmax <= 3.4028235e38f) ? ilogbf(qmax) - 14 : 0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const _Float16 lo = (_Float16)ldexpf(qv[c][2 * i], -e), hi = (_Float16)ldexpf(qv[c][2 * i + 1], -e);
        qs += (float)lo + (float)hi;
        qa[c][i] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
      }
    }
    qs += __shfl_xor(qs, 16);
    qs += __shfl_xor(qs, 32);
    qmax = ldexpf(a.scale_log2, e);  // reused: per-head score multiplier
  }
  // score lanes: head 4*grp + r, token n16 (+16 for the second token group)
  float qcorr[4], qmul[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int h = 4 * grp + r;
    qcorr[r] = 1152.0f * __shfl(qs, h & 15);
    qmul[r] = __shfl(qmax, h & 15);
  }

  // P strip rows past GQA stay zero
  for (int i = lane; i < 2 * 16 * 32; i += 64)
    if ((i & 511) / 32 >= GQA) pstrip[i] = 0;

  const rsrc_t rk = make_rsrc(a.kc + b * a.kc_b + kh * a.kc_h, (uint32_t)(t_end * a.kc_t));
  const rsrc_t rv = make_rsrc(a.vc + b * a.vc_b + kh * a.vc_h, (uint32_t)(t_end * a.vc_t));
  const rsrc_t rks = make_rsrc(reinterpret_cast<const uint16_t*>(a.ks) + b * a.ks_b + kh * a.ks_h,
                               (uint32_t)(t_end * a.ks_t * 2));
  const rsrc_t rvs = make_rsrc(reinterpret_cast<const uint16_t*>(a.vs) + b * a.vs_b + kh * a.vs_h,
                               (uint32_t)(t_end * a.vs_t * 2));

  // block registers, two sets (the next two blocks are in flight while one
  // is computed): K pieces [token group][piece], V pieces, the K and V
  // scales of the block's 32 tokens (lane t % 32). Every load is issued
  // unconditionally (past t_end it reads zeros through the bounded
  // descriptors), so the loop's wait counts stay exact instead of draining
  // all loads each block.
  u32x4_t kr[2][2][PL], vr[2][VL];
  uint16_t skr[2], svr[2];
  auto load = [&](int set, int t0) {
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
      for (int i = 0; i < PL; ++i)
        kr[set][g2][i] = buf_load16(rk, (uint32_t)((t0 + 16 * g2 + n16) * a.kc_t + 16 * (grp + 4 * i)));
#pragma unroll
    for (int v = 0; v < VL; ++v) {
      const int f = lane + 64 * v, tok = f / (D / 16), pc = f % (D / 16);
      vr[set][v] = buf_load16(rv, (uint32_t)((t0 + tok) * a.vc_t + 16 * pc));
    }
    skr[set] = buf_load2(rks, (uint32_t)((t0 + (lane & 31)) * a.ks_t * 2));
    svr[set] = buf_load2(rvs, (uint32_t)((t0 + (lane & 31)) * a.vs_t * 2));
  };

  float mrun[4], zl[4], psl[4];
  f32x4_t acc[NJ];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    mrun[r] = kNegInf;
    zl[r] = 0.0f;
    psl[r] = 0.0f;
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  const int stride = NW * 32;
  // The block's registers are read in place and refilled with the block two
  // ahead once the QK product and the scales have been taken from them, so
  // no register copy waits on the loads still in flight.
  auto block = [&](int t0, auto setc) {
    constexpr int set = decltype(setc)::value;
    __builtin_amdgcn_sched_barrier(0);  // nothing of this block moves into the previous one
    const auto& kb = kr[set];
    const auto& vb = vr[set];
    // V block to this wave's LDS copy (padded rows)
#pragma unroll
    for (int v = 0; v < VL; ++v) {
      const int f = lane + 64 * v, tok = f / (D / 16), pc = f % (D / 16);
      *reinterpret_cast<u32x4_t*>(vtile + tok * L::VROW + 16 * pc) = vb[v];
    }

    // scores: 2 token groups x NC chunks
    f32x4_t sc[2];
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2) {
      sc[g2] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const u32x4_t kp = kb[g2][c >> 1];
        const u32x4_t kf = (c & 1) ? s8x8_to_f16(kp.z, kp.w) : s8x8_to_f16(kp.x, kp.y);
        sc[g2] = mfma16x16x32_f16(qa[c], kf, sc[g2]);
      }
    }
    const float ksc0 = f16lo_to_f32(__shfl((int)skr[set], n16));
    const float ksc1 = f16lo_to_f32(__shfl((int)skr[set], 16 + n16));
    const float vsc0 = f16lo_to_f32(__shfl((int)svr[set], n16));
    const float vsc1 = f16lo_to_f32(__shfl((int)svr[set], 16 + n16));
    // the refill stays in issue order at this point (the wait counts of the
    // next blocks rely on it)
    __builtin_amdgcn_sched_barrier(0);
    load(set, t0 + 2 * stride);
    __builtin_amdgcn_sched_barrier(0);
    const bool ok0 = t0 + n16 < t_end, ok1 = t0 + 16 + n16 < t_end;

    float alpha[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float s0 = ok0 ? (sc[0][r] - qcorr[r]) * ksc0 * qmul[r] : kNegInf;
      const float s1 = ok1 ? (sc[1][r] - qcorr[r]) * ksc1 * qmul[r] : kNegInf;
      float mb = max_row16(fmaxf(s0, s1));
      mb = fmaxf(mb, mrun[r]);
      alpha[r] = exp2_guarded(mrun[r] - mb, mrun[r] != kNegInf);
      mrun[r] = mb;
      const float p0 = exp2_guarded(s0 - mb, ok0), p1 = exp2_guarded(s1 - mb, ok1);
      const float f0 = p0 * vsc0, f1 = p1 * vsc1;
      const _Float16 w0 = (_Float16)f0, w1 = (_Float16)f1;
      const _Float16 u0 = (_Float16)(f0 - (float)w0), u1 = (_Float16)(f1 - (float)w1);
      zl[r] = fmaf(zl[r], alpha[r], p0 + p1);
      psl[r] = fmaf(psl[r], alpha[r], ((float)w0 + (float)u0) + ((float)w1 + (float)u1));
      const int h = 4 * grp + r;
      if (h < GQA) {
        pstrip[h * 32 + n16] = __builtin_bit_cast(uint16_t, w0);
        pstrip[h * 32 + 16 + n16] = __builtin_bit_cast(uint16_t, w1);
        pstrip[512 + h * 32 + n16] = __builtin_bit_cast(uint16_t, u0);
        pstrip[512 + h * 32 + 16 + n16] = __builtin_bit_cast(uint16_t, u1);
      }
    }
    // PV: A = P strip row n16, tokens 8*grp .. +8
    const u32x4_t pa = *reinterpret_cast<const u32x4_t*>(pstrip + n16 * 32 + 8 * grp);
    const u32x4_t pl = *reinterpret_cast<const u32x4_t*>(pstrip + 512 + n16 * 32 + 8 * grp);
    const unsigned char* vaddr = vtile + (8 * grp + (n16 >> 1)) * L::VROW + 8 * (n16 & 1);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      acc[j][0] *= alpha[0];
      acc[j][1] *= alpha[1];
      acc[j][2] *= alpha[2];
      acc[j][3] *= alpha[3];
      typedef int v2i_t __attribute__((ext_vector_type(2)));
      const v2i_t t8 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          (__attribute__((address_space(3))) v2i_t*)(vaddr + 16 * j));
      const u32x4_t vf = s8x8_to_f16((uint32_t)t8.x, (uint32_t)t8.y);
      acc[j] = mfma16x16x32_f16(pa, vf, acc[j]);
      acc[j] = mfma16x16x32_f16(pl, vf, acc[j]);
    }
  };
  int t0 = t_begin + 32 * wave;
  // blocks in pairs with no branch in the loop body (so the wait counts
  // carried around it stay exact), then an odd last block
  const int nb = t0 < t_end ? (t_end - t0 + stride - 1) / stride : 0;
  load(0, t0);
  load(1, t0 + stride);
  int ib = 0;
  for (; ib + 2 <= nb; ib += 2, t0 += 2 * stride) {
    block(t0, std::integral_constant<int, 0>{});
    block(t0 + stride, std::integral_constant<int, 1>{});
  }
  if (ib < nb) block(t0, std::integral_constant<int, 0>{});

  // per-lane partial sums -> the 16 token lanes of each head group
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    zl[r] = sum_row16(zl[r]);
    psl[r] = sum_row16(psl[r]);
  }

  // combine the waves through LDS (the loop's LDS is free after the barrier)
  __syncthreads();
  float* wm = reinterpret_cast<float*>(smem);            // [NW][8]
  float* wz = wm + NW * 8;                               // [NW][8]
  float* wacc = wz + NW * 8;                             // [NW][8][D]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int h = 4 * grp + r;
    if (h < GQA) {
      if (n16 == 0) {
        wm[wave * 8 + h] = mrun[r];
        wz[wave * 8 + h] = zl[r];
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j) wacc[(wave * 8 + h) * D + 16 * j + n16] = acc[j][r] - 1152.0f * psl[r];
    }
  }
  __syncthreads();
  for (int e = tid; e < GQA * D; e += 64 * NW) {
    const int h = e / D, d = e - h * D;
    float mm = kNegInf;
#pragma unroll
    for (int w = 0; w < NW; ++w) mm = fmaxf(mm, wm[w * 8 + h]);
    float z = 0.0f, o = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = exp2_guarded(wm[w * 8 + h] - mm, wm[w * 8 + h] != kNegInf);
      z = fmaf(wz[w * 8 + h], wt, z);
      o = fmaf(wacc[(w * 8 + h) * D + d], wt, o);
    }
    const int64_t bh = (int64_t)b * a.Hq + kh * GQA + h;
    if (a.S == 1) {
      store_out(a.out, bh * D + d, z > 0.0f ? o / z : 0.0f, a.out_dtype);
    } else if (a.counters) {
      splitk_store(&a.pacc[(bh * a.S + split) * D + d], o);
      if (d == 0) {
        splitk_store(&a.pm[bh * a.S + split], mm);
        splitk_store(&a.pz[bh * a.S + split], z);
      }
    } else {
      a.pacc[(bh * a.S + split) * D + d] = o;
      if (d == 0) {
        a.pm[bh * a.S + split] = mm;
        a.pz[bh * a.S + split] = z;
      }
    }
  }
  if (a.S > 1 && a.counters) {
    __shared__ int s_last;
    if (splitk_arrive(a.counters + blockIdx.y, a.S, &s_last)) {
      __syncthreads();  // the combine above is done with the LDS it reused
      sdpa_fold_merge<D, GQA, 64 * NW>(a, b, kh, reinterpret_cast<float*>(smem));
      splitk_reset(a.counters + blockIdx.y);
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA prefill attention for the symmetric s8 + fp16-scale format (L > 1)
// ---------------------------------------------------------------------------
// The decode kernel's block step with the 16 MFMA rows of a wave taken by 16
// (query position, head) rows of one KV head: row rr of L*GQA is position
// rr / GQA of head rr % GQA, so a wave's rows cover 16/GQA adjacent positions
// and share most of their visible context. Each wave walks every 32-token
// block up to the last one its rows see (bottom-right causal: position i of
// L sees tokens 0 .. N-L+i; without the mask all N), two blocks in flight,
// masking each score row at its own limit, and writes its rows' outputs
// itself (no context split, no merge). A workgroup is 4 waves = 64 rows.
template <int D, int GQA>
__global__ __launch_bounds__(256, D == 256 ? 1 : 2) void sdpa_prefill_kernel(SdpaArgs a) {
  constexpr int NC = D / 32;   // k chunks of QK
  constexpr int PL = D / 64;   // 16-byte K pieces per lane per 16-token group
  constexpr int NJ = D / 16;   // 16-dim column groups of PV
  constexpr int VL = D / 32;   // 16-byte V pieces per lane per block
  using L = SdpaMfmaLds<D>;
  __shared__ __attribute__((aligned(16))) unsigned char smem[L::BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15, grp = lane >> 4;
  int bx, by;
  xcd_grid_item(a.xcd != 0, bx, by);
  const int b = by / a.Hkv, kh = by - b * a.Hkv;
  const int R = a.L * GQA;                     // query rows (position, head) of this KV head
  // the wave's first row; under the causal mask the later (longer) row
  // tiles start first
  const int row0 = (a.causal ? (int)gridDim.x - 1 - bx : bx) * 64 + wave * 16;
  // last visible token of row rr (bottom-right causal), -1 for rows past R
  auto last_tok = [&](int rr) -> int {
    return rr >= R ? -1 : (a.causal ? a.N - a.L + rr / GQA : a.N - 1);
  };
  const int t_end = row0 < R ? min(a.N, last_tok(min(row0 + 15, R - 1)) + 1) : 0;
  const int t_begin = 0;
  unsigned char* vtile = smem + wave * L::VT;
  uint16_t* pstrip = reinterpret_cast<uint16_t*>(smem + 4 * L::VT + wave * L::PT);

  // query operand: lane (head n16, k quarter grp); chunk c covers dims
  // 16*(grp + 4*(c/2)) + 8*(c%2) .. +8, matching the K piece order below
  u32x4_t qa[NC];
  float qmax = 0.0f, qs = 0.0f;
  {
    const int rr = min(row0 + n16, R - 1);
    const bool live = row0 + n16 < R;
    float qv[NC][8];
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) +
                           (((int64_t)b * a.Hq + kh * GQA + rr % GQA) * a.L + rr / GQA) * D;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d0 = 16 * (grp + 4 * (c >> 1)) + 8 * (c & 1);
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(qrow + d0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint16_t bits = (uint16_t)(w[i >> 1] >> (16 * (i & 1)));
        const float v = a.q_dtype == SPARKQ_BF16 ? bf16_to_f32(bits) : f16_to_f32(bits);
        qv[c][i] = live ? v : 0.0f;
        qmax = fmaxf(qmax, fabsf(qv[c][i]));
      }
    }
    qmax = fmaxf(qmax, __shfl_xor(qmax, 16));
    qmax = fmaxf(qmax, __shfl_xor(qmax, 32));
    const int e = (qmax > 0.0f && qmax <= 3.4028235e38f) ? ilogbf(qmax) - 14 : 0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const _Float16 lo = (_Float16)ldexpf(qv[c][2 * i], -e), hi = (_Float16)ldexpf(qv[c][2 * i + 1], -e);
        qs += (float)lo + (float)hi;
        qa[c][i] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
      }
    }
    qs += __shfl_xor(qs, 16);
    qs += __shfl_xor(qs, 32);
    qmax = ldexpf(a.scale_log2, e);  // reused: per-head score multiplier
  }
  // score lanes: head 4*grp + r, token n16 (+16 for the second token group)
  float qcorr[4], qmul[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int h = 4 * grp + r;
    qcorr[r] = 1152.0f * __shfl(qs, h & 15);
    qmul[r] = __shfl(qmax, h & 15);
  }

  // last visible token of the four score rows of this lane
  int lim[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) lim[r] = last_tok(row0 + 4 * grp + r);

  const rsrc_t rk = make_rsrc(a.kc + b * a.kc_b + kh * a.kc_h, (uint32_t)(t_end * a.kc_t));
  const rsrc_t rv = make_rsrc(a.vc + b * a.vc_b + kh * a.vc_h, (uint32_t)(t_end * a.vc_t));
  const rsrc_t rks = make_rsrc(reinterpret_cast<const uint16_t*>(a.ks) + b * a.ks_b + kh * a.ks_h,
                               (uint32_t)(t_end * a.ks_t * 2));
  const rsrc_t rvs = make_rsrc(reinterpret_cast<const uint16_t*>(a.vs) + b * a.vs_b + kh * a.vs_h,
                               (uint32_t)(t_end * a.vs_t * 2));

  // block registers, two sets (the next two blocks are in flight while one
  // is computed): K pieces [token group][piece], V pieces, the K and V
  // scales of the block's 32 tokens (lane t % 32). Every load is issued
  // unconditionally (past t_end it reads zeros through the bounded
  // descriptors), so the loop's wait counts stay exact instead of draining
  // all loads each block.
  u32x4_t kr[2][2][PL], vr[2][VL];
  uint16_t skr[2], svr[2];
  auto load = [&](int set, int t0) {
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
      for (int i = 0; i < PL; ++i)
        kr[set][g2][i] = buf_load16(rk, (uint32_t)((t0 + 16 * g2 + n16) * a.kc_t + 16 * (grp + 4 * i)));
#pragma unroll
    for (int v = 0; v < VL; ++v) {
      const int f = lane + 64 * v, tok = f / (D / 16), pc = f % (D / 16);
      vr[set][v] = buf_load16(rv, (uint32_t)((t0 + tok) * a.vc_t + 16 * pc));
    }
    skr[set] = buf_load2(rks, (uint32_t)((t0 + (lane & 31)) * a.ks_t * 2));
    svr[set] = buf_load2(rvs, (uint32_t)((t0 + (lane & 31)) * a.vs_t * 2));
  };

  float mrun[4], zl[4], psl[4];
  f32x4_t acc[NJ];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    mrun[r] = kNegInf;
    zl[r] = 0.0f;
    psl[r] = 0.0f;
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  const int stride = 32;
  // The block's registers are read in place and refilled with the block two
  // ahead once the QK product and the scales have been taken from them, so
  // no register copy waits on the loads still in flight.
  auto block = [&](int t0, auto setc) {
    constexpr int set = decltype(setc)::value;
    __builtin_amdgcn_sched_barrier(0);  // nothing of this block moves into the previous one
    const auto& kb = kr[set];
    const auto& vb = vr[set];
    // V block to this wave's LDS copy (padded rows)
#pragma unroll
    for (int v = 0; v < VL; ++v) {
      const int f = lane + 64 * v, tok = f / (D / 16), pc = f % (D / 16);
      *reinterpret_cast<u32x4_t*>(vtile + tok * L::VROW + 16 * pc) = vb[v];
    }

    // scores: 2 token groups x NC chunks
    f32x4_t sc[2];
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2) {
      sc[g2] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const u32x4_t kp = kb[g2][c >> 1];
        const u32x4_t kf = (c & 1) ? s8x8_to_f16(kp.z, kp.w) : s8x8_to_f16(kp.x, kp.y);
        sc[g2] = mfma16x16x32_f16(qa[c], kf, sc[g2]);
      }
    }
    const float ksc0 = f16lo_to_f32(__shfl((int)skr[set], n16));
    const float ksc1 = f16lo_to_f32(__shfl((int)skr[set], 16 + n16));
    const float vsc0 = f16lo_to_f32(__shfl((int)svr[set], n16));
    const float vsc1 = f16lo_to_f32(__shfl((int)svr[set], 16 + n16));
    // the refill stays in issue order at this point (the wait counts of the
    // next blocks rely on it)
    __builtin_amdgcn_sched_barrier(0);
    load(set, t0 + 2 * stride);
    __builtin_amdgcn_sched_barrier(0);

    float alpha[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok0 = t0 + n16 <= lim[r], ok1 = t0 + 16 + n16 <= lim[r];
      const float s0 = ok0 ? (sc[0][r] - qcorr[r]) * ksc0 * qmul[r] : kNegInf;
      const float s1 = ok1 ? (sc[1][r] - qcorr[r]) * ksc1 * qmul[r] : kNegInf;
      float mb = max_row16(fmaxf(s0, s1));
      mb = fmaxf(mb, mrun[r]);
      alpha[r] = exp2_guarded(mrun[r] - mb, mrun[r] != kNegInf);
      mrun[r] = mb;
      const float p0 = exp2_guarded(s0 - mb, ok0), p1 = exp2_guarded(s1 - mb, ok1);
      const float f0 = p0 * vsc0, f1 = p1 * vsc1;
      const _Float16 w0 = (_Float16)f0, w1 = (_Float16)f1;
      const _Float16 u0 = (_Float16)(f0 - (float)w0), u1 = (_Float16)(f1 - (float)w1);
      zl[r] = fmaf(zl[r], alpha[r], p0 + p1);
      psl[r] = fmaf(psl[r], alpha[r], ((float)w0 + (float)u0) + ((float)w1 + (float)u1));
      const int h = 4 * grp + r;
      pstrip[h * 32 + n16] = __builtin_bit_cast(uint16_t, w0);
      pstrip[h * 32 + 16 + n16] = __builtin_bit_cast(uint16_t, w1);
      pstrip[512 + h * 32 + n16] = __builtin_bit_cast(uint16_t, u0);
      pstrip[512 + h * 32 + 16 + n16] = __builtin_bit_cast(uint16_t, u1);
    }
    // PV: A = P strip row n16, tokens 8*grp .. +8
    const u32x4_t pa = *reinterpret_cast<const u32x4_t*>(pstrip + n16 * 32 + 8 * grp);
    const u32x4_t pl = *reinterpret_cast<const u32x4_t*>(pstrip + 512 + n16 * 32 + 8 * grp);
    const unsigned char* vaddr = vtile + (8 * grp + (n16 >> 1)) * L::VROW + 8 * (n16 & 1);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      acc[j][0] *= alpha[0];
      acc[j][1] *= alpha[1];
      acc[j][2] *= alpha[2];
      acc[j][3] *= alpha[3];
      typedef int v2i_t __attribute__((ext_vector_type(2)));
      const v2i_t t8 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          (__attribute__((address_space(3))) v2i_t*)(vaddr + 16 * j));
      const u32x4_t vf = s8x8_to_f16((uint32_t)t8.x, (uint32_t)t8.y);
      acc[j] = mfma16x16x32_f16(pa, vf, acc[j]);
      acc[j] = mfma16x16x32_f16(pl, vf, acc[j]);
    }
  };
  int t0 = t_begin;
  // blocks in pairs with no branch in the loop body (so the wait counts
  // carried around it stay exact), then an odd last block
  const int nb = t0 < t_end ? (t_end - t0 + stride - 1) / stride : 0;
  load(0, t0);
  load(1, t0 + stride);
  int ib = 0;
  for (; ib + 2 <= nb; ib += 2, t0 += 2 * stride) {
    block(t0, std::integral_constant<int, 0>{});
    block(t0 + stride, std::integral_constant<int, 1>{});
  }
  if (ib < nb) block(t0, std::integral_constant<int, 0>{});

  // per-lane partial sums -> the 16 token lanes of each head group
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    zl[r] = sum_row16(zl[r]);
    psl[r] = sum_row16(psl[r]);
  }

  // each wave owns its 16 rows: out = (acc - 1152 * sum of fp16 weights) / z
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int rr = row0 + 4 * grp + r;
    if (rr < R) {
      const int64_t orow = ((int64_t)b * a.Hq + kh * GQA + rr % GQA) * a.L + rr / GQA;
      const float inv = zl[r] > 0.0f ? 1.0f / zl[r] : 0.0f;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        store_out(a.out, orow * D + 16 * j + n16, (acc[j][r] - 1152.0f * psl[r]) * inv, a.out_dtype);
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA prefill attention over the MLX affine u8 cache (L > 1)
// ---------------------------------------------------------------------------
// The numerics of spark_affine_u8_sdpa_prefill: K and V dequantize to the
// query dtype T as T(code * scale + bias) (fp32 fma, one rounding), the
// softmax weights are rounded to T for the PV product, and the scores, the
// normalizer and the outputs stay fp32. The query is used as given (the
// softmax scale multiplies the fp32 scores instead of a rounded q * scale).
//
// A workgroup of 4 waves owns 128 consecutive (position, head) rows of one
// (sequence, KV head), 32 rows per wave, and walks the 32-token blocks up to
// the last token its last row sees. Each block is dequantized once per
// workgroup into LDS (double-buffered, one barrier per block): K token-major
// with the 16-byte chunks of a token row XOR-swizzled by the token, V
// token-major with its 32-byte runs swizzled. Both products run on the
// 16x16x32 MFMA in the transposed orientation
//     S^T (16 tokens x 16 rows) = K (16 tokens x 32 dims) . Q^T
//     O^T (16 dims x 16 rows)  += V^T (16 dims x 32 tokens) . P^T
// so that the lane holding row n16's scores for tokens 4g+r and 16+4g+r
// (lane group g) after QK holds exactly the k-slots of that row in the PV
// operand: alpha and the normalizer of a row never leave its lane. The V^T
// operand comes from ds_read_b64_tr_b16 (per 16 lanes a 4-token x 16-dim
// tile, each lane left with one dim of the 4 tokens).
template <int D>
struct AffPrefillLds {
  static constexpr int ROW = 2 * D;        // bytes of one dequantized token row
  static constexpr int TILE = 32 * ROW;    // one 32-token K or V block
  static constexpr int BUF = 2 * TILE;     // K then V
  static constexpr int BYTES = 2 * BUF;    // double-buffered
};
// 16-byte chunk swizzle of K rows and 32-byte run swizzle of V rows: the 16
// lanes of an MFMA operand read (K: 16 tokens, one chunk; V: 4 tokens x 4
// lanes per 16 lanes, 8 tokens per half wave) hit distinct banks.
template <int D>
__device__ __forceinline__ int aff_kswz(int t) { return D >= 128 ? (t & 15) : ((t >> 1) & 7); }
template <int D>
__device__ __forceinline__ int aff_vswz(int t) { return D >= 128 ? (t & 7) : ((t >> 1) & 3); }

template <typename T>
__device__ __forceinline__ f32x4_t mfma16_kv(u32x4_t a, u32x4_t b, f32x4_t c);
template <>
__device__ __forceinline__ f32x4_t mfma16_kv<BF16>(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4_t mfma16_kv<F16>(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// 16 codes (byte j of word w is code 4w+j) of one group -> 16 values of T in
// 8 packed words, each T(code * s + b) with one rounding.
template <typename T>
__device__ __forceinline__ void dequant_u8x16(u32x4_t c, uint32_t s, uint32_t b, uint32_t o[8]);
template <>
__device__ __forceinline__ void dequant_u8x16<BF16>(u32x4_t c, uint32_t s, uint32_t b, uint32_t o[8]) {
  const float sf = __uint_as_float(s << 16), bf = __uint_as_float(b << 16);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t x = c[w];
    o[2 * w] = pack_round<BF16>(fmaf((float)(x & 255u), sf, bf), fmaf((float)((x >> 8) & 255u), sf, bf));
    o[2 * w + 1] =
        pack_round<BF16>(fmaf((float)((x >> 16) & 255u), sf, bf), fmaf((float)(x >> 24), sf, bf));
  }
}
template <>
__device__ __forceinline__ void dequant_u8x16<F16>(u32x4_t c, uint32_t s, uint32_t b, uint32_t o[8]) {
  // a code byte under the fp16 exponent of 1024 reads 1024 + code; the
  // packed subtract leaves the code exactly, the packed fma rounds once
  const f16x2_t s2 = __builtin_bit_cast(f16x2_t, (s & 0xFFFFu) * 0x10001u);
  const f16x2_t b2 = __builtin_bit_cast(f16x2_t, (b & 0xFFFFu) * 0x10001u);
  const f16x2_t k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t x = c[w];
    const f16x2_t lo = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u)) - k1024;
    const f16x2_t hi = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u)) - k1024;
    o[2 * w] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(lo, s2, b2));
    o[2 * w + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(hi, s2, b2));
  }
}

// max / sum over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48);
// every lane ends with the same value
__device__ __forceinline__ float max_rows4(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_rows4(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int D, typename T, bool SPLIT>
__global__ __launch_bounds__(256, D <= 128 ? 2 : 1) void sdpa_prefill_affine_kernel(SdpaArgs a) {
  using LY = AffPrefillLds<D>;
  constexpr int NK = D / 32;                    // QK k chunks
  constexpr int NJ = D / 16;                    // PV dim tiles
  constexpr int PIECES = 2 * D;                 // 16-code pieces of one K (or V) block
  constexpr int PPT = PIECES >= 256 ? PIECES / 256 : 1;
  constexpr int NVB = NJ < 8 ? NJ : 8;          // distinct V run offsets of a lane
  __shared__ __attribute__((aligned(16))) unsigned char smem[LY::BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15, grp = lane >> 4;
  int bx, by;
  xcd_grid_item(a.xcd != 0, bx, by);
  const int b = by / a.Hkv, kh = by - b * a.Hkv;
  const int gqa = a.Hq / a.Hkv;
  const int R = a.L * gqa;  // (position, head) rows of this KV head
  // Row tiles of 128. Under the causal mask tile t walks ~t+1 times the
  // blocks of tile 0: with pairing (when the paired grid still covers the
  // chip) workgroup x takes tiles T-1-x and x in turn, so every workgroup
  // walks about the same number of blocks; otherwise the longer tiles start
  // first.
  // With a context split (S > 1, no pairing) workgroup x takes chunk x % S
  // of the blocks of tile x / S and the last chunk to finish merges.
  const int ntiles = (R + 127) / 128;
  const int S = SPLIT ? a.S : 1;
  const int xt = S > 1 ? bx / S : bx, chunk = bx - xt * S;
  const int npass = D <= 128 && a.pair && ntiles - 1 - xt != xt ? 2 : 1;
  for (int pass = 0; pass < npass; ++pass) {
  const int tile = D <= 128 && a.pair ? (pass == 0 ? ntiles - 1 - xt : xt)
                                      : (a.causal ? ntiles - 1 - xt : xt);
  const int rw0 = tile * 128;
  auto last_tok = [&](int rr) -> int {
    return rr >= R ? -1 : (a.causal ? a.N - a.L + rr / gqa : a.N - 1);
  };
  const int t_end = min(a.N, last_tok(min(rw0 + 127, R - 1)) + 1);
  const int nb_all = (t_end + 31) / 32;
  const int ib0 = (int)((int64_t)chunk * nb_all / S), ib1 = (int)((int64_t)(chunk + 1) * nb_all / S);

  // Q^T operand of each 16-row tile: lane (g, n16) holds row n16, dims
  // 32*kk + 8*g .. +8; rows past R read row R-1 and are masked out
  u32x4_t qb[2][NK];
  int lim[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int rr = rw0 + 32 * wave + 16 * rt + n16;
    lim[rt] = last_tok(rr);
    const int rq = min(rr, R - 1);
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) +
                           (((int64_t)b * a.Hq + kh * gqa + rq % gqa) * a.L + rq / gqa) * D;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) qb[rt][kk] = *reinterpret_cast<const u32x4_t*>(qrow + 32 * kk + 8 * grp);
  }

  // staging: piece p = tid + 256 i is token p / (D/16), codes 16 (p % (D/16)) ..
  // +16; loads past t_end read zeros through the bounded descriptors
  const int64_t sbase_k = (int64_t)b * a.ks_b + kh * a.ks_h, sbase_v = (int64_t)b * a.vs_b + kh * a.vs_h;
  const rsrc_t rk = make_rsrc(a.kc + b * a.kc_b + kh * a.kc_h, (uint32_t)(t_end * a.kc_t));
  const rsrc_t rv = make_rsrc(a.vc + b * a.vc_b + kh * a.vc_h, (uint32_t)(t_end * a.vc_t));
  const rsrc_t rks = make_rsrc(reinterpret_cast<const uint16_t*>(a.ks) + sbase_k, (uint32_t)(t_end * a.ks_t * 2));
  const rsrc_t rkb = make_rsrc(reinterpret_cast<const uint16_t*>(a.kb) + sbase_k, (uint32_t)(t_end * a.ks_t * 2));
  const rsrc_t rvs = make_rsrc(reinterpret_cast<const uint16_t*>(a.vs) + sbase_v, (uint32_t)(t_end * a.vs_t * 2));
  const rsrc_t rvb = make_rsrc(reinterpret_cast<const uint16_t*>(a.vb) + sbase_v, (uint32_t)(t_end * a.vs_t * 2));
  const bool stager = PIECES >= 256 || tid < PIECES;  // wave-uniform
  u32x4_t kcr[PPT], vcr[PPT];
  uint32_t ksr[PPT], kbr[PPT], vsr[PPT], vbr[PPT];
  auto load = [&](int t0) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int p = tid + 256 * i, tk = p / (D / 16), jb = p % (D / 16), g = 16 * jb / a.G;
      kcr[i] = buf_load16(rk, (uint32_t)((t0 + tk) * a.kc_t + 16 * jb));
      vcr[i] = buf_load16(rv, (uint32_t)((t0 + tk) * a.vc_t + 16 * jb));
      ksr[i] = buf_load2(rks, (uint32_t)(((t0 + tk) * a.ks_t + g) * 2));
      kbr[i] = buf_load2(rkb, (uint32_t)(((t0 + tk) * a.ks_t + g) * 2));
      vsr[i] = buf_load2(rvs, (uint32_t)(((t0 + tk) * a.vs_t + g) * 2));
      vbr[i] = buf_load2(rvb, (uint32_t)(((t0 + tk) * a.vs_t + g) * 2));
    }
  };
  // D <= 128: the next block dequantized in registers (interleaved with the
  // PV product), then written to the other buffer
  uint32_t kw[PPT][8], vw[PPT][8];
  auto dequant = [&]() {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      dequant_u8x16<T>(kcr[i], ksr[i], kbr[i], kw[i]);
      dequant_u8x16<T>(vcr[i], vsr[i], vbr[i], vw[i]);
    }
  };
  // dequant and write in one pass, each piece's values short-lived
  auto stage = [&](unsigned char* buf) {
    if (!stager) return;
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int p = tid + 256 * i, tk = p / (D / 16), jb = p % (D / 16);
      uint32_t kq[8], vq[8];
      dequant_u8x16<T>(kcr[i], ksr[i], kbr[i], kq);
      dequant_u8x16<T>(vcr[i], vsr[i], vbr[i], vq);
      unsigned char* kt = buf + tk * LY::ROW;
      const int ks = aff_kswz<D>(tk);
      *reinterpret_cast<u32x4_t*>(kt + ((2 * jb) ^ ks) * 16) = u32x4_t{kq[0], kq[1], kq[2], kq[3]};
      *reinterpret_cast<u32x4_t*>(kt + ((2 * jb + 1) ^ ks) * 16) = u32x4_t{kq[4], kq[5], kq[6], kq[7]};
      unsigned char* vt = buf + LY::TILE + tk * LY::ROW + (jb ^ aff_vswz<D>(tk)) * 32;
      *reinterpret_cast<u32x4_t*>(vt) = u32x4_t{vq[0], vq[1], vq[2], vq[3]};
      *reinterpret_cast<u32x4_t*>(vt + 16) = u32x4_t{vq[4], vq[5], vq[6], vq[7]};
    }
  };
  auto stage_write = [&](unsigned char* buf) {
    if (!stager) return;
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int p = tid + 256 * i, tk = p / (D / 16), jb = p % (D / 16);
      unsigned char* kt = buf + tk * LY::ROW;
      const int ks = aff_kswz<D>(tk);
      *reinterpret_cast<u32x4_t*>(kt + ((2 * jb) ^ ks) * 16) = u32x4_t{kw[i][0], kw[i][1], kw[i][2], kw[i][3]};
      *reinterpret_cast<u32x4_t*>(kt + ((2 * jb + 1) ^ ks) * 16) =
          u32x4_t{kw[i][4], kw[i][5], kw[i][6], kw[i][7]};
      unsigned char* vt = buf + LY::TILE + tk * LY::ROW + (jb ^ aff_vswz<D>(tk)) * 32;
      *reinterpret_cast<u32x4_t*>(vt) = u32x4_t{vw[i][0], vw[i][1], vw[i][2], vw[i][3]};
      *reinterpret_cast<u32x4_t*>(vt + 16) = u32x4_t{vw[i][4], vw[i][5], vw[i][6], vw[i][7]};
    }
  };

  // operand addresses of this lane inside a buffer. K (A of S^T): token
  // n16 (+16 for the second token tile), chunk 4 kk + g. V (A of O^T): the
  // lane feeds token 4 g + n16/4 (+16 for slots 4..7), dims 16 j + 4 (n16 % 4)
  // .. +4; run j = 8 u + v sits at va[v] + 256 u.
  int ka[NK], va[NVB];
#pragma unroll
  for (int kk = 0; kk < NK; ++kk) ka[kk] = n16 * LY::ROW + ((4 * kk + grp) ^ aff_kswz<D>(n16)) * 16;
  {
    const int tv = 4 * grp + (n16 >> 2), sw = aff_vswz<D>(tv);
#pragma unroll
    for (int v = 0; v < NVB; ++v) va[v] = LY::TILE + tv * LY::ROW + ((v ^ sw) * 32) + 8 * (n16 & 3);
  }

  float mrun[2] = {kNegInf, kNegInf}, zl[2] = {0.0f, 0.0f};
  f32x4_t acc[2][NJ];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[rt][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  typedef short s16x4_t __attribute__((ext_vector_type(4)));
  // One block. The running max of a row moves only when a block's max
  // exceeds it by more than 8 (log2 units): until then the weights
  // exp2(s - m) stay below 2^8 and the accumulators are not rescaled, so the
  // rescale (a wave-uniform branch) runs for few blocks. It moves to the
  // ceiling of the block max: with an integer offset the weights rounded to
  // T are T(exp2(s)) scaled by a power of two (rounding commutes with it), so
  // they do not depend on the block order, and every rescale factor is an
  // exact power of two.
  auto compute = [&](const unsigned char* buf, int t0) {
    f32x4_t sc[2][2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) sc[tt][rt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const u32x4_t kf = *reinterpret_cast<const u32x4_t*>(buf + ka[kk] + tt * 16 * LY::ROW);
        sc[tt][0] = mfma16_kv<T>(kf, qb[0][kk], sc[tt][0]);
        sc[tt][1] = mfma16_kv<T>(kf, qb[1][kk], sc[tt][1]);
      }
    u32x4_t pb[2];
    float alpha[2];
    bool up[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      float s[8];
      float mb = kNegInf;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        s[i] = sc[i >> 2][rt][i & 3] * a.scale_log2;
        s[i] = t0 + 16 * (i >> 2) + 4 * grp + (i & 3) <= lim[rt] ? s[i] : kNegInf;
        mb = fmaxf(mb, s[i]);
      }
      mb = max_rows4(mb);
      up[rt] = mb > mrun[rt] + 8.0f;
      const float mnew = ceilf(mb);
      alpha[rt] = up[rt] ? exp2_guarded(mrun[rt] - mnew, mrun[rt] != kNegInf) : 1.0f;
      mrun[rt] = up[rt] ? mnew : mrun[rt];
      // a row with nothing visible yet keeps m = -inf; its weights are 0
      const float mu = mrun[rt] == kNegInf ? 0.0f : mrun[rt];
      float p[8], ps = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        p[i] = __builtin_amdgcn_exp2f(s[i] - mu);
        ps += p[i];
      }
      zl[rt] = fmaf(zl[rt], alpha[rt], ps);
      pb[rt] = u32x4_t{pack_round<T>(p[0], p[1]), pack_round<T>(p[2], p[3]), pack_round<T>(p[4], p[5]),
                       pack_round<T>(p[6], p[7])};
    }
    if (__builtin_amdgcn_ballot_w64(up[0] || up[1]) != 0) {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[rt][j] *= alpha[rt];
    }
    // the next block's dequant (VALU) goes between the PV MFMAs (at D=256
    // the registers it holds cost more than the overlap gains)
    if (D <= 128) dequant();
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const unsigned char* vp = buf + va[j % NVB] + 256 * (j / NVB);
      const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4_t*)(vp));
      const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4_t*)(vp + 16 * LY::ROW));
      typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
      const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), h2 = __builtin_bit_cast(u32x2_t, hi);
      const u32x4_t vf = u32x4_t{l2.x, l2.y, h2.x, h2.y};
      acc[0][j] = mfma16_kv<T>(vf, pb[0], acc[0][j]);
      acc[1][j] = mfma16_kv<T>(vf, pb[1], acc[1][j]);
    }
    if (D <= 128) {
      constexpr int VPM = (PPT * 80) / (2 * NJ);  // dequant VALU per PV MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
        if (j + 2 < NJ) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
    }
  };
  load(32 * ib0);
  stage(smem);
  load(32 * ib0 + 32);
  __syncthreads();
  for (int ib = ib0; ib < ib1; ++ib) {
    // compute (with the next block's dequant), write the next block into
    // the other buffer, issue the loads of the block after it
    const int t0 = 32 * ib, cur = (ib - ib0) & 1;
    compute(smem + cur * LY::BUF, t0);
    if (D > 128)
      stage(smem + (cur ^ 1) * LY::BUF);
    else
      stage_write(smem + (cur ^ 1) * LY::BUF);
    load(t0 + 64);
    __syncthreads();
  }

  float zrow[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) zrow[rt] = sum_rows4(zl[rt]);
  if (SPLIT) {
    // store this chunk's (max, sum, acc) of its 128 rows, then the last
    // chunk of the tile to arrive combines all S in chunk order
    const int64_t tg = ((int64_t)b * a.Hkv + kh) * ntiles + tile;
    const int64_t pbase = tg * S;
    constexpr int NV = 2 * NJ * 4;  // accumulators per thread
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      if (grp == 0) {
        const int64_t ri = (pbase + chunk) * 128 + 32 * wave + 16 * rt + n16;
        splitk_store(a.pm + ri, mrun[rt]);
        splitk_store(a.pz + ri, zrow[rt]);
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          splitk_store(a.pacc + ((pbase + chunk) * NV + (rt * NJ + j) * 4 + r) * 256 + tid, acc[rt][j][r]);
    }
    __shared__ int s_last;
    if (!splitk_arrive(a.counters + tg, S, &s_last)) continue;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int64_t rrow = 32 * wave + 16 * rt + n16;
      float mm = kNegInf;
      for (int c = 0; c < S; ++c) mm = fmaxf(mm, splitk_load(a.pm + (pbase + c) * 128 + rrow));
      float z = 0.0f;
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[rt][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      for (int c = 0; c < S; ++c) {
        const float mc = splitk_load(a.pm + (pbase + c) * 128 + rrow);
        const float w = exp2_guarded(mc - mm, mc != kNegInf);
        z = fmaf(splitk_load(a.pz + (pbase + c) * 128 + rrow), w, z);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[rt][j][r] =
                fmaf(splitk_load(a.pacc + ((pbase + c) * NV + (rt * NJ + j) * 4 + r) * 256 + tid), w,
                     acc[rt][j][r]);
      }
      zrow[rt] = z;
    }
    splitk_reset(a.counters + tg);
  }

  // O^T lane (g, n16): row n16, dims 16 j + 4 g + r
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const float z = zrow[rt];
    const int rr = rw0 + 32 * wave + 16 * rt + n16;
    if (rr < R) {
      const int64_t orow = (((int64_t)b * a.Hq + kh * gqa + rr % gqa) * a.L + rr / gqa) * D;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = z > 0.0f ? acc[rt][j][r] / z : 0.0f;
        const int64_t idx = orow + 16 * j + 4 * grp;
        if (a.out_dtype == SPARKQ_F32) {
          *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(a.out) + idx) = f32x4_t{o[0], o[1], o[2], o[3]};
        } else {
          typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
          *reinterpret_cast<u32x2_t*>(reinterpret_cast<uint16_t*>(a.out) + idx) =
              u32x2_t{pack_round<T>(o[0], o[1]), pack_round<T>(o[2], o[3])};
        }
      }
    }
  }
  }  // pass
}

// Log-sum-exp merge of the split partials of one (sequence, query head) row:
// the split maxima and sums reduce across the workgroup, then thread
// (d, part) sums the weighted partial outputs of every 256/D-th split with
// eight loads in flight.
__global__ __launch_bounds__(256) void sdpa_merge_kernel(const float* __restrict__ pm,
                                                         const float* __restrict__ pz,
                                                         const float* __restrict__ pacc,
                                                         void* __restrict__ out, int out_dtype,
                                                         int S, int D) {
  __shared__ float wts[1024];
  __shared__ float red[8];
  __shared__ float part[256];
  const int64_t bh = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // 1. global max over the splits
  float mm = kNegInf;
  for (int s = tid; s < S; s += 256) mm = fmaxf(mm, pm[bh * S + s]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mm = fmaxf(mm, __shfl_xor(mm, o));
  if (lane == 0) red[wave] = mm;
  __syncthreads();
  mm = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // 2. split weights and the normalizer
  float z = 0.0f;
  for (int s = tid; s < S; s += 256) {
    const float m = pm[bh * S + s];
    const float w = exp2_guarded(m - mm, m != kNegInf);
    wts[s] = w;
    z = fmaf(pz[bh * S + s], w, z);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) z += __shfl_xor(z, o);
  if (lane == 0) red[4 + wave] = z;
  __syncthreads();
  z = (red[4] + red[5]) + (red[6] + red[7]);
  // 3. weighted sum of the partial outputs
  const int parts = 256 / D, d = tid % D, pi = tid / D;
  float o = 0.0f;
  if (pi < parts) {
    int s = pi;
    for (; s + 7 * parts < S; s += 8 * parts) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = pacc[(bh * S + s + u * parts) * D + d];
#pragma unroll
      for (int u = 0; u < 8; ++u) o = fmaf(v[u], wts[s + u * parts], o);
    }
    for (; s < S; s += parts) o = fmaf(pacc[(bh * S + s) * D + d], wts[s], o);
  }
  part[tid] = o;
  __syncthreads();
  if (tid < D) {
    float t = 0.0f;
    for (int q = 0; q < parts; ++q) t += part[q * D + tid];
    store_out(out, bh * D + tid, z > 0.0f ? t / z : 0.0f, out_dtype);
  }
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

// Quantize-on-append: row (b, h, l) of x [B,H,L,D] to cache token offset+l.
// S8 format: one wave per row, the kv_quantize_s8_kernel formula. Affine u8
// format: one thread per group of G values, scale = to_dtype((max-min)/255),
// bias = to_dtype(min), code = clamp(rint((x - bias) / scale), 0, 255) with
// the rounded scale and bias (0 for a zero scale), four codes per uint32
// (dim 4w+j in byte j of word w). The 4- and 2-bit affine formats use the
// same thread-per-group kernel with 15 or 3 bins and 8 or 16 codes per
// uint32 (dim cpw*w+j at bits b*j). This min/max rule is not mx.quantize's,
// which makes the larger-magnitude edge exact (negative scale, bias = edge).
struct KvAppendArgs {
  const void* x;
  void* codes;
  void* scales;
  void* biases;
  int64_t c_b, c_h, c_t;  // code strides (bytes)
  int64_t s_b, s_h, s_t;  // scale/bias strides (elements)
  int B, H, L, D, G, offset, x_dtype;
  int bits;  // affine formats: 8, 4 or 2 bits per code
};

__global__ __launch_bounds__(256) void kv_append_s8_kernel(KvAppendArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= (int64_t)a.B * a.H * a.L) return;
  const int l = (int)(row % a.L), bh = (int)(row / a.L), h = bh % a.H, b = bh / a.H;
  const int D = a.D;
  float amax = 0.0f;
  for (int d = lane; d < D; d += 64) amax = fmaxf(amax, fabsf(load_in(a.x, row * D + d, a.x_dtype)));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  uint16_t s16 = f32_to_f16(amax / 127.0f);
  if (f16_to_f32(s16) == 0.0f) s16 = 0x3C00u;
  const float s = f16_to_f32(s16);
  const int64_t t = (int64_t)a.offset + l;
  if (lane == 0)
    reinterpret_cast<uint16_t*>(a.scales)[b * a.s_b + h * a.s_h + t * a.s_t] = s16;
  int8_t* dst = reinterpret_cast<int8_t*>(a.codes) + b * a.c_b + h * a.c_h + t * a.c_t;
  for (int d = lane; d < D; d += 64) {
    float v = __builtin_rintf(load_in(a.x, row * D + d, a.x_dtype) / s);
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    dst[d] = (int8_t)v;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void kv_append_u8_kernel(KvAppendArgs a) {
  const int ng = a.D / a.G;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (int64_t)a.B * a.H * a.L * ng) return;
  const int g = (int)(gid % ng);
  const int64_t row = gid / ng;
  const int l = (int)(row % a.L), bh = (int)(row / a.L), h = bh % a.H, b = bh / a.H;
  const int64_t t = (int64_t)a.offset + l;
  const uint16_t* v = reinterpret_cast<const uint16_t*>(a.x) + row * a.D + (int64_t)g * a.G;
  float mn = T::to_f32(v[0]), mx = mn;
  for (int i = 1; i < a.G; ++i) {
    const float f = T::to_f32(v[i]);
    mn = f < mn ? f : mn;
    mx = f > mx ? f : mx;
  }
  const float nbins = (float)((1 << a.bits) - 1);
  const uint16_t s16 = T::from_f32((mx - mn) / nbins), b16 = T::from_f32(mn);
  const int64_t si = b * a.s_b + h * a.s_h + t * a.s_t + g;
  reinterpret_cast<uint16_t*>(a.scales)[si] = s16;
  reinterpret_cast<uint16_t*>(a.biases)[si] = b16;
  const float sf = T::to_f32(s16), bf = T::to_f32(b16);
  const int cpw = 32 / a.bits;  // codes per word, the lowest bits first
  uint32_t* dst = reinterpret_cast<uint32_t*>(reinterpret_cast<unsigned char*>(a.codes) +
                                              b * a.c_b + h * a.c_h + t * a.c_t) + g * a.G / cpw;
  for (int w = 0; w < a.G / cpw; ++w) {
    uint32_t word = 0;
    for (int j = 0; j < cpw; ++j) {
      float q = 0.0f;
      if (sf != 0.0f) {
        q = __builtin_rintf((T::to_f32(v[cpw * w + j]) - bf) / sf);
        q = q < 0.0f ? 0.0f : (q > nbins ? nbins : q);
      }
      word |= (uint32_t)q << (a.bits * j);
    }
    dst[w] = word;
  }
}

// The same quantizer with one wave per row (D = 64*E): lane i holds dims
// E*i .. E*i+E-1, the G/E lanes of a group reduce its min and max by a
// butterfly, and each lane writes its own E code bytes (byte j of word w of
// the packed row is dim 4w+j). Same formula and rounding as above.
template <typename T, int E>
__global__ __launch_bounds__(256) void kv_append_u8_wave_kernel(KvAppendArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= (int64_t)a.B * a.H * a.L) return;  // whole waves leave together
  const int l = (int)(row % a.L), bh = (int)(row / a.L), h = bh % a.H, b = bh / a.H;
  const int64_t t = (int64_t)a.offset + l;
  const uint16_t* v = reinterpret_cast<const uint16_t*>(a.x) + row * (64 * E) + E * lane;
  float f[E];
#pragma unroll
  for (int e = 0; e < E; ++e) f[e] = T::to_f32(v[e]);
  float mn = f[0], mx = f[0];
#pragma unroll
  for (int e = 1; e < E; ++e) {
    mn = f[e] < mn ? f[e] : mn;
    mx = f[e] > mx ? f[e] : mx;
  }
  const int LG = a.G / E;  // lanes per group: 8, 16, 32 or 64
  for (int o = LG >> 1; o > 0; o >>= 1) {
    const float pn = __shfl_xor(mn, o), px = __shfl_xor(mx, o);
    mn = pn < mn ? pn : mn;
    mx = px > mx ? px : mx;
  }
  const uint16_t s16 = T::from_f32((mx - mn) / 255.0f), b16 = T::from_f32(mn);
  const int g = lane / LG;
  if (lane % LG == 0) {
    const int64_t si = b * a.s_b + h * a.s_h + t * a.s_t + g;
    reinterpret_cast<uint16_t*>(a.scales)[si] = s16;
    reinterpret_cast<uint16_t*>(a.biases)[si] = b16;
  }
  const float sf = T::to_f32(s16), bf = T::to_f32(b16);
  uint32_t bytes = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    float q = 0.0f;
    if (sf != 0.0f) {
      q = __builtin_rintf((f[e] - bf) / sf);
      q = q < 0.0f ? 0.0f : (q > 255.0f ? 255.0f : q);
    }
    bytes |= (uint32_t)q << (8 * e);
  }
  unsigned char* dst = reinterpret_cast<unsigned char*>(a.codes) + b * a.c_b + h * a.c_h +
                       t * a.c_t + E * lane;
  if constexpr (E == 4)
    *reinterpret_cast<uint32_t*>(dst) = bytes;
  else if constexpr (E == 2)
    *reinterpret_cast<uint16_t*>(dst) = (uint16_t)bytes;
  else
    *dst = (unsigned char)bytes;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
// Context splits: about 64 per sequence batch-wide (512 workgroups with 8 KV
// heads), at least 128 tokens per split (one 32-token block per wave), at
// most 1024 splits, and no empty split.
static int sdpa_splits(int64_t B, int64_t N, int64_t* tps_out = nullptr) {
  // 64 splits over the batch, at most 32 per sequence and at least 256
  // tokens per split: past that the merge of the partials costs more than
  // the extra workgroups gain (B=1 N=32768: 28.0 us at 64 splits, 23.1 at
  // 32; B=1 N=4096: 12.2 us at 32, 11.2 at 16)
  int64_t S = cdiv(env_int("SPARKQ_SDPA_SPLITS", 64), B);
  const int64_t cap = env_int("SPARKQ_SDPA_SPLITS", 0) ? std::min<int64_t>(cdiv(N, 128), 1024)
                                                       : std::min<int64_t>(cdiv(N, 256), 32);
  if (S > cap) S = cap;
  if (S < 1) S = 1;
  const int64_t tps = cdiv(N, S);
  S = cdiv(N, tps);
  if (tps_out) *tps_out = tps;
  return (int)S;
}

// Workspace of a split decode: the per-(batch, KV head) counters of the
// in-kernel merge first (zero before the first call, left zero), then the
// partial maxima, sums and outputs.
size_t sdpa_workspace(int64_t B, int64_t Hq, int64_t N, int64_t D) {
  if (B <= 0 || Hq <= 0 || N <= 0 || D <= 0) return 0;
  const int S = sdpa_splits(B, N);
  if (S == 1) return 0;
  const size_t rows = (size_t)B * Hq * S;
  return kCounterBytes + round_up(rows * 4, 256) * 2 + round_up(rows * D * 4, 256);
}

template <int D, int GQA>
static void launch_decode_g(const SdpaArgs& a, int fmt, dim3 grid, hipStream_t st) {
  if (fmt == SPARKQ_KV_S8_F16SCALE)
    hipLaunchKernelGGL((sdpa_decode_kernel<D, GQA, 0>), grid, dim3(256), 0, st, a);
  else if (fmt == SPARKQ_KV_AFFINE_U8)
    hipLaunchKernelGGL((sdpa_decode_kernel<D, GQA, 1>), grid, dim3(256), 0, st, a);
  else if (fmt == SPARKQ_KV_AFFINE_U4)
    hipLaunchKernelGGL((sdpa_decode_kernel<D, GQA, 2>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((sdpa_decode_kernel<D, GQA, 3>), grid, dim3(256), 0, st, a);
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

template <int D, int NW>
static void launch_mfma_w(const SdpaArgs& a, int gqa, dim3 grid, hipStream_t st) {
  const dim3 block(64 * NW);
  switch (gqa) {
    case 1: hipLaunchKernelGGL((sdpa_mfma_kernel<D, 1, NW>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((sdpa_mfma_kernel<D, 2, NW>), grid, block, 0, st, a); break;
    case 4: hipLaunchKernelGGL((sdpa_mfma_kernel<D, 4, NW>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((sdpa_mfma_kernel<D, 8, NW>), grid, block, 0, st, a); break;
  }
}
template <int D>
static void launch_mfma_d(const SdpaArgs& a, int gqa, dim3 grid, hipStream_t st) {
  if constexpr (D <= 128) {
    // eight waves when the grid fills at most half the CUs (each wave then
    // has half the blocks): B=1 N=4096 (128 workgroups) 11.0 -> 10.2 us; at
    // one workgroup per CU (B=1 N=32768) no gain
    if (2 * (int64_t)grid.x * grid.y <= device_cus() && !env_int("SPARKQ_SDPA_NO_NW8", 0)) {
      launch_mfma_w<D, 8>(a, gqa, grid, st);
      return;
    }
  }
  launch_mfma_w<D, 4>(a, gqa, grid, st);
}

// the matrix-core decode over the affine caches (sdpa_affine.hip)
bool sdpa_affine_mfma_ok(const SdpaArgs& a, int64_t D, int fmt);
int sdpa_affine_mfma_occupancy(int64_t D, int G);
void launch_sdpa_affine_mfma(const SdpaArgs& a, int64_t D, int fmt, dim3 grid, hipStream_t st);

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
  const int gqa = (int)(Hq / Hkv);
  const bool mfma = fmt == SPARKQ_KV_S8_F16SCALE && (qdt == SPARKQ_BF16 || qdt == SPARKQ_F16) &&
                    !env_int("SPARKQ_SDPA_NO_MFMA", 0);
  const bool amfma = !env_int("SPARKQ_SDPA_NO_MFMA", 0) && sdpa_affine_mfma_ok(a, D, fmt);
  if (amfma && S > 1 && !env_int("SPARKQ_SDPA_SPLITS", 0)) {
    // a kernel built for one workgroup per CU takes no more splits than fill
    // the CUs once: a second round of workgroups costs more than the longer
    // splits (B=8 N=4096, u8 G32: 8 splits in two rounds vs 4 in one)
    const int64_t fit = device_cus() * (int64_t)sdpa_affine_mfma_occupancy(D, G) / (B * Hkv);
    if (fit < S) {
      int64_t s2 = std::max<int64_t>(fit, 1);
      tps = cdiv(N, s2);
      s2 = cdiv(N, tps);
      a.S = (int)s2;
      a.tps = (int)tps;
    }
  }
  const int S2 = a.S;
  if (S2 > 1) {
    const size_t rows = (size_t)B * Hq * S2;
    unsigned char* base = reinterpret_cast<unsigned char*>(ws);
    // the MFMA kernels merge the splits themselves when their LDS holds the
    // split weights and the counters cover every (batch, KV head)
    if ((mfma || amfma) && (int64_t)gqa * S2 <= 2048 && B * Hkv <= kMaxCounterTiles &&
        !env_int("SPARKQ_SDPA_MERGE_KERNEL", 0))
      a.counters = reinterpret_cast<unsigned*>(base);
    base += kCounterBytes;
    a.pm = reinterpret_cast<float*>(base);
    a.pz = reinterpret_cast<float*>(base + round_up(rows * 4, 256));
    a.pacc = reinterpret_cast<float*>(base + 2 * round_up(rows * 4, 256));
  }
  dim3 grid((unsigned)S2, (unsigned)(B * Hkv));
  if (amfma) {
    launch_sdpa_affine_mfma(a, D, fmt, grid, st);
  } else if (mfma) {
    if (D == 64)
      launch_mfma_d<64>(a, gqa, grid, st);
    else if (D == 128)
      launch_mfma_d<128>(a, gqa, grid, st);
    else
      launch_mfma_d<256>(a, gqa, grid, st);
  } else if (D == 64)
    launch_decode_d<64>(a, gqa, fmt, grid, st);
  else if (D == 128)
    launch_decode_d<128>(a, gqa, fmt, grid, st);
  else
    launch_decode_d<256>(a, gqa, fmt, grid, st);
  if (int rc = check_launch("sdpa_decode_kernel")) return rc;
  if (S2 > 1 && !a.counters) {
    hipLaunchKernelGGL(sdpa_merge_kernel, dim3((unsigned)(B * Hq)), dim3(256), 0, st, a.pm,
                       a.pz, a.pacc, out, odt, S2, (int)D);
    if (int rc = check_launch("sdpa_merge_kernel")) return rc;
  }
  return SPARKQ_OK;
}

template <int D>
static void launch_prefill_d(const SdpaArgs& a, int gqa, dim3 grid, hipStream_t st) {
  switch (gqa) {
    case 1: hipLaunchKernelGGL((sdpa_prefill_kernel<D, 1>), grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL((sdpa_prefill_kernel<D, 2>), grid, dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL((sdpa_prefill_kernel<D, 4>), grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((sdpa_prefill_kernel<D, 8>), grid, dim3(256), 0, st, a); break;
  }
}

int int8kv_sdpa_prefill(const void* q, const void* kc, const void* ks, const void* vc,
                        const void* vs, void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                        int64_t N, int64_t D, int causal, int qdt, int odt, float scale,
                        const int64_t* strides, hipStream_t st) {
  SdpaArgs a{};
  a.q = q;
  a.kc = reinterpret_cast<const uint8_t*>(kc);
  a.ks = ks;
  a.vc = reinterpret_cast<const uint8_t*>(vc);
  a.vs = vs;
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
  a.L = (int)L;
  a.causal = causal ? 1 : 0;
  a.q_dtype = qdt;
  a.out_dtype = odt;
  a.S = 1;
  a.tps = (int)N;
  a.scale_log2 = scale * 1.4426950408889634f;
  // the row tiles of one (sequence, KV head) on one XCD, sharing its L2 for
  // the K/V blocks every wave re-reads (B=1 causal, 32/8 heads, D=128: L=N=2048
  // 185 -> 246 TFLOP/s; L=512 N=4096 unchanged)
  a.xcd = !env_int("SPARKQ_PREFILL_NO_XCD", 0);
  const int gqa = (int)(Hq / Hkv);
  dim3 grid((unsigned)cdiv(L * gqa, 64), (unsigned)(B * Hkv));
  if (D == 64)
    launch_prefill_d<64>(a, gqa, grid, st);
  else if (D == 128)
    launch_prefill_d<128>(a, gqa, grid, st);
  else
    launch_prefill_d<256>(a, gqa, grid, st);
  return check_launch("sdpa_prefill_kernel");
}

template <int D, bool SPLIT>
static void launch_prefill_affine_s(const SdpaArgs& a, int qdt, dim3 grid, hipStream_t st) {
  if (qdt == SPARKQ_BF16)
    hipLaunchKernelGGL((sdpa_prefill_affine_kernel<D, BF16, SPLIT>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((sdpa_prefill_affine_kernel<D, F16, SPLIT>), grid, dim3(256), 0, st, a);
}
template <int D>
static void launch_prefill_affine_d(const SdpaArgs& a, int qdt, dim3 grid, hipStream_t st) {
  if (a.S > 1)
    launch_prefill_affine_s<D, true>(a, qdt, grid, st);
  else
    launch_prefill_affine_s<D, false>(a, qdt, grid, st);
}

// Launch plan of the affine prefill: causal row tiles are paired when the
// paired grid still has a workgroup for every CU (D <= 128); a grid short of
// one workgroup per CU splits each tile's blocks over S <= 8 workgroups,
// merged in the same launch through the workspace (tile counters, then the
// per-chunk maxima, sums and accumulators).
struct AffPrefillPlan {
  int pair, S;
  int64_t ntiles_all;
  size_t bytes;
};
static AffPrefillPlan plan_prefill_affine(int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                                          int64_t D, int causal) {
  AffPrefillPlan p{};
  const int64_t ntiles = cdiv(L * (Hq / Hkv), 128);
  p.ntiles_all = ntiles * B * Hkv;
  p.pair = D <= 128 && causal && ntiles >= 2 && cdiv(ntiles, 2) * B * Hkv >= 256 ? 1 : 0;
  p.S = 1;
  static const int64_t target = [] {
    const char* e = std::getenv("SPARKQ_PREFILL_SPLIT_TARGET");
    return e ? std::max(1, std::atoi(e)) : 256;
  }();
  if (!p.pair && p.ntiles_all < target && p.ntiles_all <= (int64_t)(kCounterBytes / 4))
    p.S = (int)std::min<int64_t>(8, cdiv(target, p.ntiles_all));
  p.bytes = p.S > 1 ? kCounterBytes + round_up((size_t)p.ntiles_all * p.S * 128 * 4, 256) * 2 +
                          (size_t)p.ntiles_all * p.S * 128 * D * 4
                    : 0;
  return p;
}

size_t int8kv_sdpa_prefill_affine_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                                            int64_t D, int causal) {
  return plan_prefill_affine(B, Hq, Hkv, L, D, causal).bytes;
}

int int8kv_sdpa_prefill_affine(const void* q, const void* kc, const void* ks, const void* kb,
                               const void* vc, const void* vs, const void* vb, void* out,
                               int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t N,
                               int64_t D, int G, int causal, int qdt, int odt, float scale,
                               const int64_t* strides, void* ws, size_t wsb, hipStream_t st) {
  const AffPrefillPlan plan = plan_prefill_affine(B, Hq, Hkv, L, D, causal);
  if (plan.S > 1 && (ws == nullptr || wsb < plan.bytes))
    return set_error(SPARKQ_ERR_WORKSPACE, "int8kv_sdpa_prefill_affine: workspace too small");
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
  a.L = (int)L;
  a.causal = causal ? 1 : 0;
  a.q_dtype = qdt;
  a.out_dtype = odt;
  a.S = plan.S;
  a.pair = plan.pair;
  a.tps = (int)N;
  a.scale_log2 = scale * 1.4426950408889634f;
  // XCD-grouped work order (L=512 N=4096: D=128 275 -> 286, D=256 332 -> 344
  // TFLOP/s; L=N=2048 unchanged)
  a.xcd = !env_int("SPARKQ_PREFILL_NO_XCD", 0);
  if (plan.S > 1) {
    unsigned char* base = reinterpret_cast<unsigned char*>(ws);
    const size_t rows = round_up((size_t)plan.ntiles_all * plan.S * 128 * 4, 256);
    a.counters = reinterpret_cast<unsigned*>(base);
    a.pm = reinterpret_cast<float*>(base + kCounterBytes);
    a.pz = reinterpret_cast<float*>(base + kCounterBytes + rows);
    a.pacc = reinterpret_cast<float*>(base + kCounterBytes + 2 * rows);
  }
  const int64_t ntiles = cdiv(L * (Hq / Hkv), 128);
  dim3 grid((unsigned)(plan.pair ? cdiv(ntiles, 2) : ntiles * plan.S), (unsigned)(B * Hkv));
  if (D == 64)
    launch_prefill_affine_d<64>(a, qdt, grid, st);
  else if (D == 128)
    launch_prefill_affine_d<128>(a, qdt, grid, st);
  else
    launch_prefill_affine_d<256>(a, qdt, grid, st);
  return check_launch("sdpa_prefill_affine_kernel");
}

template <typename T>
static void launch_append_u8(int D, const KvAppendArgs& a, dim3 grid, hipStream_t st) {
  if (D == 64)
    hipLaunchKernelGGL((kv_append_u8_wave_kernel<T, 1>), grid, dim3(256), 0, st, a);
  else if (D == 128)
    hipLaunchKernelGGL((kv_append_u8_wave_kernel<T, 2>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((kv_append_u8_wave_kernel<T, 4>), grid, dim3(256), 0, st, a);
}

int kv_append(const void* x, void* codes, void* scales, void* biases, int64_t B, int64_t H,
              int64_t L, int64_t D, int64_t offset, int G, int fmt, int xdt,
              const int64_t* strides, hipStream_t st) {
  KvAppendArgs a{};
  a.x = x;
  a.codes = codes;
  a.scales = scales;
  a.biases = biases;
  a.c_b = strides[0];
  a.c_h = strides[1];
  a.c_t = strides[2];
  a.s_b = strides[3];
  a.s_h = strides[4];
  a.s_t = strides[5];
  a.B = (int)B;
  a.H = (int)H;
  a.L = (int)L;
  a.D = (int)D;
  a.G = G;
  a.offset = (int)offset;
  a.x_dtype = xdt;
  a.bits = fmt == SPARKQ_KV_AFFINE_U4 ? 4 : fmt == SPARKQ_KV_AFFINE_U2 ? 2 : 8;
  const int64_t rows = B * H * L;
  if (fmt == SPARKQ_KV_S8_F16SCALE) {
    hipLaunchKernelGGL(kv_append_s8_kernel, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, st, a);
  } else if (a.bits == 8 && (D == 64 || D == 128 || D == 256) && G % (D / 64) == 0 &&
             G / (D / 64) <= 64 && !env_int("SPARKQ_KV_APPEND_THREAD", 0)) {
    const dim3 grid((unsigned)cdiv(rows, 4));
    if (xdt == SPARKQ_BF16)
      launch_append_u8<BF16>((int)D, a, grid, st);
    else
      launch_append_u8<F16>((int)D, a, grid, st);
  } else {
    const unsigned grid = (unsigned)cdiv(rows * (D / G), 256);
    if (xdt == SPARKQ_BF16)
      hipLaunchKernelGGL(kv_append_u8_kernel<BF16>, dim3(grid), dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL(kv_append_u8_kernel<F16>, dim3(grid), dim3(256), 0, st, a);
  }
  return check_launch("kv_append_kernel");
}

int kv_quantize_s8(const void* x, int8_t* codes, void* scales, int64_t R, int64_t D, int xdt,
                   hipStream_t st) {
  hipLaunchKernelGGL(kv_quantize_s8_kernel, dim3((unsigned)cdiv(R, 4)), dim3(256), 0, st, x,
                     codes, (uint16_t*)scales, R, D, xdt);
  return check_launch("kv_quantize_s8_kernel");
}

// ---------------------------------------------------------------------------
// Allocation-free decode: the workspace is a file-scope device array, one
// copy per GPU, held until the process ends. Its counters start at zero (the
// first use on a device clears them with a fill kernel) and every decode
// leaves them zero; the partials need no clearing. The host never passes
// the array's name to a kernel: it is a host-side stand-in, and the device
// address comes from hipGetSymbolAddress, resolved once per device.
// ---------------------------------------------------------------------------
constexpr size_t kDecodeScratchBytes = 8u << 20;
static __device__ __align__(256) unsigned char g_decode_scratch[kDecodeScratchBytes];

__global__ __launch_bounds__(256) void fill_zero_kernel(uint32_t* p, int64_t words) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < words; i += (int64_t)gridDim.x * 256)
    p[i] = 0u;
}

static void* g_decode_scratch_ptr[64];
static std::mutex g_decode_scratch_mu;

// Device address of this GPU's scratch array, resolved (and its counters
// cleared on stream st) on the first call per device; null on failure.
static void* decode_scratch(hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(g_decode_scratch_mu);
  if (g_decode_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_decode_scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error(SPARKQ_ERR_DEVICE, "hipGetSymbolAddress(decode scratch): %s", hipGetErrorString(e));
      return nullptr;
    }
    hipLaunchKernelGGL(fill_zero_kernel, dim3(16), dim3(256), 0, st, (uint32_t*)ptr,
                       (int64_t)(kCounterBytes / 4));
    if (hipGetLastError() != hipSuccess) {
      set_error(SPARKQ_ERR_DEVICE, "decode scratch: clearing the counters failed");
      return nullptr;
    }
    g_decode_scratch_ptr[dev] = ptr;
  }
  return g_decode_scratch_ptr[dev];
}

size_t decode_scratch_bytes() { return kDecodeScratchBytes; }

int int8kv_sdpa_decode_noalloc(const void* q, const void* kc, const void* ks, const void* kb,
                               const void* vc, const void* vs, const void* vb, void* out,
                               int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D, int G,
                               int fmt, int qdt, int odt, float scale, const int64_t* strides,
                               hipStream_t st) {
  const size_t need = sdpa_workspace(B, Hq, N, D);
  if (need > kDecodeScratchBytes)
    return set_error(SPARKQ_ERR_UNSUPPORTED,
                     "int8kv_sdpa_decode_noalloc: B=%lld Hq=%lld N=%lld D=%lld needs %zu bytes of "
                     "scratch, above the fixed %zu",
                     (long long)B, (long long)Hq, (long long)N, (long long)D, need,
                     kDecodeScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    ws = decode_scratch(st);
    if (ws == nullptr) return SPARKQ_ERR_DEVICE;
  }
  return int8kv_sdpa_decode(q, kc, ks, kb, vc, vs, vb, out, B, Hq, Hkv, N, D, G, fmt, qdt, odt,
                            scale, strides, ws, need > 0 ? kDecodeScratchBytes : 0, st);
}

}  // namespace sparkq
