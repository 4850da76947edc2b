// sdpa_affine.hip -- decode attention (one query token) on the matrix cores
// over the MLX affine KV caches: u8, u4 or u2 codes, code j of a uint32 word
// at bits * j, with one scale and one bias per group of G dims and token, in
// the query dtype (bf16 or fp16 queries).
//
// The numerics of spark_affine_u8_sdpa_decode
// (X/spark_mlx_ext/_int8_sdpa_sources.py:45-118): per group the score term
// is sk * sum(q * code) + bk * sum(q) in fp32, an online softmax in fp32,
// and the value term p * (code * sv + bv) accumulated in fp32. Here:
//  * QK on v_mfma_f32_16x16x32_f16, the GQA query heads as the (zero-padded)
//    16-row side. A k-chunk is one 32-dim window, so every chunk lies inside
//    one group (G >= 32); a lane supplies 8 dims of a window. The codes
//    become exact fp16 values 1024 + code with one byte permute under the
//    fp16 1024 pattern (4- and 2-bit codes after a mask and shift; the query
//    is permuted to the order the decode leaves them in); the query is
//    shifted per head by a power of two so that it is an exact fp16 operand.
//    The windows of a group accumulate together and the group's fp32 result
//    takes sk * acc + (bk - 1024 sk) * sum(q'), which is the reference's
//    factorization with the code offset folded into the bias term.
//  * PV on v_mfma_f32_16x16x32_bf16: A = p * sv (one value per head, token
//    and group) as the sum of three bf16 terms (24 significant bits and the
//    fp32 exponent range, so any bf16 or fp16 scale), transposed to
//    row-major through per-wave LDS strips; B = the codes themselves, exact
//    in bf16, read from a per-wave LDS copy of the block with
//    ds_read_b64_tr_b8 (the 8 bytes of a lane are one code byte of 8 tokens)
//    and converted with v_cvt_f32_ubyte. The bias term p * bv is an fp32 sum
//    per (head, group).
//  * Rows: when (heads per KV head) * (groups per row) <= 16 the 16 MFMA rows
//    are (head, group) pairs: the QK rows of one head repeat, each row's
//    strip weighs its own group's value scale, and one strip per block feeds
//    the PV product of every column; the epilogue keeps, for each column,
//    the rows of its group. Otherwise the rows are the heads and the PV
//    product runs once per group with that group's strip.
// Each workgroup (4 waves) owns one (sequence, KV head) and one context
// split; a wave walks 32-token blocks with the next blocks in flight. Waves
// combine through LDS; a split's partial is merged by the last workgroup of
// its (sequence, KV head) as in the s8 kernel.
#include <type_traits>

#include "sdpa_common.h"

namespace sparkq {

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t buf_load4(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ u32x2_t buf_load8(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}

// Dim (within the lane's 8 dims of a window) held by k-slot i after the K
// decode below: natural order for 8-bit codes; for 4-bit codes the even dims
// then the odd ones; for 2-bit codes the pairs (m, m + 4).
template <int BITS>
__host__ __device__ constexpr int aff_kslot_dim(int i) {
  return BITS == 8 ? i : (BITS == 4 ? (i < 4 ? 2 * i : 2 * (i - 4) + 1) : 4 * (i & 1) + (i >> 1));
}

// The lane's 8 codes of a window (u8: two words; u4: one word; u2: the low
// 16 bits of w0) -> 8 exact fp16 values 1024 + code in k-slot order.
template <int BITS>
__device__ __forceinline__ u32x4_t aff_kdecode(uint32_t w0, uint32_t w1) {
  constexpr uint32_t M = 0x64646464u;  // fp16 exponent byte of 1024
  constexpr uint32_t LO = 0x04010400u, HI = 0x04030402u;
  if constexpr (BITS == 8) {
    return u32x4_t{__builtin_amdgcn_perm(M, w0, LO), __builtin_amdgcn_perm(M, w0, HI),
                   __builtin_amdgcn_perm(M, w1, LO), __builtin_amdgcn_perm(M, w1, HI)};
  } else if constexpr (BITS == 4) {
    const uint32_t ev = w0 & 0x0F0F0F0Fu, od = (w0 >> 4) & 0x0F0F0F0Fu;
    return u32x4_t{__builtin_amdgcn_perm(M, ev, LO), __builtin_amdgcn_perm(M, ev, HI),
                   __builtin_amdgcn_perm(M, od, LO), __builtin_amdgcn_perm(M, od, HI)};
  } else {
    return u32x4_t{__builtin_amdgcn_perm(M, w0 & 0x0303u, LO),
                   __builtin_amdgcn_perm(M, (w0 >> 2) & 0x0303u, LO),
                   __builtin_amdgcn_perm(M, (w0 >> 4) & 0x0303u, LO),
                   __builtin_amdgcn_perm(M, (w0 >> 6) & 0x0303u, LO)};
  }
}

// Four code bytes -> two packed bf16 pairs (bytes 0,1 and 2,3): each byte
// converted exactly to fp32, the pair's high halves taken.
__device__ __forceinline__ void aff_bytes_bf16(uint32_t x, uint32_t& p01, uint32_t& p23) {
  const float f0 = (float)(x & 255u), f1 = (float)((x >> 8) & 255u);
  const float f2 = (float)((x >> 16) & 255u), f3 = (float)(x >> 24);
  p01 = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
  p23 = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
}

// The tr8 read of a lane (lo: code bytes of k-slots 0..3, hi: 4..7) ->
// the B operand of sub-dim m (the m-th code of each byte) as bf16 codes.
template <int BITS>
__device__ __forceinline__ u32x4_t aff_vdecode(uint32_t lo, uint32_t hi, int m) {
  constexpr uint32_t MASK = BITS == 8 ? 0xFFFFFFFFu : (BITS == 4 ? 0x0F0F0F0Fu : 0x03030303u);
  const uint32_t l = BITS == 8 ? lo : (lo >> (BITS * m)) & MASK;
  const uint32_t h = BITS == 8 ? hi : (hi >> (BITS * m)) & MASK;
  uint32_t r0, r1, r2, r3;
  aff_bytes_bf16(l, r0, r1);
  aff_bytes_bf16(h, r2, r3);
  return u32x4_t{r0, r1, r2, r3};
}

__device__ __forceinline__ f32x4_t mfma16x16x32_bf16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// 16-bit value i of a packed scale vector as fp32
template <typename T>
__device__ __forceinline__ float aff_elem(const uint32_t* v, int i) {
  return (i & 1) ? hi16<T>(v[i >> 1]) : lo16<T>(v[i >> 1]);
}

template <int D, int BITS>
struct AffDecodeLds {
  static constexpr int NW = 4;
  static constexpr int RB = D * BITS / 8;             // code bytes of a token row
  static constexpr int VROW = RB + 16;                // padded row of the V copy
  static constexpr int VT = 32 * VROW;                // one wave's V block
  static constexpr int PT = 3 * 16 * 32 * 2;          // one wave's P strips (3 terms) [16 heads][32] bf16
  static constexpr int LOOP = NW * (VT + PT);
  static constexpr int MERGE = NW * 8 * 4 * 2 + NW * 8 * D * 4;
  static constexpr int BYTES = LOOP > MERGE ? LOOP : MERGE;
};

// Blocks in flight beyond the one computed (register sets) and workgroups
// per CU the registers are sized for.
template <int D, int FMT, int G>
__host__ __device__ constexpr int aff_pipe() { return D == 256 ? 1 : 2; }
template <int D, int FMT, int G>
__host__ __device__ constexpr int aff_occ() { return D == 256 || G == 32 ? 1 : 2; }

// T: the query (and scale) dtype tag; FMT 1/2/3: u8/u4/u2 codes. PACK: the
// 16 MFMA rows are (query head, group of dims) pairs, head-major, which
// needs (heads per KV head) * D/G <= 16; otherwise the rows are the query
// heads and the PV product runs once per group (see below).
template <int D, int FMT, int G, typename T, bool PACK>
__global__ __launch_bounds__(256, (aff_occ<D, FMT, G>())) void sdpa_affine_mfma_kernel(SdpaArgs a) {
  constexpr int BITS = FMT == 1 ? 8 : (FMT == 2 ? 4 : 2);
  constexpr int NW = 4;
  using L = AffDecodeLds<D, BITS>;
  constexpr int RB = L::RB;
  constexpr int NWIN = D / 32;                  // QK windows (k chunks)
  constexpr int NGR = D / G;                    // groups of a row
  constexpr int WPG = G / 32;                   // windows per group
  constexpr int KD = BITS == 8 ? 2 : 1;         // code words of a lane's window
  constexpr int VW = RB / 2 < 16 ? RB / 2 : 16; // bytes of one V piece
  constexpr int PPR = RB / VW;                  // V pieces per token row
  constexpr int VL = 32 * PPR / 64;             // V pieces per lane and block
  constexpr int DPB = 8 / BITS;                 // dims per code byte
  constexpr int CSPAN = 16 * DPB;               // dims of a 16-byte PV column block
  constexpr int NJ = D / 16;                    // PV accumulators
  constexpr int SWD = NGR >= 2 ? NGR / 2 : 1;   // words of one packed scale vector
  constexpr int SB = 2 * NGR;                   // bytes of one scale vector
  constexpr int PIPE = aff_pipe<D, FMT, G>();
  constexpr int NPE = PACK ? 1 : NGR;           // bias sums per row
  static_assert(VL >= 1 && 64 * VL == 32 * PPR, "V pieces");
  __shared__ __attribute__((aligned(16))) unsigned char smem[L::BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15, grp = lane >> 4;
  const int gqa = a.Hq / a.Hkv;
  const int split = blockIdx.x;
  const int b = blockIdx.y / a.Hkv, kh = blockIdx.y - b * a.Hkv;
  const int t_begin = split * a.tps;
  const int t_end = min(a.N, t_begin + a.tps);
  unsigned char* vtile = smem + wave * L::VT;
  uint32_t* pstrip = reinterpret_cast<uint32_t*>(smem + NW * L::VT + wave * L::PT);

  const rsrc_t rk = make_rsrc(a.kc + b * a.kc_b + kh * a.kc_h, (uint32_t)(t_end * a.kc_t));
  const rsrc_t rv = make_rsrc(a.vc + b * a.vc_b + kh * a.vc_h, (uint32_t)(t_end * a.vc_t));
  const uint16_t* ksb = reinterpret_cast<const uint16_t*>(a.ks) + b * a.ks_b + kh * a.ks_h;
  const uint16_t* kbb = reinterpret_cast<const uint16_t*>(a.kb) + b * a.ks_b + kh * a.ks_h;
  const uint16_t* vsb = reinterpret_cast<const uint16_t*>(a.vs) + b * a.vs_b + kh * a.vs_h;
  const uint16_t* vbb = reinterpret_cast<const uint16_t*>(a.vb) + b * a.vs_b + kh * a.vs_h;
  const rsrc_t rks = make_rsrc(ksb, (uint32_t)(t_end * a.ks_t * 2));
  const rsrc_t rkb = make_rsrc(kbb, (uint32_t)(t_end * a.ks_t * 2));
  const rsrc_t rvs = make_rsrc(vsb, (uint32_t)(t_end * a.vs_t * 2));
  const rsrc_t rvb = make_rsrc(vbb, (uint32_t)(t_end * a.vs_t * 2));

  // block registers, two sets: K codes [token group][window][word], V
  // pieces, and the four packed scale vectors of the lane's two tokens. Every
  // load is issued unconditionally (past t_end the bounded descriptors return
  // zeros) so that the loop's wait counts stay exact.
  uint32_t kr[PIPE][2][NWIN][KD];
  typedef std::conditional_t<VW == 16, u32x4_t, u32x2_t> vpiece_t;
  vpiece_t vr[PIPE][VL];
  uint32_t skr[PIPE][2][SWD], bkr[PIPE][2][SWD], svr[PIPE][2][SWD], bvr[PIPE][2][SWD];
  auto load_vec = [&](rsrc_t r, uint32_t off, uint32_t* dst) {
    if constexpr (SB == 2) {
      dst[0] = buf_load2(r, off);
    } else if constexpr (SB == 4) {
      dst[0] = buf_load4(r, off);
    } else if constexpr (SB == 8) {
      const u32x2_t v = buf_load8(r, off);
      dst[0] = v[0];
      dst[1] = v[1];
    } else {
      const u32x4_t v = buf_load16(r, off);
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i] = v[i];
    }
  };
  auto load = [&](int set, int t0) {
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2) {
      const uint32_t tok = (uint32_t)(t0 + 16 * g2 + n16);
#pragma unroll
      for (int w = 0; w < NWIN; ++w) {
        const uint32_t off = tok * (uint32_t)a.kc_t + (uint32_t)((32 * w + 8 * grp) * BITS / 8);
        if constexpr (BITS == 8) {
          const u32x2_t v = buf_load8(rk, off);
          kr[set][g2][w][0] = v[0];
          kr[set][g2][w][KD - 1] = v[1];
        } else if constexpr (BITS == 4) {
          kr[set][g2][w][0] = buf_load4(rk, off);
        } else {
          kr[set][g2][w][0] = buf_load2(rk, off);
        }
      }
    }
#pragma unroll
    for (int v = 0; v < VL; ++v) {
      const int f = lane + 64 * v, tok = f / PPR, pc = f % PPR;
      const uint32_t off = (uint32_t)((t0 + tok) * a.vc_t + VW * pc);
      if constexpr (VW == 16)
        vr[set][v] = buf_load16(rv, off);
      else
        vr[set][v] = buf_load8(rv, off);
    }
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2) {
      const uint32_t tok = (uint32_t)(t0 + 16 * g2 + n16);
      load_vec(rks, tok * (uint32_t)a.ks_t * 2u, skr[set][g2]);
      load_vec(rkb, tok * (uint32_t)a.ks_t * 2u, bkr[set][g2]);
      load_vec(rvs, tok * (uint32_t)a.vs_t * 2u, svr[set][g2]);
      load_vec(rvb, tok * (uint32_t)a.vs_t * 2u, bvr[set][g2]);
    }
  };
  // the first blocks are in flight while the query operand is built (their
  // loads do not depend on it)
  const int stride = NW * 32;
  int t0 = t_begin + 32 * wave;
  load(0, t0);
  if constexpr (PIPE == 2) load(1, t0 + stride);

  // query operand: lane (row n16, k quarter grp) holds dims 32 w + 8 grp ..
  // +8 of window w of the row's head in k-slot order; per window the sum of
  // the fp16 values
  u32x4_t qa[NWIN];
  float qsw[NWIN];
  float qmul_h;
  {
    const int h = PACK ? n16 / NGR : n16;
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) +
                           ((int64_t)b * a.Hq + kh * gqa + min(h, gqa - 1)) * D;
    float qv[NWIN][8];
    float qmax = 0.0f;
#pragma unroll
    for (int w = 0; w < NWIN; ++w) {
      const u32x4_t x = *reinterpret_cast<const u32x4_t*>(qrow + 32 * w + 8 * grp);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = (i & 1) ? hi16<T>(x[i >> 1]) : lo16<T>(x[i >> 1]);
        qv[w][i] = h < gqa ? v : 0.0f;
        qmax = fmaxf(qmax, fabsf(qv[w][i]));
      }
    }
    qmax = fmaxf(qmax, __shfl_xor(qmax, 16));
    qmax = fmaxf(qmax, __shfl_xor(qmax, 32));
    const int e = (qmax > 0.0f && qmax <= 3.4028235e38f) ? ilogbf(qmax) - 14 : 0;
#pragma unroll
    for (int w = 0; w < NWIN; ++w) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const _Float16 lo = (_Float16)ldexpf(qv[w][aff_kslot_dim<BITS>(2 * i)], -e);
        const _Float16 hi = (_Float16)ldexpf(qv[w][aff_kslot_dim<BITS>(2 * i + 1)], -e);
        s += (float)lo + (float)hi;
        qa[w][i] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
      }
      s += __shfl_xor(s, 16);
      s += __shfl_xor(s, 32);
      qsw[w] = s;
    }
    qmul_h = ldexpf(a.scale_log2, e);
  }
  // score lanes: row 4 grp + r, token n16 (+16 for the second token group);
  // per row and group of dims the sum of the row's query
  float qg[4][NGR], qmul[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int src = (4 * grp + r) & 15;
    qmul[r] = __shfl(qmul_h, src);
#pragma unroll
    for (int g = 0; g < NGR; ++g) {
      float s = 0.0f;
#pragma unroll
      for (int w = 0; w < WPG; ++w) s += qsw[g * WPG + w];
      qg[r][g] = __shfl(s, src);
    }
  }


  float mrun[4], zl[4], pe[4][NPE];
  f32x4_t acc[NJ];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    mrun[r] = kNegInf;
    zl[r] = 0.0f;
#pragma unroll
    for (int g = 0; g < NPE; ++g) pe[r][g] = 0.0f;
  }
  // PACK: the group of dims of score row 4 grp + r, and that group's element
  // of a packed scale vector
  auto row_group = [&](int r) -> int { return NGR <= 4 ? r % NGR : (4 * grp + r) % NGR; };
  auto row_elem = [&](const uint32_t* v, int r) -> float {
    if constexpr (NGR <= 4) {
      return aff_elem<T>(v, r % NGR);
    } else {
      const uint32_t w = (grp & 1) ? v[2 + (r >> 1)] : v[r >> 1];
      return (r & 1) ? hi16<T>(w) : lo16<T>(w);
    }
  };
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  auto block = [&](int t0, auto setc) {
    constexpr int set = decltype(setc)::value;
    __builtin_amdgcn_sched_barrier(0);
    // V block to this wave's LDS copy: token t at row 2 (t % 16) + t / 16,
    // the k-slot order of the P strips
#pragma unroll
    for (int v = 0; v < VL; ++v) {
      const int f = lane + 64 * v, tok = f / PPR, pc = f % PPR;
      const int row = 2 * (tok & 15) + (tok >> 4);
      *reinterpret_cast<vpiece_t*>(vtile + row * L::VROW + VW * pc) = vr[set][v];
    }
    // QK per token group and group of dims, each group's product scaled
    // into the token's score as soon as it is done
    float sc[2][4];
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[g2][r] = 0.0f;
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
      for (int g = 0; g < NGR; ++g) {
        f32x4_t sa = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = g * WPG; w < (g + 1) * WPG; ++w)
          sa = mfma16x16x32_f16(qa[w], aff_kdecode<BITS>(kr[set][g2][w][0], kr[set][g2][w][KD - 1]), sa);
        const float ks = aff_elem<T>(skr[set][g2], g);
        const float ke = fmaf(-1024.0f, ks, aff_elem<T>(bkr[set][g2], g));
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[g2][r] = fmaf(ks, sa[r], fmaf(ke, qg[r][g], sc[g2][r]));
      }
    // the value scales and biases stay packed until used
    uint32_t svl[2][SWD], bvl[2][SWD];
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
      for (int i = 0; i < SWD; ++i) {
        svl[g2][i] = svr[set][g2][i];
        bvl[g2][i] = bvr[set][g2][i];
      }
    // the refill stays in issue order here (the next blocks' wait counts
    // rely on it)
    __builtin_amdgcn_sched_barrier(0);
    load(set, t0 + PIPE * stride);
    __builtin_amdgcn_sched_barrier(0);
    const bool ok0 = t0 + n16 < t_end, ok1 = t0 + 16 + n16 < t_end;

    float alpha[4], p0[4], p1[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float s0 = ok0 ? sc[0][r] * qmul[r] : kNegInf;
      const float s1 = ok1 ? sc[1][r] * qmul[r] : kNegInf;
      float mb = max_row16(fmaxf(s0, s1));
      mb = fmaxf(mb, mrun[r]);
      alpha[r] = exp2_guarded(mrun[r] - mb, mrun[r] != kNegInf);
      mrun[r] = mb;
      // rows past the heads (padding) get zero weights, so their strip rows
      // are zero
      const bool live = (PACK ? (4 * grp + r) / NGR : 4 * grp + r) < gqa;
      p0[r] = exp2_guarded(s0 - mb, ok0 && live);
      p1[r] = exp2_guarded(s1 - mb, ok1 && live);
      zl[r] = fmaf(zl[r], alpha[r], p0[r] + p1[r]);
      if constexpr (PACK) {
        pe[r][0] = fmaf(pe[r][0], alpha[r], fmaf(p0[r], row_elem(bvl[0], r), p1[r] * row_elem(bvl[1], r)));
      } else {
#pragma unroll
        for (int g = 0; g < NGR; ++g)
          pe[r][g] = fmaf(pe[r][g], alpha[r],
                          fmaf(p0[r], aff_elem<T>(bvl[0], g), p1[r] * aff_elem<T>(bvl[1], g)));
      }
    }
    // rescaled every block: a wave-uniform branch that skipped this when no
    // row maximum moved measured slower (it splits the block's wait counts)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      acc[j][0] *= alpha[0];
      acc[j][1] *= alpha[1];
      acc[j][2] *= alpha[2];
      acc[j][3] *= alpha[3];
    }
    // PV through the wave's strips (three bf16 terms of the weights, rows as
    // above): position 2 n16 + g2 holds token 16 g2 + n16 (one 32-bit write
    // per lane, row and term)
    const unsigned char* vaddr = vtile + (8 * grp + (n16 >> 1)) * L::VROW + 8 * (n16 & 1);
    auto strip_row = [&](int r, float sv0, float sv1) {
      const int row = 4 * grp + r;
      const float f0 = p0[r] * sv0, f1 = p1[r] * sv1;
      const uint32_t hi = pack_round<BF16>(f0, f1);
      const float r0 = f0 - lo16<BF16>(hi), r1 = f1 - hi16<BF16>(hi);
      const uint32_t mid = pack_round<BF16>(r0, r1);
      const uint32_t lo = pack_round<BF16>(r0 - lo16<BF16>(mid), r1 - hi16<BF16>(mid));
      pstrip[row * 16 + n16] = hi;
      pstrip[256 + row * 16 + n16] = mid;
      pstrip[512 + row * 16 + n16] = lo;
    };
    // the B operands of column block cb (its DPB sub-dims) into the
    // accumulators, with the columns outside group g zeroed when a block
    // spans two groups (g < 0: all columns)
    auto pv_block = [&](int cb, int g, const u32x4_t& pa, const u32x4_t& pm, const u32x4_t& pl) {
      typedef int v2i_t __attribute__((ext_vector_type(2)));
      const v2i_t t8 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          (__attribute__((address_space(3))) v2i_t*)(vaddr + 16 * cb));
      const bool mine = g < 0 || CSPAN <= G || ((CSPAN * cb + DPB * n16) / G == g);
#pragma unroll
      for (int m = 0; m < DPB; ++m) {
        u32x4_t vb = aff_vdecode<BITS>((uint32_t)t8.x, (uint32_t)t8.y, m);
        if (!mine) vb = u32x4_t{0u, 0u, 0u, 0u};
        acc[cb * DPB + m] = mfma16x16x32_bf16(pa, vb, acc[cb * DPB + m]);
        acc[cb * DPB + m] = mfma16x16x32_bf16(pm, vb, acc[cb * DPB + m]);
        acc[cb * DPB + m] = mfma16x16x32_bf16(pl, vb, acc[cb * DPB + m]);
      }
    };
    if constexpr (PACK) {
      // one strip: row (head, group) weighs its group's value scale; every
      // output row is computed for every column, the epilogue keeps the
      // rows of each column's group
#pragma unroll
      for (int r = 0; r < 4; ++r) strip_row(r, row_elem(svl[0], r), row_elem(svl[1], r));
      const u32x4_t pa = *reinterpret_cast<const u32x4_t*>(pstrip + n16 * 16 + 4 * grp);
      const u32x4_t pm = *reinterpret_cast<const u32x4_t*>(pstrip + 256 + n16 * 16 + 4 * grp);
      const u32x4_t pl = *reinterpret_cast<const u32x4_t*>(pstrip + 512 + n16 * 16 + 4 * grp);
#pragma unroll
      for (int cb = 0; cb < NJ / DPB; ++cb) pv_block(cb, -1, pa, pm, pl);
    } else {
      // rows are heads: one strip per group, each through the column blocks
      // holding the group's dims
#pragma unroll
      for (int g = 0; g < NGR; ++g) {
#pragma unroll
        for (int r = 0; r < 4; ++r) strip_row(r, aff_elem<T>(svl[0], g), aff_elem<T>(svl[1], g));
        const u32x4_t pa = *reinterpret_cast<const u32x4_t*>(pstrip + n16 * 16 + 4 * grp);
        const u32x4_t pm = *reinterpret_cast<const u32x4_t*>(pstrip + 256 + n16 * 16 + 4 * grp);
        const u32x4_t pl = *reinterpret_cast<const u32x4_t*>(pstrip + 512 + n16 * 16 + 4 * grp);
        constexpr int NCB = CSPAN <= G ? G / CSPAN : 1;
#pragma unroll
        for (int cb = g * G / CSPAN; cb < g * G / CSPAN + NCB; ++cb) pv_block(cb, g, pa, pm, pl);
      }
    }
  };
  const int nb = t0 < t_end ? (t_end - t0 + stride - 1) / stride : 0;
  if constexpr (PIPE == 2) {
    // blocks in pairs with no branch in the loop body (so the wait counts
    // carried around it stay exact), then an odd last block
    int ib = 0;
    for (; ib + 2 <= nb; ib += 2, t0 += 2 * stride) {
      block(t0, std::integral_constant<int, 0>{});
      block(t0 + stride, std::integral_constant<int, 1>{});
    }
    if (ib < nb) block(t0, std::integral_constant<int, 0>{});
  } else {
    for (int ib = 0; ib < nb; ++ib, t0 += stride) block(t0, std::integral_constant<int, 0>{});
  }

  // per-lane partial sums -> the 16 token lanes of each head group
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    zl[r] = sum_row16(zl[r]);
#pragma unroll
    for (int g = 0; g < NPE; ++g) pe[r][g] = sum_row16(pe[r][g]);
  }

  // combine the waves through LDS (the loop's LDS is free after the barrier)
  __syncthreads();
  float* wm = reinterpret_cast<float*>(smem);            // [NW][8]
  float* wz = wm + NW * 8;                               // [NW][8]
  float* wacc = wz + NW * 8;                             // [NW][8][D]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = 4 * grp + r;
    const int h = PACK ? row / NGR : row;
    const int rg = PACK ? row_group(r) : 0;  // the row's group (PACK)
    if (h < gqa) {
      if (n16 == 0 && rg == 0) {
        wm[wave * 8 + h] = mrun[r];
        wz[wave * 8 + h] = zl[r];
      }
#pragma unroll
      for (int cb = 0; cb < NJ / DPB; ++cb)
#pragma unroll
        for (int m = 0; m < DPB; ++m) {
          const int d = CSPAN * cb + DPB * n16 + m;
          if constexpr (PACK) {
            // the column's group: fixed per block unless a block spans two
            const int gd = CSPAN <= G ? CSPAN * cb / G : (CSPAN * cb + DPB * n16) / G;
            if (gd == rg) wacc[(wave * 8 + h) * D + d] = acc[cb * DPB + m][r] + pe[r][0];
          } else {
            float bias;
            if constexpr (CSPAN <= G) {
              bias = pe[r][CSPAN * cb / G];
            } else {
              bias = n16 >= 8 ? pe[r][(CSPAN * cb + CSPAN / 2) / G] : pe[r][CSPAN * cb / G];
            }
            wacc[(wave * 8 + h) * D + d] = acc[cb * DPB + m][r] + bias;
          }
        }
    }
  }
  __syncthreads();
  for (int e = tid; e < gqa * D; e += 64 * NW) {
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
    const int64_t bh = (int64_t)b * a.Hq + kh * gqa + h;
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
      // register arrays sized for the actual head count (more splits in
      // flight per output with fewer heads)
      float* sm = reinterpret_cast<float*>(smem);
      if (gqa <= 2)
        sdpa_fold_merge<D, 2, 64 * NW>(a, b, kh, sm, gqa);
      else if (gqa <= 4)
        sdpa_fold_merge<D, 4, 64 * NW>(a, b, kh, sm, gqa);
      else
        sdpa_fold_merge<D, 8, 64 * NW>(a, b, kh, sm, gqa);
      splitk_reset(a.counters + blockIdx.y);
    }
  }
}

// rows as (head, group) pairs when they fit in 16; the per-group passes
// otherwise (instantiated only where some head count needs them)
template <int D, int FMT, int G, typename T>
static void launch_affine_p(const SdpaArgs& a, dim3 grid, hipStream_t st) {
  constexpr bool NEED_HEADS = 8 * (D / G) > 16;
  if (NEED_HEADS && (a.Hq / a.Hkv) * (D / G) > 16)
    hipLaunchKernelGGL((sdpa_affine_mfma_kernel<D, FMT, G, T, !NEED_HEADS>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((sdpa_affine_mfma_kernel<D, FMT, G, T, true>), grid, dim3(256), 0, st, a);
}

template <int D, int FMT, typename T>
static void launch_affine_g(const SdpaArgs& a, dim3 grid, hipStream_t st) {
  if (a.G == 32) {
    launch_affine_p<D, FMT, 32, T>(a, grid, st);
  } else if (a.G == 64) {
    launch_affine_p<D, FMT, 64, T>(a, grid, st);
  } else if constexpr (D >= 128) {
    launch_affine_p<D, FMT, 128, T>(a, grid, st);
  }
}

template <int D, typename T>
static void launch_affine_f(const SdpaArgs& a, int fmt, dim3 grid, hipStream_t st) {
  if (fmt == SPARKQ_KV_AFFINE_U8)
    launch_affine_g<D, 1, T>(a, grid, st);
  else if (fmt == SPARKQ_KV_AFFINE_U4)
    launch_affine_g<D, 2, T>(a, grid, st);
  else
    launch_affine_g<D, 3, T>(a, grid, st);
}

// The matrix-core decode takes the affine formats for 16-bit queries when
// every scale and bias vector of a token is aligned to its byte width (the
// contiguous [.., N, D/G] layout is) and the code rows are 16-byte aligned.
bool sdpa_affine_mfma_ok(const SdpaArgs& a, int64_t D, int fmt) {
  if (fmt != SPARKQ_KV_AFFINE_U8 && fmt != SPARKQ_KV_AFFINE_U4 && fmt != SPARKQ_KV_AFFINE_U2) return false;
  if (a.q_dtype != SPARKQ_BF16 && a.q_dtype != SPARKQ_F16) return false;
  if (D != 64 && D != 128 && D != 256) return false;
  if (a.G != 32 && a.G != 64 && a.G != 128) return false;
  if (D % a.G != 0) return false;
  const int64_t ngr = D / a.G;  // elements of one scale vector
  for (int64_t s : {a.ks_b, a.ks_h, a.ks_t, a.vs_b, a.vs_h, a.vs_t})
    if (s % ngr != 0) return false;
  for (const void* p : {a.ks, a.kb, a.vs, a.vb})
    if (reinterpret_cast<uintptr_t>(p) % (2 * ngr) != 0) return false;
  for (int64_t s : {a.kc_b, a.kc_h, a.kc_t, a.vc_b, a.vc_h, a.vc_t})
    if (s % 16 != 0) return false;
  for (const void* p : {(const void*)a.kc, (const void*)a.vc, a.q})
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
  return true;
}

// workgroups per CU the kernel for (D, G) is built for
int sdpa_affine_mfma_occupancy(int64_t D, int G) {
  if (D == 256) return aff_occ<256, 1, 32>();
  return G == 32 ? aff_occ<128, 1, 32>() : aff_occ<128, 1, 64>();
}

void launch_sdpa_affine_mfma(const SdpaArgs& a, int64_t D, int fmt, dim3 grid, hipStream_t st) {
  const bool bf = a.q_dtype == SPARKQ_BF16;
  if (D == 64)
    bf ? launch_affine_f<64, BF16>(a, fmt, grid, st) : launch_affine_f<64, F16>(a, fmt, grid, st);
  else if (D == 128)
    bf ? launch_affine_f<128, BF16>(a, fmt, grid, st) : launch_affine_f<128, F16>(a, fmt, grid, st);
  else
    bf ? launch_affine_f<256, BF16>(a, fmt, grid, st) : launch_affine_f<256, F16>(a, fmt, grid, st);
}

}  // namespace sparkq
