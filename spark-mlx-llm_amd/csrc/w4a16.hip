// w4a16.hip -- MLX-affine W4A16 quantized linear on gfx950.
//
// y[m,n] = sum_g s[n,g] * (sum_{k in g} x[m,k] * q[n,k]) + b[n,g] * X_g[m]
// with X_g[m] = sum_{k in g} x[m,k]. The MFMA consumes the 4-bit codes as the
// exact 16-bit values OFFSET+q (one byte-permute and one and-or per pair), so
// the per-group epilogue uses b' = b - OFFSET*s in place of b. Products of
// codes and activations are exact; accumulation and the epilogue are fp32.
//
// Kernels
//   w4_dequant_kernel   fp32 fmaf(q, s, b) (debug / bit-exact check entry)
//   w4_quantize_kernel  affine 4-bit quantizer (format producer)
//   w4_gemv_kernel      M <= 4 decode: 4 rows x 256 contiguous bytes per load
//                       instruction, v_mfma_f32_4x4x4_16b blocks, activations
//                       and (scale, bias) staged once per workgroup in LDS,
//                       whole rows per workgroup (no split-K)
//   w4_gemv_stream_kernel  M = 1, rows over 2560 k: one 16-wave workgroup per
//                       CU over a contiguous range of row quads, (row quad,
//                       span) items dealt evenly, every load issued at the
//                       start, per-item lane sums through LDS
//   w4_decode_stream_kernel  2 <= M <= 16: the same layout with each decoded
//                       piece feeding eight MFMAs per row quartet and lane
//                       sums kept in registers over a run of spans
//   w4_decode_phased_kernel  5 <= M <= 8 with rows whose activations exceed
//                       the staging registers or LDS: the same, activations
//                       staged a K phase at a time (opt-in)
//   w4_skinny_kernel    M <= 32: weight streaming, 32 rows x 64 k per wave
//                       step, MFMA 32x32x16, in-workgroup split-K over waves,
//                       cross-workgroup split-K combined in the same launch by
//                       the last workgroup of each tile
//   gemm_prep_kernel    bf16 GEMM prologue: fp16 activations and scales
//                       under per-row power-of-two shifts, bias slots
//   w4_gemm_x16w_kernel bf16, M > 32: 128x256 tiles of exact fp16 operands
//                       (weights decoded to s'*(q-8) in registers, activations
//                       through LDS), fp16 MFMA 32x32x16 with no per-group
//                       epilogue, the bias slots on the bf16 MFMA, split-K
//                       combined in the same launch when tiles are few
//   xsum_kernel         group sums X_g[m] for the fp16 GEMM, layout [K/G][M]
//   w4_gemm_kernel      fp16, M > 32: 128x128x64 LDS tiles (B decoded to the
//                       exact q), per-group fp32 scale and bias epilogue
#include <algorithm>
#include <type_traits>
#include <cmath>
#include <cstdlib>

#include "common.h"

namespace sparkq {

// ---------------------------------------------------------------------------
// exact dequantization
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void w4_dequant_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
    const uint16_t* __restrict__ b, float* __restrict__ out, int64_t N,
    int64_t K, int G) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t kw = K / 8;
  if (idx >= N * kw) return;
  const int64_t n = idx / kw;
  const int64_t k0 = (idx - n * kw) * 8;
  const int64_t gi = n * (K / G) + k0 / G;
  const float sv = T::to_f32(s[gi]);
  const float bv = T::to_f32(b[gi]);
  const uint32_t v = w[idx];
  float o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = fmaf((float)((v >> (4 * j)) & 15u), sv, bv);
  f32x4_t* dst = reinterpret_cast<f32x4_t*>(out + n * K + k0);
  dst[0] = f32x4_t{o[0], o[1], o[2], o[3]};
  dst[1] = f32x4_t{o[4], o[5], o[6], o[7]};
}

// ---------------------------------------------------------------------------
// affine 4-bit quantizer: one thread per group, the benchmark's min/max
// formula (scale (max-min)/15, bias min); mx.quantize's rule, which makes the
// larger-magnitude edge exact, gives different tuples in the same layout
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void w4_quantize_kernel(
    const uint16_t* __restrict__ w, uint32_t* __restrict__ wq,
    uint16_t* __restrict__ s, uint16_t* __restrict__ b, int64_t N, int64_t K,
    int G) {
  const int64_t ng = K / G;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= N * ng) return;
  const int64_t n = gid / ng, g = gid - n * ng;
  const uint16_t* v = w + n * K + g * G;
  float mn = T::to_f32(v[0]), mx = mn;
  for (int i = 1; i < G; ++i) {
    const float f = T::to_f32(v[i]);
    mn = f < mn ? f : mn;
    mx = f > mx ? f : mx;
  }
  const uint16_t s16 = T::from_f32((mx - mn) / 15.0f);
  const uint16_t b16 = T::from_f32(mn);
  s[gid] = s16;
  b[gid] = b16;
  const float sf = T::to_f32(s16), bf = T::to_f32(b16);
  uint32_t* dst = wq + n * (K / 8) + g * (G / 8);
  for (int i = 0; i < G / 8; ++i) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float q = 0.0f;
      if (sf != 0.0f) {
        q = __builtin_rintf((T::to_f32(v[8 * i + j]) - bf) / sf);
        q = q < 0.0f ? 0.0f : (q > 15.0f ? 15.0f : q);
      }
      word |= (uint32_t)q << (4 * j);
    }
    dst[i] = word;
  }
}

// ---------------------------------------------------------------------------
// decode GEMV (M <= 4): 4x4x4 MFMA blocks over 256-byte row spans
// ---------------------------------------------------------------------------
// The weight rows are read in spans of 256 bytes (512 k). Lane l = 4b + j
// (block b = l/4, quad row j = l%4) loads the 16 bytes at byte 16b of a span
// of weight row 4q+j, so one load instruction covers 4 rows x 256 contiguous
// bytes (whole cache lines). v_mfma_f32_4x4x4_16b runs 16 independent 4x4x4
// products: block b multiplies the activation rows (A: lane 4b+i holds
// x[i]) by the 4 weight rows (B: lane 4b+j holds row j) over 4 k of the 32 k
// in that 16-byte piece; eight of them cover the piece, and lane 4b+j ends
// with D[i] = sum over the piece of x[i,k] * (OFFSET + q[4q+j,k]) for i = 0..3.
// A 16-byte piece never straddles a group (G >= 32), so the lane applies its
// own group's scale and bias: acc[i] += s*D[i] + (b - OFFSET*s)*X[i] with X[i]
// the sum of x[i] over the piece. The sixteen blocks are summed by lane
// shuffles once per row quad.
//
// A vector memory instruction costs the texture unit about the same whatever
// its width, so the weights are the only per-wave global loads. The
// activations, their per-piece sums and the (scale, bias) pairs of the
// workgroup's rows are staged in LDS once per workgroup: the activations in
// the k order of the decoded pairs, the pairs interleaved into one dword.
// Work split: a workgroup owns R rows over the whole K; each wave owns one
// span group (SG groups of up to US consecutive spans per row) for RQW row
// quads and keeps that group's activations in registers. With SG > 1 the SG
// waves of a row quad add their sums through LDS. Every global load is a
// buffer load issued before any compute; lanes with nothing to read use an
// out-of-range offset and read zeros.
struct GemvArgs {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* sc;
  const uint16_t* bi;
  void* y;
  int y_dtype;
  int M, N, K;
  int SG;       // span groups per row (1, 2 or 4)
  int USr;      // spans per group (the last group may have fewer)
  int R;        // rows per workgroup
  // plain GEMV: 16-bit residual [M][N] added to the rounded output (or null)
  const uint16_t* res;
  // fused layer steps (GemvFuse)
  const uint16_t* xr;   // kFfnGateUp: residual added to x before the norm (or null)
  const uint16_t* nw;   // kFfnGateUp: RMSNorm weight [K]
  uint16_t* hid;        // kFfnGateUp: x + xr [M][K], written by workgroup 0 (or null)
  uint16_t* nrm;        // kFfnGateUp: the normed activations [M][K], workgroup 0 (or null)
  float eps;
  const uint32_t* w2;   // kFfnGateUp: the up projection's weights, scales, biases
  const uint16_t* sc2;
  const uint16_t* bi2;
  void* y2;             // kQkvRope: key and value outputs
  void* y3;
  int heads;            // kQkvRope: heads of the query and key sections
  int hd, rd;           // kQkvRope: head_dim and rope_dims
  int q_rows, kv_rows;  // kQkvRope: q_size and kv_size
  float log2_base;      // kQkvRope: log2 of the RoPE base
  float pos;            // kQkvRope: the token's position (the cache offset)
};

// Decoder-layer steps fused into the GEMV (template parameter FUSE):
//  kFfnGateUp  the residual add and RMSNorm of the FFN input in the prologue;
//              gate and up row quads interleaved (even virtual quad t -> gate
//              quad t/2, odd -> up quad t/2) and gelu(gate) * up written as
//              the output (spark_mlx_llm/ops/ffn.py:98-102);
//  kQkvRope    the QKV projection of one token with rotary embedding of the
//              query and key heads in the epilogue: within each head the row
//              quad of dims i..i+3 and the one of i + rope_dims/2 are an
//              even/odd virtual pair (X/src/spark_qkv_rope.cpp:83-101).
enum GemvFuse { kPlain = 0, kFfnGateUp = 1, kQkvRope = 2 };

// Real row quad of virtual quad vq under the kQkvRope pairing: head h of the
// query and key sections holds hd/4 quads; its first rope_dims/4 virtual
// quads are the pairs (p, p + rope_dims/8), the rest keep their place, and so
// do the value rows.
__device__ __forceinline__ int qkv_real_quad(int vq, int hq, int P, int heads) {
  const int h = vq / hq, w = vq - h * hq;
  if (h >= heads || w >= 2 * P) return vq;
  return h * hq + (w >> 1) + (w & 1) * P;
}

constexpr int kGemvXP = 2;   // staged activation pieces (64 B) per thread, at most
constexpr int kGemvSP = 4;   // staged (scale, bias) pieces (16 B each) per thread, at most
constexpr int kFfnXC1 = 2;   // FFN prologue chunks (16 B) per thread at one row, at most
constexpr int kFfnXC4 = 4;   // ... at two to four rows

// LDS slot (dword index) of 16-byte chunk w of activation piece pi. The
// pieces of a span sit chunk-major (16 pieces x 16 B per chunk), so the 16
// lane blocks of a wave, which read 16 consecutive pieces, hit 256
// contiguous bytes per read instead of 16 addresses at a 64-byte stride.
__device__ __forceinline__ int gemv_xslot(int pi, int w) {
  return 256 * (pi >> 4) + 64 * w + 4 * (pi & 15);
}

// LDS layout of the decode GEMV (byte offsets)
struct GemvLds {
  int xp;    // activations [M][K] in pair order (2 B each)
  int xs;    // sums of each 32-k piece: [K/32][4] fp32 (rows past M unused)
  int sb;    // (scale, bias) of the workgroup's rows: [R][K/G] dwords
  int red;   // cross-wave partial sums: [NW][RQW][4][4] fp32
  int fz;    // fused epilogues: final sums of the workgroup's rows [R][4] fp32
  int st;    // FFN prologue: the normed rows [M][K] in natural order
  int bytes;
};
__host__ __device__ __forceinline__ GemvLds gemv_lds(int M, int K, int R, int G, int NW, int RQW,
                                                     bool ffn = false) {
  GemvLds l;
  l.xp = 0;
  l.xs = l.xp + ((M * K * 2 + 1023) & ~1023);
  l.sb = l.xs + (K / 32) * 16;
  l.red = l.sb + ((R * (K / G) * 4 + 15) & ~15);
  l.fz = l.red + NW * RQW * 64;
  l.st = l.fz + R * 16;
  l.bytes = l.st + (ffn ? M * K * 2 : 0);
  return l;
}


template <typename T, int G, int MQ, int US, int RQW, int NW, int FUSE = kPlain>
__global__ __launch_bounds__(64 * NW, 3) void w4_gemv_kernel(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int NT = 64 * NW;
  // FFN prologue: 16-byte chunks of x, the residual and the norm weight per
  // thread, spread over the whole workgroup
  constexpr int XC = FUSE == kFfnGateUp ? (MQ == 1 ? kFfnXC1 : kFfnXC4) : 1;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = lane >> 2, j = lane & 3;
  const int M = a.M, N = a.N, K = a.K, SG = a.SG, R = a.R;
  // rows of one weight matrix (the gate and up matrices each hold N/2)
  const int NR = FUSE == kFfnGateUp ? N >> 1 : N;
  const int RB = K >> 1;                       // bytes per weight row
  const int U = (RB + 255) >> 8;               // spans per row
  const int ng = K / G;                        // groups per row
  const int r0 = blockIdx.x * R;               // first row of the workgroup
  const int sg = wave % SG;
  const int q0 = (r0 >> 2) + (wave / SG) * RQW;  // first row quad of the wave
  const int u0 = sg * a.USr;
  const int ns = min(a.USr, U - u0);           // spans of this wave (wave-uniform)
  const GemvLds L = gemv_lds(M, K, R, G, NW, RQW, FUSE == kFfnGateUp);

  const rsrc_t rx = make_rsrc(a.x, (uint32_t)M * K * 2);
  const rsrc_t rw = make_rsrc(a.w, (uint32_t)NR * RB);
  const rsrc_t rs = make_rsrc(a.sc, (uint32_t)NR * ng * 2);
  const rsrc_t rb = make_rsrc(a.bi, (uint32_t)NR * ng * 2);

  // 1. staging loads: activation pieces (64 B) and (scale, bias) pieces
  const int nxp = M * (K >> 5);                // activation pieces
  const int nsp = (R * ng) >> 3;               // 16-byte scale pieces of the workgroup
  u32x4_t xr[kGemvXP][4];
  u32x4_t xc[XC], rc[XC], nc[XC];              // FFN prologue chunks
  u32x4_t sr[kGemvSP], br[kGemvSP];
  const int nxc = nxp * 4;                     // 16-byte activation chunks
  // a wave with no piece to fetch skips the instruction (the texture unit
  // charges per instruction, lanes or not); the condition is wave-uniform
  if constexpr (FUSE == kFfnGateUp) {
    const rsrc_t rr_ = make_rsrc(a.xr, a.xr ? (uint32_t)M * K * 2 : 0u);
    const rsrc_t rn_ = make_rsrc(a.nw, (uint32_t)K * 2);
#pragma unroll
    for (int c = 0; c < XC; ++c) {
      const int ci = tid + c * NT;
      if (c * NT + 64 * wave < nxc) {
        const uint32_t off = ci < nxc ? 16u * ci : kOob;
        xc[c] = buf_load16(rx, off);
        rc[c] = buf_load16(rr_, off);
        nc[c] = buf_load16(rn_, ci < nxc ? 16u * (ci % (K >> 3)) : kOob);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kGemvXP; ++i) {
      const int pi = tid + i * NT;
      if (i * NT + 64 * wave < nxp) {
        const uint32_t off = pi < nxp ? 64u * pi : kOob;
#pragma unroll
        for (int w = 0; w < 4; ++w) xr[i][w] = buf_load16(rx, off + 16 * w);
      }
    }
  }
  if constexpr (FUSE == kPlain) {
#pragma unroll
    for (int i = 0; i < kGemvSP; ++i) {
      const int pi = tid + i * NT;
      if (i * NT + 64 * wave < nsp) {
        const uint32_t off = pi < nsp ? 2u * (uint32_t)r0 * ng + 16u * pi : kOob;
        sr[i] = buf_load16(rs, off);
        br[i] = buf_load16(rb, off);
      }
    }
  } else {
    // the workgroup's virtual quads are not contiguous rows: wave w stages
    // the scale block of virtual quads w and w + NW (4 contiguous rows, ng/2
    // pieces of 16 bytes, one per lane), from that quad's matrix; the quad's
    // matrix and rows are wave-uniform
    const int hp = ng >> 1;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int vql = wave + t * NW;
      if (vql < (R >> 2)) {
        const int vq = min((r0 >> 2) + vql, (N >> 2) - 1);
        rsrc_t rsq = rs, rbq = rb;
        int rq;
        if constexpr (FUSE == kFfnGateUp) {
          rq = vq >> 1;
          if (vq & 1) {
            rsq = make_rsrc(a.sc2, (uint32_t)NR * ng * 2);
            rbq = make_rsrc(a.bi2, (uint32_t)NR * ng * 2);
          }
        } else {
          rq = qkv_real_quad(vq, a.hd >> 2, a.rd >> 3, a.heads);
        }
        const uint32_t off = lane < hp ? (uint32_t)rq * 8 * ng + 16 * lane : kOob;
        sr[t] = buf_load16(rsq, off);
        br[t] = buf_load16(rbq, off);
      }
    }
  }

  // 2. the wave's weights: RQW row quads x US spans
  u32x4_t wv[RQW][US];
#pragma unroll
  for (int r = 0; r < RQW; ++r) {
    const int vq = q0 + r;
    int rq = vq;
    rsrc_t rwr = rw;
    if constexpr (FUSE == kFfnGateUp) {
      rq = vq >> 1;
      if (vq & 1) rwr = make_rsrc(a.w2, (uint32_t)NR * RB);
    } else if constexpr (FUSE == kQkvRope) {
      rq = qkv_real_quad(vq, a.hd >> 2, a.rd >> 3, a.heads);
    }
    const int row = 4 * rq + j;
#pragma unroll
    for (int s = 0; s < US; ++s) {
      const int p = 256 * (u0 + s) + 16 * b;
      const bool ok = row < NR && s < ns && p + 16 <= RB;
      wv[r][s] = buf_load16(rwr, ok ? (uint32_t)row * RB + p : kOob);
    }
  }

  // keep every load above ahead of the arithmetic below
  __builtin_amdgcn_sched_barrier(0);

  // 2b. FFN prologue: hidden = x + residual and its RMSNorm,
  // w * T(hidden * rsqrt(mean(hidden^2) + eps)) (mx.fast.rms_norm,
  // spark_mlx_llm/ops/ffn.py:98-99), over 16-byte chunks spread across the
  // workgroup; the normed rows go to an LDS stage in natural order, from
  // which the activation pieces are read below. Every workgroup reduces the
  // sums of squares in the same order, so all of them normalise alike.
  if constexpr (FUSE == kFfnGateUp) {
    const bool has_res = a.xr != nullptr;
    float ss[MQ];
#pragma unroll
    for (int m = 0; m < MQ; ++m) ss[m] = 0.0f;
#pragma unroll
    for (int c = 0; c < XC; ++c) {
      const int ci = tid + c * NT;
      if (ci < nxc) {
        float q = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint32_t p = xc[c][e];
          if (has_res)
            p = pack_round<T>(lo16<T>(p) + lo16<T>(rc[c][e]), hi16<T>(p) + hi16<T>(rc[c][e]));
          xc[c][e] = p;
          const float h0 = lo16<T>(p), h1 = hi16<T>(p);
          q = fmaf(h0, h0, q);
          q = fmaf(h1, h1, q);
        }
        const int m = MQ == 1 ? 0 : ci / (K >> 3);
#pragma unroll
        for (int mm = 0; mm < MQ; ++mm) ss[mm] += mm == m ? q : 0.0f;
        if (blockIdx.x == 0 && a.hid) *reinterpret_cast<u32x4_t*>(a.hid + 8 * ci) = xc[c];
      }
    }
    float* red = reinterpret_cast<float*>(smem + L.red);
#pragma unroll
    for (int m = 0; m < MQ; ++m) {
      const float v = wave_sum(ss[m]);
      if (lane == 0) red[wave * 4 + m] = v;
    }
    __syncthreads();
    float inv[MQ];
#pragma unroll
    for (int m = 0; m < MQ; ++m) {
      float t = 0.0f;
      for (int w = 0; w < NW; ++w) t += red[w * 4 + m];
      inv[m] = (float)(1.0 / sqrt((double)(t / (float)K + a.eps)));
    }
    uint16_t* stage = reinterpret_cast<uint16_t*>(smem + L.st);
#pragma unroll
    for (int c = 0; c < XC; ++c) {
      const int ci = tid + c * NT;
      if (ci < nxc) {
        const int m = MQ == 1 ? 0 : ci / (K >> 3);
        float im = inv[0];
#pragma unroll
        for (int mm = 1; mm < MQ; ++mm) im = mm == m ? inv[mm] : im;
        u32x4_t nv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t p = xc[c][e], wt = nc[c][e];
          const uint32_t n = pack_round<T>(lo16<T>(p) * im, hi16<T>(p) * im);
          nv[e] = pack_round<T>(lo16<T>(wt) * lo16<T>(n), hi16<T>(wt) * hi16<T>(n));
        }
        *reinterpret_cast<u32x4_t*>(stage + 8 * ci) = nv;
        if (blockIdx.x == 0 && a.nrm) *reinterpret_cast<u32x4_t*>(a.nrm + 8 * ci) = nv;
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kGemvXP; ++i) {
      const int pi = tid + i * NT;
      if (pi < nxp) {
#pragma unroll
        for (int w = 0; w < 4; ++w) xr[i][w] = *reinterpret_cast<const u32x4_t*>(stage + 32 * pi + 8 * w);
      }
    }
  }

  // 3. write the staged data to LDS
  {
    uint32_t* xp = reinterpret_cast<uint32_t*>(smem + L.xp);
    float* xs = reinterpret_cast<float*>(smem + L.xs);
#pragma unroll
    for (int i = 0; i < kGemvXP; ++i) {
      const int pi = tid + i * NT;
      if (pi < nxp) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const u32x4_t r = xr[i][w];
          const u32x4_t o = {__builtin_amdgcn_perm(r.z, r.x, 0x05040100u),   // (x0, x4)
                             __builtin_amdgcn_perm(r.z, r.x, 0x07060302u),   // (x1, x5)
                             __builtin_amdgcn_perm(r.w, r.y, 0x05040100u),   // (x2, x6)
                             __builtin_amdgcn_perm(r.w, r.y, 0x07060302u)};  // (x3, x7)
          *reinterpret_cast<u32x4_t*>(xp + gemv_xslot(pi, w)) = o;
#pragma unroll
          for (int e = 0; e < 4; ++e) sum = pair_sum<T>(r[e], sum);
        }
        const int m = pi / (K >> 5), piece = pi - m * (K >> 5);
        xs[4 * piece + m] = sum;
      }
    }
    uint32_t* sb = reinterpret_cast<uint32_t*>(smem + L.sb);
    const int hp = ng >> 1;
#pragma unroll
    for (int i = 0; i < kGemvSP; ++i) {
      // plain: piece tid + i*NT; fused: piece lane of virtual quad wave + i*NW
      const int pi = FUSE == kPlain ? tid + i * NT : (wave + i * NW) * hp + lane;
      const bool ok = FUSE == kPlain ? pi < nsp : i < 2 && wave + i * NW < (R >> 2) && lane < hp;
      if (ok) {
        const u32x4_t s = sr[i], c = br[i];
        u32x4_t lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo[e] = __builtin_amdgcn_perm(c[e], s[e], 0x05040100u);  // (s0, b0)
          hi[e] = __builtin_amdgcn_perm(c[e], s[e], 0x07060302u);                 // (s1, b1)
        }
        *reinterpret_cast<u32x4_t*>(sb + 8 * pi) = u32x4_t{lo[0], hi[0], lo[1], hi[1]};
        *reinterpret_cast<u32x4_t*>(sb + 8 * pi + 4) = u32x4_t{lo[2], hi[2], lo[3], hi[3]};
      }
    }
  }
  __syncthreads();

  // 4. the wave's activations (pair order) and piece sums, from LDS
  uint32_t xa[US][4][4];
  float xm[US][MQ];
  {
    const unsigned char* xp = smem + L.xp;
    const float* xs = reinterpret_cast<const float*>(smem + L.xs);
#pragma unroll
    for (int s = 0; s < US; ++s) {
      const int piece = min(16 * (u0 + s) + b, (K >> 5) - 1);
      const int pi = min(j, M - 1) * (K >> 5) + piece;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xp + 4 * gemv_xslot(pi, w));
        xa[s][w][0] = v.x;
        xa[s][w][1] = v.y;
        xa[s][w][2] = v.z;
        xa[s][w][3] = v.w;
      }
      if constexpr (MQ == 1) {
        xm[s][0] = xs[4 * piece];
      } else {
        const f32x4_t v = *reinterpret_cast<const f32x4_t*>(xs + 4 * piece);
        xm[s][0] = v.x;
        xm[s][1] = v.y;
        xm[s][2] = v.z;
        xm[s][3] = v.w;
      }
    }
  }

  // 4b. the rotation of each output row of the wave (kQkvRope) does not
  // depend on the projection: its angle is taken here, while the weights are
  // still arriving
  float rcs[RQW], rsn[RQW];
  if constexpr (FUSE == kQkvRope) {
#pragma unroll
    for (int r = 0; r < RQW; ++r) {
      const int vq = q0 + r, hq = a.hd >> 2, P = a.rd >> 3;
      const int h = vq / hq, w = vq - h * hq;
      rcs[r] = 1.0f;
      rsn[r] = 0.0f;
      if (lane < 4 && h < a.heads && w < 2 * P)
        sincosf(a.pos * rope_inv_freq(4 * (w >> 1) + lane, a.rd >> 1, a.log2_base), &rsn[r],
                &rcs[r]);
      // materialise the values here rather than where the epilogue uses them
      asm volatile("" ::"v"(rcs[r]), "v"(rsn[r]));
    }
  }

  // 5. per row quad: decode and 8 MFMAs per span, then the group epilogue.
  // A 4x4x4 MFMA takes ~48 cycles to feed its result to the next one, but
  // issues every ~10 cycles when independent: the spans of a row quad keep
  // separate accumulators (two each when there are fewer than three spans)
  // and their MFMAs are interleaved. Template spans beyond the wave's group
  // (s >= ns) are computed too and dropped by the epilogue.
  const uint32_t* sb = reinterpret_cast<const uint32_t*>(smem + L.sb);
  const DecodeConsts dc = decode_consts<T>();
  constexpr int NA = US < 3 ? 2 : 1;     // accumulators per span
  float out[RQW][MQ];
#pragma unroll
  for (int r = 0; r < RQW; ++r) {
    const int rl = 4 * (q0 + r) + j - r0;      // row within the workgroup
    f32x4_t d[US][NA];
#pragma unroll
    for (int s = 0; s < US; ++s)
#pragma unroll
      for (int h = 0; h < NA; ++h) d[s][h] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t pr[US][4];
#pragma unroll
      for (int s = 0; s < US; ++s) decode_w4_strided<T>(wv[r][s][w], dc, pr[s]);
#pragma unroll
      for (int s = 0; s < US; ++s)
        d[s][0] = mfma4x4<T>(xa[s][w][0], xa[s][w][1], pr[s][0], pr[s][1], d[s][0]);
#pragma unroll
      for (int s = 0; s < US; ++s)
        d[s][NA - 1] = mfma4x4<T>(xa[s][w][2], xa[s][w][3], pr[s][2], pr[s][3], d[s][NA - 1]);
    }
    float acc[MQ];
#pragma unroll
    for (int m = 0; m < MQ; ++m) acc[m] = 0.0f;
#pragma unroll
    for (int s = 0; s < US; ++s) {
      const int p = 256 * (u0 + s) + 16 * b;
      const bool ok = s < ns && p + 16 <= RB;
      // pieces past the row end carry zero codes and unrelated activations
      const uint32_t pair = ok ? sb[rl * ng + (2 * p) / G] : 0u;
      const float sf = T::to_f32((uint16_t)(pair & 0xFFFFu));
      const float bf = fmaf(-T::OFFSET, sf, T::to_f32((uint16_t)(pair >> 16)));
#pragma unroll
      for (int m = 0; m < MQ; ++m) {
        const float dm = NA == 2 ? d[s][0][m] + d[s][NA - 1][m] : d[s][0][m];
        const float t = fmaf(sf, dm, fmaf(bf, xm[s][m], acc[m]));
        acc[m] = ok ? t : acc[m];
      }
    }
    // sum the sixteen blocks (lanes j, j+4, ..., j+60)
#pragma unroll
    for (int m = 0; m < MQ; ++m) out[r][m] = sum_blocks(acc[m]);
  }

  if (SG > 1) {
    float* red = reinterpret_cast<float*>(smem + L.red);
    if (lane < 4) {
#pragma unroll
      for (int r = 0; r < RQW; ++r)
#pragma unroll
        for (int m = 0; m < MQ; ++m) red[((wave * RQW + r) * 4 + lane) * 4 + m] = out[r][m];
    }
    __syncthreads();
    if (sg == 0 && lane < 4) {
#pragma unroll
      for (int r = 0; r < RQW; ++r)
#pragma unroll
        for (int m = 0; m < MQ; ++m) {
          float v = out[r][m];
          for (int o = 1; o < SG; ++o) v += red[(((wave + o) * RQW + r) * 4 + lane) * 4 + m];
          out[r][m] = v;
        }
    }
  }

  if constexpr (FUSE != kPlain) {
    // the partner of virtual quad vq is vq ^ 1: the wave's other quad, or
    // (one quad per wave) the neighbouring wave's, exchanged through LDS
    float pv[RQW][MQ];
    if constexpr (RQW == 2) {
#pragma unroll
      for (int m = 0; m < MQ; ++m) {
        pv[0][m] = out[1][m];
        pv[1][m] = out[0][m];
      }
    } else {
      float* fz = reinterpret_cast<float*>(smem + L.fz);
      const int ql = q0 - (r0 >> 2);
      if (sg == 0 && lane < 4) {
#pragma unroll
        for (int m = 0; m < MQ; ++m) fz[(ql * 4 + lane) * 4 + m] = out[0][m];
      }
      __syncthreads();
#pragma unroll
      for (int m = 0; m < MQ; ++m) pv[0][m] = fz[((ql ^ 1) * 4 + lane) * 4 + m];
    }
    if (sg != 0 || lane >= 4) return;
#pragma unroll
    for (int r = 0; r < RQW; ++r) {
      const int vq = q0 + r;
      if constexpr (FUSE == kFfnGateUp) {
        // the gate quad's lanes write gelu(gate) * up for rows 4*(vq/2) + lane
        const int row = 2 * (vq & ~1) + lane;
        if ((vq & 1) == 0 && row < NR) {
#pragma unroll
          for (int m = 0; m < MQ; ++m)
            if (m < M) store_out(a.y, (int64_t)m * NR + row, gelu_mul<T>(out[r][m], pv[r][m]), a.y_dtype);
        }
      } else {
        const int hq = a.hd >> 2, P = a.rd >> 3;
        const int h = vq / hq, w = vq - h * hq;
        const int row = 4 * qkv_real_quad(vq, hq, P, a.heads) + lane;
        float v = out[r][0];
        if (h < a.heads && w < 2 * P) {
          // mx.fast.rope on the 16-bit projections (non-traditional):
          // x1 = dim i, x2 = dim i + rope_dims/2 of the head
          const float sn = rsn[r], cs = rcs[r];
          const float self = T::to_f32(T::from_f32(v)), other = T::to_f32(T::from_f32(pv[r][0]));
          v = (w & 1) == 0 ? self * cs - other * sn : other * sn + self * cs;
        }
        if (row < a.q_rows)
          store_out(a.y, row, v, a.y_dtype);
        else if (row < a.q_rows + a.kv_rows)
          store_out(a.y2, row - a.q_rows, v, a.y_dtype);
        else if (row < N)
          store_out(a.y3, row - a.q_rows - a.kv_rows, v, a.y_dtype);
      }
    }
    return;
  }
  if (sg != 0) return;
  if (lane < 4) {
#pragma unroll
    for (int r = 0; r < RQW; ++r) {
      const int row = 4 * (q0 + r) + lane;
      if (row < N) {
#pragma unroll
        for (int m = 0; m < MQ; ++m)
          if (m < M) {
            const int64_t idx = (int64_t)m * N + row;
            const float v = out[r][m];
            store_out(a.y, idx, a.res ? add_rounded<T>(v, a.res[idx]) : v, a.y_dtype);
          }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// streaming decode GEMV (M = 1)
// ---------------------------------------------------------------------------
// One workgroup of 16 waves per CU. Workgroup w owns the row quads
// [w*nq/P, (w+1)*nq/P) (sizes differ by at most one), so every CU streams
// the same number of bytes. Its work items are (row quad, span) pairs in
// quad-major order, dealt to the waves round-robin: each wave gets NI or
// fewer 1 KB items whatever the row length. The activations (pair order,
// chunk-major spans) with their piece sums, and the (scale, bias) pairs of
// the workgroup's rows, are staged in LDS once per workgroup.
// Every wave issues all of its weight loads at the start, right after the
// staging loads, and computes its items in issue order, each as soon as its
// own load has landed: the decode and MFMAs of early items overlap the
// arrival of later ones, and the work left after the last byte lands is one
// item per wave.
// An item is the w4_gemv_kernel step for one span of one row quad: one
// 16-byte piece per lane (activations read from LDS), eight 4x4x4 MFMAs and
// the lane's group epilogue. Its 64 lane sums go to an LDS slot; at the end
// each row adds its slots over the spans in order, then over the 16 blocks
// by a fixed shuffle tree.
struct GemvStreamArgs {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* sc;
  const uint16_t* bi;
  void* y;
  int y_dtype;
  int N, K;
  int nq;  // row quads
  int P;   // workgroups
  int QW;  // row quads of the largest workgroup
  const uint16_t* res;  // 16-bit residual added to the rounded output (or null)
  int RR;  // 1: workgroup i owns rows [i*N/P, (i+1)*N/P) (quads from its first row)
};

constexpr int kStreamXP = 1;   // staged activation pieces (64 B) per thread, at most
constexpr int kStreamSP = 2;   // staged (scale, bias) pieces (16 B each) per thread, at most

// LDS layout of the streaming GEMV (byte offsets)
struct StreamLds {
  int xp;    // activations [K], gemv_xslot order
  int xs;    // piece sums [K/32] fp32
  int sb;    // (scale, bias) of the workgroup's rows: [4*QW][K/G] dwords
  int part;  // lane sums of the items: [QW*U][64] fp32
  int bytes;
};
__host__ __device__ __forceinline__ StreamLds stream_lds(int K, int QW, int G) {
  const int U = ((K >> 1) + 255) >> 8;
  StreamLds l;
  l.xp = 0;
  l.xs = (K * 2 + 1023) & ~1023;
  l.sb = l.xs + ((K / 32) * 4 + 15) / 16 * 16;
  l.part = l.sb + ((4 * QW * (K / G) * 4 + 15) & ~15);
  l.bytes = l.part + QW * U * 64 * 4;
  return l;
}

// FULL: K % 512 == 0 and N % 4 == 0 (every piece of every item is in range)
template <typename T, int G, int NI, int NW, bool FULL>
__global__ __launch_bounds__(64 * NW) void w4_gemv_stream_kernel(GemvStreamArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int NT = 64 * NW;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = lane >> 2, j = lane & 3;
  const int N = a.N, K = a.K;
  const int RB = K >> 1;             // bytes per weight row
  const int U = (RB + 255) >> 8;     // spans per row
  const int ng = K / G;              // groups per row
  // the workgroup's rows [r0, r1), taken as row quads from r0
  int r0, r1;
  if (a.RR) {
    r0 = (int)((int64_t)blockIdx.x * N / a.P);
    r1 = (int)((int64_t)(blockIdx.x + 1) * N / a.P);
  } else {
    r0 = 4 * (int)((int64_t)blockIdx.x * a.nq / a.P);
    r1 = min(N, 4 * (int)((int64_t)(blockIdx.x + 1) * a.nq / a.P));
  }
  const int nql = (r1 - r0 + 3) >> 2;
  const int nitems = nql * U;
  const StreamLds L = stream_lds(K, a.QW, G);

  const rsrc_t rx = make_rsrc(a.x, (uint32_t)K * 2);
  const rsrc_t rw = make_rsrc(a.w, (uint32_t)N * RB);
  const rsrc_t rs = make_rsrc(a.sc, (uint32_t)N * ng * 2);
  const rsrc_t rb = make_rsrc(a.bi, (uint32_t)N * ng * 2);

  // 1. staging loads: activation pieces and (scale, bias) pieces; a wave
  // with no piece to fetch skips the instruction
  const int nxp = K >> 5;
  const int nsp = (4 * nql * ng) >> 3;
  u32x4_t xr[kStreamXP][4];
  u32x4_t sr[kStreamSP], br[kStreamSP];
#pragma unroll
  for (int i = 0; i < kStreamXP; ++i) {
    const int pi = tid + i * NT;
    if (i * NT + 64 * wave < nxp) {
      const uint32_t off = pi < nxp ? 64u * pi : kOob;
#pragma unroll
      for (int w = 0; w < 4; ++w) xr[i][w] = buf_load16(rx, off + 16 * w);
    }
  }
#pragma unroll
  for (int i = 0; i < kStreamSP; ++i) {
    const int pi = tid + i * NT;
    if (i * NT + 64 * wave < nsp) {
      const uint32_t off = pi < nsp ? 2u * (uint32_t)r0 * ng + 16u * pi : kOob;
      sr[i] = buf_load16(rs, off);
      br[i] = buf_load16(rb, off);
    }
  }

  // 2. every weight load of the wave: item wave + 16 i is (row quad ql[i],
  // span sp[i]); slots past the wave's last item read nothing
  const int nmy = nitems > wave ? (nitems - wave + NW - 1) / NW : 0;
  int ql[NI], sp[NI];
  u32x4_t wv[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int it = wave + i * NW;
    ql[i] = it / U;
    sp[i] = it - ql[i] * U;
    const int row = r0 + 4 * ql[i] + j, p = 256 * sp[i] + 16 * b;
    const bool ok = i < nmy && row < r1 && (FULL || p + 16 <= RB);
    wv[i] = buf_load16(rw, ok ? (uint32_t)row * RB + p : kOob);
  }

  // keep every load above ahead of the arithmetic below
  __builtin_amdgcn_sched_barrier(0);

  // 3. write the staged data to LDS
  {
    uint32_t* xp = reinterpret_cast<uint32_t*>(smem + L.xp);
    float* xs = reinterpret_cast<float*>(smem + L.xs);
#pragma unroll
    for (int i = 0; i < kStreamXP; ++i) {
      const int pi = tid + i * NT;
      if (pi < nxp) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const u32x4_t r = xr[i][w];
          const u32x4_t o = {__builtin_amdgcn_perm(r.z, r.x, 0x05040100u),   // (x0, x4)
                             __builtin_amdgcn_perm(r.z, r.x, 0x07060302u),   // (x1, x5)
                             __builtin_amdgcn_perm(r.w, r.y, 0x05040100u),   // (x2, x6)
                             __builtin_amdgcn_perm(r.w, r.y, 0x07060302u)};  // (x3, x7)
          *reinterpret_cast<u32x4_t*>(xp + gemv_xslot(pi, w)) = o;
#pragma unroll
          for (int e = 0; e < 4; ++e) sum = pair_sum<T>(r[e], sum);
        }
        xs[pi] = sum;
      }
    }
    uint32_t* sb = reinterpret_cast<uint32_t*>(smem + L.sb);
#pragma unroll
    for (int i = 0; i < kStreamSP; ++i) {
      const int pi = tid + i * NT;
      if (pi < nsp) {
        const u32x4_t s = sr[i], c = br[i];
        u32x4_t lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo[e] = __builtin_amdgcn_perm(c[e], s[e], 0x05040100u);  // (s0, b0)
          hi[e] = __builtin_amdgcn_perm(c[e], s[e], 0x07060302u);  // (s1, b1)
        }
        *reinterpret_cast<u32x4_t*>(sb + 8 * pi) = u32x4_t{lo[0], hi[0], lo[1], hi[1]};
        *reinterpret_cast<u32x4_t*>(sb + 8 * pi + 4) = u32x4_t{lo[2], hi[2], lo[3], hi[3]};
      }
    }
  }
  __syncthreads();

  // 4. the wave's items, in issue order
  const unsigned char* xp = smem + L.xp;
  const float* xs = reinterpret_cast<const float*>(smem + L.xs);
  const uint32_t* sb = reinterpret_cast<const uint32_t*>(smem + L.sb);
  float* part = reinterpret_cast<float*>(smem + L.part);
  const DecodeConsts dc = decode_consts<T>();
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    if (i < nmy) {
      const int s = sp[i];
      const int p = 256 * s + 16 * b;
      const bool ok = r0 + 4 * ql[i] + j < r1 && (FULL || p + 16 <= RB);
      const int piece = FULL ? 16 * s + b : min(16 * s + b, (K >> 5) - 1);
      uint32_t xa[4][4];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xp + 4 * gemv_xslot(piece, w));
        xa[w][0] = v.x;
        xa[w][1] = v.y;
        xa[w][2] = v.z;
        xa[w][3] = v.w;
      }
      const float xm = xs[piece];
      // pieces past the row end carry zero codes and unrelated activations
      const uint32_t pair = ok ? sb[(4 * ql[i] + j) * ng + (2 * p) / G] : 0u;
      f32x4_t d0 = {0.0f, 0.0f, 0.0f, 0.0f}, d1 = d0;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        uint32_t pr[4];
        decode_w4_strided<T>(wv[i][w], dc, pr);
        d0 = mfma4x4<T>(xa[w][0], xa[w][1], pr[0], pr[1], d0);
        d1 = mfma4x4<T>(xa[w][2], xa[w][3], pr[2], pr[3], d1);
      }
      const float sf = T::to_f32((uint16_t)(pair & 0xFFFFu));
      const float bf = fmaf(-T::OFFSET, sf, T::to_f32((uint16_t)(pair >> 16)));
      const float v = fmaf(sf, d0[0] + d1[0], bf * xm);
      part[(ql[i] * U + s) * 64 + lane] = ok ? v : 0.0f;
    }
  }
  __syncthreads();

  // 5. row r of the workgroup, block bb: the sum of its slots over the spans
  // in order, then over the 16 blocks by a shuffle tree (lanes 16t..16t+15
  // hold the blocks of one row)
  for (int t0 = 0; t0 < 64 * nql; t0 += NT) {
    const int t = t0 + tid;
    const int rl = t >> 4, bb = t & 15;
    float v = 0.0f;
    if (rl < 4 * nql) {
      const float* src = part + (rl >> 2) * U * 64 + 4 * bb + (rl & 3);
      for (int s = 0; s < U; ++s) v += src[s * 64];
    }
    v = sum_row16(v);
    const int row = r0 + rl;
    if (bb == 0 && row < r1)
      store_out(a.y, row, a.res ? add_rounded<T>(v, a.res[row]) : v, a.y_dtype);
  }
}

// ---------------------------------------------------------------------------
// streaming decode GEMV, several activation rows (2 <= M <= 16)
// ---------------------------------------------------------------------------
// The M = 1 streaming layout (one workgroup of 16 waves per CU, a contiguous
// range of row quads per workgroup, 1 KB (row quad, span) items, every
// weight load issued at the start) with the activation rows taken four at a
// time: each decoded piece feeds eight 4x4x4 MFMAs per row quartet (MQ
// quartets), so the decode is shared by all M rows. A wave takes a
// contiguous run of items in quad-major order and keeps per-lane sums in
// registers while the row quad stays the same; when it changes (and at the
// end) the sixteen blocks are added by lane shuffles and the quad's sums go
// to the LDS slot of the run's first span (the other slots of the run stay
// zero). Each output is the sum of its quad's slots in span order.
struct DecodeStreamArgs {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* sc;
  const uint16_t* bi;
  void* y;
  int y_dtype;
  int M, N, K;
  int nq;  // row quads
  int P;   // workgroups
  int QW;  // row quads of the largest workgroup
  const uint16_t* res;  // 16-bit residual added to the rounded output (or null)
  int RR;  // 1: workgroup i owns rows [i*N/P, (i+1)*N/P) (quads from its first row)
  int PH;   // K phases (phased kernel): the activations are staged SPH spans at a time
  int SPH;  // spans per phase (the last phase may hold fewer)
};

constexpr int kDecNW = 16;  // waves per workgroup
constexpr int kDecXP = 2;   // staged activation pieces (64 B) per thread, at most
constexpr int kDecSP = 2;   // staged (scale, bias) pieces (16 B each) per thread, at most

// LDS layout of the multi-row streaming GEMV (byte offsets)
struct DecLds {
  int xp;    // activations [M][K], gemv_xslot order
  int xs;    // piece sums [K/32][4*MQ] fp32
  int sb;    // (scale, bias) of the workgroup's rows: [4*QW][K/G] dwords
  int part;  // quad sums: [QW][U][4][4*MQ] fp32
  int bytes;
};
__host__ __device__ __forceinline__ DecLds dec_lds(int M, int K, int QW, int G, int MQ) {
  const int U = ((K >> 1) + 255) >> 8;
  DecLds l;
  l.xp = 0;
  l.xs = (M * K * 2 + 1023) & ~1023;
  l.sb = l.xs + (K / 32) * 16 * MQ;
  l.part = l.sb + ((4 * QW * (K / G) * 4 + 15) & ~15);
  l.bytes = l.part + QW * U * 4 * 4 * MQ * 4;
  return l;
}
// the same layout with npw 32-k pieces of each activation row staged at once
// (K phases: xp [M][npw], xs [npw][4*MQ])
__host__ __device__ __forceinline__ DecLds dec_lds_phased(int M, int K, int QW, int G, int MQ,
                                                          int npw) {
  const int U = ((K >> 1) + 255) >> 8;
  DecLds l;
  l.xp = 0;
  l.xs = (M * npw * 64 + 1023) & ~1023;
  l.sb = l.xs + npw * 16 * MQ;
  l.part = l.sb + ((4 * QW * (K / G) * 4 + 15) & ~15);
  l.bytes = l.part + QW * U * 4 * 4 * MQ * 4;
  return l;
}

// D: weight items of a wave in flight (D < NI: the first D go out ahead of the
// staging loads, each later one as the item D before it is taken up)
template <typename T, int G, int MQ, int NI, bool FULL, int D>
__global__ __launch_bounds__(64 * kDecNW) void w4_decode_stream_kernel(DecodeStreamArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int NT = 64 * kDecNW;
  constexpr int MR = 4 * MQ;         // activation rows held (rows past M repeat row M-1)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = lane >> 2, j = lane & 3;
  const int M = a.M, N = a.N, K = a.K;
  const int RB = K >> 1;             // bytes per weight row
  const int U = (RB + 255) >> 8;     // spans per row
  const int ng = K / G;              // groups per row
  const int np = K >> 5;             // 32-k pieces per row
  // the workgroup's rows [r0, r1), taken as row quads from r0
  int r0, r1;
  if (a.RR) {
    r0 = (int)((int64_t)blockIdx.x * N / a.P);
    r1 = (int)((int64_t)(blockIdx.x + 1) * N / a.P);
  } else {
    r0 = 4 * (int)((int64_t)blockIdx.x * a.nq / a.P);
    r1 = min(N, 4 * (int)((int64_t)(blockIdx.x + 1) * a.nq / a.P));
  }
  const int nql = (r1 - r0 + 3) >> 2;
  const int nitems = nql * U;
  const int i0 = (int)((int64_t)wave * nitems / kDecNW);
  const int nmy = (int)((int64_t)(wave + 1) * nitems / kDecNW) - i0;
  const DecLds L = dec_lds(M, K, a.QW, G, MQ);

  const rsrc_t rx = make_rsrc(a.x, (uint32_t)M * K * 2);
  const rsrc_t rw = make_rsrc(a.w, (uint32_t)N * RB);
  const rsrc_t rs = make_rsrc(a.sc, (uint32_t)N * ng * 2);
  const rsrc_t rb = make_rsrc(a.bi, (uint32_t)N * ng * 2);

  // the wave's items (slots past its last item read nothing)
  int ql[NI], sp[NI];
  u32x4_t wv[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int it = i0 + i;
    ql[i] = it / U;
    sp[i] = it - ql[i] * U;
  }
  auto wload = [&](int i) {
    const int row = r0 + 4 * ql[i] + j, p = 256 * sp[i] + 16 * b;
    const bool ok = i < nmy && row < r1 && (FULL || p + 16 <= RB);
    wv[i] = buf_load16(rw, ok ? (uint32_t)row * RB + p : kOob);
  };
  if constexpr (D < NI) {
#pragma unroll
    for (int i = 0; i < D; ++i) wload(i);
  }

  // 1. staging loads (a wave with no piece to fetch skips the instruction)
  const int nxp = M * np;
  const int nsp = (4 * nql * ng) >> 3;
  u32x4_t xr[kDecXP][4];
  u32x4_t sr[kDecSP], br[kDecSP];
#pragma unroll
  for (int i = 0; i < kDecXP; ++i) {
    const int pi = tid + i * NT;
    if (i * NT + 64 * wave < nxp) {
      const uint32_t off = pi < nxp ? 64u * pi : kOob;
#pragma unroll
      for (int w = 0; w < 4; ++w) xr[i][w] = buf_load16(rx, off + 16 * w);
    }
  }
#pragma unroll
  for (int i = 0; i < kDecSP; ++i) {
    const int pi = tid + i * NT;
    if (i * NT + 64 * wave < nsp) {
      const uint32_t off = pi < nsp ? 2u * (uint32_t)r0 * ng + 16u * pi : kOob;
      sr[i] = buf_load16(rs, off);
      br[i] = buf_load16(rb, off);
    }
  }

  // 2. with every item in flight at once (D = NI), the weight loads
  if constexpr (D == NI) {
#pragma unroll
    for (int i = 0; i < NI; ++i) wload(i);
  }

  // keep every load above ahead of the arithmetic below
  __builtin_amdgcn_sched_barrier(0);

  // 3. write the staged data to LDS; clear the quad slots
  {
    float* part = reinterpret_cast<float*>(smem + L.part);
    const int nslot = nql * U * 16 * MQ;
    for (int e = tid; e < nslot; e += NT) part[e] = 0.0f;
    uint32_t* xp = reinterpret_cast<uint32_t*>(smem + L.xp);
    float* xs = reinterpret_cast<float*>(smem + L.xs);
#pragma unroll
    for (int i = 0; i < kDecXP; ++i) {
      const int pi = tid + i * NT;
      if (pi < nxp) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const u32x4_t r = xr[i][w];
          const u32x4_t o = {__builtin_amdgcn_perm(r.z, r.x, 0x05040100u),   // (x0, x4)
                             __builtin_amdgcn_perm(r.z, r.x, 0x07060302u),   // (x1, x5)
                             __builtin_amdgcn_perm(r.w, r.y, 0x05040100u),   // (x2, x6)
                             __builtin_amdgcn_perm(r.w, r.y, 0x07060302u)};  // (x3, x7)
          *reinterpret_cast<u32x4_t*>(xp + gemv_xslot(pi, w)) = o;
#pragma unroll
          for (int e = 0; e < 4; ++e) sum = pair_sum<T>(r[e], sum);
        }
        const int m = pi / np, piece = pi - m * np;
        xs[piece * MR + m] = sum;
      }
    }
    uint32_t* sb = reinterpret_cast<uint32_t*>(smem + L.sb);
#pragma unroll
    for (int i = 0; i < kDecSP; ++i) {
      const int pi = tid + i * NT;
      if (pi < nsp) {
        const u32x4_t s = sr[i], c = br[i];
        u32x4_t lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo[e] = __builtin_amdgcn_perm(c[e], s[e], 0x05040100u);  // (s0, b0)
          hi[e] = __builtin_amdgcn_perm(c[e], s[e], 0x07060302u);  // (s1, b1)
        }
        *reinterpret_cast<u32x4_t*>(sb + 8 * pi) = u32x4_t{lo[0], hi[0], lo[1], hi[1]};
        *reinterpret_cast<u32x4_t*>(sb + 8 * pi + 4) = u32x4_t{lo[2], hi[2], lo[3], hi[3]};
      }
    }
  }
  __syncthreads();

  // 4. the wave's items in order; per-lane sums while the row quad stays
  const unsigned char* xp = smem + L.xp;
  const float* xs = reinterpret_cast<const float*>(smem + L.xs);
  const uint32_t* sb = reinterpret_cast<const uint32_t*>(smem + L.sb);
  float* part = reinterpret_cast<float*>(smem + L.part);
  const DecodeConsts dc = decode_consts<T>();
  f32x4_t acc[MQ];
#pragma unroll
  for (int q = 0; q < MQ; ++q) acc[q] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  int first = nmy > 0 ? sp[0] : 0;   // first span of the current run
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    if (i + D < NI) wload(i + D);
    if (i < nmy) {
      const int s = sp[i];
      const int p = 256 * s + 16 * b;
      const bool ok = r0 + 4 * ql[i] + j < r1 && (FULL || p + 16 <= RB);
      const int piece = FULL ? 16 * s + b : min(16 * s + b, np - 1);
      // pieces past the row end carry zero codes and unrelated activations
      const uint32_t pair = ok ? sb[(4 * ql[i] + j) * ng + (2 * p) / G] : 0u;
      const float sf = T::to_f32((uint16_t)(pair & 0xFFFFu));
      const float bf = fmaf(-T::OFFSET, sf, T::to_f32((uint16_t)(pair >> 16)));
      uint32_t pr[4][4];
#pragma unroll
      for (int w = 0; w < 4; ++w) decode_w4_strided<T>(wv[i][w], dc, pr[w]);
#pragma unroll
      for (int q = 0; q < MQ; ++q) {
        const int pi = min(4 * q + j, M - 1) * np + piece;
        f32x4_t d0 = {0.0f, 0.0f, 0.0f, 0.0f}, d1 = d0;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xp + 4 * gemv_xslot(pi, w));
          d0 = mfma4x4<T>(v.x, v.y, pr[w][0], pr[w][1], d0);
          d1 = mfma4x4<T>(v.z, v.w, pr[w][2], pr[w][3], d1);
        }
        const f32x4_t xm = *reinterpret_cast<const f32x4_t*>(xs + piece * MR + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float t = fmaf(sf, d0[e] + d1[e], bf * xm[e]);
          acc[q][e] += ok ? t : 0.0f;
        }
      }
      // end of a run: next item in another row quad, or the wave's last
      const bool last = i + 1 >= nmy || (i + 1 < NI && ql[i + 1] != ql[i]);
      if (last) {
        float* dst = part + ((ql[i] * U + first) * 4) * MR;
#pragma unroll
        for (int q = 0; q < MQ; ++q) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float v = sum_blocks(acc[q][e]);
            if (lane < 4) dst[lane * MR + 4 * q + e] = v;
          }
          acc[q] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
        if (i + 1 < NI) first = sp[i + 1];
      }
    }
  }
  __syncthreads();

  // 5. each output: the sum of its quad's slots in span order
  for (int t = tid; t < 4 * nql * M; t += NT) {
    const int rl = t / M, m = t - rl * M;
    const int row = r0 + rl;
    if (row < r1) {
      const float* src = part + (((rl >> 2) * U) * 4 + (rl & 3)) * MR + m;
      float v = 0.0f;
      for (int s = 0; s < U; ++s) v += src[s * 4 * MR];
      const int64_t idx = (int64_t)m * N + row;
      store_out(a.y, idx, a.res ? add_rounded<T>(v, a.res[idx]) : v, a.y_dtype);
    }
  }
}

// K-phased variant (5..8 rows, two row quartets, at most two items a wave
// per phase): for rows whose activation slab exceeds the staging registers or
// LDS (the down projection at 7 and 8 rows), the activations are staged SPH
// spans (16*SPH pieces) at a time. Each phase deals its own (row quad, span)
// items to the waves, in quad-major order over the phase's spans, with every
// item of a wave in flight. Once a phase's activations are in LDS, each wave
// issues the next phase's staging and weight loads and then takes up its
// items of the current phase; a barrier ends the current phase's reads before
// the next one's activations overwrite them. Runs of items end at phase
// boundaries, so each output is still the sum of its quad's span slots in
// span order. (A separate kernel: folding the phases into the one above
// changed its code and cost its 5..8-row shapes 2-3%.)
template <typename T, int G>
__global__ __launch_bounds__(64 * kDecNW) void w4_decode_phased_kernel(DecodeStreamArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int NT = 64 * kDecNW;
  constexpr int MQ = 2, MR = 8;      // two row quartets (rows past M repeat row M-1)
  constexpr int NI = 2;              // items of a wave per phase, at most
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = lane >> 2, j = lane & 3;
  const int M = a.M, N = a.N, K = a.K;
  const int RB = K >> 1;             // bytes per weight row (a multiple of 256)
  const int U = RB >> 8;             // spans per row
  const int ng = K / G;              // groups per row
  const int np = K >> 5;             // 32-k pieces per row
  const int PH = a.PH, SPH = a.SPH;  // phases, spans per phase
  const int npw = 16 * SPH;          // pieces of a row staged at once
  // the workgroup's rows [r0, r1), taken as row quads from r0
  int r0, r1;
  if (a.RR) {
    r0 = (int)((int64_t)blockIdx.x * N / a.P);
    r1 = (int)((int64_t)(blockIdx.x + 1) * N / a.P);
  } else {
    r0 = 4 * (int)((int64_t)blockIdx.x * a.nq / a.P);
    r1 = min(N, 4 * (int)((int64_t)(blockIdx.x + 1) * a.nq / a.P));
  }
  const int nql = (r1 - r0 + 3) >> 2;
  const DecLds L = dec_lds_phased(M, K, a.QW, G, MQ, npw);

  const rsrc_t rx = make_rsrc(a.x, (uint32_t)M * K * 2);
  const rsrc_t rw = make_rsrc(a.w, (uint32_t)N * RB);
  const rsrc_t rs = make_rsrc(a.sc, (uint32_t)N * ng * 2);
  const rsrc_t rb = make_rsrc(a.bi, (uint32_t)N * ng * 2);

  // the wave's items of phase ph, (row quad, span) pairs; returns their count
  // (slots past the last item read nothing)
  auto take_items = [&](int ph, int (&qv)[NI], int (&sv)[NI]) {
    const int s0 = ph * SPH, us = min(U - s0, SPH);
    const int nitems = nql * us;
    const int i0 = (int)((int64_t)wave * nitems / kDecNW);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      qv[i] = (i0 + i) / us;
      sv[i] = s0 + i0 + i - qv[i] * us;
    }
    return (int)((int64_t)(wave + 1) * nitems / kDecNW) - i0;
  };
  auto wload = [&](int q, int s, bool live) {
    const int row = r0 + 4 * q + j;
    return buf_load16(rw, live && row < r1 ? (uint32_t)row * RB + 256 * s + 16 * b : kOob);
  };
  // staged activation pieces of phase ph: pi = m * npw + (piece - 16 * s0)
  const int nxp = M * npw;
  u32x4_t xr[kDecXP][4];
  auto xload = [&](int ph) {
    const int s0 = ph * SPH, us = min(U - s0, SPH);
#pragma unroll
    for (int i = 0; i < kDecXP; ++i) {
      const int pi = tid + i * NT;
      if (i * NT + 64 * wave < nxp) {
        const int m = pi / npw, lp = pi - m * npw;
        const uint32_t off =
            pi < nxp && lp < 16 * us ? 64u * (uint32_t)(m * np + 16 * s0 + lp) : kOob;
#pragma unroll
        for (int w = 0; w < 4; ++w) xr[i][w] = buf_load16(rx, off + 16 * w);
      }
    }
  };

  // 1. the first phase's staging loads, the scales and biases, its weights
  int ql[NI], sp[NI];
  int nmy = take_items(0, ql, sp);
  xload(0);
  const int nsp = (4 * nql * ng) >> 3;
  u32x4_t sr[kDecSP], br[kDecSP];
#pragma unroll
  for (int i = 0; i < kDecSP; ++i) {
    const int pi = tid + i * NT;
    if (i * NT + 64 * wave < nsp) {
      const uint32_t off = pi < nsp ? 2u * (uint32_t)r0 * ng + 16u * pi : kOob;
      sr[i] = buf_load16(rs, off);
      br[i] = buf_load16(rb, off);
    }
  }
  u32x4_t wv[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) wv[i] = wload(ql[i], sp[i], i < nmy);
  __builtin_amdgcn_sched_barrier(0);

  // 2. clear the quad slots; the scales and biases to LDS (once, so that their
  // registers are free before the phase loop)
  {
    float* part = reinterpret_cast<float*>(smem + L.part);
    const int nslot = nql * U * 16 * MQ;
    for (int e = tid; e < nslot; e += NT) part[e] = 0.0f;
    uint32_t* sb = reinterpret_cast<uint32_t*>(smem + L.sb);
#pragma unroll
    for (int i = 0; i < kDecSP; ++i) {
      const int pi = tid + i * NT;
      if (pi < nsp) {
        const u32x4_t s = sr[i], c = br[i];
        u32x4_t lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo[e] = __builtin_amdgcn_perm(c[e], s[e], 0x05040100u);  // (s0, b0)
          hi[e] = __builtin_amdgcn_perm(c[e], s[e], 0x07060302u);  // (s1, b1)
        }
        *reinterpret_cast<u32x4_t*>(sb + 8 * pi) = u32x4_t{lo[0], hi[0], lo[1], hi[1]};
        *reinterpret_cast<u32x4_t*>(sb + 8 * pi + 4) = u32x4_t{lo[2], hi[2], lo[3], hi[3]};
      }
    }
  }

  const DecodeConsts dc = decode_consts<T>();
  const unsigned char* xpc = smem + L.xp;
  const float* xsc = reinterpret_cast<const float*>(smem + L.xs);
  const uint32_t* sb = reinterpret_cast<const uint32_t*>(smem + L.sb);
  float* part = reinterpret_cast<float*>(smem + L.part);
  for (int ph = 0; ph < PH; ++ph) {
    const int s0 = ph * SPH;  // the phase's first span
    // 3. the phase's activations to LDS, with the sums of their pieces
    {
      uint32_t* xp = reinterpret_cast<uint32_t*>(smem + L.xp);
      float* xs = reinterpret_cast<float*>(smem + L.xs);
#pragma unroll
      for (int i = 0; i < kDecXP; ++i) {
        const int pi = tid + i * NT;
        if (pi < nxp) {
          float sum = 0.0f;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const u32x4_t r = xr[i][w];
            const u32x4_t o = {__builtin_amdgcn_perm(r.z, r.x, 0x05040100u),   // (x0, x4)
                               __builtin_amdgcn_perm(r.z, r.x, 0x07060302u),   // (x1, x5)
                               __builtin_amdgcn_perm(r.w, r.y, 0x05040100u),   // (x2, x6)
                               __builtin_amdgcn_perm(r.w, r.y, 0x07060302u)};  // (x3, x7)
            *reinterpret_cast<u32x4_t*>(xp + gemv_xslot(pi, w)) = o;
#pragma unroll
            for (int e = 0; e < 4; ++e) sum = pair_sum<T>(r[e], sum);
          }
          const int m = pi / npw, piece = pi - m * npw;
          xs[piece * MR + m] = sum;
        }
      }
    }
    __syncthreads();

    // the next phase's staging and weight loads go out behind this phase's
    int qn[NI], sn[NI], nn = 0;
    u32x4_t wn[NI];
    const bool more = ph + 1 < PH;
    if (more) {
      nn = take_items(ph + 1, qn, sn);
      xload(ph + 1);
#pragma unroll
      for (int i = 0; i < NI; ++i) wn[i] = wload(qn[i], sn[i], i < nn);
    }

    // 4. the wave's items in order; per-lane sums while the row quad stays
    f32x4_t acc[MQ];
#pragma unroll
    for (int q = 0; q < MQ; ++q) acc[q] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    int first = nmy > 0 ? sp[0] : 0;   // first span of the current run
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      if (i < nmy) {
        const int s = sp[i];
        const int p = 256 * s + 16 * b;
        const bool ok = r0 + 4 * ql[i] + j < r1;
        const int lpc = 16 * (s - s0) + b;   // the piece's place in the staged slab
        const uint32_t pair = ok ? sb[(4 * ql[i] + j) * ng + (2 * p) / G] : 0u;
        const float sf = T::to_f32((uint16_t)(pair & 0xFFFFu));
        const float bf = fmaf(-T::OFFSET, sf, T::to_f32((uint16_t)(pair >> 16)));
        uint32_t pr[4][4];
#pragma unroll
        for (int w = 0; w < 4; ++w) decode_w4_strided<T>(wv[i][w], dc, pr[w]);
#pragma unroll
        for (int q = 0; q < MQ; ++q) {
          const int pi = min(4 * q + j, M - 1) * npw + lpc;
          f32x4_t d0 = {0.0f, 0.0f, 0.0f, 0.0f}, d1 = d0;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xpc + 4 * gemv_xslot(pi, w));
            d0 = mfma4x4<T>(v.x, v.y, pr[w][0], pr[w][1], d0);
            d1 = mfma4x4<T>(v.z, v.w, pr[w][2], pr[w][3], d1);
          }
          const f32x4_t xm = *reinterpret_cast<const f32x4_t*>(xsc + lpc * MR + 4 * q);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float t = fmaf(sf, d0[e] + d1[e], bf * xm[e]);
            acc[q][e] += ok ? t : 0.0f;
          }
        }
        // end of a run: next item in another row quad, or the wave's last
        const bool last = i + 1 >= nmy || (i + 1 < NI && ql[i + 1] != ql[i]);
        if (last) {
          float* dst = part + ((ql[i] * U + first) * 4) * MR;
#pragma unroll
          for (int q = 0; q < MQ; ++q) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float v = sum_blocks(acc[q][e]);
              if (lane < 4) dst[lane * MR + 4 * q + e] = v;
            }
            acc[q] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
          }
          if (i + 1 < NI) first = sp[i + 1];
        }
      }
    }

    if (more) {
      nmy = nn;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        ql[i] = qn[i];
        sp[i] = sn[i];
        wv[i] = wn[i];
      }
      __syncthreads();
    }
  }
  __syncthreads();

  // 5. each output: the sum of its quad's slots in span order
  for (int t = tid; t < 4 * nql * M; t += NT) {
    const int rl = t / M, m = t - rl * M;
    const int row = r0 + rl;
    if (row < r1) {
      const float* src = part + (((rl >> 2) * U) * 4 + (rl & 3)) * MR + m;
      float v = 0.0f;
      for (int s = 0; s < U; ++s) v += src[s * 4 * MR];
      const int64_t idx = (int64_t)m * N + row;
      store_out(a.y, idx, a.res ? add_rounded<T>(v, a.res[idx]) : v, a.y_dtype);
    }
  }
}

// ---------------------------------------------------------------------------
// skinny kernel (M <= MB <= 32)
// ---------------------------------------------------------------------------
// Workgroup = 4 waves; tile = 32 weight rows; the workgroup's K range (a
// split of 4*CPW 64-k chunks) is dealt to the waves round-robin, CPW chunks
// each. The code is straight-line: every wave issues all of its weight and
// scale loads first (unconditionally, so the compiler waits for exactly the
// load each chunk needs), then stages x and the group sums of x into LDS
// behind one barrier, then computes its chunks in order.
// Chunk step: lane (n = l%32, j = l/32) holds 16 bytes = 32 codes of row n at
// k = 64c + 32j, i.e. four MFMA k-slots of 8; the A operand is the matching
// 16 bytes of x row m = l%32 from the LDS slab (rows past M read a zero row).
// Four MFMAs accumulate x.(OFFSET+q); the chunk ends with the fp32 epilogue
// acc += s*T + (b - OFFSET*s)*X over its group(s), X being the group sums.
// Splits of K combine in the same launch: every workgroup writes its fp32
// partial, and the last one to arrive at the tile's counter sums the partials
// in split order (deterministic) and resets the counter to zero.

struct SkinnyArgs {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* sc;
  const uint16_t* bi;
  float* part;          // [S][M][N] fp32 partials (S > 1)
  unsigned* counters;   // [ceil(N/32)] zero on entry, zero on exit (S > 1)
  void* y;
  int y_dtype;
  int M, N, K;
  int cps;              // 64-k chunks per split (4 * CPW)
  int S;
};

template <typename T, int G>
struct ChunkMeta {
  // (s, b) of the group(s) covering chunk c for a lane's row; for G = 32 the
  // low half is group 2c and the high half group 2c+1.
  __device__ static __forceinline__ void load(const uint16_t* srow,
                                              const uint16_t* brow, int c,
                                              uint32_t& s, uint32_t& b) {
    if constexpr (G == 32) {
      s = *reinterpret_cast<const uint32_t*>(srow + 2 * c);
      b = *reinterpret_cast<const uint32_t*>(brow + 2 * c);
    } else if constexpr (G == 64) {
      s = srow[c];
      b = brow[c];
    } else {
      s = srow[c >> 1];
      b = brow[c >> 1];
    }
  }
};

// Rows of the 32x32 output a lane holds for row-bucket MB: accumulators v <
// VM cover rows 8*(v/4) + 4*(l/32) + v%4 < MB (MB = 1 keeps v = 0 only).
template <int MB>
struct RowBucket {
  static constexpr int VM = MB >= 8 ? MB / 2 : 1;
  static constexpr int ROWS = MB >= 8 ? MB : 8;  // group-sum rows kept in LDS
};

template <typename T, int G, int MB, int CPW>
__global__ __launch_bounds__(256, 2) void w4_skinny_kernel(SkinnyArgs a) {
  constexpr int VM = RowBucket<MB>::VM;
  constexpr int XR = RowBucket<MB>::ROWS;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ float red[4][VM][64];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane >> 5;
  const int M = a.M, N = a.N, K = a.K;
  const int n0 = blockIdx.x * 32;
  const int split = blockIdx.y;
  const int nchunks = K >> 6;
  const int c_begin = split * a.cps;
  const int nc = min(a.cps, nchunks - c_begin);
  const int ngroups = K / G;
  // this wave's chunks are wave, wave+4, ...: my_n <= CPW of them (fewer
  // only in a tail split)
  const int my_n = nc > wave ? min(CPW, (nc - wave + 3) >> 2) : 0;

  // LDS: x slab [M+1][nc*64 + 8] (16-bit, row M zero), then the half-chunk
  // (32-k) sums of x [2*nc][XR] fp32 (rows past M zero)
  const int xpitch = nc * 64 + 8;
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  float* xh = reinterpret_cast<float*>(smem + (size_t)(M + 1) * xpitch * 2);

  const int n = n0 + (lane & 31);
  const int nr = n < N ? n : N - 1;
  const uint32_t* wrow = a.w + (int64_t)nr * (K >> 3) + (int64_t)c_begin * 8 + 4 * j;
  const uint16_t* srow = a.sc + (int64_t)nr * ngroups;
  const uint16_t* brow = a.bi + (int64_t)nr * ngroups;

  u32x4_t wv[CPW];
  uint32_t sv[CPW], bv[CPW];
  if (my_n > 0) {
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      // past the wave's last chunk (tail split only) re-read that chunk
      const int cl = wave + 4 * min(i, my_n - 1);
      wv[i] = *reinterpret_cast<const u32x4_t*>(wrow + (int64_t)cl * 8);
      ChunkMeta<T, G>::load(srow, brow, c_begin + cl, sv[i], bv[i]);
    }
  }

  // stage x (plus the zero row) and the half-chunk sums, behind one barrier
  {
    const int ppr = nc * 8;
    for (int p = tid; p < (M + 1) * ppr; p += 256) {
      const int m = p / ppr, pc = p - m * ppr;
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (m < M)
        v = *reinterpret_cast<const u32x4_t*>(a.x + (int64_t)m * K + (int64_t)c_begin * 64 + pc * 8);
      *reinterpret_cast<u32x4_t*>(xs + m * xpitch + pc * 8) = v;
    }
    for (int p = tid; p < 2 * nc * XR; p += 256) {
      const int h = p / XR, m = p - h * XR;
      float sum = 0.0f;
      if (m < M) {
        const u32x4_t* src = reinterpret_cast<const u32x4_t*>(
            a.x + (int64_t)m * K + (int64_t)c_begin * 64 + h * 32);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4_t v = src[q];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            sum += T::to_f32((uint16_t)(v[e] & 0xFFFFu)) + T::to_f32((uint16_t)(v[e] >> 16));
        }
      }
      xh[h * XR + m] = sum;
    }
  }
  __syncthreads();

  float acc[VM];
#pragma unroll
  for (int v = 0; v < VM; ++v) acc[v] = 0.0f;

  const int am = lane & 31;
  const uint16_t* arow = xs + (am < M ? am : M) * xpitch + 32 * j;
  const DecodeConsts dc = decode_consts<T>();
  const u32x4_t zero = {0u, 0u, 0u, 0u};

#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    if (i < my_n) {
      const int cl = wave + 4 * i;
      f32x16_t t0 = {}, t1 = {};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const u32x4_t bq = decode_w4<T>(wv[i][t], dc);
        const u32x4_t av = *reinterpret_cast<const u32x4_t*>(arow + cl * 64 + 8 * t);
        if constexpr (G == 32) {
          t0 = mfma32x32x16<T>(j == 0 ? av : zero, bq, t0);
          t1 = mfma32x32x16<T>(j == 1 ? av : zero, bq, t1);
        } else {
          t0 = mfma32x32x16<T>(av, bq, t0);
        }
      }
      const float s0 = T::to_f32((uint16_t)(sv[i] & 0xFFFFu));
      const float b0 = fmaf(-T::OFFSET, s0, T::to_f32((uint16_t)(bv[i] & 0xFFFFu)));
      // group sums of the rows this lane holds: rows 8*(v/4) + 4*j + v%4
      const float* h0 = xh + (2 * cl) * XR + 4 * j;
      const float* h1 = h0 + XR;
      if constexpr (G == 32) {
        const float s1 = T::to_f32((uint16_t)(sv[i] >> 16));
        const float b1 = fmaf(-T::OFFSET, s1, T::to_f32((uint16_t)(bv[i] >> 16)));
#pragma unroll
        for (int v = 0; v < VM; ++v) {
          const int off = 8 * (v >> 2) + (v & 3);
          float r = fmaf(s0, t0[v], acc[v]);
          r = fmaf(b0, h0[off], r);
          r = fmaf(s1, t1[v], r);
          acc[v] = fmaf(b1, h1[off], r);
        }
      } else {
#pragma unroll
        for (int v = 0; v < VM; ++v) {
          const int off = 8 * (v >> 2) + (v & 3);
          acc[v] = fmaf(b0, h0[off] + h1[off], fmaf(s0, t0[v], acc[v]));
        }
      }
    }
  }

  // cross-wave reduction through LDS
#pragma unroll
  for (int v = 0; v < VM; ++v) red[wave][v][lane] = acc[v];
  __syncthreads();
  for (int e = tid; e < VM * 64; e += 256) {
    const int v = e >> 6, l = e & 63;
    const float s = red[0][v][l] + red[1][v][l] + red[2][v][l] + red[3][v][l];
    const int m = mfma32_row(l, v);
    const int nn = n0 + (l & 31);
    if (m < M && nn < N) {
      if (a.S == 1)
        store_out(a.y, (int64_t)m * N + nn, s, a.y_dtype);
      else
        splitk_store(&a.part[((int64_t)split * M + m) * N + nn], s);
    }
  }
  if (a.S == 1) return;

  // split-K: the last workgroup of this tile sums the partials in split order
  if (!splitk_arrive(&a.counters[blockIdx.x], a.S, &s_last)) return;
  const int64_t MN = (int64_t)M * N;
  for (int e = tid; e < M * 32; e += 256) {
    const int m = e >> 5, nn = n0 + (e & 31);
    if (nn < N) {
      const float s = splitk_sum(a.part + (int64_t)m * N + nn, MN, a.S);
      store_out(a.y, (int64_t)m * N + nn, s, a.y_dtype);
    }
  }
  splitk_reset(&a.counters[blockIdx.x]);
}

// ---------------------------------------------------------------------------
// GEMM (M > 32)
// ---------------------------------------------------------------------------
// group sums X_g[m] in fp32, stored [K/G][M]; one thread per (m, g)
template <typename T>
__global__ __launch_bounds__(256) void xsum_kernel(const uint16_t* __restrict__ x,
                                                   float* __restrict__ xsum,
                                                   int M, int K, int G) {
  const int ng = K / G;
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= (int64_t)M * ng) return;
  const int m = (int)(id / ng), g = (int)(id - (int64_t)m * ng);
  const u32x4_t* src = reinterpret_cast<const u32x4_t*>(x + (int64_t)m * K + (int64_t)g * G);
  float s = 0.0f;
  for (int i = 0; i < G / 8; ++i) {
    const u32x4_t v = src[i];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s += T::to_f32((uint16_t)(v[e] & 0xFFFFu));
      s += T::to_f32((uint16_t)(v[e] >> 16));
    }
  }
  xsum[(int64_t)g * M + m] = s;
}

constexpr int kBM = 128, kBN = 128, kBK = 64;

// element offset of the 16-byte piece (row, kc) in a swizzled [128][64] tile
__device__ __forceinline__ int tile_off(int row, int kc) {
  return row * 64 + ((kc ^ (row & 7)) << 3);
}

// ---------------------------------------------------------------------------
// bf16 prefill GEMM on exact fp16 operands
// ---------------------------------------------------------------------------
// With w = s*q + b = s*(q-8) + b', b' = b + 8s, the affine dot splits into
//   y[m,n] = sum_k x[m,k] * s[n,g(k)]*(q-8)  +  sum_g b'[n,g] * X_g[m]
// (X_g[m] the sum of x[m,:] over group g). Both parts run on the MFMA with
// products that are exact in fp32:
//  * s*(q-8) is a bf16 significand (8 bits) times |q-8| <= 8: at most 11
//    significant bits, exact in fp16. A per-row power of two 2^-es[n] brings
//    max_g |s[n,g]| into [2^10, 2^11), so |s'*(q-8)| and |24*s'| stay finite.
//    Activations scale the same way per row, 2^-ex[m] putting max_k |x[m,k]|
//    into [2^15, 2^16). The fp16 MFMA then accumulates exact products and the
//    epilogue multiplies by 2^(ex[m]+es[n]) (an exponent add). The only
//    rounding this adds is for values below 2^-24 after the shift (fp16
//    subnormals): scales under 2^-27 of their row's largest and activations
//    under 2^-39 of theirs.
//  * the bias part is a GEMM over K2 = 3*K/G "bias slots" on the bf16 MFMA,
//    with both factors split into bf16 pairs so that the three products
//    Xh*bh + Xh*bl + Xl*bh reproduce X*b' to ~2^-17 relative:
//      A2[m][3g .. 3g+2] = (Xh, Xh, Xl),  B2[n][3g .. 3g+2] = (bh, bl, bh),
//    zero-padded to K2p = a multiple of 16 slots.
// Weights decode per uint32 word as dword i = (code i, code i+4) (one shift
// and one and-or under the fp16 1024 pattern, then a packed subtract of 1032
// and a packed multiply by s'); the prologue stores x' with the same
// in-chunk order, dword i = (x[8c+i], x[8c+i+4]), so the MFMA pairs them.
__host__ __device__ __forceinline__ int bias_slots(int K, int G) { return (3 * (K / G) + 15) & ~15; }

struct GemmPrepArgs {
  const uint16_t* x;   // [M][K] bf16
  const uint16_t* sc;  // [N][K/G] bf16
  const uint16_t* bi;  // [N][K/G] bf16
  uint16_t* xh;        // [M][K] fp16, scaled and chunk-permuted
  int* ex;             // [M]
  uint16_t* a2;        // [M][K2p] bf16
  uint16_t* sp;        // [N][K/G] fp16 scaled scales
  int* es;             // [N]
  uint16_t* b2;        // [N][K2p] bf16
  int M, N, K, G, K2p;
  int rw;  // weight rows per block
};

__device__ __forceinline__ void split_bf16(float v, uint16_t& hi, uint16_t& lo) {
  hi = f32_to_bf16(v);
  lo = f32_to_bf16(v - bf16_to_f32(hi));
}

// exponent that brings a positive finite maximum into [2^top, 2^(top+1))
__device__ __forceinline__ int row_shift(float amax, int top) {
  return (amax > 0.0f && amax <= 3.4028235e38f) ? ilogbf(amax) - top : 0;
}

__device__ __forceinline__ float block_max256(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  return v;
}

// Blocks [0, nwb = ceil(N / rw)): rw weight rows each (dispatched first: they
// run longer than a row block); blocks [nwb, nwb + M): one activation row
// each (the conversion pass reads the row again, from L2). In a weight block
// the (scale, bias) pairs are read coalesced into LDS, each row's
// maximum reduced by four threads, and the outputs written coalesced: the
// fp16 scales straight from the pair index, the bias slots through LDS as
// whole 4-byte slot pairs.
// NCH > 0: the activation row's 16-byte chunks (at most 256 * NCH) are all
// loaded at once and kept in registers for the conversion; NCH = 0 loops
// over the row twice (the second pass from L2). NCH is the exact chunk
// count per thread (an out-of-range load still costs an issue). Measured per
// call, prologue and GEMM, against the two passes: QKV 3584x2560 M = 512
// 33.5 -> 32.6 us, down 2560x9728 M = 2048 163 -> 161.5 us, the other shapes
// within 0.5%.
template <int NCH>
__global__ __launch_bounds__(256) void gemm_prep_kernel(GemmPrepArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* red = reinterpret_cast<float*>(smem);
  const int tid = threadIdx.x;
  const int ng = a.K / a.G;
  const int nwb = (a.N + a.rw - 1) / a.rw;  // weight blocks come first
  if ((int)blockIdx.x >= nwb) {
    const int m = blockIdx.x - nwb;
    const u32x4_t* xr = reinterpret_cast<const u32x4_t*>(a.x + (int64_t)m * a.K);
    const int nc = a.K / 8;
    constexpr int NR = NCH > 0 ? NCH : 1;
    u32x4_t xv[NR];
    float amax = 0.0f;
    if constexpr (NCH > 0) {
      // every load unconditional (past the row: the out-of-range offset reads zeros)
      const rsrc_t rx = make_rsrc(a.x + (int64_t)m * a.K, (uint32_t)a.K * 2u);
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int c = tid + 256 * i;
        xv[i] = buf_load16(rx, c < nc ? 16u * (uint32_t)c : kOob);
      }
#pragma unroll
      for (int i = 0; i < NCH; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          amax = fmaxf(amax, fmaxf(fabsf(bf16_to_f32((uint16_t)xv[i][e])),
                                   fabsf(bf16_to_f32((uint16_t)(xv[i][e] >> 16)))));
    } else {
      for (int c = tid; c < nc; c += 256) {
        const u32x4_t v = xr[c];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          amax = fmaxf(amax, fmaxf(fabsf(bf16_to_f32((uint16_t)v[e])),
                                   fabsf(bf16_to_f32((uint16_t)(v[e] >> 16)))));
      }
    }
    const int e = row_shift(block_max256(amax, red), 15);
    if (tid == 0) a.ex[m] = e;
    u32x4_t* dst = reinterpret_cast<u32x4_t*>(a.xh + (int64_t)m * a.K);
    uint16_t* a2 = a.a2 + (int64_t)m * a.K2p;
    const int cpg = a.G / 8;  // chunks per group: 4, 8 or 16 consecutive lanes
    // (256 and nc are multiples of cpg: the lanes of a group are active together)
    auto convert = [&](int c, const u32x4_t v) {
      float f[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[2 * i] = bf16_to_f32((uint16_t)v[i]);
        f[2 * i + 1] = bf16_to_f32((uint16_t)(v[i] >> 16));
      }
      u32x4_t o;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        o[i] = (uint32_t)f32_to_f16(ldexpf(f[i], -e)) |
               ((uint32_t)f32_to_f16(ldexpf(f[i + 4], -e)) << 16);
      dst[c] = o;
      float s = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
      for (int o2 = 1; o2 < cpg; o2 <<= 1) s += __shfl_xor(s, o2);
      if ((c & (cpg - 1)) == 0) {
        const int g = c / cpg;
        uint16_t hi, lo;
        split_bf16(s, hi, lo);
        a2[3 * g] = hi;
        a2[3 * g + 1] = hi;
        a2[3 * g + 2] = lo;
      }
    };
    if constexpr (NCH > 0) {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int c = tid + 256 * i;
        if (c < nc) convert(c, xv[i]);
      }
    } else {
      for (int c = tid; c < nc; c += 256) convert(c, xr[c]);
    }
    for (int sl = 3 * ng + tid; sl < a.K2p; sl += 256) a2[sl] = 0;
    return;
  }
  // weight rows [n0, n0 + nr)
  const int rw = a.rw;
  const int n0 = (int)blockIdx.x * rw;
  const int nr = min(rw, a.N - n0);
  const int nel = nr * ng;
  uint32_t* pair = reinterpret_cast<uint32_t*>(smem + 16);          // [rw * ng] (s | b << 16)
  int* rexp = reinterpret_cast<int*>(pair + rw * ng);               // [rw]
  uint32_t* slots = reinterpret_cast<uint32_t*>(rexp + rw);         // [rw * K2p / 2]
  const rsrc_t rs = make_rsrc(a.sc + (int64_t)n0 * ng, (uint32_t)nel * 2u);
  const rsrc_t rb = make_rsrc(a.bi + (int64_t)n0 * ng, (uint32_t)nel * 2u);
  for (int i0 = 0; i0 < nel; i0 += 4 * 256) {
    uint32_t sv[4], bv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + 256 * u + tid;
      sv[u] = __builtin_amdgcn_raw_buffer_load_b16(rs, i < nel ? 2 * i : (int)kOob, 0, 0);
      bv[u] = __builtin_amdgcn_raw_buffer_load_b16(rb, i < nel ? 2 * i : (int)kOob, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + 256 * u + tid;
      if (i < nel) pair[i] = (sv[u] & 0xFFFFu) | (bv[u] << 16);
    }
  }
  __syncthreads();
  {
    const int r = tid >> 2, part = tid & 3;
    float smax = 0.0f;
    if (r < nr)
      for (int g = part; g < ng; g += 4) smax = fmaxf(smax, fabsf(bf16_to_f32((uint16_t)pair[r * ng + g])));
    smax = fmaxf(smax, __shfl_xor(smax, 1));
    smax = fmaxf(smax, __shfl_xor(smax, 2));
    if (r < nr && part == 0) {
      const int e = row_shift(smax, 10);
      rexp[r] = e;
      a.es[n0 + r] = e;
    }
  }
  // rw <= 64 rows: the four threads of a row are the threads above
  __syncthreads();
  uint16_t* spr = a.sp + (int64_t)n0 * ng;
  uint16_t* sl16 = reinterpret_cast<uint16_t*>(slots);
  const int K2p = a.K2p;
  for (int i = tid; i < nel; i += 256) {
    const int r = i / ng, g = i - r * ng;
    const uint32_t pv = pair[i];
    const float sf = bf16_to_f32((uint16_t)pv);
    spr[i] = f32_to_f16(ldexpf(sf, -rexp[r]));
    uint16_t hi, lo;
    split_bf16(fmaf(8.0f, sf, bf16_to_f32((uint16_t)(pv >> 16))), hi, lo);
    sl16[r * K2p + 3 * g] = hi;
    sl16[r * K2p + 3 * g + 1] = lo;
    sl16[r * K2p + 3 * g + 2] = hi;
  }
  for (int i = tid; i < nr * (K2p - 3 * ng); i += 256) {
    const int r = i / (K2p - 3 * ng);
    sl16[r * K2p + 3 * ng + (i - r * (K2p - 3 * ng))] = 0;
  }
  __syncthreads();
  uint32_t* b2 = reinterpret_cast<uint32_t*>(a.b2 + (int64_t)n0 * K2p);
  for (int i = tid; i < nr * K2p / 2; i += 256) b2[i] = slots[i];
}

// rows per weight block of the prologue (at most 64: four threads per row
// reduce the row maximum; 16 by default) and its LDS bytes: the most rows
// within 32 KB, else one row (rows of up to ~6500 groups fit in 64 KB).
// Measured on the MI355X against one row per wave, the prologue of gate+up
// 19456 x 2560 takes 13.5 -> 10.5 us at M = 512 and 17.7 -> 12.0 us at
// M = 2048; QKV and down (few rows or long activation rows) are unchanged
// within noise, as are 4 and 64 rows per block.
struct PrepPlan {
  int rw;
  size_t lds;
};
static PrepPlan plan_prep(int K, int G) {
  const size_t ng = (size_t)(K / G), row = ng * 4 + 4 + (size_t)bias_slots(K, G) * 2;
  PrepPlan p{};
  for (p.rw = (int)std::min<int64_t>(env_int("SPARKQ_PREP_RW", 16), 64); p.rw > 1; p.rw /= 2)
    if (16 + p.rw * row <= 32768) break;
  p.lds = 16 + p.rw * row;
  return p;
}

struct GemmX16Args {
  const uint16_t* xh;  // [M][K] fp16 from the prologue
  const uint32_t* w;   // [N][K/8]
  const uint16_t* sp;  // [N][K/G] fp16
  const int* ex;       // [M]
  const int* es;       // [N]
  const uint16_t* a2;  // [M][K2p]
  const uint16_t* b2;  // [N][K2p]
  void* y;
  int y_dtype, M, N, K, K2p;
  // work items (a 1-D grid): items [0, full) are whole output tiles, tile t
  // at column block t % tiles_n and row block t / tiles_n; the tiles
  // [full, tiles) are split along k into S pieces each, piece-major (item
  // full + p * (tiles - full) + i is piece p of tile full + i, so the
  // workgroups that run at the same time read the same k range), whose fp32
  // partials and one counter per split tile live in the workspace
  int tiles_n, tiles, full, S;
  int gm;  // tile rows per group of the XCD-grouped tile order (0: row-major)
  float* part;
  unsigned* counters;
};

// Wide variant: a (32*MX) x (64*NWV) tile per workgroup of NWV waves, each
// wave owning 32*MX rows x 64 columns (MX even: the staged output goes in
// halves of 64 rows). Activations go through LDS (shared by the
// waves); each wave loads its own packed weights straight into registers and
// decodes them there. The k order inside a 64-k step is permuted so that one
// 16-byte load per lane covers the whole step: lane half j of sub-step ss
// reads chunk 4j+ss (the A fragments use the same chunk), so a lane's four
// consecutive weight words are its operands of sub-steps 0..3. Every lane
// scales its own words, so any group size works with this order.
//
// Decode, three VALU ops per pair of weights: code q goes to fp16 mantissa
// bits 9..6 under exponent 4, which reads as exactly 16+q, and one packed fma
// (16+q)*s' + (-24*s') = s'*(q-8) is exact (the exact product sum is
// representable, so its single rounding changes nothing). Pair i of a word
// holds codes i and i+4, 16 bits apart, so one shift places both.
//
// LDS rows are 128 bytes; chunk c of row r sits at c ^ ((t ^ (t >> 3)) & 7)
// with t = r mod 32, which keeps any 16 consecutive rows of an aligned block
// at one chunk index on distinct banks, and repeats every 32 rows so that a
// fragment 32*x rows further down is a constant offset away.
__device__ __forceinline__ int atile_off(int row, int kc) {
  const int t = row & 31;
  return row * 64 + ((kc ^ ((t ^ (t >> 3)) & 7)) << 3);
}

__device__ __forceinline__ uint32_t bf16x2_rne(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// PD: 1 = the loads of step s+1 go out during step s, 2 = those of step s+2.
// SCH (schedule variants, PD = 1): bit 0 raises the wave priority over the
// MFMA phase of each step; bit 1 keeps four A slots in LDS, fills slot s+2
// during step s and synchronises the workgroup after every second step only.
template <int G, int NWV, int MX, int PD, int SCH = 0>
__global__ __launch_bounds__(64 * NWV, 2) void w4_gemm_x16w_kernel(GemmX16Args a) {
  constexpr int NT = 64 * NWV;
  constexpr int BM = 32 * MX;                // tile rows: MX 32-row fragments per wave
  constexpr int AL = BM * kBK / 8 / NT;      // 16-byte A pieces per thread per step
  constexpr bool PRIO = (SCH & 1) != 0;
  constexpr bool BAR2 = (SCH & 2) != 0 && PD == 1;
  constexpr int NSLOT = BAR2 ? 4 : 2;
  // the A slots, at least 8 KB per wave for the staged bf16 output
  constexpr int AS = NSLOT * BM * kBK > NWV * 64 * 64 ? NSLOT * BM * kBK : NWV * 64 * 64;
  __shared__ __attribute__((aligned(16))) uint16_t As[AS];

  const int tid = threadIdx.x, lane = tid & 63;
  // wave-uniform, so that the per-wave buffer descriptors live in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane >> 5, l32 = lane & 31;
  const int K = a.K, ng = K / G;
  // work item -> (tile, piece) and this workgroup's 64-k steps [s_begin, nsteps)
  const int item = blockIdx.x;
  const bool split = item >= a.full;
  const int nsplit = a.tiles - a.full;
  const int tile = split ? a.full + (item - a.full) % nsplit : item;
  const int piece = split ? (item - a.full) / nsplit : 0;
  const int S = split ? a.S : 1;
  int tm = tile / a.tiles_n, tn = tile - tm * a.tiles_n;
  if (a.gm > 0) {
    // XCD-contiguous chunks of the tile order (work item i runs on XCD i % 8),
    // each walking groups of gm tile rows column by column
    const int T = a.tiles;
    const int v = (T & 7) == 0 ? (tile & 7) * (T >> 3) + (tile >> 3) : tile;
    const int tiles_m = T / a.tiles_n, width = a.gm * a.tiles_n;
    const int g = v / width, fm = g * a.gm, gs = min(tiles_m - fm, a.gm), r = v - g * width;
    tm = fm + r % gs;
    tn = r / gs;
  }
  const int n0 = tn * (64 * NWV), m0 = tm * BM;
  const int s_begin = (int)((int64_t)piece * (K / kBK) / S);
  const int nsteps = (int)((int64_t)(piece + 1) * (K / kBK) / S);
  const int mrows = min(BM, a.M - m0);
  const int wn0 = n0 + 64 * wave;  // this wave's first column
  const int nrows = __builtin_amdgcn_readfirstlane(max(0, min(64, a.N - wn0)));
  // rows past the tile's last one read as zero
  const rsrc_t rx = make_rsrc(a.xh + (int64_t)m0 * K, (uint32_t)mrows * (uint32_t)K * 2u);
  const rsrc_t rw = make_rsrc(a.w + (int64_t)wn0 * (K / 8), (uint32_t)nrows * (uint32_t)K / 2u);
  const rsrc_t rs = make_rsrc(a.sp + (int64_t)wn0 * ng, (uint32_t)(nrows * ng) * 2u);
  const uint32_t mask = vgpr_const(0x03C003C0u), magic = vgpr_const(0x4C004C00u);

  // loop-invariant per-lane offsets; the k offset of a step is a scalar
  uint32_t xoff[AL], lds_w[AL];
#pragma unroll
  for (int i = 0; i < AL; ++i) {
    const int p = tid + NT * i, row = p >> 3, kc = p & 7;
    xoff[i] = (uint32_t)(row * K + kc * 8) * 2u;
    lds_w[i] = (uint32_t)atile_off(row, kc) * 2u;
  }
  uint32_t woff[2], soff[2], lds_r[4];
#pragma unroll
  for (int y = 0; y < 2; ++y) {
    const int col = 32 * y + l32;
    woff[y] = (uint32_t)(col * (K / 2) + 16 * j);
    soff[y] = (uint32_t)(col * ng + (G == 32 ? j : 0)) * 2u;
  }
#pragma unroll
  for (int ss = 0; ss < 4; ++ss) lds_r[ss] = (uint32_t)atile_off(l32, 4 * j + ss) * 2u;

  // PD register sets of one step's loads. With two, the loads of step s+2
  // go out at the start of step s into the set step s has just taken its
  // operands from, on every path (past the last step at an out-of-range
  // offset, which reads zeros), so the wait counts stay exact across the loop.
  constexpr int NW = PD, NA = PD;
  u32x4_t ra[NA][AL], rb[NW][2];
  uint32_t rsv[NW][2];
  auto load_a = [&](int step, int set) {
    const bool live = PD == 1 || step < nsteps;
    const int k0 = live ? step * kBK : 0;
#pragma unroll
    for (int i = 0; i < AL; ++i)
      ra[set][i] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(live ? xoff[i] : kOob), 2 * k0, 0));
  };
  // set 0 at step's offset, or the out-of-range offset (zeros) when not live
  auto load_a_at = [&](int step, bool live) {
    const int k0 = live ? step * kBK : 0;
#pragma unroll
    for (int i = 0; i < AL; ++i)
      ra[0][i] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(live ? xoff[i] : kOob), 2 * k0, 0));
  };
  auto load_w = [&](int step, int set) {
    const bool live = (PD == 1 && !BAR2) || step < nsteps;
    const int k0 = live ? step * kBK : 0;
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      rb[set][y] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(live ? woff[y] : kOob), k0 / 2, 0));
      rsv[set][y] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)(live ? soff[y] : kOob), 2 * (k0 / G), 0);
    }
  };
  auto lds_at = [&](uint32_t byte_off) -> u32x4_t* {
    return reinterpret_cast<u32x4_t*>(reinterpret_cast<unsigned char*>(As) + byte_off);
  };

  f32x16_t acc[MX][2];
#pragma unroll
  for (int x = 0; x < MX; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) acc[x][y] = f32x16_t{};

  auto body = [&](int step, auto stc) {
    constexpr int st = decltype(stc)::value;
    constexpr int rs0 = NW == 1 ? 0 : (st & 1);  // weight set holding this step
    // nothing of a step moves into the one before (it would wait there for
    // the loads still in flight)
    if constexpr (PD > 1) __builtin_amdgcn_sched_barrier(0);
    const u32x4_t wb0 = rb[rs0][0], wb1 = rb[rs0][1];
    const f16x2_t s0 = __builtin_bit_cast(f16x2_t, rsv[rs0][0] * 0x10001u);
    const f16x2_t s1 = __builtin_bit_cast(f16x2_t, rsv[rs0][1] * 0x10001u);
    const f16x2_t c0 = s0 * f16x2_t{(_Float16)-24.0f, (_Float16)-24.0f};
    const f16x2_t c1 = s1 * f16x2_t{(_Float16)-24.0f, (_Float16)-24.0f};
    if constexpr (BAR2) {
      // A two steps ahead, the weights one; past the end the loads read the
      // out-of-range offset (zeros), so no branch splits the wait counts
      load_a_at(step + 2, step + 2 < nsteps);
      load_w(step + 1, 0);
    } else if constexpr (PD == 1) {
      if (step + 1 < nsteps) {
        load_a(step + 1, 0);
        load_w(step + 1, 0);
      }
    } else {
      load_a(step + 2, st);
      load_w(step + 2, st);
    }
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ss = 0; ss < 4; ++ss) {
      u32x4_t bf0, bf1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int sh = 6 - 4 * i;
        const uint32_t t0 = ((sh >= 0 ? wb0[ss] << sh : wb0[ss] >> -sh) & mask) | magic;
        const uint32_t t1 = ((sh >= 0 ? wb1[ss] << sh : wb1[ss] >> -sh) & mask) | magic;
        bf0[i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2_t, t0), s0, c0));
        bf1[i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2_t, t1), s1, c1));
      }
#pragma unroll
      for (int x = 0; x < MX; ++x) {
        const u32x4_t af = *lds_at(lds_r[ss] + (uint32_t)(st * BM * kBK * 2 + x * 32 * 128));
        acc[x][0] = mfma32x32x16<F16>(af, bf0, acc[x][0]);
        acc[x][1] = mfma32x32x16<F16>(af, bf1, acc[x][1]);
      }
    }
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    if constexpr (BAR2) {
      if (step + 2 < nsteps) {
#pragma unroll
        for (int i = 0; i < AL; ++i) *lds_at(lds_w[i] + (uint32_t)(((st + 2) & 3) * BM * kBK * 2)) = ra[0][i];
      }
      // slot s+2 is refilled at the end of step s, after the barrier that
      // followed every wave's reads of step s-2; it is read in step s+2,
      // after the barrier that ends step s or s+1
      if constexpr ((st & 1) == 1) __syncthreads();
    } else {
      if (step + 1 < nsteps) {
        constexpr int rs1 = NA == 1 ? 0 : st ^ 1;  // activation set holding the next step
#pragma unroll
        for (int i = 0; i < AL; ++i) *lds_at(lds_w[i] + (uint32_t)((st ^ 1) * BM * kBK * 2)) = ra[rs1][i];
      }
      __syncthreads();
    }
  };

  if constexpr (BAR2) {
    // slots 0 and 1 hold the first two steps; the loop starts on slot 0
    load_a_at(s_begin, true);
    load_w(s_begin, 0);
#pragma unroll
    for (int i = 0; i < AL; ++i) *lds_at(lds_w[i]) = ra[0][i];
    load_a_at(s_begin + 1, s_begin + 1 < nsteps);
#pragma unroll
    for (int i = 0; i < AL; ++i) *lds_at(lds_w[i] + (uint32_t)(BM * kBK * 2)) = ra[0][i];
    __syncthreads();
    int step = s_begin;
    for (; step + 4 <= nsteps; step += 4) {
      body(step, std::integral_constant<int, 0>{});
      body(step + 1, std::integral_constant<int, 1>{});
      body(step + 2, std::integral_constant<int, 2>{});
      body(step + 3, std::integral_constant<int, 3>{});
    }
    if (step < nsteps) body(step, std::integral_constant<int, 0>{});
    if (step + 1 < nsteps) body(step + 1, std::integral_constant<int, 1>{});
    if (step + 2 < nsteps) body(step + 2, std::integral_constant<int, 2>{});
    __syncthreads();  // every wave is past its last A read before the output staging
  } else {
  load_a(s_begin, 0);
  load_w(s_begin, 0);
  if constexpr (PD > 1) {
    __builtin_amdgcn_sched_barrier(0);  // the sets go out in step order
    load_a(s_begin + 1, 1);
    load_w(s_begin + 1, 1);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int i = 0; i < AL; ++i) *lds_at(lds_w[i]) = ra[0][i];
  __syncthreads();
  if constexpr (PD == 1) {
    for (int step = s_begin; step < nsteps; step += 2) {
      body(step, std::integral_constant<int, 0>{});
      if (step + 1 < nsteps) body(step + 1, std::integral_constant<int, 1>{});
    }
  } else {
    // pairs of steps with no branch around the loads, then an odd last step
    int step = s_begin;
    for (; step + 2 <= nsteps; step += 2) {
      body(step, std::integral_constant<int, 0>{});
      body(step + 1, std::integral_constant<int, 1>{});
    }
    if (step < nsteps) body(step, std::integral_constant<int, 0>{});
  }
  }

  if (split) {
    // every piece stores its raw tile (16-byte stores through to the
    // device-coherent level, sc1, like the split-K atomics); the last to
    // arrive adds the pieces in piece order (deterministic; its own from
    // registers), resets the counter and finishes the tile. A lane's
    // accumulator chunk c (16 bytes) sits at (c * NT + tid) * 16, so each
    // store and load instruction moves 1 KB per wave.
    const int stile = tile - a.full;
    constexpr uint32_t PB = MX * 2 * 16 * 4 * NT;  // bytes per piece
    const rsrc_t rp = make_rsrc(a.part + (size_t)stile * S * (PB / 4), (uint32_t)S * PB);
#pragma unroll
    for (int x = 0; x < MX; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4_t v = {__float_as_uint(acc[x][y][4 * q]), __float_as_uint(acc[x][y][4 * q + 1]),
                             __float_as_uint(acc[x][y][4 * q + 2]), __float_as_uint(acc[x][y][4 * q + 3])};
          __builtin_amdgcn_raw_buffer_store_b128(v, rp, (uint32_t)tid * 16u,
                                                 piece * PB + ((x * 2 + y) * 4 + q) * NT * 16, 16);
        }
    __shared__ int s_last;
    if (!splitk_arrive(a.counters + stile, S, &s_last)) return;
#pragma unroll
    for (int xy = 0; xy < 2 * MX; ++xy) {
      f32x16_t t = f32x16_t{};
      for (int z = 0; z < S; ++z) {
        if (z == piece) {
          t += acc[xy >> 1][xy & 1];
          continue;
        }
        u32x4_t v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
          v[c] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                 rp, (uint32_t)tid * 16u, z * PB + (xy * 4 + c) * NT * 16, 16));
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e) t[4 * c + e] += __uint_as_float(v[c][e]);
      }
      acc[xy >> 1][xy & 1] = t;
    }
    splitk_reset(a.counters + stile);
  }

  // undo the row shifts: y = 2^(ex[m] + es[n]) * acc
  const rsrc_t rex = make_rsrc(a.ex + m0, (uint32_t)mrows * 4u);
  const rsrc_t res = make_rsrc(a.es + wn0, (uint32_t)nrows * 4u);
#pragma unroll
  for (int y = 0; y < 2; ++y) {
    const int esn = (int)__builtin_amdgcn_raw_buffer_load_b32(res, (32 * y + l32) * 4, 0, 0);
#pragma unroll
    for (int x = 0; x < MX; ++x)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const u32x4_t e4 = buf_load16(rex, (uint32_t)(x * 32 + 8 * q4 + 4 * j) * 4u);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[x][y][4 * q4 + r] = ldexpf(acc[x][y][4 * q4 + r], (int)e4[r] + esn);
      }
  }
  // bias slots: acc += A2 * B2^T on the bf16 MFMA
  const int K2p = a.K2p;
  const rsrc_t ra2 = make_rsrc(a.a2 + (int64_t)m0 * K2p, (uint32_t)mrows * (uint32_t)K2p * 2u);
  const rsrc_t rb2 = make_rsrc(a.b2 + (int64_t)wn0 * K2p, (uint32_t)nrows * (uint32_t)K2p * 2u);
  for (int ks = 0; ks < K2p; ks += 16) {
    u32x4_t bf[2];
#pragma unroll
    for (int y = 0; y < 2; ++y)
      bf[y] = buf_load16(rb2, (uint32_t)((32 * y + l32) * K2p + ks + 8 * j) * 2u);
#pragma unroll
    for (int x = 0; x < MX; ++x) {
      const u32x4_t af = buf_load16(ra2, (uint32_t)((32 * x + l32) * K2p + ks + 8 * j) * 2u);
      acc[x][0] = mfma32x32x16<BF16>(af, bf[0], acc[x][0]);
      acc[x][1] = mfma32x32x16<BF16>(af, bf[1], acc[x][1]);
    }
  }

  const int gn0 = wn0 + l32;
  if (a.y_dtype == SPARKQ_BF16 && a.N % 8 == 0 && ((uintptr_t)a.y & 15) == 0) {
    // bf16 output through LDS (the A buffers are idle after the main loop's
    // closing barrier): in halves of 64 rows, each wave writes its 64 x 64
    // piece into its own 8 KB of LDS and stores whole 16-byte row segments,
    // 1 KB per wave instruction, instead of one 2-byte value per lane (a
    // wave's LDS stores and loads are performed in order)
    unsigned char* ot = reinterpret_cast<unsigned char*>(As) + wave * 8192;
    uint16_t* yb = reinterpret_cast<uint16_t*>(a.y);
#pragma unroll
    for (int h = 0; h < MX / 2; ++h) {
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            *reinterpret_cast<uint16_t*>(ot + (32 * x + mfma32_row(lane, v)) * 128 + (32 * y + l32) * 2) =
                (uint16_t)bf16x2_rne(acc[2 * h + x][y][v], 0.0f);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int pc = lane + 64 * i, row = pc >> 3, seg = pc & 7;
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ot + row * 128 + seg * 16);
        const int gm = m0 + 64 * h + row, gn = wn0 + 8 * seg;
        if (gm < a.M && gn < a.N) *reinterpret_cast<u32x4_t*>(yb + (int64_t)gm * a.N + gn) = v;
      }
    }
    return;
  }
#pragma unroll
  for (int x = 0; x < MX; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int gn = gn0 + 32 * y;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int gm = m0 + 32 * x + mfma32_row(lane, v);
        if (gm < a.M && gn < a.N) {
          const int64_t idx = (int64_t)gm * a.N + gn;
          if (a.y_dtype == SPARKQ_BF16)
            reinterpret_cast<uint16_t*>(a.y)[idx] = (uint16_t)bf16x2_rne(acc[x][y][v], 0.0f);
          else
            store_out(a.y, idx, acc[x][y][v], a.y_dtype);
        }
      }
    }
}

template <typename T, int G>
__global__ __launch_bounds__(256, 2) void w4_gemm_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ sc, const uint16_t* __restrict__ bi,
    const float* __restrict__ xsum, void* __restrict__ y, int y_dtype, int M,
    int N, int K) {
  constexpr int GPS = G == 32 ? 2 : 1;  // groups starting inside one k-step
  __shared__ __attribute__((aligned(16))) uint16_t As[2][kBM * kBK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][kBN * kBK];
  __shared__ __attribute__((aligned(16))) float SBs[2][GPS][kBN][2];
  __shared__ __attribute__((aligned(16))) float XSs[2][GPS][kBM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane >> 5;
  const int wm = wave & 1, wn = wave >> 1;
  const int n0 = blockIdx.x * kBN, m0 = blockIdx.y * kBM;
  const int ngroups = K / G;
  const int nsteps = K / kBK;

  const DecodeConsts dc = decode_consts<T>();
  // global -> register staging
  u32x4_t ra[4], rb;
  float rs = 0.0f, rbias = 0.0f, rx = 0.0f;

  auto load = [&](int step) {
    const int k0 = step * kBK;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = tid + 256 * i, row = p >> 3, kc = p & 7;
      const int gm = m0 + row;
      ra[i] = u32x4_t{0u, 0u, 0u, 0u};
      if (gm < M) ra[i] = *reinterpret_cast<const u32x4_t*>(x + (int64_t)gm * K + k0 + kc * 8);
    }
    {
      const int row = tid >> 1, half = tid & 1, gn = n0 + row;
      rb = u32x4_t{0u, 0u, 0u, 0u};
      if (gn < N) rb = *reinterpret_cast<const u32x4_t*>(w + (int64_t)gn * (K >> 3) + (k0 >> 3) + 4 * half);
    }
    if (tid < 128 * GPS) {
      const int gi = tid >> 7, row = tid & 127;
      const int g = (G == 32) ? 2 * step + gi : (k0 / G);
      const int gn = n0 + row, gm = m0 + row;
      rs = 0.0f;
      rbias = 0.0f;
      rx = 0.0f;
      if (gn < N) {
        rs = T::to_f32(sc[(int64_t)gn * ngroups + g]);
        rbias = T::to_f32(bi[(int64_t)gn * ngroups + g]);
      }
      if (gm < M) rx = xsum[(int64_t)g * M + gm];
    }
  };
  auto store = [&](int st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = tid + 256 * i, row = p >> 3, kc = p & 7;
      *reinterpret_cast<u32x4_t*>(&As[st][tile_off(row, kc)]) = ra[i];
    }
    {
      const int row = tid >> 1, half = tid & 1;
#pragma unroll
      for (int wi = 0; wi < 4; ++wi)
        *reinterpret_cast<u32x4_t*>(&Bs[st][tile_off(row, 4 * half + wi)]) = decode_w4<T>(rb[wi], dc);
    }
    if (tid < 128 * GPS) {
      const int gi = tid >> 7, row = tid & 127;
      SBs[st][gi][row][0] = rs;
      SBs[st][gi][row][1] = fmaf(-T::OFFSET, rs, rbias);
      XSs[st][gi][row] = rx;
    }
  };

  f32x16_t acc[2][2], tmp[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      acc[a][b] = f32x16_t{};
      tmp[a][b] = f32x16_t{};
    }

  load(0);
  store(0);
  __syncthreads();

  for (int step = 0; step < nsteps; ++step) {
    const int st = step & 1;
    if (step + 1 < nsteps) load(step + 1);
#pragma unroll
    for (int ss = 0; ss < 4; ++ss) {
      const int kc = 2 * ss + j;
      u32x4_t af[2], bf[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int ar = wm * 64 + t * 32 + (lane & 31);
        const int br = wn * 64 + t * 32 + (lane & 31);
        af[t] = *reinterpret_cast<const u32x4_t*>(&As[st][tile_off(ar, kc)]);
        bf[t] = *reinterpret_cast<const u32x4_t*>(&Bs[st][tile_off(br, kc)]);
      }
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) tmp[a][b] = mfma32x32x16<T>(af[a], bf[b], tmp[a][b]);

      const bool group_end =
          (G == 32) ? (ss == 1 || ss == 3) : (G == 64 ? ss == 3 : (ss == 3 && (step & 1)));
      if (group_end) {
        const int gi = (G == 32) ? (ss >> 1) : 0;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const int br = wn * 64 + b * 32 + (lane & 31);
          const float s = SBs[st][gi][br][0], bp = SBs[st][gi][br][1];
#pragma unroll
          for (int a = 0; a < 2; ++a) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
              const int mr = wm * 64 + a * 32 + 8 * q4 + 4 * j;
              const f32x4_t xv = *reinterpret_cast<const f32x4_t*>(&XSs[st][gi][mr]);
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int v = 4 * q4 + r;
                const float t = fmaf(s, tmp[a][b][v], acc[a][b][v]);
                acc[a][b][v] = fmaf(bp, xv[r], t);
              }
            }
            tmp[a][b] = f32x16_t{};
          }
        }
      }
    }
    if (step + 1 < nsteps) store(st ^ 1);
    __syncthreads();
  }

  // epilogue
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int gn = n0 + wn * 64 + b * 32 + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int gm = m0 + wm * 64 + a * 32 + mfma32_row(lane, v);
        if (gm < M && gn < N) store_out(y, (int64_t)gm * N + gn, acc[a][b][v], y_dtype);
      }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct SkinnyPlan {
  int MB;      // row bucket: 1, 8, 16 or 32
  int CPW;     // chunks per wave: 1, 2, 4, 5 or 8
  int S;       // workgroup splits of K
  int cps;     // 64-k chunks per split (4 * CPW)
  size_t lds;  // dynamic LDS: the x slab and its group sums
  size_t part_bytes;
};

// Workgroups aimed at per launch; SPARKQ_W4_TARGET_WGS overrides it and
// SPARKQ_W4_CPW forces the chunks per wave, both for tuning.
static SkinnyPlan plan_skinny(int64_t M, int64_t N, int64_t K) {
  static const int kCpw[] = {1, 2, 4, 5, 8};
  SkinnyPlan p;
  p.MB = M == 1 ? 1 : (M <= 8 ? 8 : (M <= 16 ? 16 : 32));
  const int64_t tiles = cdiv(N, 32);
  const int64_t nchunks = K / 64;
  const int64_t target = env_int("SPARKQ_W4_TARGET_WGS", 1024);
  const int64_t forced = env_int("SPARKQ_W4_CPW", 0);
  const int64_t xr = M >= 8 ? (M <= 16 ? 16 : 32) : 8;
  double best = 1e30;
  p.CPW = 1;
  for (int cpw : kCpw) {
    if (forced && cpw != forced) continue;
    const int64_t cps = 4 * (int64_t)cpw;
    // x slab (M rows + a zero row) and the sums in LDS <= 40 KB
    const size_t lds = (size_t)(M + 1) * (cps * 64 + 8) * 2 + (size_t)2 * cps * xr * 4;
    if (lds > 40960 && !forced) continue;
    const int64_t S = cdiv(nchunks, cps);
    if (S > 1 && tiles > kMaxCounterTiles) continue;
    const int64_t wgs = tiles * S;
    // distance from the target workgroup count, plus idle slots of a tail
    const int64_t tail = S * cps - nchunks;
    const double cost = std::fabs(std::log((double)wgs / (double)target)) +
                        (double)tail / (double)(S * cps);
    if (cost < best) {
      best = cost;
      p.CPW = cpw;
    }
  }
  p.cps = 4 * p.CPW;
  p.S = (int)cdiv(nchunks, p.cps);
  p.lds = (size_t)(M + 1) * (p.cps * 64 + 8) * 2 + (size_t)2 * p.cps * xr * 4;
  p.part_bytes = p.S > 1 ? round_up((size_t)p.S * M * N * 4, 256) : 0;
  return p;
}

// Decode GEMV plan. A row has U = ceil(K/512) spans; a wave keeps at most 5
// spans of activations in registers, so rows of up to 20 spans (K <= 10240)
// split into SG = 1, 2 or 4 span groups. Workgroups of 4 waves (8 when the
// activations need the larger staging budget) cover R = 4 * (waves / SG) *
// RQW rows; two row quads per wave (M = 1 only) once that still leaves
// >= 2048 waves. The staged activations, (scale, bias)
// pieces and LDS must fit the kernel's fixed budgets, and the scale tensors
// must end on a 16-byte boundary (they are staged in 16-byte loads).
struct GemvPlan {
  bool ok;
  int SG, USr, US, RQW, MQ, NW, R;
  size_t lds;
  int64_t wgs;
};

static GemvPlan plan_gemv(int64_t M, int64_t N, int64_t K, int G) {
  GemvPlan p{};
  if (M > 4 || env_int("SPARKQ_W4_NO_GEMV", 0)) return p;
  // every tensor must stay below the out-of-range offset of the buffer loads
  if (N * (K / 2) >= (int64_t)kOob || M * K * 2 >= (int64_t)kOob) return p;
  const int64_t ng = K / G;
  if ((N * ng * 2) % 16 != 0) return p;
  const int64_t U = cdiv(K / 2, 256);
  if (U <= 5)
    p.SG = 1;
  else if (U <= 10)
    p.SG = 2;
  else if (U <= 20)
    p.SG = 4;
  else
    return p;
  p.USr = (int)cdiv(U, p.SG);
  p.US = p.USr <= 1 ? 1 : (p.USr <= 2 ? 2 : 5);
  // 4 waves: three workgroups fit a CU, so the whole grid is resident at
  // once (8-wave workgroups fit one per CU and ran long rows in two rounds);
  // 8 only when the activations need the larger staging budget
  p.NW = M * (K / 32) > kGemvXP * 256 ? 8 : 4;
  if (env_int("SPARKQ_W4_GEMV_NW", 0)) p.NW = env_int("SPARKQ_W4_GEMV_NW", 4) == 8 ? 8 : 4;
  const int64_t nq = cdiv(N, 4);
  // two row quads per wave only at M = 1: with four activation rows the
  // second quad's registers spill at three waves per SIMD (measured: gate+up
  // at M = 4 takes 15.4 us with two, 11.1 us with one)
  p.RQW = M == 1 && cdiv(nq, 2) * p.SG >= 2048 ? 2 : 1;
  if (env_int("SPARKQ_W4_GEMV_RQW", 0)) p.RQW = env_int("SPARKQ_W4_GEMV_RQW", 1) == 2 ? 2 : 1;
  p.MQ = M == 1 ? 1 : 4;
  p.R = 4 * (p.NW / p.SG) * p.RQW;
  const int64_t nt = 64 * p.NW;
  if (M * (K / 32) > kGemvXP * nt || p.R * ng / 8 > kGemvSP * nt) return p;
  const GemvLds l = gemv_lds((int)M, (int)K, p.R, G, p.NW, p.RQW);
  if (l.bytes > 65536) return p;
  p.lds = (size_t)l.bytes;
  p.wgs = cdiv(N, p.R);
  p.ok = true;
  return p;
}

template <typename T, int G, int MQ, int US, int RQW, int NW, int F = kPlain>
static void launch_gemv_w(const GemvPlan& p, const GemvArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((w4_gemv_kernel<T, G, MQ, US, RQW, NW, F>), dim3((unsigned)p.wgs),
                     dim3(64 * NW), p.lds, st, a);
}
template <typename T, int G, int MQ, int US, int RQW>
static void launch_gemv_r(const GemvPlan& p, const GemvArgs& a, hipStream_t st) {
  if (p.NW == 4)
    launch_gemv_w<T, G, MQ, US, RQW, 4>(p, a, st);
  else
    launch_gemv_w<T, G, MQ, US, RQW, 8>(p, a, st);
}
template <typename T, int G, int MQ, int US>
static void launch_gemv_u(const GemvPlan& p, const GemvArgs& a, hipStream_t st) {
  if (p.RQW == 1)
    launch_gemv_r<T, G, MQ, US, 1>(p, a, st);
  else
    launch_gemv_r<T, G, MQ, US, 2>(p, a, st);
}
template <typename T, int G, int MQ>
static void launch_gemv_m(const GemvPlan& p, const GemvArgs& a, hipStream_t st) {
  if (p.US == 1)
    launch_gemv_u<T, G, MQ, 1>(p, a, st);
  else if (p.US == 2)
    launch_gemv_u<T, G, MQ, 2>(p, a, st);
  else
    launch_gemv_u<T, G, MQ, 5>(p, a, st);
}
template <typename T, int G>
static void launch_gemv_g(const GemvPlan& p, const GemvArgs& a, hipStream_t st) {
  if (p.MQ == 1)
    launch_gemv_m<T, G, 1>(p, a, st);
  else
    launch_gemv_m<T, G, 4>(p, a, st);
}
template <typename T>
static void launch_gemv(const GemvPlan& p, int G, const GemvArgs& a, hipStream_t st) {
  if (G == 32)
    launch_gemv_g<T, 32>(p, a, st);
  else if (G == 64)
    launch_gemv_g<T, 64>(p, a, st);
  else
    launch_gemv_g<T, 128>(p, a, st);
}

// Plan of a fused GEMV (w4_gemv_kernel with FUSE != kPlain) over NV
// virtual rows: the plain plan, with rows of 3 or more spans per wave (US 5,
// every K >= 1536 up to the plain limit), an even number of groups per row
// (scale pieces are staged per row quad), and workgroups of whole virtual
// quad pairs (R % 8 == 0; eight waves when four would give R = 4).
static GemvPlan plan_fused(int64_t M, int64_t NV, int64_t K, int G, int fuse) {
  GemvPlan p = plan_gemv(M, NV, K, G);
  const GemvPlan bad{};
  if (!p.ok || p.US != 5 || (K / G) % 2 != 0 || NV % 8 != 0) return bad;
  if (p.R % 8 != 0) {
    p.NW = 8;
    p.R = 4 * (p.NW / p.SG) * p.RQW;
    if (p.R % 8 != 0) return bad;
  }
  const int xc = p.MQ == 1 ? kFfnXC1 : kFfnXC4;
  if (fuse == kFfnGateUp && M * (K / 8) > xc * 64 * p.NW && p.NW == 4 && p.SG == 1) {
    p.NW = 8;  // more threads for the prologue's chunks
    p.R = 4 * (p.NW / p.SG) * p.RQW;
  }
  const int64_t nt = 64 * p.NW, ng = K / G;
  if (fuse == kFfnGateUp && M * (K / 8) > xc * nt) return bad;
  // scale staging: one lane per 16-byte piece of a quad, two quads per wave
  if (ng / 2 > 64 || p.R / 4 > 2 * p.NW) return bad;
  if (M * (K / 32) > kGemvXP * nt || p.R * ng / 8 > kGemvSP * nt) return bad;
  const GemvLds l = gemv_lds((int)M, (int)K, p.R, G, p.NW, p.RQW, fuse == kFfnGateUp);
  if (l.bytes > 65536) return bad;
  p.lds = (size_t)l.bytes;
  p.wgs = cdiv(NV, p.R);
  return p;
}

template <typename T, int G, int MQ, int F>
static void launch_fused_g(const GemvPlan& p, const GemvArgs& a, hipStream_t st) {
  // two row quads per wave only at one activation row (plan_gemv)
  if (MQ > 1 || p.RQW == 1) {
    if (p.NW == 4)
      launch_gemv_w<T, G, MQ, 5, 1, 4, F>(p, a, st);
    else
      launch_gemv_w<T, G, MQ, 5, 1, 8, F>(p, a, st);
  } else if constexpr (MQ == 1) {
    if (p.NW == 4)
      launch_gemv_w<T, G, MQ, 5, 2, 4, F>(p, a, st);
    else
      launch_gemv_w<T, G, MQ, 5, 2, 8, F>(p, a, st);
  }
}
template <typename T, int MQ, int F>
static void launch_fused(const GemvPlan& p, int G, const GemvArgs& a, hipStream_t st) {
  if (G == 32)
    launch_fused_g<T, 32, MQ, F>(p, a, st);
  else if (G == 64)
    launch_fused_g<T, 64, MQ, F>(p, a, st);
  else
    launch_fused_g<T, 128, MQ, F>(p, a, st);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Residual add, RMSNorm and the gate/up projections of the FFN with
// gelu(gate) * up in one launch, for M <= 4 rows (spark_mlx_llm/ops/ffn.py:
// 98-102). Writes act [M][I]; workgroup 0 also writes hidden = x + xres and
// the normed rows [M][K] when those pointers are given. Returns 1 when no
// fused plan serves the shape (the caller composes the steps instead).
int w4_ffn_gate_up(const void* x, const void* xres, const void* nw, float eps,
                   const uint32_t* wg, const void* sg, const void* bg, const uint32_t* wu,
                   const void* su, const void* bu, void* act, void* hid, void* nrm, int64_t M,
                   int64_t K, int64_t I, int G, int dt, hipStream_t st) {
  if (M < 1 || M > 4 || env_int("SPARKQ_NO_FUSED_FFN", 0)) return 1;
  if (!aligned16(sg) || !aligned16(bg) || !aligned16(su) || !aligned16(bu)) return 1;
  if (I * (K / 2) >= (int64_t)kOob) return 1;
  const GemvPlan p = plan_fused(M, 2 * I, K, G, kFfnGateUp);
  if (!p.ok) return 1;
  GemvArgs a{};
  a.x = (const uint16_t*)x;
  a.w = wg;
  a.sc = (const uint16_t*)sg;
  a.bi = (const uint16_t*)bg;
  a.w2 = wu;
  a.sc2 = (const uint16_t*)su;
  a.bi2 = (const uint16_t*)bu;
  a.xr = (const uint16_t*)xres;
  a.nw = (const uint16_t*)nw;
  a.hid = (uint16_t*)hid;
  a.nrm = (uint16_t*)nrm;
  a.eps = eps;
  a.y = act;
  a.y_dtype = dt;
  a.M = (int)M;
  a.N = (int)(2 * I);
  a.K = (int)K;
  a.SG = p.SG;
  a.USr = p.USr;
  a.R = p.R;
  if (dt == SPARKQ_BF16) {
    if (p.MQ == 1)
      launch_fused<BF16, 1, kFfnGateUp>(p, G, a, st);
    else
      launch_fused<BF16, 4, kFfnGateUp>(p, G, a, st);
  } else {
    if (p.MQ == 1)
      launch_fused<F16, 1, kFfnGateUp>(p, G, a, st);
    else
      launch_fused<F16, 4, kFfnGateUp>(p, G, a, st);
  }
  return check_launch("w4_gemv_kernel<ffn gate/up>");
}

// QKV projection of one token with RoPE on the query and key heads in one
// launch (X/src/spark_qkv_rope.cpp:83-101). q, k, v receive the [heads][D]
// rows of each section. Returns 1 when no fused plan serves the shape.
int w4_qkv_rope(const void* x, const uint32_t* w, const void* s, const void* b, void* q,
                void* k, void* v, int64_t K, int nh, int nkv, int hd, int rd, float log2_base,
                int64_t pos, int G, int dt, hipStream_t st) {
  if (env_int("SPARKQ_NO_FUSED_QKV", 0)) return 1;
  if (hd % 8 != 0 || rd % 8 != 0 || !aligned16(s) || !aligned16(b)) return 1;
  const int64_t N = (int64_t)(nh + 2 * nkv) * hd;
  if (N * (K / 2) >= (int64_t)kOob) return 1;
  const GemvPlan p = plan_fused(1, N, K, G, kQkvRope);
  if (!p.ok) return 1;
  GemvArgs a{};
  a.x = (const uint16_t*)x;
  a.w = w;
  a.sc = (const uint16_t*)s;
  a.bi = (const uint16_t*)b;
  a.y = q;
  a.y2 = k;
  a.y3 = v;
  a.y_dtype = dt;
  a.M = 1;
  a.N = (int)N;
  a.K = (int)K;
  a.SG = p.SG;
  a.USr = p.USr;
  a.R = p.R;
  a.heads = nh + nkv;
  a.hd = hd;
  a.rd = rd;
  a.q_rows = nh * hd;
  a.kv_rows = nkv * hd;
  a.log2_base = log2_base;
  a.pos = (float)pos;
  if (dt == SPARKQ_BF16)
    launch_fused<BF16, 1, kQkvRope>(p, G, a, st);
  else
    launch_fused<F16, 1, kQkvRope>(p, G, a, st);
  return check_launch("w4_gemv_kernel<qkv rope>");
}

// Streaming GEMV plan (M = 1, rows longer than 5 spans): one workgroup per
// CU, each owning a contiguous range of row quads, its items dealt NI or
// fewer to a wave. The
// staged activations and the (scale, bias) pieces of the largest workgroup
// must fit the staging budgets and LDS; the scale tensors must end on a
// 16-byte boundary and every workgroup's first scale on one (K/G even),
// since they are staged in 16-byte loads.
struct StreamPlan {
  bool ok;
  int P, QW, NI, NW, RR;
  bool full;
  size_t lds;
};

static StreamPlan plan_stream(int64_t M, int64_t N, int64_t K, int G) {
  StreamPlan p{};
  if (M != 1 || env_int("SPARKQ_W4_NO_STREAM", 0)) return p;
  if (N * (K / 2) >= (int64_t)kOob || K * 2 >= (int64_t)kOob) return p;
  const int64_t ng = K / G;
  if (ng % 2 != 0 || (N * ng * 2) % 16 != 0) return p;
  const int64_t nq = cdiv(N, 4), U = cdiv(K / 2, 256);
  // Rows of up to 5 spans (K <= 2560) keep w4_gemv_kernel, whose
  // activations fit one wave's registers and are staged by many small
  // workgroups at little cost (measured: gate+up 19456x2560 8.5 us there
  // against 9.1 us here). Longer rows stage up to 20 KB of activations per
  // workgroup there, once per CU here (down 2560x9728: 6.9 -> 6.1 us).
  if (U <= 5 && !env_int("SPARKQ_W4_STREAM_ALL", 0)) return p;
  p.NW = env_int("SPARKQ_W4_STREAM_NW", 16) == 8 ? 8 : 16;
  p.P = (int)std::min<int64_t>(nq, device_cus() * (16 / p.NW));
  p.QW = (int)cdiv(nq, p.P);
  // Row ranges instead of whole quads (every CU streams the same bytes:
  // down 2560 x 9728 gives each CU 10 rows instead of 8 or 12) when the
  // (scale, bias) rows of any first row start on a 16-byte boundary: down
  // 6.2-6.4 -> 5.9 us, bit-identical. The one-round kernel of the 5-span rows
  // (gate+up, QKV) showed no gain from the same split.
  p.RR = !env_int("SPARKQ_W4_STREAM_QUADS", 0) && ng % 8 == 0 && N >= 4 * (int64_t)p.P;
  if (p.RR) p.QW = (int)cdiv(cdiv(N, p.P), 4);
  const int64_t ni = cdiv(p.QW * U, p.NW);
  if (ni > 8) return p;
  p.NI = ni <= 2 ? 2 : (ni <= 4 ? (int)ni : (ni <= 6 ? 6 : 8));
  const int64_t nt = 64 * p.NW;
  if (K / 32 > kStreamXP * nt || 4 * p.QW * ng / 8 > kStreamSP * nt) return p;
  const StreamLds l = stream_lds((int)K, p.QW, G);
  if (l.bytes > 65536) return p;
  p.lds = (size_t)l.bytes;
  p.full = K % 512 == 0 && N % 4 == 0;
  p.ok = true;
  return p;
}

template <typename T, int G, int NI, int NW>
static void launch_stream_w(const StreamPlan& p, const GemvStreamArgs& a, hipStream_t st) {
  if (p.full)
    hipLaunchKernelGGL((w4_gemv_stream_kernel<T, G, NI, NW, true>), dim3((unsigned)p.P),
                       dim3(64 * NW), p.lds, st, a);
  else
    hipLaunchKernelGGL((w4_gemv_stream_kernel<T, G, NI, NW, false>), dim3((unsigned)p.P),
                       dim3(64 * NW), p.lds, st, a);
}
template <typename T, int G, int NI>
static void launch_stream_n(const StreamPlan& p, const GemvStreamArgs& a, hipStream_t st) {
  if (p.NW == 16)
    launch_stream_w<T, G, NI, 16>(p, a, st);
  else
    launch_stream_w<T, G, NI, 8>(p, a, st);
}
template <typename T, int G>
static void launch_stream_g(const StreamPlan& p, const GemvStreamArgs& a, hipStream_t st) {
  switch (p.NI) {
    case 2: launch_stream_n<T, G, 2>(p, a, st); break;
    case 3: launch_stream_n<T, G, 3>(p, a, st); break;
    case 4: launch_stream_n<T, G, 4>(p, a, st); break;
    case 6: launch_stream_n<T, G, 6>(p, a, st); break;
    default: launch_stream_n<T, G, 8>(p, a, st); break;
  }
}
template <typename T>
static void launch_stream(const StreamPlan& p, int G, const GemvStreamArgs& a, hipStream_t st) {
  if (G == 32)
    launch_stream_g<T, 32>(p, a, st);
  else if (G == 64)
    launch_stream_g<T, 64>(p, a, st);
  else
    launch_stream_g<T, 128>(p, a, st);
}

// Multi-row streaming plan (2 <= M <= 16): the layout of plan_stream with
// all M activation rows staged per workgroup. K % 512 == 0 and N % 4 == 0
// (whole spans and row quads); LDS up to 160 KB.
struct DecPlan {
  bool ok;
  int P, QW, MQ, NI, RR, D;
  int PH, SPH;  // K phases and spans per phase (PH = 1: the whole row staged)
  size_t lds;
};

constexpr int kDecMaxLds = 160 * 1024;

static DecPlan plan_dec(int64_t M, int64_t N, int64_t K, int G) {
  DecPlan p{};
  if (M < (env_int("SPARKQ_W4_DEC_M1", 0) ? 1 : 2) || M > 16 || env_int("SPARKQ_W4_NO_DEC", 0))
    return p;
  if (K % 512 != 0 || N % 4 != 0) return p;
  // Up to four rows of at most 5 spans keep w4_gemv_kernel (measured at
  // M = 4: QKV 3584x2560 4.5 against 5.2 us here, gate+up 19456x2560 11.1
  // against 11.4 us); longer rows (down 2560x9728: 12.0 -> 9.0 us) and more
  // rows (M = 8: QKV 8.6 -> 6.8 us, gate+up 17.9 -> 16.4 us) come here.
  if (M <= 4 && K <= 2560 && !env_int("SPARKQ_W4_DEC_ALL", 0)) return p;
  if (N * (K / 2) >= (int64_t)kOob || M * K * 2 >= (int64_t)kOob) return p;
  const int64_t ng = K / G;
  if (ng % 2 != 0 || (N * ng * 2) % 16 != 0) return p;
  const int64_t nq = N / 4, U = K / 512;
  p.P = (int)std::min<int64_t>(nq, device_cus());
  p.QW = (int)cdiv(nq, p.P);
  // equal row ranges (not whole quads) per workgroup, as in the M = 1
  // streaming kernel; measured within noise here (down 2560x9728 M = 2:
  // 7.3-7.7 us with whole quads, 7.3 us with ranges; M = 4 and 8 equal), as
  // every workgroup still issues whole quads of items
  p.RR = !env_int("SPARKQ_W4_DEC_QUADS", 0) && ng % 8 == 0;
  if (p.RR) p.QW = (int)cdiv(cdiv(N, p.P), 4);
  p.MQ = (int)cdiv(M, 4);
  const int64_t nt = 64 * kDecNW;
  if (4 * p.QW * ng / 8 > kDecSP * nt) return p;
  // K phases: the fewest whose staged activation slab fits the staging
  // registers and LDS. More than one for 5..8 rows and at most two items per
  // wave and phase only: the phased kernel holds the next phase's staging and
  // weight registers beside the current ones (126 VGPRs there; three row
  // quartets or four items spill). Phases are opt-in (SPARKQ_W4_DEC_PHASES=n:
  // at least n): the phased down projection at 7 and 8 rows was faster than
  // the skinny kernel back to back (12.57 -> 12.2 us at 7 rows) but not inside
  // the decode sweep (QKV, gate+up, down per layer: 8 rows 1146 -> 1161 us, 7
  // rows equal), so those rows keep the skinny kernel by default.
  const int64_t want0 = env_int("SPARKQ_W4_DEC_PHASES", 0);
  const int64_t phmax = want0 < 1 || p.MQ != 2 ? 1 : 4;
  for (int64_t want = std::max<int64_t>(1, want0); want <= phmax; ++want) {
    const int64_t sph = cdiv(U, want), npw = 16 * sph;
    if (M * npw > kDecXP * nt) continue;
    if (cdiv(U, sph) > 1 && cdiv(p.QW * sph, kDecNW) > 2) continue;
    const DecLds l = dec_lds_phased((int)M, (int)K, p.QW, G, p.MQ, (int)npw);
    if (l.bytes > kDecMaxLds) continue;
    p.SPH = (int)sph;
    p.PH = (int)cdiv(U, sph);
    p.lds = (size_t)l.bytes;
    break;
  }
  if (p.PH == 0) return p;
  const int64_t ni = cdiv(p.QW * p.SPH, kDecNW);
  if (ni > 8) return p;
  p.NI = ni <= 2 ? 2 : (ni <= 4 ? 4 : 8);
  // one weight item per wave in flight, the next issued as an item is taken
  // up, for waves of four or more items: every item in flight at once kept
  // the waves at issue while the CU's memory queue drained and put the items'
  // arithmetic after the stream (M = 2 / 4 / 6 / 8 sweeps 2073 / 2054 / 1530 /
  // 1419 -> 2119 / 2104 / 1604 / 1467 GB/s, gate+up at 8 rows 14.3-14.6 ->
  // 13.2-14.2 us, down at 4 rows 8.5 -> 8.1 us); two items a wave (QKV at 8
  // rows) stay all in flight (6.1 -> 6.2 us at one). SPARKQ_W4_DEC_DEPTH: 1 or
  // 8 (all).
  const int64_t dd = env_int("SPARKQ_W4_DEC_DEPTH", p.NI >= 4 ? 1 : 8);
  p.D = dd == 1 && p.PH == 1 ? 1 : p.NI;
  p.ok = true;
  return p;
}

template <typename T, int G, int MQ, int NI, int D>
static void launch_dec_k(const DecPlan& p, const DecodeStreamArgs& a, hipStream_t st) {
  auto* k = w4_decode_stream_kernel<T, G, MQ, NI, true, D>;
  // dynamic LDS above 64 KB must be enabled per kernel
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, kDecMaxLds);
  (void)attr;
  hipLaunchKernelGGL(k, dim3((unsigned)p.P), dim3(64 * kDecNW), p.lds, st, a);
}
template <typename T, int G, int MQ, int NI>
static void launch_dec_n(const DecPlan& p, const DecodeStreamArgs& a, hipStream_t st) {
  if (p.D == 1)
    launch_dec_k<T, G, MQ, NI, 1>(p, a, st);
  else
    launch_dec_k<T, G, MQ, NI, NI>(p, a, st);
}
template <typename T, int G, int MQ>
static void launch_dec_m(const DecPlan& p, const DecodeStreamArgs& a, hipStream_t st) {
  if (p.NI == 2)
    launch_dec_n<T, G, MQ, 2>(p, a, st);
  else if (p.NI == 4)
    launch_dec_n<T, G, MQ, 4>(p, a, st);
  else
    launch_dec_n<T, G, MQ, 8>(p, a, st);
}
template <typename T, int G>
static void launch_dec_g(const DecPlan& p, const DecodeStreamArgs& a, hipStream_t st) {
  if (p.PH > 1) {
    auto* k = w4_decode_phased_kernel<T, G>;
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, kDecMaxLds);
    (void)attr;
    hipLaunchKernelGGL(k, dim3((unsigned)p.P), dim3(64 * kDecNW), p.lds, st, a);
    return;
  }
  switch (p.MQ) {
    case 1: launch_dec_m<T, G, 1>(p, a, st); break;
    case 2: launch_dec_m<T, G, 2>(p, a, st); break;
    case 3: launch_dec_m<T, G, 3>(p, a, st); break;
    default: launch_dec_m<T, G, 4>(p, a, st); break;
  }
}
template <typename T>
static void launch_dec(const DecPlan& p, int G, const DecodeStreamArgs& a, hipStream_t st) {
  if (G == 32)
    launch_dec_g<T, 32>(p, a, st);
  else if (G == 64)
    launch_dec_g<T, 64>(p, a, st);
  else
    launch_dec_g<T, 128>(p, a, st);
}

// Workspace of the bf16 GEMM after the counter block: the prologue's
// scaled fp16 activations, row shifts, scaled scales and bias slots.
struct GemmX16Layout {
  size_t xh, ex, a2, sp, es, b2, bytes;
};
static GemmX16Layout gemm_x16_layout(int64_t M, int64_t N, int64_t K, int G) {
  const int64_t ng = K / G, k2p = bias_slots((int)K, G);
  GemmX16Layout l;
  l.xh = 0;
  l.ex = l.xh + round_up((size_t)(M * K * 2), 256);
  l.a2 = l.ex + round_up((size_t)(M * 4), 256);
  l.sp = l.a2 + round_up((size_t)(M * k2p * 2), 256);
  l.es = l.sp + round_up((size_t)(N * ng * 2), 256);
  l.b2 = l.es + round_up((size_t)(N * 4), 256);
  l.bytes = l.b2 + round_up((size_t)(N * k2p * 2), 256);
  return l;
}

// The weight half of that prologue (scaled fp16 scales, row shifts and bias
// slots) depends on the scales and biases only, so a caller can compute it
// once per weight set (w4a16_prepare) and hand it to every later call; the
// per-call prologue then converts the activation rows only.
struct PreparedLayout {
  size_t sp, es, b2, bytes;
};
static PreparedLayout prepared_layout(int64_t N, int64_t K, int G) {
  const int64_t ng = K / G, k2p = bias_slots((int)K, G);
  PreparedLayout l;
  l.sp = 0;
  l.es = round_up((size_t)(N * ng * 2), 256);
  l.b2 = l.es + round_up((size_t)(N * 4), 256);
  l.bytes = l.b2 + round_up((size_t)(N * k2p * 2), 256);
  return l;
}

// Work plan of the wide GEMM (up to two workgroups per CU).
//
// Grids of 128-row tiles that would fill less than a quarter of the slots
// (QKV 3584 x 2560 and down 2560 x 9728 at M = 512) take 64-row tiles and
// split every tile along k into the number of pieces S that minimises
// ceil(T*S / CUs) * ceil(steps / S) + 2*S: the longest chain of 64-k steps
// on one CU (two workgroups sharing a CU each run at about half speed) plus
// the cost of a piece's partial round trip. Measured on the MI355X (whole
// call, prologue included): QKV M = 512 two pieces 35.0 us (one 45.0,
// three 39.4, four 35.6), down M = 512 three pieces 76.2 us (two 92.0, four
// 93.1, six 77.5).
//
// Larger grids keep 128-row tiles: whole rounds of tiles run unsplit, and
// the tiles of a last round that leaves at least three quarters of the
// slots idle (half, for rows of 64 steps or more) are split into S = slots
// / tail tiles, capped at four pieces and at twelve 64-k steps per piece.
// The last piece of a tile reads the others' partials in dependent rounds
// of loads, which costs time when a quarter or more of the slots are busy
// anyway (QKV at M = 2048 in two pieces: 59.5 -> 71.3 us; gate+up 19456 x
// 2560 at M = 512: 89.8 -> 98.6 us); down at M = 2048 (160 tiles of 152
// steps) gains from three pieces (190.6 -> 161.9 us).
//
// Split tiles need their counters in the fixed block, else nothing splits.
struct WidePlan {
  int MX, tiles_n, tiles, full, S, items;
  size_t part_bytes;
};
static WidePlan plan_wide(int64_t M, int64_t N, int64_t K) {
  WidePlan p{};
  const int64_t cus = device_cus(), P = 2 * cus;
  p.MX = cdiv(N, 256) * cdiv(M, 128) < P / 4 && M > 64 && !env_int("SPARKQ_W4_GEMM_MX4", 0) ? 2 : 4;
  if (env_int("SPARKQ_W4_GEMM_MX2", 0)) p.MX = 2;
  const int64_t BM = 32 * p.MX;
  const int64_t tn = cdiv(N, 256), T = tn * cdiv(M, BM), nsteps = K / kBK;
  int64_t tail = T % P, S = 1;
  if (p.MX == 2) {
    tail = T;
    int64_t best = -1;
    for (int64_t s = 1; s <= std::min<int64_t>(8, std::max<int64_t>(nsteps / 8, 1)); ++s) {
      const int64_t cost = cdiv(T * s, cus) * cdiv(nsteps, s) + 2 * s;
      if (best < 0 || cost < best) best = cost, S = s;
    }
  } else if (T > cus && T < P && !env_int("SPARKQ_W4_GEMM_NO_CU1", 0)) {
    // one round of more tiles than CUs: a workgroup pair on a CU runs at
    // well over half the speed of one alone, so the CUs holding two whole
    // tiles set the time; instead one whole tile per CU, and the tiles past
    // the CUs in k pieces (at most 3: each piece adds a 128 KB partial to
    // the last one's reads). gate+up 19456x2560: M = 512 (304 tiles) 86-88
    // -> 78 us (three pieces; two 79.7, five 80-82, eight 90), M = 640
    // (380 tiles, two pieces) 91-93 -> 87 us
    tail = T - cus;
    S = std::min<int64_t>(std::min<int64_t>(cus / tail, 3), std::max<int64_t>(nsteps / 8, 1));
  } else if (tail && (tail <= P / 4 || (nsteps >= 64 && tail < P / 2))) {
    S = std::min<int64_t>(P / tail, std::min<int64_t>(env_int("SPARKQ_W4_GEMM_MAXS", 4), nsteps / 12));
  }
  if (env_int("SPARKQ_W4_SPLITS", 0)) S = std::min<int64_t>(env_int("SPARKQ_W4_SPLITS", 1), nsteps);
  if (tail > kMaxCounterTiles) S = 1;
  p.tiles_n = (int)tn;
  p.tiles = (int)T;
  p.S = (int)std::max<int64_t>(S, 1);
  p.full = (int)(p.S > 1 ? T - tail : T);
  p.items = (int)(p.full + (T - p.full) * p.S);
  if (p.S > 1) p.part_bytes = round_up((size_t)(T - p.full) * p.S * BM * 256 * 4, 256);
  return p;
}

int64_t w4_mr_workspace(int64_t M, int64_t N, int64_t K, int G);
int w4_mr_linear(const void* x, const uint32_t* w, const void* s, const void* b, void* y,
                 int64_t M, int64_t N, int64_t K, int G, int xdt, int ydt, hipStream_t st,
                 const void* res, void* ws, size_t wsb);

size_t w4a16_workspace(int64_t M, int64_t N, int64_t K, int G) {
  if (M <= 0 || N <= 0 || K <= 0 || G <= 0) return 0;
  // in dispatch order
  if (plan_stream(M, N, K, G).ok) return 0;
  const int64_t mr = w4_mr_workspace(M, N, K, G);
  if (mr >= 0) return (size_t)mr;
  if (plan_dec(M, N, K, G).ok || plan_gemv(M, N, K, G).ok) return 0;
  // every workspace of this entry point starts with the counter block, so a
  // GEMM call never writes over the counters a later split-K call relies on
  if (M <= 32 && M < env_int("SPARKQ_W4_GEMM_FROM", 33)) {
    const SkinnyPlan p = plan_skinny(M, N, K);
    return p.S > 1 ? kCounterBytes + p.part_bytes : 0;
  }
  const GemmX16Layout l = gemm_x16_layout(M, N, K, G);
  return kCounterBytes +
         std::max(round_up((size_t)(K / G) * M * 4, 256), l.bytes + plan_wide(M, N, K).part_bytes);
}

template <typename T, int G, int MB, int CPW>
static void launch_skinny_c(const SkinnyPlan& p, const SkinnyArgs& a, hipStream_t st) {
  dim3 grid((unsigned)cdiv(a.N, 32), (unsigned)p.S);
  hipLaunchKernelGGL((w4_skinny_kernel<T, G, MB, CPW>), grid, dim3(256), p.lds, st, a);
}

template <typename T, int G, int MB>
static void launch_skinny_t(const SkinnyPlan& p, const SkinnyArgs& a, hipStream_t st) {
  switch (p.CPW) {
    case 1: launch_skinny_c<T, G, MB, 1>(p, a, st); break;
    case 2: launch_skinny_c<T, G, MB, 2>(p, a, st); break;
    case 4: launch_skinny_c<T, G, MB, 4>(p, a, st); break;
    case 5: launch_skinny_c<T, G, MB, 5>(p, a, st); break;
    default: launch_skinny_c<T, G, MB, 8>(p, a, st); break;
  }
}

template <typename T, int G>
static void launch_skinny_g(const SkinnyPlan& p, const SkinnyArgs& a, hipStream_t st) {
  switch (p.MB) {
    case 1: launch_skinny_t<T, G, 1>(p, a, st); break;
    case 8: launch_skinny_t<T, G, 8>(p, a, st); break;
    case 16: launch_skinny_t<T, G, 16>(p, a, st); break;
    default: launch_skinny_t<T, G, 32>(p, a, st); break;
  }
}

template <typename T>
static void launch_skinny(const SkinnyPlan& p, int G, const SkinnyArgs& a, hipStream_t st) {
  if (G == 32)
    launch_skinny_g<T, 32>(p, a, st);
  else if (G == 64)
    launch_skinny_g<T, 64>(p, a, st);
  else
    launch_skinny_g<T, 128>(p, a, st);
}

template <typename T>
static void launch_gemm(int G, const void* x, const uint32_t* w, const void* s,
                        const void* b, float* xs, void* y, int ydt, int M, int N,
                        int K, hipStream_t st) {
  const int64_t nxs = (int64_t)M * (K / G);
  hipLaunchKernelGGL(xsum_kernel<T>, dim3((unsigned)cdiv(nxs, 256)), dim3(256), 0, st,
                     (const uint16_t*)x, xs, M, K, G);
  dim3 grid((unsigned)cdiv(N, kBN), (unsigned)cdiv(M, kBM));
#define SPARKQ_GEMM(GG)                                                              \
  hipLaunchKernelGGL((w4_gemm_kernel<T, GG>), grid, dim3(256), 0, st, (const uint16_t*)x, \
                     w, (const uint16_t*)s, (const uint16_t*)b, xs, y, ydt, M, N, K)
  if (G == 32)
    SPARKQ_GEMM(32);
  else if (G == 64)
    SPARKQ_GEMM(64);
  else
    SPARKQ_GEMM(128);
#undef SPARKQ_GEMM
}

// One launch of the prologue over M activation rows and the weight rows of
// p.N (p.N = 0: activation rows only; p.M = 0: weight rows only).
static void launch_gemm_prep(const GemmPrepArgs& p, hipStream_t st) {
  const PrepPlan pp = plan_prep(p.K, p.G);
  GemmPrepArgs q = p;
  q.rw = pp.rw;
  // the activation row in registers up to 2048 chunks of 16 bytes (K <= 16384)
  const int64_t nch = env_int("SPARKQ_PREP_NO_REG", 0) ? 0 : cdiv(p.K / 8, 256);
  const dim3 pg((unsigned)(p.M + cdiv(p.N, pp.rw)));
  switch (nch) {
#define SPARKQ_PREP_CASE(n) \
  case n: hipLaunchKernelGGL(gemm_prep_kernel<n>, pg, dim3(256), pp.lds, st, q); break;
    SPARKQ_PREP_CASE(1) SPARKQ_PREP_CASE(2) SPARKQ_PREP_CASE(3) SPARKQ_PREP_CASE(4)
    SPARKQ_PREP_CASE(5) SPARKQ_PREP_CASE(6) SPARKQ_PREP_CASE(7) SPARKQ_PREP_CASE(8)
#undef SPARKQ_PREP_CASE
    default: hipLaunchKernelGGL(gemm_prep_kernel<0>, pg, dim3(256), pp.lds, st, q);
  }
}

// prep: the weight half made by w4a16_prepare for these scales and biases,
// or null to compute it in this call's prologue
static void launch_gemm_x16(int G, const void* x, const uint32_t* w, const void* s,
                            const void* b, const unsigned char* prep, unsigned* counters,
                            unsigned char* ws, void* y, int ydt, int M, int N, int K,
                            hipStream_t st) {
  const GemmX16Layout l = gemm_x16_layout(M, N, K, G);
  GemmPrepArgs p{};
  p.x = (const uint16_t*)x;
  p.sc = (const uint16_t*)s;
  p.bi = (const uint16_t*)b;
  p.xh = reinterpret_cast<uint16_t*>(ws + l.xh);
  p.ex = reinterpret_cast<int*>(ws + l.ex);
  p.a2 = reinterpret_cast<uint16_t*>(ws + l.a2);
  p.M = M;
  p.N = N;
  p.K = K;
  p.G = G;
  p.K2p = bias_slots(K, G);
  if (prep != nullptr) {
    const PreparedLayout pl = prepared_layout(N, K, G);
    p.sp = const_cast<uint16_t*>(reinterpret_cast<const uint16_t*>(prep + pl.sp));
    p.es = const_cast<int*>(reinterpret_cast<const int*>(prep + pl.es));
    p.b2 = const_cast<uint16_t*>(reinterpret_cast<const uint16_t*>(prep + pl.b2));
    p.N = 0;  // the prologue converts the activation rows only
  } else {
    p.sp = reinterpret_cast<uint16_t*>(ws + l.sp);
    p.es = reinterpret_cast<int*>(ws + l.es);
    p.b2 = reinterpret_cast<uint16_t*>(ws + l.b2);
  }
  launch_gemm_prep(p, st);
  GemmX16Args a{};
  a.xh = p.xh;
  a.w = w;
  a.sp = p.sp;
  a.ex = p.ex;
  a.es = p.es;
  a.a2 = p.a2;
  a.b2 = p.b2;
  a.y = y;
  a.y_dtype = ydt;
  a.M = M;
  a.N = N;
  a.K = K;
  a.K2p = p.K2p;
  const WidePlan wp = plan_wide(M, N, K);
  a.tiles_n = wp.tiles_n;
  a.tiles = wp.tiles;
  a.full = wp.full;
  a.S = wp.S;
  // XCD-grouped tile order, groups of four tile rows: the tiles an XCD runs
  // together share their activation rows and weight columns in its L2 (M =
  // 2048: down 160.2 -> 151.1 us, QKV 60.8 -> 59.6, gate+up 232 -> 230; M = 512
  // unchanged); SPARKQ_W4_GEMM_ROWMAJOR keeps the row-major order
  a.gm = env_int("SPARKQ_W4_GEMM_ROWMAJOR", 0) ? 0 : (int)env_int("SPARKQ_W4_GEMM_GM", 4);
  a.part = reinterpret_cast<float*>(ws + l.bytes);
  a.counters = counters;
  dim3 gw((unsigned)wp.items);
#define SPARKQ_X16W(GG, MM, PP) \
  hipLaunchKernelGGL((w4_gemm_x16w_kernel<GG, 4, MM, PP>), gw, dim3(256), 0, st, a)
#define SPARKQ_X16S(GG, SS) \
  hipLaunchKernelGGL((w4_gemm_x16w_kernel<GG, 4, 4, 1, SS>), gw, dim3(256), 0, st, a)
  // the 64-row tiles (grids of at most one workgroup per CU, whose steps
  // wait on their loads) keep two steps of loads in flight: QKV 3584 x 2560
  // at M = 512 35.0 -> 32.2 us, down 2560 x 9728 78.3 -> 70.0 us, bit-identical;
  // the 128-row tiles have no registers for it (weights alone two steps
  // ahead measured 0-1% slower at M = 512 and 2048)
  const int pd = env_int("SPARKQ_W4_GEMM_PD", wp.MX == 2 ? 2 : 1);
  if (wp.MX == 2 && pd == 2) {
    if (G == 32) SPARKQ_X16W(32, 2, 2);
    else if (G == 64) SPARKQ_X16W(64, 2, 2);
    else SPARKQ_X16W(128, 2, 2);
  } else if (wp.MX == 2) {
    if (G == 32) SPARKQ_X16W(32, 2, 1);
    else if (G == 64) SPARKQ_X16W(64, 2, 1);
    else SPARKQ_X16W(128, 2, 1);
  } else {
    // schedule variant (SCH bits): priority over the MFMA phase with four A
    // slots and a barrier every second step is the default, measured per
    // call with prepared weights against the plain schedule: gate+up 19456 x
    // 2560 M = 2048 231.2 -> 227.0 us, M = 512 75.2-76.2 -> 73.6-75.0 us,
    // QKV and down at M = 2048 within 1%. The four slots alone ran slower
    // (240 us), the priority alone the same (231.2 us).
    // SPARKQ_W4_GEMM_SCH = 1..3 picks a variant, any other value the plain one
    const int sch = env_int("SPARKQ_W4_GEMM_SCH", 3);
    if (sch == 1) {
      if (G == 32) SPARKQ_X16S(32, 1);
      else if (G == 64) SPARKQ_X16S(64, 1);
      else SPARKQ_X16S(128, 1);
    } else if (sch == 2) {
      if (G == 32) SPARKQ_X16S(32, 2);
      else if (G == 64) SPARKQ_X16S(64, 2);
      else SPARKQ_X16S(128, 2);
    } else if (sch == 3) {
      if (G == 32) SPARKQ_X16S(32, 3);
      else if (G == 64) SPARKQ_X16S(64, 3);
      else SPARKQ_X16S(128, 3);
    } else {
      if (G == 32) SPARKQ_X16W(32, 4, 1);
      else if (G == 64) SPARKQ_X16W(64, 4, 1);
      else SPARKQ_X16W(128, 4, 1);
    }
  }
#undef SPARKQ_X16S
#undef SPARKQ_X16W
}

// one row quad per wave, every quad in one round (w4q.hip); 1 = not taken
int w4_gemvq_linear(const void* x, const uint32_t* w, const void* s, const void* b, void* y,
                    int64_t M, int64_t N, int64_t K, int G, int xdt, int ydt, hipStream_t st,
                    const void* res);

int w4a16_linear(const void* x, const uint32_t* w, const void* s, const void* b,
                 void* y, int64_t M, int64_t N, int64_t K, int G, int xdt, int ydt,
                 void* ws, size_t wsb, hipStream_t st, const void* res, bool* res_done,
                 const void* prep) {
  // res (16-bit [M][N], y of the same type) is added to the rounded output by
  // the decode kernels; *res_done says whether the chosen kernel did it
  if (res_done) *res_done = false;
  const size_t need = w4a16_workspace(M, N, K, G);
  if (need > 0 && (ws == nullptr || wsb < need))
    return set_error(SPARKQ_ERR_WORKSPACE,
                     "w4a16_linear needs a workspace of %zu bytes (got %zu)", need, wsb);
  {
    const int rc = w4_gemvq_linear(x, w, s, b, y, M, N, K, G, xdt, ydt, st, res);
    if (rc != 1) {
      if (res_done) *res_done = rc == 0 && res != nullptr;
      return rc;
    }
  }
  const StreamPlan sp = plan_stream(M, N, K, G);
  if (sp.ok) {
    GemvStreamArgs a{};
    a.x = (const uint16_t*)x;
    a.w = w;
    a.sc = (const uint16_t*)s;
    a.bi = (const uint16_t*)b;
    a.y = y;
    a.y_dtype = ydt;
    a.N = (int)N;
    a.K = (int)K;
    a.nq = (int)cdiv(N, 4);
    a.P = sp.P;
    a.QW = sp.QW;
    a.RR = sp.RR;
    a.res = (const uint16_t*)res;
    if (res_done) *res_done = res != nullptr;
    if (xdt == SPARKQ_BF16)
      launch_stream<BF16>(sp, G, a, st);
    else
      launch_stream<F16>(sp, G, a, st);
    return check_launch("w4_gemv_stream_kernel");
  }
  {
    const int rc = w4_mr_linear(x, w, s, b, y, M, N, K, G, xdt, ydt, st, res, ws, wsb);
    if (rc != 1) {
      if (res_done) *res_done = rc == 0 && res != nullptr;
      return rc;
    }
  }
  const DecPlan dp = plan_dec(M, N, K, G);
  if (dp.ok) {
    DecodeStreamArgs a{};
    a.x = (const uint16_t*)x;
    a.w = w;
    a.sc = (const uint16_t*)s;
    a.bi = (const uint16_t*)b;
    a.y = y;
    a.y_dtype = ydt;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.nq = (int)(N / 4);
    a.P = dp.P;
    a.QW = dp.QW;
    a.RR = dp.RR;
    a.PH = dp.PH;
    a.SPH = dp.SPH;
    a.res = (const uint16_t*)res;
    if (res_done) *res_done = res != nullptr;
    if (xdt == SPARKQ_BF16)
      launch_dec<BF16>(dp, G, a, st);
    else
      launch_dec<F16>(dp, G, a, st);
    return check_launch("w4_decode_stream_kernel");
  }
  const GemvPlan gp = plan_gemv(M, N, K, G);
  if (gp.ok) {
    GemvArgs a{};
    a.x = (const uint16_t*)x;
    a.w = w;
    a.sc = (const uint16_t*)s;
    a.bi = (const uint16_t*)b;
    a.y = y;
    a.y_dtype = ydt;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.SG = gp.SG;
    a.USr = gp.USr;
    a.R = gp.R;
    a.res = (const uint16_t*)res;
    if (res_done) *res_done = res != nullptr;
    if (xdt == SPARKQ_BF16)
      launch_gemv<BF16>(gp, G, a, st);
    else
      launch_gemv<F16>(gp, G, a, st);
    return check_launch("w4_gemv_kernel");
  }
  if (M <= 32 && M < env_int("SPARKQ_W4_GEMM_FROM", 33)) {
    const SkinnyPlan p = plan_skinny(M, N, K);
    if (p.S > 1 && cdiv(N, 32) > kMaxCounterTiles)
      return set_error(SPARKQ_ERR_UNSUPPORTED,
                       "w4a16_linear: N=%lld with M=%lld and K=%lld needs more split-K tile "
                       "counters than the workspace holds (N <= %lld)",
                       (long long)N, (long long)M, (long long)K, (long long)(32 * kMaxCounterTiles));
    SkinnyArgs a{};
    a.x = (const uint16_t*)x;
    a.w = w;
    a.sc = (const uint16_t*)s;
    a.bi = (const uint16_t*)b;
    a.y = y;
    a.y_dtype = ydt;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.cps = p.cps;
    a.S = p.S;
    if (p.S > 1) {
      a.counters = reinterpret_cast<unsigned*>(ws);
      a.part = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(ws) + kCounterBytes);
    }
    if (xdt == SPARKQ_BF16)
      launch_skinny<BF16>(p, G, a, st);
    else
      launch_skinny<F16>(p, G, a, st);
    return check_launch("w4_skinny_kernel");
  }
  unsigned char* wsp = reinterpret_cast<unsigned char*>(ws) + kCounterBytes;
  if (xdt == SPARKQ_BF16 && !env_int("SPARKQ_W4_NO_X16", 0)) {
    launch_gemm_x16(G, x, w, s, b, reinterpret_cast<const unsigned char*>(prep),
                    reinterpret_cast<unsigned*>(ws), wsp, y, ydt, (int)M, (int)N,
                    (int)K, st);
    return check_launch("w4_gemm_x16w_kernel");
  }
  float* xs = reinterpret_cast<float*>(wsp);
  if (xdt == SPARKQ_BF16)
    launch_gemm<BF16>(G, x, w, s, b, xs, y, ydt, (int)M, (int)N, (int)K, st);
  else
    launch_gemm<F16>(G, x, w, s, b, xs, y, ydt, (int)M, (int)N, (int)K, st);
  return check_launch("w4_gemm_kernel");
}

size_t w4a16_prepared_bytes(int64_t N, int64_t K, int G) {
  if (N <= 0 || K <= 0 || G <= 0) return 0;
  return prepared_layout(N, K, G).bytes;
}

// The weight half of the bf16 GEMM prologue for one weight set, into prep
// (w4a16_prepared_bytes); the same kernel and code path as the per-call
// prologue, so a prepared call gives bit-identical results.
int w4a16_prepare(const void* s, const void* b, void* prep, int64_t N, int64_t K, int G,
                  hipStream_t st) {
  const PreparedLayout pl = prepared_layout(N, K, G);
  unsigned char* pb = reinterpret_cast<unsigned char*>(prep);
  GemmPrepArgs p{};
  p.sc = (const uint16_t*)s;
  p.bi = (const uint16_t*)b;
  p.sp = reinterpret_cast<uint16_t*>(pb + pl.sp);
  p.es = reinterpret_cast<int*>(pb + pl.es);
  p.b2 = reinterpret_cast<uint16_t*>(pb + pl.b2);
  p.M = 0;  // weight rows only
  p.N = (int)N;
  p.K = (int)K;
  p.G = G;
  p.K2p = bias_slots((int)K, G);
  launch_gemm_prep(p, st);
  return check_launch("gemm_prep_kernel");
}

int w4a16_dequantize(const uint32_t* w, const void* s, const void* b, float* out,
                     int64_t N, int64_t K, int G, int sdt, hipStream_t st) {
  const int64_t words = N * K / 8;
  dim3 grid((unsigned)cdiv(words, 256));
  if (sdt == SPARKQ_BF16)
    hipLaunchKernelGGL(w4_dequant_kernel<BF16>, grid, dim3(256), 0, st, w,
                       (const uint16_t*)s, (const uint16_t*)b, out, N, K, G);
  else
    hipLaunchKernelGGL(w4_dequant_kernel<F16>, grid, dim3(256), 0, st, w,
                       (const uint16_t*)s, (const uint16_t*)b, out, N, K, G);
  return check_launch("w4_dequant_kernel");
}

int w4_quantize(const void* w, uint32_t* wq, void* s, void* b, int64_t N, int64_t K,
                int G, int dt, hipStream_t st) {
  const int64_t groups = N * (K / G);
  dim3 grid((unsigned)cdiv(groups, 256));
  if (dt == SPARKQ_BF16)
    hipLaunchKernelGGL(w4_quantize_kernel<BF16>, grid, dim3(256), 0, st,
                       (const uint16_t*)w, wq, (uint16_t*)s, (uint16_t*)b, N, K, G);
  else
    hipLaunchKernelGGL(w4_quantize_kernel<F16>, grid, dim3(256), 0, st,
                       (const uint16_t*)w, wq, (uint16_t*)s, (uint16_t*)b, N, K, G);
  return check_launch("w4_quantize_kernel");
}

}  // namespace sparkq
