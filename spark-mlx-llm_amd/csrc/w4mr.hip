// w4mr.hip -- W4A16 decode GEMV for 9..16 activation rows on the
// 16x16x32 MFMA (speculative-verify and small-batch decode).
//
// The 4x4x4 decode kernels share each decoded weight piece across the
// activation rows four at a time; at 8..16 rows their activation reads from
// LDS (16 KB per 1 KB item and wave at M = 16) bound them. Here one
// v_mfma_f32_16x16x32 takes 16 weight rows x 16 activation rows x 32 k:
//
//  * Items: a row tile of 16 weight rows x one 128-k segment (64 bytes a
//    row). Lane l loads 16 bytes of row l%16 at byte 16*(l/16) of the
//    segment: one load instruction per item, every load issued at the start.
//  * A 4x4 transpose of the loaded words across the four 16-lane rows
//    (v_permlane32_swap, then v_permlane16_swap) leaves in lane (g, r) word
//    g of each 32-k chunk c, so MFMA c covers exactly chunk c: its k range
//    lies inside one quantization group (G >= 32) and the group's scale and
//    bias apply to the MFMA result, s*D + (b - OFFSET*s)*X with X the group
//    sum of each activation row (the decode of 3.1: codes read as OFFSET + q).
//  * The A operand is 8 activations of row l%16 read from LDS (rows padded
//    by 16 bytes); rows past M read row M-1 and their outputs are dropped.
//  * Layout as the streaming kernels: one workgroup of 16 waves per CU, a
//    contiguous range of row tiles per workgroup, the (tile, segment) items
//    dealt to the waves in contiguous runs. A wave sums its run of a tile in
//    registers and leaves the sum in an LDS slot (a run touches at most two
//    tiles); each output is the sum of its tile's slots in wave order.
//  * Rows whose activations exceed the staging budget (the down projection,
//    K = 9728) split K into KS ranges of whole 128-k segments
//    and whole groups (grid.y): each workgroup stages the M rows of its range
//    only, stores its outputs as fp32 partials, and the last workgroup of a
//    tile range to arrive adds the KS partials in range order (coherent
//    loads, deterministic) and writes the outputs.
#include "common.h"

namespace sparkq {

struct MrArgs {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* sc;
  const uint16_t* bi;
  void* y;
  const uint16_t* res;  // 16-bit residual added to the rounded output (or null)
  int y_dtype;
  int M, N, K;
  int nt;  // row tiles of 16
  int P;   // workgroups (tile ranges)
  int TW;  // tiles of the largest workgroup
  int IW;  // items per wave
  int KS;  // K ranges (grid.y)
  float* part;         // [KS][M][N] partial outputs (KS > 1)
  unsigned* counters;  // one per tile range, zero on entry and exit (KS > 1)
};

constexpr int kMrNW = 16;              // waves per workgroup
constexpr int kMrXC = 8;               // staged activation chunks (16 B) per thread, at most
constexpr int kMrSP = 2;               // staged (scale, bias) pieces per thread, at most
constexpr int kMrMaxLds = 160 * 1024;

// LDS layout (byte offsets); K is the workgroup's K range
struct MrLds {
  int xrow;  // padded activation row (bytes)
  int xa;    // activations [M][K]
  int xs;    // group sums [K/G][16] fp32 (rows past M zero)
  int sb;    // (scale, bias) of the workgroup's rows [16*TW][K/G] dwords
  int part;  // run sums [waves][2][16][16] fp32
  int flag;  // the split handshake's last-arrival flag
  int bytes;
};
__host__ __device__ __forceinline__ MrLds mr_lds(int M, int K, int TW, int G) {
  MrLds l;
  l.xrow = 2 * K + 16;
  l.xa = 0;
  l.xs = (M * l.xrow + 15) & ~15;
  l.sb = l.xs + (K / G) * 64;
  l.part = l.sb + ((TW * 16 * (K / G) * 4 + 15) & ~15);
  l.flag = l.part + kMrNW * 2 * 256 * 4;
  l.bytes = l.flag + 16;
  return l;
}

template <typename T>
__device__ __forceinline__ f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c);
template <>
__device__ __forceinline__ f32x4_t mfma16x16x32<BF16>(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4_t mfma16x16x32<F16>(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// 4x4 transpose of the words of a 16-byte piece across the four 16-lane rows
// of the wave: afterwards lane (row g) holds in word c what row c held in
// word g. The 32-lane swap exchanges the off-diagonal 2x2 blocks, the 16-lane
// swap transposes each block.
__device__ __forceinline__ u32x4_t transpose_rows(u32x4_t v) {
  uint32_t w0 = v.x, w1 = v.y, w2 = v.z, w3 = v.w;
  auto r = __builtin_amdgcn_permlane32_swap(w0, w2, false, false);
  w0 = r[0];
  w2 = r[1];
  r = __builtin_amdgcn_permlane32_swap(w1, w3, false, false);
  w1 = r[0];
  w3 = r[1];
  r = __builtin_amdgcn_permlane16_swap(w0, w1, false, false);
  w0 = r[0];
  w1 = r[1];
  r = __builtin_amdgcn_permlane16_swap(w2, w3, false, false);
  w2 = r[0];
  w3 = r[1];
  return u32x4_t{w0, w1, w2, w3};
}

// D: weight items of a wave in flight (D < NI: the first D go out with the
// staging loads, each later one as the item D before it is taken up)
template <typename T, int G, int NI, int D>
__global__ __launch_bounds__(64 * kMrNW) void w4_mr16_kernel(MrArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int NT = 64 * kMrNW;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r16 = lane & 15;
  const int M = a.M, N = a.N, K = a.K, KS = a.KS;
  const int Kl = K / KS, kbase = blockIdx.y * Kl;      // this workgroup's K range
  const int ng = K / G, ngl = Kl / G, SEG = Kl >> 7, RB = K >> 1;
  const int t0 = blockIdx.x * a.nt / a.P;
  const int ntl = (blockIdx.x + 1) * a.nt / a.P - t0;  // tiles of this workgroup
  const int IW = a.IW;
  const int i0 = wave * IW;
  const int ni = max(0, min(IW, ntl * SEG - i0));      // items of this wave
  const MrLds L = mr_lds(M, Kl, a.TW, G);

  const rsrc_t rx = make_rsrc(a.x, (uint32_t)M * K * 2);
  const rsrc_t rw = make_rsrc(a.w, (uint32_t)N * RB);
  const rsrc_t rs = make_rsrc(a.sc, (uint32_t)N * ng * 2);
  const rsrc_t rb = make_rsrc(a.bi, (uint32_t)N * ng * 2);

  // 1. staging loads: activation chunks of the K range and the (scale,
  // bias) pieces of the workgroup's rows (16 * ntl contiguous rows): 16-byte
  // pieces of whole rows with one range, 4-byte pairs of groups with several
  const int nxc = (M * Kl) >> 3;
  const int nsp = KS == 1 ? (ntl * 16 * ng) >> 3 : (ntl * 16 * ngl) >> 1;
  // every thread issues the same loads (lanes with nothing to read use the
  // out-of-range offset): branches around loads here made the compiler
  // spill the staging registers
  u32x4_t xr[kMrXC], sr[kMrSP], br[kMrSP];
#pragma unroll
  for (int c = 0; c < kMrXC; ++c) {
    const int ci = tid + c * NT;
    const int m = ci / (Kl >> 3), kk = (ci - m * (Kl >> 3)) << 3;
    xr[c] = buf_load16(rx, ci < nxc ? 2u * (uint32_t)(m * K + kbase + kk) : kOob);
  }
  if (KS == 1) {
#pragma unroll
    for (int i = 0; i < kMrSP; ++i) {
      const int pi = tid + i * NT;
      const uint32_t off = pi < nsp ? 32u * (uint32_t)t0 * ng + 16u * pi : kOob;
      sr[i] = buf_load16(rs, off);
      br[i] = buf_load16(rb, off);
    }
  } else {
    // pair pi: row 16 t0 + pi / (ngl/2), groups kbase/G + 2 (pi % (ngl/2)) .. +1
#pragma unroll
    for (int i = 0; i < kMrSP; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int pi = tid + (4 * i + e) * NT;
        const int rl = pi / (ngl >> 1), gp = pi - rl * (ngl >> 1);
        const uint32_t off = pi < nsp ? 2u * (uint32_t)((16 * t0 + rl) * ng + kbase / G + 2 * gp) : kOob;
        sr[i][e] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)off, 0, 0);
        br[i][e] = __builtin_amdgcn_raw_buffer_load_b32(rb, (int)off, 0, 0);
      }
  }
  // 2. the wave's weight items: the first D now. With every item's load in
  // flight at once, the CU's memory queue (activations, scales and weights:
  // ~200 KB a CU for gate+up at 16 rows) kept each wave waiting at issue for
  // up to ~7 us, the staging barrier waited for the last of them, and the
  // items' arithmetic (3-5 us) ran after the stream; with one or two in
  // flight the staging completes early (barrier ~6.6 -> ~4.4 us) and the
  // items are computed as the weights arrive (gate+up at 16 rows 15.0 ->
  // 13.3 us, down 13.6 -> 12.8-13.2).
  u32x4_t wv[NI];
  auto wload = [&](int k) {
    const int it = i0 + k, tl = it / SEG, s = it - tl * SEG;
    const int row = 16 * (t0 + tl) + r16;
    const bool ok = k < ni && row < N;
    wv[k] = buf_load16(rw, ok ? (uint32_t)row * RB + (uint32_t)(kbase >> 1) + 64u * s + 16u * g : kOob);
  };
#pragma unroll
  for (int k = 0; k < D; ++k) wload(k);
  __builtin_amdgcn_sched_barrier(0);

  // 3. activations and (scale, bias) pairs to LDS, then the group sums
  uint32_t* sb = reinterpret_cast<uint32_t*>(smem + L.sb);
  float* xs = reinterpret_cast<float*>(smem + L.xs);
#pragma unroll
  for (int c = 0; c < kMrXC; ++c) {
    const int ci = tid + c * NT;
    if (ci < nxc) {
      const int m = ci / (Kl >> 3), kk = (ci - m * (Kl >> 3)) << 3;
      *reinterpret_cast<u32x4_t*>(smem + L.xa + m * L.xrow + 2 * kk) = xr[c];
    }
  }
  if (KS == 1) {
#pragma unroll
    for (int i = 0; i < kMrSP; ++i) {
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
  } else {
#pragma unroll
    for (int i = 0; i < kMrSP; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int pi = tid + (4 * i + e) * NT;
        if (pi < nsp) {
          sb[2 * pi] = __builtin_amdgcn_perm(br[i][e], sr[i][e], 0x05040100u);
          sb[2 * pi + 1] = __builtin_amdgcn_perm(br[i][e], sr[i][e], 0x07060302u);
        }
      }
  }
  __syncthreads();
  for (int e = tid; e < ngl * 16; e += NT) {
    const int grp = e >> 4, m = e & 15;
    float s = 0.0f;
    if (m < M) {
      const unsigned char* p = smem + L.xa + m * L.xrow + 2 * G * grp;
      for (int q = 0; q < G / 8; ++q) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(p + 16 * q);
#pragma unroll
        for (int h = 0; h < 4; ++h) s = pair_sum<T>(v[h], s);
      }
    }
    xs[e] = s;
  }
  __syncthreads();

  // 4. the items: per 32-k chunk one MFMA, per group the scale epilogue
  float* part = reinterpret_cast<float*>(smem + L.part);
  const unsigned char* arow = smem + L.xa + min(r16, M - 1) * L.xrow + 16 * g;
  const DecodeConsts dc = decode_consts<T>();
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  int cur = -1, slot = 0;
  auto flush = [&]() {
#pragma unroll
    for (int r = 0; r < 4; ++r) part[(wave * 2 + slot) * 256 + (4 * g + r) * 16 + r16] = acc[r];
  };
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    if (k + D < NI) wload(k + D);
    if (k < ni) {
      const int it = i0 + k, tl = it / SEG, s = it - tl * SEG;
      if (tl != cur) {
        if (cur >= 0) {
          flush();
          slot = 1;
        }
        cur = tl;
        acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
      const u32x4_t wt = transpose_rows(wv[k]);
      f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int kb = 128 * s + 32 * c;
        const u32x4_t bop = decode_w4<T>(wt[c], dc);
        const u32x4_t aop = *reinterpret_cast<const u32x4_t*>(arow + 2 * kb);
        d = mfma16x16x32<T>(aop, bop, d);
        if (((c + 1) * 32) % G == 0) {
          const int grp = kb / G;
          const uint32_t pair = sb[(tl * 16 + r16) * ngl + grp];
          const float sf = T::to_f32((uint16_t)(pair & 0xFFFFu));
          const float bf = fmaf(-T::OFFSET, sf, T::to_f32((uint16_t)(pair >> 16)));
          const f32x4_t xg = *reinterpret_cast<const f32x4_t*>(xs + grp * 16 + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] = fmaf(sf, d[r], fmaf(bf, xg[r], acc[r]));
          d = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
      }
      // one item at a time: hoisting later items' decodes would spill
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (cur >= 0) flush();
  __syncthreads();

  // 5. each output: the sum of its tile's run slots in wave order (with
  // several K ranges, this range's partial)
  const int64_t MN = (int64_t)M * N;
  for (int e = tid; e < ntl * 256; e += NT) {
    const int tl = e >> 8, m = (e >> 4) & 15, j = e & 15;
    const int n = 16 * (t0 + tl) + j;
    if (m >= M || n >= N) continue;
    const int v0 = (tl * SEG) / IW, v1 = ((tl + 1) * SEG - 1) / IW;
    float v = 0.0f;
    for (int w = v0; w <= v1; ++w) {
      const int sl = (w * IW) / SEG == tl ? 0 : 1;
      v += part[(w * 2 + sl) * 256 + m * 16 + j];
    }
    const int64_t idx = (int64_t)m * N + n;
    if (KS == 1)
      store_out(a.y, idx, a.res ? add_rounded<T>(v, a.res[idx]) : v, a.y_dtype);
    else
      splitk_store(&a.part[blockIdx.y * MN + idx], v);
  }
  if (KS == 1) return;
  // (the flag lives in the dynamic LDS: a static variable would take from
  // the 160 KB the dynamic allocation is allowed)
  if (!splitk_arrive(&a.counters[blockIdx.x], KS, reinterpret_cast<int*>(smem + L.flag))) return;
  for (int e = tid; e < ntl * 256; e += NT) {
    const int tl = e >> 8, m = (e >> 4) & 15, j = e & 15;
    const int n = 16 * (t0 + tl) + j;
    if (m >= M || n >= N) continue;
    const int64_t idx = (int64_t)m * N + n;
    const float v = splitk_sum(a.part + idx, MN, KS);
    store_out(a.y, idx, a.res ? add_rounded<T>(v, a.res[idx]) : v, a.y_dtype);
  }
  splitk_reset(&a.counters[blockIdx.x]);
}

// ---------------------------------------------------------------------------
// Segment-major variant (w4_mr16s_kernel), the default. The tile-major
// kernel above stages the M activation rows of its K range in LDS for every
// workgroup (80 KB at 16 x 2560), passes them once more for the group sums,
// and reads them back per item; at one or two row tiles per workgroup (QKV
// 3584 x 2560: 224 tiles on 256 CUs) that chain, not the weight stream, sets
// its time. Here:
//  * the weight loads of the wave go out first (a 16-byte piece of row r16
//    of every tile of the workgroup at byte 16*(l/16) of each of the wave's
//    128-k segments, contiguous segments per wave);
//  * then the segment's activations, straight into registers in the A
//    operand layout (row l%16, k 8*(l/16) .. +7 of each 32-k chunk; rows
//    past M read zeros), each loaded once per workgroup and reused by all of
//    its tiles;
//  * the group sums X_g come from one more 16x16x32 MFMA per chunk against
//    an all-ones operand (exact products, fp32 sums), lane (g, r) receiving
//    the sums of activation rows 4g .. 4g+3 that its outputs need;
//  * per group the epilogue s*D + (b - OFFSET*s)*X_g of the tile-major kernel;
//  * every wave leaves its per-tile sums in an LDS slot, and each output is
//    the sum of the waves' slots in wave order (deterministic).
// Waves: NW = ceil(SEG / NS) with NS = ceil(SEG / 16) segments each, so the
// segments divide evenly (K = 2560: 10 waves of two segments; K = 9728: 16
// waves of five, the last of one).
struct MrsArgs {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* sc;
  const uint16_t* bi;
  void* y;
  const uint16_t* res;  // 16-bit residual added to the rounded output (or null)
  int y_dtype;
  int M, N, K;
  int nt;  // row tiles of 16
  int P;   // workgroups (tile ranges)
  int TW;  // tiles of the largest workgroup
  int NS;  // segments per wave
};

struct MrsLds {
  int sb;    // (scale, bias) of the workgroup's rows [16*TW][K/G] dwords
  int part;  // per-wave tile sums [NW][TW][16][16] fp32
  int bytes;
};
__host__ __device__ __forceinline__ MrsLds mrs_lds(int K, int TW, int NW, int G) {
  MrsLds l;
  l.sb = 0;
  l.part = (TW * 16 * (K / G) * 4 + 15) & ~15;
  l.bytes = l.part + NW * TW * 1024;
  return l;
}

template <typename T, int G, int TWM, int NSM>
__global__ __launch_bounds__(1024) void w4_mr16s_kernel(MrsArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int nthr = blockDim.x, NW = nthr >> 6;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r16 = lane & 15;
  const int M = a.M, N = a.N, K = a.K;
  const int ng = K / G, SEG = K >> 7, RB = K >> 1;
  const int t0 = (int)((int64_t)blockIdx.x * a.nt / a.P);
  const int ntl = (int)((int64_t)(blockIdx.x + 1) * a.nt / a.P) - t0;  // tiles of this workgroup
  const int s0 = wave * a.NS;
  const int ns = max(0, min(a.NS, SEG - s0));                           // segments of this wave
  const MrsLds L = mrs_lds(K, a.TW, NW, G);

  const rsrc_t rx = make_rsrc(a.x, (uint32_t)M * K * 2);
  const rsrc_t rw = make_rsrc(a.w, (uint32_t)N * RB);
  const rsrc_t rs = make_rsrc(a.sc, (uint32_t)N * ng * 2);
  const rsrc_t rb = make_rsrc(a.bi, (uint32_t)N * ng * 2);

  // 1. loads, every one issued on every path (out-of-range offsets read
  // zeros): weights, activations, then the (scale, bias) pieces of the
  // workgroup's 16 * ntl contiguous rows
  u32x4_t wv[NSM][TWM];
#pragma unroll
  for (int i = 0; i < NSM; ++i)
#pragma unroll
    for (int t = 0; t < TWM; ++t) {
      const int row = 16 * (t0 + t) + r16;
      const bool ok = i < ns && t < ntl && row < N;
      wv[i][t] = buf_load16(rw, ok ? (uint32_t)row * RB + 64u * (uint32_t)(s0 + i) + 16u * g : kOob);
    }
  u32x4_t av[NSM][4];
#pragma unroll
  for (int i = 0; i < NSM; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bool ok = i < ns && r16 < M;
      av[i][c] = buf_load16(rx, ok ? 2u * (uint32_t)(r16 * K + 128 * (s0 + i) + 32 * c + 8 * g) : kOob);
    }
  const int nsp = (ntl * 16 * ng) >> 3;
  u32x4_t sr[2], br[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int pi = tid + h * nthr;
    const uint32_t off = pi < nsp ? 32u * (uint32_t)t0 * ng + 16u * pi : kOob;
    sr[h] = buf_load16(rs, off);
    br[h] = buf_load16(rb, off);
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. (scale, bias) pairs to LDS
  uint32_t* sb = reinterpret_cast<uint32_t*>(smem + L.sb);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int pi = tid + h * nthr;
    if (pi < nsp) {
      u32x4_t lo, hi;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo[e] = __builtin_amdgcn_perm(br[h][e], sr[h][e], 0x05040100u);  // (s0, b0)
        hi[e] = __builtin_amdgcn_perm(br[h][e], sr[h][e], 0x07060302u);  // (s1, b1)
      }
      *reinterpret_cast<u32x4_t*>(sb + 8 * pi) = u32x4_t{lo[0], hi[0], lo[1], hi[1]};
      *reinterpret_cast<u32x4_t*>(sb + 8 * pi + 4) = u32x4_t{lo[2], hi[2], lo[3], hi[3]};
    }
  }
  __syncthreads();

  // 3. per segment and 32-k chunk: the group-sum MFMA, one MFMA per tile,
  // and per group the scale epilogue of every tile
  const DecodeConsts dc = decode_consts<T>();
  const uint32_t one2 = T::code == SPARKQ_BF16 ? 0x3F803F80u : 0x3C003C00u;
  const u32x4_t ones = {one2, one2, one2, one2};
  f32x4_t acc[TWM];
#pragma unroll
  for (int t = 0; t < TWM; ++t) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int GPS = 128 / G;  // groups per segment
  constexpr int CPG = G / 32;   // 32-k chunks per group
#pragma unroll
  for (int i = 0; i < NSM; ++i) {
    if (i < ns) {
      const int s = s0 + i;
      // the segment's group sums first, then one tile at a time (a single
      // tile's partial product stays live across the chunks of a group)
      f32x4_t xg[GPS];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        xg[c / CPG] = mfma16x16x32<T>(av[i][c], ones,
                                      c % CPG == 0 ? f32x4_t{0.0f, 0.0f, 0.0f, 0.0f} : xg[c / CPG]);
#pragma unroll
      for (int t = 0; t < TWM; ++t) {
        if (t < ntl) {
          const u32x4_t wt = transpose_rows(wv[i][t]);
          f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            d = mfma16x16x32<T>(av[i][c], decode_w4<T>(wt[c], dc), d);
            if ((c + 1) % CPG == 0) {
              const uint32_t pair = sb[(t * 16 + r16) * ng + s * GPS + c / CPG];
              const float sf = T::to_f32((uint16_t)(pair & 0xFFFFu));
              const float bf = fmaf(-T::OFFSET, sf, T::to_f32((uint16_t)(pair >> 16)));
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(sf, d[r], fmaf(bf, xg[c / CPG][r], acc[t][r]));
              d = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            }
          }
        }
      }
    }
  }

  // 4. per-wave tile sums to LDS (every wave writes its slots, zeros when it
  // had no segment), then each output adds the waves' slots in wave order
  float* part = reinterpret_cast<float*>(smem + L.part);
#pragma unroll
  for (int t = 0; t < TWM; ++t)
    if (t < ntl)
#pragma unroll
      for (int r = 0; r < 4; ++r) part[(wave * a.TW + t) * 256 + (4 * g + r) * 16 + r16] = acc[t][r];
  __syncthreads();
  for (int e = tid; e < ntl * 256; e += nthr) {
    const int t = e >> 8, m = (e >> 4) & 15, j = e & 15;
    const int n = 16 * (t0 + t) + j;
    if (m >= M || n >= N) continue;
    float v = 0.0f;
    for (int w = 0; w < NW; ++w) v += part[(w * a.TW + t) * 256 + m * 16 + j];
    const int64_t idx = (int64_t)m * N + n;
    store_out(a.y, idx, a.res ? add_rounded<T>(v, a.res[idx]) : v, a.y_dtype);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
// Plan: 9..16 rows (from 2 with SPARKQ_W4_MR_MIN), K a multiple of 128, the
// activations, scales and run slots within 160 KB of LDS, at most 8 items per
// wave and no wave run longer than a row (so it touches at most two tiles).
// The fewest K ranges (1, 2, 4 or 8) whose activation slice fits the staging
// registers; with several, about one workgroup per CU over all ranges: down
// 2560x9728 takes 13.5 us at 16 rows and 13.3 at 12 in four ranges, against
// 17.1 and 15.5 on the skinny split-K kernel (at 8 rows two ranges took 14.4
// against its 12.7, so fewer rows stay there). Measured per projection (bf16,
// G64): QKV 3584x2560 and gate+up
// 19456x2560 take 6.9-7.1 and 14.2-14.8 us from 5 to 16 rows, against 6.1
// and 13.0 us at 5 rows, 6.2 and 14.4 at 8, 7.6 and 18.2 at 12 and 8.8 and
// 21.8 at 16 on the 4x4x4 multi-row kernel; down 2560x9728 at 5 rows 12.2
// against 9.2 us.
struct MrPlan {
  bool ok;
  int P, TW, IW, NI, KS, D;
  size_t lds, ws;
};

static MrPlan plan_mr(int64_t M, int64_t N, int64_t K, int G) {
  MrPlan p{};
  if (M < env_int("SPARKQ_W4_MR_MIN", 9) || M > 16 || env_int("SPARKQ_W4_NO_MR", 0)) return p;
  if (K % 128 != 0 || K % G != 0) return p;
  if (N * (K / 2) >= (int64_t)kOob || M * K * 2 >= (int64_t)kOob) return p;
  const int64_t ng = K / G;
  if ((N * ng * 2) % 16 != 0) return p;
  const int64_t nt = cdiv(N, 16), cus = device_cus();
  for (int KS = 1; KS <= 8; KS *= 2) {
    const int64_t Kl = K / KS, ngl = Kl / G, SEG = Kl / 128;
    if (K % KS != 0 || Kl % 128 != 0 || Kl % G != 0) continue;
    if (KS > 1 && (ngl % 2 != 0 || ng % 2 != 0 || env_int("SPARKQ_W4_MR_NO_SPLIT", 0))) continue;
    if (M * Kl / 8 > (int64_t)kMrXC * 64 * kMrNW) continue;
    p.P = (int)std::min<int64_t>(nt, KS == 1 ? cus : std::max<int64_t>(1, cus / KS));
    if (KS > 1 && p.P > kMaxCounterTiles) continue;
    p.TW = (int)cdiv(nt, p.P);
    const int64_t iw = cdiv(p.TW * SEG, kMrNW);
    if (iw > 8 || iw > SEG) continue;
    const int64_t pieces = KS == 1 ? p.TW * 16 * ng / 8 : p.TW * 16 * ngl / 2;
    if (pieces > (int64_t)kMrSP * 64 * kMrNW * (KS == 1 ? 1 : 4)) continue;
    const MrLds l = mr_lds((int)M, (int)Kl, p.TW, G);
    if (l.bytes > kMrMaxLds) continue;
    p.IW = (int)iw;
    p.NI = iw <= 2 ? 2 : (iw <= 4 ? 4 : 8);
    p.KS = KS;
    // weight items in flight per wave (SPARKQ_W4_MR_DEPTH: 1, 2, or 0 for
    // all); one measured best (M = 9 / 12 / 16 sweeps 1365 / 1397 / 1340 ->
    // 1492 / 1505 / 1458 GB/s; two 1475 / 1485 / 1430)
    const char* de = getenv("SPARKQ_W4_MR_DEPTH");
    const int dv = de ? atoi(de) : 1;
    p.D = dv == 0 || p.NI <= 2 ? p.NI : (dv == 1 ? 1 : 2);
    p.lds = (size_t)l.bytes;
    p.ws = KS > 1 ? kCounterBytes + round_up((size_t)KS * M * N * 4, 256) : 0;
    p.ok = true;
    return p;
  }
  return p;
}

template <typename T, int G, int NI, int D>
static void launch_mr_d(const MrPlan& p, const MrArgs& a, hipStream_t st) {
  auto* k = w4_mr16_kernel<T, G, NI, D>;
  // dynamic LDS above 64 KB must be enabled per kernel
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, kMrMaxLds);
  (void)attr;
  hipLaunchKernelGGL(k, dim3((unsigned)p.P, (unsigned)p.KS), dim3(64 * kMrNW), p.lds, st, a);
}
template <typename T, int G, int NI>
static void launch_mr_n(const MrPlan& p, const MrArgs& a, hipStream_t st) {
  if (p.D == NI)
    launch_mr_d<T, G, NI, NI>(p, a, st);
  else if (p.D == 1)
    launch_mr_d<T, G, NI, 1>(p, a, st);
  else
    launch_mr_d<T, G, NI, 2>(p, a, st);
}
template <typename T, int G>
static void launch_mr_g(const MrPlan& p, const MrArgs& a, hipStream_t st) {
  if (p.NI == 2)
    launch_mr_n<T, G, 2>(p, a, st);
  else if (p.NI == 4)
    launch_mr_n<T, G, 4>(p, a, st);
  else
    launch_mr_n<T, G, 8>(p, a, st);
}
template <typename T>
static void launch_mr(const MrPlan& p, int G, const MrArgs& a, hipStream_t st) {
  if (G == 32)
    launch_mr_g<T, 32>(p, a, st);
  else if (G == 64)
    launch_mr_g<T, 64>(p, a, st);
  else
    launch_mr_g<T, 128>(p, a, st);
}

// Plan of the segment-major kernel: 5..16 rows (SPARKQ_W4_MR_MIN sets the
// least), K a multiple of 128 with at most 8 segments per wave, one workgroup
// per CU over contiguous tile ranges, the (scale, bias) pieces within two per
// thread, the register arrays (tiles x segments) within 16 pieces, LDS within
// 160 KB. SPARKQ_W4_MR_TILED keeps the tile-major kernel. From 5 rows, not 9
// as the tile-major kernel: per projection at 5 / 6 / 7 / 8 rows (bf16, G64,
// 36 weight sets) QKV 3584 x 2560 took 4.98 / 5.12 / 5.23 / 5.31 us against
// 6.04 / 6.07 / 6.15 / 6.24 on the 4x4x4 multi-row streaming kernel, and the
// 2560 x 2560 linear 4.87 / 5.00 / 5.12 / 5.21 against 5.33 / 5.37 / 5.45 /
// 5.53 (2..4 rows keep the one-round kernel, equal within 0.05 us).
struct MrsPlan {
  bool ok;
  int P, TW, NS, NW, TWM, NSM;
  size_t lds;
};

static MrsPlan plan_mrs(int64_t M, int64_t N, int64_t K, int G) {
  MrsPlan p{};
  if (M < env_int("SPARKQ_W4_MR_MIN", 5) || M > 16 || env_int("SPARKQ_W4_NO_MR", 0) ||
      env_int("SPARKQ_W4_MR_TILED", 0))
    return p;
  if (K % 128 != 0 || K % G != 0) return p;
  if (N * (K / 2) >= (int64_t)kOob || M * K * 2 >= (int64_t)kOob) return p;
  const int64_t ng = K / G, SEG = K / 128;
  if ((N * ng * 2) % 16 != 0) return p;
  const int64_t nt = cdiv(N, 16), cus = device_cus();
  p.NS = (int)cdiv(SEG, 16);
  p.NW = (int)cdiv(SEG, p.NS);
  p.P = (int)std::min<int64_t>(nt, cus);
  p.TW = (int)cdiv(nt, p.P);
  // It pays where the tile-major kernel's staging outweighs its weight
  // stream: one row tile per workgroup over rows of at most 32 segments.
  // Measured per projection at 9 / 12 / 16 rows (bf16, G64, 36 weight
  // sets), segment-major against tile-major: QKV 3584 x 2560 5.3 / 5.7 /
  // 6.1 against 7.1 / 7.1 / 7.5 us; gate+up 19456 x 2560 (five tiles per
  // workgroup) 14.4 / 14.8 / 15.3 against 14.2 / 14.4 / 15.1; down 2560 x
  // 9728 (one tile, 76 segments, 311 KB of activations per workgroup)
  // 13.3 / 14.9 / 16.6 against 14.8 / 13.3 / 13.6 in four K ranges.
  // SPARKQ_W4_MR_SEG takes every shape the instantiations below fit: (1, 2),
  // (2, 2), (5, 2) and (1, 5) tiles x segments stay within the 128 VGPRs of
  // 16-wave workgroups.
  const bool all = env_int("SPARKQ_W4_MR_SEG", 0) != 0;
  if (!all && (p.TW > 1 || p.NS > 2)) return p;
  p.TWM = p.TW <= 1 ? 1 : p.TW <= 2 ? 2 : 5;
  p.NSM = p.NS <= 2 ? 2 : 5;
  if (p.NS > 5 || p.TW > 5 || (p.NSM == 5 && p.TWM > 1)) return p;
  if ((int64_t)p.TW * 16 * ng / 8 > 2LL * 64 * p.NW) return p;
  const MrsLds l = mrs_lds((int)K, p.TW, p.NW, G);
  if (l.bytes > kMrMaxLds) return p;
  p.lds = (size_t)l.bytes;
  p.ok = true;
  return p;
}

template <typename T, int G, int TWM, int NSM>
static void launch_mrs_k(const MrsPlan& p, const MrsArgs& a, hipStream_t st) {
  auto* k = w4_mr16s_kernel<T, G, TWM, NSM>;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, kMrMaxLds);
  (void)attr;
  hipLaunchKernelGGL(k, dim3((unsigned)p.P), dim3(64 * p.NW), p.lds, st, a);
}
template <typename T, int G>
static void launch_mrs_g(const MrsPlan& p, const MrsArgs& a, hipStream_t st) {
  if (p.NSM == 5)
    launch_mrs_k<T, G, 1, 5>(p, a, st);
  else if (p.TWM == 1)
    launch_mrs_k<T, G, 1, 2>(p, a, st);
  else if (p.TWM == 2)
    launch_mrs_k<T, G, 2, 2>(p, a, st);
  else
    launch_mrs_k<T, G, 5, 2>(p, a, st);
}
template <typename T>
static void launch_mrs(const MrsPlan& p, int G, const MrsArgs& a, hipStream_t st) {
  if (G == 32)
    launch_mrs_g<T, 32>(p, a, st);
  else if (G == 64)
    launch_mrs_g<T, 64>(p, a, st);
  else
    launch_mrs_g<T, 128>(p, a, st);
}

// Workspace of the plan (split counters and partials), or -1 when the shape
// is not served.
int64_t w4_mr_workspace(int64_t M, int64_t N, int64_t K, int G) {
  if (plan_mrs(M, N, K, G).ok) return 0;
  const MrPlan p = plan_mr(M, N, K, G);
  return p.ok ? (int64_t)p.ws : -1;
}

// Returns 1 when the shape is not served (the caller picks another kernel).
int w4_mr_linear(const void* x, const uint32_t* w, const void* s, const void* b, void* y,
                 int64_t M, int64_t N, int64_t K, int G, int xdt, int ydt, hipStream_t st,
                 const void* res, void* ws, size_t wsb) {
  const MrsPlan sp = plan_mrs(M, N, K, G);
  if (sp.ok) {
    MrsArgs a{};
    a.x = (const uint16_t*)x;
    a.w = w;
    a.sc = (const uint16_t*)s;
    a.bi = (const uint16_t*)b;
    a.y = y;
    a.res = (const uint16_t*)res;
    a.y_dtype = ydt;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.nt = (int)cdiv(N, 16);
    a.P = sp.P;
    a.TW = sp.TW;
    a.NS = sp.NS;
    if (xdt == SPARKQ_BF16)
      launch_mrs<BF16>(sp, G, a, st);
    else
      launch_mrs<F16>(sp, G, a, st);
    return check_launch("w4_mr16s_kernel");
  }
  const MrPlan p = plan_mr(M, N, K, G);
  if (!p.ok) return 1;
  if (p.ws > 0 && (ws == nullptr || wsb < p.ws))
    return set_error(SPARKQ_ERR_WORKSPACE, "w4a16_linear needs a workspace of %zu bytes (got %zu)",
                     p.ws, wsb);
  MrArgs a{};
  a.x = (const uint16_t*)x;
  a.w = w;
  a.sc = (const uint16_t*)s;
  a.bi = (const uint16_t*)b;
  a.y = y;
  a.res = (const uint16_t*)res;
  a.y_dtype = ydt;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.nt = (int)cdiv(N, 16);
  a.P = p.P;
  a.TW = p.TW;
  a.IW = p.IW;
  a.KS = p.KS;
  if (p.KS > 1) {
    a.counters = reinterpret_cast<unsigned*>(ws);
    a.part = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(ws) + kCounterBytes);
  }
  if (xdt == SPARKQ_BF16)
    launch_mr<BF16>(p, G, a, st);
  else
    launch_mr<F16>(p, G, a, st);
  return check_launch("w4_mr16_kernel");
}

}  // namespace sparkq
