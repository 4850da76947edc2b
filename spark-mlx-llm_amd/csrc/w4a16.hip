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
//   w4_skinny_kernel    M <= 32: weight streaming, 32 rows x 64 k per wave
//                       step, MFMA 32x32x16, in-workgroup split-K over waves,
//                       cross-workgroup split-K combined in the same launch by
//                       the last workgroup of each tile
//   xsum_kernel         group sums X_g[m] for the GEMM, layout [K/G][M]
//   w4_gemm_kernel      M > 32: 128x128x64 LDS tiles (A bf16/f16, B decoded
//                       to OFFSET+q), double-buffered, MFMA 32x32x16
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
// affine 4-bit quantizer: one thread per group
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

size_t w4a16_workspace(int64_t M, int64_t N, int64_t K, int G) {
  if (M <= 0 || N <= 0 || K <= 0 || G <= 0) return 0;
  // every workspace of this entry point starts with the counter block, so a
  // GEMM call never writes over the counters a later split-K call relies on
  if (M <= 32) {
    const SkinnyPlan p = plan_skinny(M, N, K);
    return p.S > 1 ? kCounterBytes + p.part_bytes : 0;
  }
  return kCounterBytes + round_up((size_t)(K / G) * M * 4, 256);
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

int w4a16_linear(const void* x, const uint32_t* w, const void* s, const void* b,
                 void* y, int64_t M, int64_t N, int64_t K, int G, int xdt, int ydt,
                 void* ws, size_t wsb, hipStream_t st) {
  const size_t need = w4a16_workspace(M, N, K, G);
  if (need > 0 && (ws == nullptr || wsb < need))
    return set_error(SPARKQ_ERR_WORKSPACE,
                     "w4a16_linear needs a workspace of %zu bytes (got %zu)", need, wsb);
  if (M <= 32) {
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
  float* xs = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(ws) + kCounterBytes);
  if (xdt == SPARKQ_BF16)
    launch_gemm<BF16>(G, x, w, s, b, xs, y, ydt, (int)M, (int)N, (int)K, st);
  else
    launch_gemm<F16>(G, x, w, s, b, xs, y, ydt, (int)M, (int)N, (int)K, st);
  return check_launch("w4_gemm_kernel");
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
