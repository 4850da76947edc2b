// w8a8.hip -- W8A8 projection on gfx950: per-token int8 activations,
// per-channel int8 weights, exact int32 accumulation on the int8 MFMA.
//
// Kernels
//   i8_gemv_kernel       M <= 2 decode (M <= 4 when K % 64 != 0; 16-bit
//                        activations up to K = 4096, longer rows go to the
//                        rows kernel's one launch): whole
//                        rows per workgroup, 4 rows x
//                        256 bytes per load, v_dot4_i32_i8, activation
//                        quantizer fused (one launch per projection)
//   i8_gemvq_kernel      M = 2 over whole 256-k spans up to K = 2560: one
//                        row quad per wave over its whole row, quantizer fused
//   i8_gemv_stream_kernel  M = 1 over rows longer than 4096 k, M = 2 over
//                        runs of at most 48 KB a CU: one 16-wave workgroup
//                        per CU streams a contiguous run of weight rows in
//                        1 KB items, all loads in flight; quantizer fused
//   a8_quantize_kernel   one workgroup per token row (a8_quantize_reg_kernel
//                        for rows of up to 32 KB: one load round trip): amax, scale = amax/127
//                        (1 when 0), q = clamp(rint(x/scale), -127, 127);
//                        bit-exact with X/src/kernels/w8a8_quantize.metal:11-27
//   i8_skinny_kernel     32 weight rows per workgroup, 4 waves split K; lane
//                        (n = l%32, j = l/32) feeds 16 bytes of row n straight
//                        into v_mfma_i32_32x32x32_i8; the A operand is the
//                        matching 16 bytes of the int8 activations from LDS;
//                        m-blocks of 32 rows go to grid.z. Output is either the
//                        raw int32 sums or the fused epilogue
//                        fmaf(float(acc)*sa[m], sw[n], bias[n]); splits of K
//                        combine in the same launch (the last workgroup of a
//                        tile sums the int32 partials).
//   i8_rows_kernel       3..16 token rows: 16 weight rows per workgroup, 8
//                        (16) waves split K, both operands straight from
//                        global memory into v_mfma_i32_16x16x64_i8.
//   i8_rows_q_kernel     3..16 token rows over at least two row tiles per
//                        workgroup slot (gate+up): one round of workgroups
//                        owning up to three tiles each, the activation tile
//                        staged once per workgroup in LDS.
#include "common.h"

namespace sparkq {

// ---------------------------------------------------------------------------
// per-token quantizer
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void a8_quantize_kernel(
    const void* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ scales,
    int64_t K, int x_dtype) {
  __shared__ float wmax[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  float amax = 0.0f;
  for (int64_t k = tid; k < K; k += 256) amax = fmaxf(amax, fabsf(load_in(x, row * K + k, x_dtype)));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  if ((tid & 63) == 0) wmax[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
  if (tid == 0) scales[row] = scale;
  for (int64_t k = tid; k < K; k += 256) {
    float v = __builtin_rintf(load_in(x, row * K + k, x_dtype) / scale);
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    q[row * K + k] = (int8_t)v;
  }
}

// ---------------------------------------------------------------------------
// int8 weight-streaming MFMA kernel
// ---------------------------------------------------------------------------
enum I8Out { kOutRaw = 0, kOutEpilogue = 1 };

struct I8Args {
  const int8_t* a;      // [M,K] int8 activations
  const int8_t* b;      // [N,K] int8 weights
  int32_t* c_raw;       // [M,N] (kOutRaw)
  int32_t* part;        // [S][M][N] partials (S > 1)
  unsigned* counters;   // per (m-block, n-tile), zero on entry and exit (S > 1)
  void* y;              // [M,N] (kOutEpilogue)
  const float* sa;      // [M]
  const float* sw;      // [N]
  const void* bias;     // [N] or null
  int bias_dtype;
  int y_dtype;
  int M, N, K;
  int cps;              // 32-k chunks per split
  int slab;             // 32-k chunks per LDS slab of activations
  int S;
  int mode;
  int wgs;              // workgroups of the one-round rows kernel
  int tiles_n, tiles;   // tiled GEMM: column tiles, tiles (split items are piece-major)
  int gm;               // tiled GEMM: tile rows per group of the tile order (0: row-major)
  int full;             // tiled GEMM: items [0, full) are whole tiles, the tiles past them split in S
  // one launch with the quantizer (3..16 rows): producer workgroups [0, np)
  // write the int8 rows of x into a (and their scales into sa); counters[0]
  // counts the rows written, counters[1] the workgroups done (both zero on
  // entry and exit)
  const void* x;
  int xt;               // 0 bf16, 1 fp16
  int np;               // producer workgroups (0: a already holds the int8 rows)
  int spin;             // polls of counters[0] before a workgroup quantizes itself
};

__device__ __forceinline__ i32x16_t mfma_i8(u32x4_t a, u32x4_t b, i32x16_t c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4_t, a),
                                               __builtin_bit_cast(i32x4_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ void i8_store(const I8Args& args, int gm, int nn, int32_t s) {
  if (args.mode == kOutRaw) {
    args.c_raw[(int64_t)gm * args.N + nn] = s;
  } else {
    const float bias = args.bias ? load_in(args.bias, nn, args.bias_dtype) : 0.0f;
    const float t = (float)s * args.sa[gm];
    store_out(args.y, (int64_t)gm * args.N + nn, fmaf(t, args.sw[nn], bias), args.y_dtype);
  }
}

constexpr int kI8U = 8;

__global__ __launch_bounds__(256, 2) void i8_skinny_kernel(I8Args args) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ int32_t red[4][16][64];
  __shared__ int s_last;
  constexpr int U = kI8U;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane >> 5;
  const int M = args.M, N = args.N, K = args.K;
  const int n0 = blockIdx.x * 32;
  const int split = blockIdx.y;
  const int m0 = blockIdx.z * 32;
  const int mrows = min(32, M - m0);
  const int nchunks = K >> 5;
  const int c_begin = split * args.cps;
  const int nc = min(args.cps, nchunks - c_begin);

  // the split's x rows live in LDS in slabs of at most args.slab chunks
  const int pitch = min(nc, args.slab) * 32 + 16;
  int8_t* xs = reinterpret_cast<int8_t*>(smem);

  const int n = n0 + (lane & 31);
  const int nr = n < N ? n : N - 1;
  const int8_t* brow = args.b + (int64_t)nr * K + (int64_t)c_begin * 32 + 16 * j;

  u32x4_t wa[U], wb[U];
  int lim = 0;  // end (exclusive) of the chunks of the current slab
  auto load_batch = [&](int cl0, u32x4_t* wv) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int cl = cl0 + 4 * u;
      if (cl < lim) wv[u] = *reinterpret_cast<const u32x4_t*>(brow + (int64_t)cl * 32);
    }
  };

  const int am = lane & 31;
  const bool a_ok = am < mrows;
  i32x16_t acc = {};

  for (int s0 = 0; s0 < nc; s0 += args.slab) {
    lim = min(nc, s0 + args.slab);
    load_batch(s0 + wave, wa);
    load_batch(s0 + wave + 4 * U, wb);
    {
      const int pieces = (lim - s0) * 2;  // 16-byte pieces per row
      for (int p = tid; p < mrows * pieces; p += 256) {
        const int m = p / pieces, pc = p - m * pieces;
        *reinterpret_cast<u32x4_t*>(xs + m * pitch + pc * 16) = *reinterpret_cast<const u32x4_t*>(
            args.a + (int64_t)(m0 + m) * K + (int64_t)(c_begin + s0) * 32 + pc * 16);
      }
    }
    __syncthreads();
    const int8_t* arow = xs + (a_ok ? am : 0) * pitch + 16 * j - s0 * 32;
    auto compute_batch = [&](int cl0, const u32x4_t* wv) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int cl = cl0 + 4 * u;
        if (cl < lim) {
          u32x4_t av = {0u, 0u, 0u, 0u};
          if (a_ok) av = *reinterpret_cast<const u32x4_t*>(arow + cl * 32);
          acc = mfma_i8(av, wv[u], acc);
        }
      }
    };
    for (int base = s0 + wave; base < lim; base += 8 * U) {
      compute_batch(base, wa);
      load_batch(base + 8 * U, wa);
      compute_batch(base + 4 * U, wb);
      load_batch(base + 12 * U, wb);
    }
    __syncthreads();  // the slab is consumed before the next one is staged
  }

#pragma unroll
  for (int v = 0; v < 16; ++v) red[wave][v][lane] = acc[v];
  __syncthreads();
  const int64_t MN = (int64_t)M * N;
  for (int e = tid; e < 16 * 64; e += 256) {
    const int v = e >> 6, l = e & 63;
    const int m = mfma32_row(l, v);
    const int nn = n0 + (l & 31);
    if (m < mrows && nn < N) {
      const int32_t s = red[0][v][l] + red[1][v][l] + red[2][v][l] + red[3][v][l];
      if (args.S == 1)
        i8_store(args, m0 + m, nn, s);
      else
        splitk_store(&args.part[split * MN + (int64_t)(m0 + m) * N + nn], s);
    }
  }
  if (args.S == 1) return;

  // split-K: the last workgroup of this (m-block, n-tile) sums the partials
  const int tile = blockIdx.z * gridDim.x + blockIdx.x;
  if (!splitk_arrive(&args.counters[tile], args.S, &s_last)) return;
  for (int e = tid; e < mrows * 32; e += 256) {
    const int gm = m0 + (e >> 5), nn = n0 + (e & 31);
    if (nn < N) i8_store(args, gm, nn, splitk_sum(args.part + (int64_t)gm * N + nn, MN, args.S));
  }
  splitk_reset(&args.counters[tile]);
}

// ---------------------------------------------------------------------------
// decode GEMV (M <= 2; M <= 4 when K % 64 != 0), activation quantizer fused
// ---------------------------------------------------------------------------
// A workgroup owns R whole weight rows. Lane l = 4b + j loads the 16 bytes at
// byte 16b of a 256-byte span of weight row 4q+j (4 rows x 256 contiguous
// bytes per load instruction) and multiplies them by the 16 matching int8
// activations of each row m with four v_dot4_i32_i8; int32 sums are exact in
// any order, so the sixteen lanes of a row and the span groups of a row quad
// are added by shuffles and LDS. The workgroup quantizes the activations
// itself (per-token amax over the whole row, scale = amax/127 with IEEE
// division, rint, clamp to +-127, as a8_quantize_kernel), so one launch does
// the whole projection. The weights are the only per-wave global loads; the
// activations are staged once per workgroup through LDS. All loads are
// bounds-checked buffer loads issued before any arithmetic.
struct I8GemvArgs {
  const void* x;        // [M,K] activations in x_dtype, or int8 for the raw mode
  const int8_t* w;      // [N,K]
  const float* sw;      // [N]
  const void* bias;     // [N] or null
  void* y;              // [M,N] (epilogue)
  int32_t* c_raw;       // [M,N] (raw)
  int x_dtype, bias_dtype, y_dtype;
  int M, N, K;
  int SG, USr, R;
  int mode;
  int nq, P;  // one-round kernel: row quads, workgroups
};

constexpr int kI8XP = 4;  // staged 16-byte activation pieces per thread, at most

// x element e of a 16-byte piece as fp32 (XT: 0 bf16, 1 f16, 2 f32)
template <int XT>
__device__ __forceinline__ float piece_elem(const u32x4_t& v, int e) {
  if constexpr (XT == 2) return __uint_as_float(v[e]);
  const uint32_t word = v[e >> 1];
  const uint16_t h = (e & 1) ? (uint16_t)(word >> 16) : (uint16_t)(word & 0xFFFFu);
  return XT == 0 ? bf16_to_f32(h) : f16_to_f32(h);
}

// Sum over the 64 lanes of a wave (int32, exact): quads by DPP, the sixteen
// quads by row rotations and the row and half swaps; lane 0's value.
__device__ __forceinline__ int wave_sum_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x124, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false);
  const auto r16 = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
  v = (int)r16[0] + (int)r16[1];
  const auto r32 = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
  return __builtin_amdgcn_readfirstlane((int)r32[0] + (int)r32[1]);
}

// Maximum over the 64 lanes of a wave (fmaxf: a NaN lane is ignored, as in a
// chain of fmaxf), lane 0's value.
__device__ __forceinline__ float wave_max(float v) {
  v = max_row16(v);
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float m = fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(m)));
}

// Per-token amax of the staged activation pieces (piece pi of token row
// pi*EP/K): each thread's maxima per row, reduced over the wave, then one
// LDS atomic max per wave and row (exact in any order). All lanes active.
template <int MQ, int NP, int XT>
__device__ __forceinline__ void staged_amax(const u32x4_t (&xr)[NP], int nxp, int K, unsigned* amax) {
  constexpr int EP = XT == 2 ? 4 : 8;
  const int tid = threadIdx.x, NT = blockDim.x;
  float mx[MQ];
#pragma unroll
  for (int m = 0; m < MQ; ++m) mx[m] = 0.0f;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int pi = tid + i * NT;
    if (pi < nxp) {
      float v = 0.0f;
#pragma unroll
      for (int e = 0; e < EP; ++e) v = fmaxf(v, fabsf(piece_elem<XT>(xr[i], e)));
      const int r = (pi * EP) / K;
#pragma unroll
      for (int m = 0; m < MQ; ++m)
        if (r == m) mx[m] = fmaxf(mx[m], v);
    }
  }
#pragma unroll
  for (int m = 0; m < MQ; ++m) {
    const float w = wave_max(mx[m]);
    if ((tid & 63) == 0)
      __hip_atomic_fetch_max(&amax[m], __float_as_uint(w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

template <int MQ, int US, int NW, int XT>  // XT 3: int8 activations (raw int32 mode)
__global__ __launch_bounds__(64 * NW) void i8_gemv_kernel(I8GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int NT = 64 * NW;
  constexpr int ES = XT == 2 ? 4 : (XT == 3 ? 1 : 2);   // activation element bytes
  constexpr int EP = 16 / ES;                            // elements per piece
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = lane >> 2, j = lane & 3;
  const int M = a.M, N = a.N, K = a.K, SG = a.SG, R = a.R;
  const int U = (K + 255) >> 8;
  const int r0 = blockIdx.x * R;
  const int sg = wave % SG;
  const int q = (r0 >> 2) + wave / SG;
  const int u0 = sg * a.USr;
  const int ns = min(a.USr, U - u0);
  int8_t* xq = reinterpret_cast<int8_t*>(smem);                     // [M][K]
  unsigned* amax = reinterpret_cast<unsigned*>(smem + ((M * K + 15) & ~15));
  int32_t* red = reinterpret_cast<int32_t*>(amax + 4);               // [NW][4][4]

  const rsrc_t rx = make_rsrc(a.x, (uint32_t)M * K * ES);
  const rsrc_t rw = make_rsrc(a.w, (uint32_t)N * K);

  // 1. staging loads of the activations
  const int nxp = (M * K * ES) >> 4;
  u32x4_t xr[kI8XP];
#pragma unroll
  for (int i = 0; i < kI8XP; ++i) {
    const int pi = tid + i * NT;
    // waves with no piece skip the instruction (wave-uniform condition)
    if (i * NT + 64 * wave < nxp) xr[i] = buf_load16(rx, pi < nxp ? 16u * pi : kOob);
  }
  // 2. the wave's weights: one row quad x US spans
  u32x4_t wv[US];
  {
    const int row = 4 * q + j;
#pragma unroll
    for (int s = 0; s < US; ++s) {
      const int p = 256 * (u0 + s) + 16 * b;
      const bool ok = row < N && s < ns && p + 16 <= K;
      wv[s] = buf_load16(rw, ok ? (uint32_t)row * K + p : kOob);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 3. per-token amax (exact in any order), then the quantized rows in LDS
  if (tid < 4) amax[tid] = 0u;
  __syncthreads();
  if constexpr (XT != 3) {
    staged_amax<MQ, kI8XP, XT>(xr, nxp, K, amax);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < kI8XP; ++i) {
    const int pi = tid + i * NT;
    if (pi < nxp) {
      if constexpr (XT == 3) {
        *reinterpret_cast<u32x4_t*>(xq + 16 * pi) = xr[i];
      } else {
        const float am = __uint_as_float(amax[(pi * EP) / K]);
        const float scale = am > 0.0f ? am / 127.0f : 1.0f;
        uint32_t packed[EP / 4];
#pragma unroll
        for (int e = 0; e < EP / 4; ++e) packed[e] = 0u;
#pragma unroll
        for (int e = 0; e < EP; ++e) {
          float v = __builtin_rintf(piece_elem<XT>(xr[i], e) / scale);
          v = fminf(fmaxf(v, -127.0f), 127.0f);
          packed[e >> 2] |= ((uint32_t)(int32_t)v & 0xFFu) << (8 * (e & 3));
        }
        if constexpr (EP == 8) {
          *reinterpret_cast<uint2*>(xq + 8 * pi) = uint2{packed[0], packed[1]};
        } else {
          *reinterpret_cast<uint32_t*>(xq + 4 * pi) = packed[0];
        }
      }
    }
  }
  __syncthreads();

  // 4. int8 dot products, 16 activations x 16 weights per lane per span
  int32_t acc[MQ];
#pragma unroll
  for (int m = 0; m < MQ; ++m) acc[m] = 0;
#pragma unroll
  for (int s = 0; s < US; ++s) {
    const int p = 256 * (u0 + s) + 16 * b;
    if (s < ns && p + 16 <= K) {
#pragma unroll
      for (int m = 0; m < MQ; ++m) {
        if (m < M) {
          const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(xq + m * K + p);
          int32_t t = acc[m];
          t = __builtin_amdgcn_sdot4((int)wv[s].x, (int)xv.x, t, false);
          t = __builtin_amdgcn_sdot4((int)wv[s].y, (int)xv.y, t, false);
          t = __builtin_amdgcn_sdot4((int)wv[s].z, (int)xv.z, t, false);
          t = __builtin_amdgcn_sdot4((int)wv[s].w, (int)xv.w, t, false);
          acc[m] = t;
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MQ; ++m) {
    int32_t v = acc[m];
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 8);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    acc[m] = v;
  }
  if (SG > 1) {
    if (lane < 4) {
#pragma unroll
      for (int m = 0; m < MQ; ++m) red[(wave * 4 + lane) * 4 + m] = acc[m];
    }
    __syncthreads();
    if (sg != 0) return;
    if (lane < 4) {
#pragma unroll
      for (int m = 0; m < MQ; ++m)
        for (int o = 1; o < SG; ++o) acc[m] += red[((wave + o) * 4 + lane) * 4 + m];
    }
  }
  // 5. epilogue: lanes 0..3 hold rows 4q..4q+3
  if (lane < 4) {
    const int row = 4 * q + lane;
    if (row < N) {
      float sw = 0.0f, bias = 0.0f;
      if (a.mode == kOutEpilogue) {
        sw = a.sw[row];
        bias = a.bias ? load_in(a.bias, row, a.bias_dtype) : 0.0f;
      }
#pragma unroll
      for (int m = 0; m < MQ; ++m) {
        if (m < M) {
          if (a.mode == kOutRaw) {
            a.c_raw[(int64_t)m * N + row] = acc[m];
          } else {
            const float am = __uint_as_float(amax[m]);
            const float sa = am > 0.0f ? am / 127.0f : 1.0f;
            store_out(a.y, (int64_t)m * N + row, fmaf((float)acc[m] * sa, sw, bias), a.y_dtype);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// streaming int8 GEMV (M <= 2, rows of at least 1024 k), quantizer fused
// ---------------------------------------------------------------------------
// One workgroup of 16 waves per CU owns the rows [i*N/P, (i+1)*N/P), whose
// weights are one contiguous run of bytes. The run is dealt to the waves in
// 1 KB items (lane l: bytes 16l..16l+15 of the item; item t to wave t % 16),
// and every weight load of a wave is issued at the start, right after the
// activation staging loads, so each CU streams the same bytes with all of
// them in flight. The workgroup quantizes the activations itself (per-token
// amax over the whole row, scale = amax/127 with IEEE division, rint, clamp
// to +-127, as a8_quantize_kernel) into LDS. Each lane meets its 16 weights
// with the 16 activations of their columns in four v_dot4_i32_i8 per token
// row; an item covers at most two weight rows (K >= 1024), whose lane sums
// are added over the wave and into the rows' LDS sums (int32 addition is
// exact in any order, so the output equals i8_gemv_kernel's bit for bit).
constexpr int kI8SXP = 4;  // staged 16-byte activation pieces per thread, at most

template <int MQ, int NI, int XT>
__global__ __launch_bounds__(1024) void i8_gemv_stream_kernel(I8GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int NW = 16, NT = 64 * NW;
  constexpr int ES = XT == 2 ? 4 : 2;  // activation element bytes
  constexpr int EP = 16 / ES;          // elements per piece
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = a.N, K = a.K;
  const int r0 = (int)((int64_t)blockIdx.x * N / gridDim.x);
  const int r1 = (int)((int64_t)(blockIdx.x + 1) * N / gridDim.x);
  const int nr = r1 - r0;
  const uint32_t base = (uint32_t)r0 * K;    // first byte of the run
  const uint32_t B = (uint32_t)nr * K;       // bytes of the run
  const int nit = (int)((B + 1023u) >> 10);  // items
  int8_t* xq = reinterpret_cast<int8_t*>(smem);                    // [MQ][K]
  unsigned* amax = reinterpret_cast<unsigned*>(smem + ((MQ * K + 15) & ~15));
  int* rsum = reinterpret_cast<int*>(amax + 4);                     // [nr][MQ]

  const rsrc_t rx = make_rsrc(a.x, (uint32_t)MQ * K * ES);
  const rsrc_t rw = make_rsrc(a.w, (uint32_t)N * K);

  // 1. staging loads of the activations (a wave with no piece skips them)
  const int nxp = (MQ * K * ES) >> 4;
  u32x4_t xr[kI8SXP];
#pragma unroll
  for (int i = 0; i < kI8SXP; ++i) {
    const int pi = tid + i * NT;
    if (i * NT + 64 * wave < nxp) xr[i] = buf_load16(rx, pi < nxp ? 16u * pi : kOob);
  }
  // 2. every weight load of the wave; bytes past the run read nothing
  u32x4_t wv[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const uint32_t o = 1024u * (uint32_t)(wave + NW * i) + 16u * lane;
    wv[i] = buf_load16(rw, o < B ? base + o : kOob);
  }
  __builtin_amdgcn_sched_barrier(0);

  // 3. per-token amax (exact in any order), then the quantized rows in LDS
  if (tid < 4) amax[tid] = 0u;
  for (int t = tid; t < nr * MQ; t += NT) rsum[t] = 0;
  __syncthreads();
  staged_amax<MQ, kI8SXP, XT>(xr, nxp, K, amax);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kI8SXP; ++i) {
    const int pi = tid + i * NT;
    if (pi < nxp) {
      const float am = __uint_as_float(amax[(pi * EP) / K]);
      const float scale = am > 0.0f ? am / 127.0f : 1.0f;
      uint32_t packed[EP / 4];
#pragma unroll
      for (int e = 0; e < EP / 4; ++e) packed[e] = 0u;
#pragma unroll
      for (int e = 0; e < EP; ++e) {
        float v = __builtin_rintf(piece_elem<XT>(xr[i], e) / scale);
        v = fminf(fmaxf(v, -127.0f), 127.0f);
        packed[e >> 2] |= ((uint32_t)(int32_t)v & 0xFFu) << (8 * (e & 3));
      }
      if constexpr (EP == 8) {
        *reinterpret_cast<uint2*>(xq + 8 * pi) = uint2{packed[0], packed[1]};
      } else {
        *reinterpret_cast<uint32_t*>(xq + 4 * pi) = packed[0];
      }
    }
  }
  __syncthreads();

  // 4. the wave's items in issue order: lane row and column by a float
  // quotient corrected once (o < 2^24), the item's first row from lane 0
  const float invk = 1.0f / (float)K;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int it = wave + NW * i;
    if (it < nit) {
      const int o = 1024 * it + 16 * lane;
      int rl = (int)((float)o * invk);
      int col = o - rl * K;
      if (col >= K) { col -= K; ++rl; }
      if (col < 0) { col += K; --rl; }
      const int ra = __builtin_amdgcn_readfirstlane(rl);
      const bool two = __builtin_amdgcn_readlane(rl, 63) != ra && ra + 1 < nr;
#pragma unroll
      for (int m = 0; m < MQ; ++m) {
        const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(xq + m * K + col);
        int t = 0;
        t = __builtin_amdgcn_sdot4((int)wv[i].x, (int)xv.x, t, false);
        t = __builtin_amdgcn_sdot4((int)wv[i].y, (int)xv.y, t, false);
        t = __builtin_amdgcn_sdot4((int)wv[i].z, (int)xv.z, t, false);
        t = __builtin_amdgcn_sdot4((int)wv[i].w, (int)xv.w, t, false);
        const int ta = rl == ra ? t : 0;
        const int sa = wave_sum_i32(ta);
        if (lane == 0) atomicAdd(&rsum[ra * MQ + m], sa);
        if (two) {
          const int sb = wave_sum_i32(t - ta);
          if (lane == 0) atomicAdd(&rsum[(ra + 1) * MQ + m], sb);
        }
      }
    }
  }
  __syncthreads();

  // 5. epilogue: one thread per (row, token row)
  for (int t = tid; t < nr * MQ; t += NT) {
    const int rl = t / MQ, m = t - rl * MQ, row = r0 + rl;
    const float sw = a.sw[row];
    const float bias = a.bias ? load_in(a.bias, row, a.bias_dtype) : 0.0f;
    const float am = __uint_as_float(amax[m]);
    const float sa = am > 0.0f ? am / 127.0f : 1.0f;
    store_out(a.y, (int64_t)m * N + row, fmaf((float)rsum[t] * sa, sw, bias), a.y_dtype);
  }
}

// ---------------------------------------------------------------------------
// one-round int8 GEMV (M <= 2, rows of up to 2560 k), quantizer fused
// ---------------------------------------------------------------------------
// The layout of the W4 and W8A16 one-round GEMVs: every workgroup owns a
// contiguous range of row quads, one quad per wave, and the grid holds every
// quad at once. The workgroup stages and quantizes the activations as
// i8_gemv_kernel does (per-token amax, IEEE division, rint, clamp); a wave
// walks its quad's 256-byte spans in order (lane 4b+j: bytes 256s + 16b of
// row 4q+j) with D spans' loads in flight (the first D ahead of the staging
// loads, each later one issued as the span D before it is taken up; all of
// them right after the staging loads when D = U), four v_dot4_i32_i8 per
// span and token row, and adds the quad's lanes by shuffles (int32: exact,
// so the output equals i8_gemv_kernel's bit for bit).
constexpr int kI8QXP = 4;  // staged 16-byte activation pieces per thread, at most

template <int MQ, int U, int D, int XT>
__global__ __launch_bounds__(1024) void i8_gemvq_kernel(I8GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int ES = XT == 2 ? 4 : 2;  // activation element bytes
  constexpr int EP = 16 / ES;          // elements per piece
  const int NT = blockDim.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = lane >> 2, j = lane & 3;
  const int N = a.N, K = a.K;
  const int ns = K >> 8;  // spans per row (<= U)
  const int qa = (int)((int64_t)blockIdx.x * a.nq / a.P);
  const int nql = (int)((int64_t)(blockIdx.x + 1) * a.nq / a.P) - qa;
  int8_t* xq = reinterpret_cast<int8_t*>(smem);                    // [MQ][K]
  unsigned* amax = reinterpret_cast<unsigned*>(smem + ((MQ * K + 15) & ~15));

  const rsrc_t rx = make_rsrc(a.x, (uint32_t)MQ * K * ES);
  const rsrc_t rw = make_rsrc(a.w, (uint32_t)N * K);

  const bool has_quad = wave < nql;
  const int row = 4 * (qa + wave) + j;
  const uint32_t wbase = has_quad && row < N ? (uint32_t)row * K + 16u * b : kOob;
  u32x4_t wv[U];
  if constexpr (D < U) {
#pragma unroll
    for (int s = 0; s < D; ++s) wv[s] = buf_load16(rw, s < ns ? wbase + 256u * s : kOob);
  }
  // staging loads: the MQ rows' 16-byte pieces; a wave with none skips them
  const int nxp = (MQ * K * ES) >> 4;
  u32x4_t xr[kI8QXP];
#pragma unroll
  for (int i = 0; i < kI8QXP; ++i) {
    const int pi = tid + i * NT;
    if (i * NT + 64 * wave < nxp) xr[i] = buf_load16(rx, pi < nxp ? 16u * pi : kOob);
  }
  if constexpr (D == U) {
#pragma unroll
    for (int s = 0; s < U; ++s) wv[s] = buf_load16(rw, s < ns ? wbase + 256u * s : kOob);
  }
  // keep every load above ahead of the arithmetic below
  __builtin_amdgcn_sched_barrier(0);

  // per-token amax, then the quantized rows in LDS
  if (tid < 4) amax[tid] = 0u;
  __syncthreads();
  staged_amax<MQ, kI8QXP, XT>(xr, nxp, K, amax);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kI8QXP; ++i) {
    const int pi = tid + i * NT;
    if (pi < nxp) {
      const float am = __uint_as_float(amax[(pi * EP) / K]);
      const float scale = am > 0.0f ? am / 127.0f : 1.0f;
      uint32_t packed[EP / 4];
#pragma unroll
      for (int e = 0; e < EP / 4; ++e) packed[e] = 0u;
#pragma unroll
      for (int e = 0; e < EP; ++e) {
        float v = __builtin_rintf(piece_elem<XT>(xr[i], e) / scale);
        v = fminf(fmaxf(v, -127.0f), 127.0f);
        packed[e >> 2] |= ((uint32_t)(int32_t)v & 0xFFu) << (8 * (e & 3));
      }
      if constexpr (EP == 8) {
        *reinterpret_cast<uint2*>(xq + 8 * pi) = uint2{packed[0], packed[1]};
      } else {
        *reinterpret_cast<uint32_t*>(xq + 4 * pi) = packed[0];
      }
    }
  }
  __syncthreads();
  if (!has_quad) return;

  int32_t acc[MQ];
#pragma unroll
  for (int m = 0; m < MQ; ++m) acc[m] = 0;
#pragma unroll
  for (int s = 0; s < U; ++s) {
    // span s + D's load goes out as span s is taken up
    if (s + D < U) wv[s + D] = buf_load16(rw, s + D < ns ? wbase + 256u * (s + D) : kOob);
    if (s < ns) {
      const int p = 256 * s + 16 * b;
#pragma unroll
      for (int m = 0; m < MQ; ++m) {
        const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(xq + m * K + p);
        int32_t t = acc[m];
        t = __builtin_amdgcn_sdot4((int)wv[s].x, (int)xv.x, t, false);
        t = __builtin_amdgcn_sdot4((int)wv[s].y, (int)xv.y, t, false);
        t = __builtin_amdgcn_sdot4((int)wv[s].z, (int)xv.z, t, false);
        t = __builtin_amdgcn_sdot4((int)wv[s].w, (int)xv.w, t, false);
        acc[m] = t;
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MQ; ++m) {
    int32_t v = acc[m];
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 8);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    acc[m] = v;
  }
  // lanes 0..3 hold rows 4q..4q+3
  const int orow = 4 * (qa + wave) + lane;
  if (lane < 4 && orow < N) {
    const float sw = a.sw[orow];
    const float bias = a.bias ? load_in(a.bias, orow, a.bias_dtype) : 0.0f;
#pragma unroll
    for (int m = 0; m < MQ; ++m) {
      const float am = __uint_as_float(amax[m]);
      const float sa = am > 0.0f ? am / 127.0f : 1.0f;
      store_out(a.y, (int64_t)m * N + orow, fmaf((float)acc[m] * sa, sw, bias), a.y_dtype);
    }
  }
}


// Per-token quantizer for rows of up to 2048 16-byte pieces: every load of
// the row is issued at once into registers (one round trip instead of one
// per element), the amax reduced across the workgroup, and the codes
// written from the same registers. The formula is a8_quantize_kernel's.
constexpr int kQPieces = 8;  // 16-byte pieces per thread

template <int XT>
__global__ __launch_bounds__(256) void a8_quantize_reg_kernel(const void* __restrict__ x,
                                                              int8_t* __restrict__ q,
                                                              float* __restrict__ scales, int K) {
  constexpr int ES = XT == 2 ? 4 : 2, EP = 16 / ES;
  __shared__ float wmax[4];
  const int row = blockIdx.x, tid = threadIdx.x;
  const int np = K * ES / 16;
  const rsrc_t rx = make_rsrc(reinterpret_cast<const unsigned char*>(x) + (int64_t)row * K * ES,
                              (uint32_t)(K * ES));
  u32x4_t v[kQPieces];
#pragma unroll
  for (int i = 0; i < kQPieces; ++i) {
    const int p = tid + 256 * i;
    v[i] = buf_load16(rx, p < np ? 16u * (uint32_t)p : kOob);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < kQPieces; ++i)
#pragma unroll
    for (int e = 0; e < EP; ++e) amax = fmaxf(amax, fabsf(piece_elem<XT>(v[i], e)));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  if ((tid & 63) == 0) wmax[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
  if (tid == 0) scales[row] = scale;
  int8_t* qrow = q + (int64_t)row * K;
#pragma unroll
  for (int i = 0; i < kQPieces; ++i) {
    const int p = tid + 256 * i;
    if (p < np) {
      uint32_t packed[EP / 4];
#pragma unroll
      for (int e = 0; e < EP / 4; ++e) packed[e] = 0u;
#pragma unroll
      for (int e = 0; e < EP; ++e) {
        float t = __builtin_rintf(piece_elem<XT>(v[i], e) / scale);
        t = fminf(fmaxf(t, -127.0f), 127.0f);
        packed[e >> 2] |= ((uint32_t)(int32_t)t & 0xFFu) << (8 * (e & 3));
      }
      if constexpr (EP == 8)
        *reinterpret_cast<uint2*>(qrow + 8 * p) = uint2{packed[0], packed[1]};
      else
        *reinterpret_cast<uint32_t*>(qrow + 4 * p) = packed[0];
    }
  }
}

// ---------------------------------------------------------------------------
// one launch for 3..16 token rows: the quantizer runs in producer
// workgroups while the others stream their weights
// ---------------------------------------------------------------------------
// The first np workgroups of the grid each quantize rows b, b + np, ... of x
// (one whole row per pass: per-token amax, scale = amax/127 with IEEE
// division, rint, clamp to +-127, as a8_quantize_kernel) into the int8
// buffer with stores at the device coherence level (sc1), count the rows
// done, and exit. Every other workgroup issues its weight loads, then polls
// the count (at most args.spin times); past the bound it quantizes all rows
// itself, writing the same bytes, so no workgroup waits on one that may not
// be resident. Its activation loads and scale reads then go to the same
// coherence level. The last workgroup to finish resets both counters.
constexpr int kA8PP = 4;  // 16-byte activation pieces per producer thread, at most
constexpr int kSc1 = 16;  // buffer cache policy sc1: the device coherence level (split-K partials use it too)

// LEAN: one piece at a time, loaded twice (the fallback, which runs while a
// workgroup holds its weights in registers)
template <int XT, bool LEAN = false>
__device__ void a8_produce_row(const I8Args& a, int row, float* red) {
  typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
  const int K = a.K, np = K >> 3, NT = blockDim.x, tid = threadIdx.x;
  if constexpr (!LEAN) {
    // a workgroup narrower than the row's single pass needs (the rows
    // kernel's width set below 512 threads) takes the looping form, which
    // covers every piece whatever the width
    if (np > kA8PP * NT) {
      a8_produce_row<XT, true>(a, row, red);
      return;
    }
  }
  const rsrc_t rx = make_rsrc(reinterpret_cast<const unsigned char*>(a.x) + (int64_t)row * K * 2,
                              (uint32_t)K * 2);
  constexpr int NV = LEAN ? 1 : kA8PP;
  u32x4_t v[NV];
  float mx = 0.0f;
  if constexpr (LEAN) {
    for (int p = tid; p < np; p += NT) {
      const u32x4_t t = buf_load16(rx, 16u * (uint32_t)p);
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(piece_elem<XT>(t, e)));
    }
  } else {
#pragma unroll
    for (int i = 0; i < kA8PP; ++i) {
      const int p = tid + i * NT;
      v[i] = buf_load16(rx, p < np ? 16u * (uint32_t)p : kOob);
    }
#pragma unroll
    for (int i = 0; i < kA8PP; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(piece_elem<XT>(v[i], e)));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  float am = 0.0f;
  for (int w = 0; w < (NT >> 6); ++w) am = fmaxf(am, red[w]);
  const float scale = am > 0.0f ? am / 127.0f : 1.0f;
  const rsrc_t rq = make_rsrc(a.a + (int64_t)row * K, (uint32_t)K);
#pragma unroll
  for (int i = 0; i < (LEAN ? (np + NT - 1) / NT : kA8PP); ++i) {
    const int p = tid + i * NT;
    if (p < np) {
      const u32x4_t pv = LEAN ? buf_load16(rx, 16u * (uint32_t)p) : v[LEAN ? 0 : i];
      uint32_t packed[2] = {0u, 0u};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float t = __builtin_rintf(piece_elem<XT>(pv, e) / scale);
        t = fminf(fmaxf(t, -127.0f), 127.0f);
        packed[e >> 2] |= ((uint32_t)(int32_t)t & 0xFFu) << (8 * (e & 3));
      }
      __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{packed[0], packed[1]}, rq, 8 * p, 0, kSc1);
    }
  }
  if (tid == 0) splitk_store(const_cast<float*>(a.sa) + row, scale);
  __syncthreads();  // red is reused by the next row
}

// producer workgroup b: rows b, b + np, ...; then counts them
template <int XT>
__device__ void a8_producer(const I8Args& a, float* red) {
  int rows = 0;
  for (int row = blockIdx.x; row < a.M; row += a.np, ++rows) a8_produce_row<XT>(a, row, red);
  __builtin_amdgcn_s_waitcnt(0);  // the stores have reached the coherence level
  __syncthreads();
  if (threadIdx.x == 0 && rows > 0)
    __hip_atomic_fetch_add(&a.counters[0], (unsigned)rows, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// consumer: returns once all M rows are written (by the producers or, past
// the poll bound, by this workgroup). A fallback may rewrite rows that a
// producer or another fallback also writes, or that other consumers are
// reading: every writer stores the same bytes (the quantizer is a pure
// function of the row), so the overlap changes no value that is read.
template <int XT>
__device__ void a8_wait_rows(const I8Args& a, int* flag, float* red) {
  if (threadIdx.x == 0) {
    int ok = 0;
    for (int it = 0; it < a.spin; ++it) {
      if (splitk_load(&a.counters[0]) >= (unsigned)a.M) {
        ok = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(8);
    }
    *flag = ok;
  }
  __syncthreads();
  if (*flag == 0) {
    for (int row = 0; row < a.M; ++row) a8_produce_row<XT, true>(a, row, red);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
}

// every workgroup at its end; the last one resets the counters
__device__ __forceinline__ void a8_done(const I8Args& a) {
  __syncthreads();
  if (threadIdx.x == 0) {
    __builtin_amdgcn_s_waitcnt(0);
    if (__hip_atomic_fetch_add(&a.counters[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
        gridDim.x - 1) {
      __hip_atomic_store(&a.counters[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&a.counters[1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// fp32 epilogue with the scale read at the coherence level
__device__ __forceinline__ void i8_store_sync(const I8Args& args, int gm, int nn, int32_t s) {
  const float bias = args.bias ? load_in(args.bias, nn, args.bias_dtype) : 0.0f;
  const float t = (float)s * splitk_load(args.sa + gm);
  store_out(args.y, (int64_t)gm * args.N + nn, fmaf(t, args.sw[nn], bias), args.y_dtype);
}

// ---------------------------------------------------------------------------
// 3..16 token rows: i8_rows_kernel
// ---------------------------------------------------------------------------
// One workgroup per 16 weight rows; its 8 or 16 waves split K. Both
// int8 operands go from global memory straight into
// v_mfma_i32_16x16x64_i8 (lane l: row l%16 of the weights / of the
// activations, k 16*(l/16) .. +16 of each 64-k chunk); the quantized
// activations (at most 16 x K bytes) stay in L2 for every workgroup. Each
// wave issues the loads of up to eight (ten) chunks (all of them in flight before
// the first MFMA waits) and then their MFMAs; rows past M or N read zeros
// through the bounded descriptors. The waves' int32 sums are added through
// LDS (exact in any order) and wave 0 writes the epilogue.
//
// Measured on the MI355X (36 distinct weight sets per graph replay, bf16
// activations, quantizer launch included): QKV 3584 x 2560 at M = 8 9.2 us,
// gate+up 19456 x 2560 19.1 us, down 2560 x 9728 16.0 us. Slower, and not
// kept: splitting K across two to four workgroups per row tile when the
// tiles do not fill the chip (QKV 9.2 -> 13.1 us: the partials' round trip),
// 32-row tiles sharing each activation load (gate+up 19.1 -> 22.6 us), and
// a single launch whose workgroups quantize the activations themselves and
// run 4x4x4 MFMAs over 256-byte row spans (QKV 9.1 -> 15.0 us at M = 8,
// 25.7 us at M = 16: every workgroup re-reads the M x K activations).
// XT < 0: the int8 rows are in args.a already; 0 / 1: one launch with the
// quantizer (bf16 / fp16 x), producers first in the grid
template <int RW, int RPD, int XT>  // waves per workgroup (K split), 64-k chunks in flight per wave
__global__ __launch_bounds__(64 * RW) void i8_rows_kernel(I8Args args) {
  __shared__ i32x4_t red[RW - 1][64];
  __shared__ float sred[16];
  __shared__ int sflag;
  if constexpr (XT >= 0) {
    if ((int)blockIdx.x < args.np) {
      a8_producer<XT>(args, sred);
      a8_done(args);
      return;
    }
  }
  const int bx = XT >= 0 ? (int)blockIdx.x - args.np : (int)blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15, grp = lane >> 4;
  const int K = args.K, N = args.N, M = args.M;
  const int n0 = bx * 16;
  const int nch = K / 64;
  const int c0 = wave * nch / RW, c1 = (wave + 1) * nch / RW;
  const int nrows = min(16, N - n0);
  const rsrc_t rb = make_rsrc(args.b + (int64_t)n0 * K, (uint32_t)nrows * (uint32_t)K);
  const rsrc_t ra = make_rsrc(args.a, (uint32_t)M * (uint32_t)K);
  const uint32_t off = (uint32_t)(n16 * K + 16 * grp);
  i32x4_t acc = {0, 0, 0, 0};
  bool waited = XT < 0;
  for (int c = c0; c < c1; c += RPD) {
    u32x4_t av[RPD], bv[RPD];
    if (!waited) {
      // one launch: the weights first, then the rows once they are written
#pragma unroll
      for (int u = 0; u < RPD; ++u)
        bv[u] = buf_load16(rb, c + u < c1 ? off + 64u * (uint32_t)(c + u) : kOob);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (XT >= 0) a8_wait_rows<XT>(args, &sflag, sred);
      waited = true;
#pragma unroll
      for (int u = 0; u < RPD; ++u)
        av[u] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                         ra, (int)(c + u < c1 ? off + 64u * (uint32_t)(c + u) : kOob), 0, kSc1));
    } else {
#pragma unroll
      for (int u = 0; u < RPD; ++u) {
        const bool ok = c + u < c1;  // wave-uniform
        bv[u] = buf_load16(rb, ok ? off + 64u * (uint32_t)(c + u) : kOob);
        av[u] = XT < 0 ? buf_load16(ra, ok ? off + 64u * (uint32_t)(c + u) : kOob)
                       : __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                         ra, (int)(ok ? off + 64u * (uint32_t)(c + u) : kOob),
                                                         0, kSc1));
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < RPD; ++u)
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4_t, av[u]),
                                                  __builtin_bit_cast(i32x4_t, bv[u]), acc, 0, 0, 0);
  }
  if constexpr (XT >= 0) {
    // a wave with no chunk still takes part in the wait (it has barriers)
    if (!waited) a8_wait_rows<XT>(args, &sflag, sred);
  }
  if (wave > 0) red[wave - 1][lane] = acc;
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 0; w < RW - 1; ++w) acc += red[w][lane];
    // lane (grp, n16) holds token rows 4grp .. 4grp+3 of weight row n0 + n16
    const int nn = n0 + n16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * grp + r;
      if (m < M && nn < N) {
        if constexpr (XT < 0)
          i8_store(args, m, nn, acc[r]);
        else
          i8_store_sync(args, m, nn, acc[r]);
      }
    }
  }
  if constexpr (XT >= 0) a8_done(args);
}

// ---------------------------------------------------------------------------
// 3..16 token rows over many row tiles: i8_rows_q_kernel (one round)
// ---------------------------------------------------------------------------
// When the weights hold at least two 16-row tiles per workgroup slot of the
// chip (gate+up), i8_rows_kernel re-reads the activations from L2 in every
// wave and runs its tiles in several rounds. Here P = twice the CUs
// workgroups each own the contiguous tiles [i*T/P, (i+1)*T/P) (at most
// three), all resident at once:
//  * the workgroup stages the 16 x K int8 activation tile once in LDS (rows
//    past M read zeros through the bounded descriptor), padded rows;
//  * wave w owns quarter w%4 of K of tile w/4 and issues all of its 16-byte
//    weight loads (16 rows x 64 bytes per instruction) before any
//    arithmetic, then reads the matching activations from LDS into
//    v_mfma_i32_16x16x64_i8;
//  * the four quarters' int32 sums are added through LDS (exact in any
//    order) and the first wave of each tile writes the epilogue.
// Measured on gate+up 19456 x 2560 (36 weight sets per graph replay, the
// quantizer launch included): M = 16 22.0 -> 17.9 us, M = 8 19.0 -> 17.0,
// M = 4 17.4 -> 16.7, M = 3 the same. The same kernel quantizing the 16-bit
// activations itself (one launch, each workgroup repeating the per-token
// amax and the IEEE divisions) took 24-27 us at M = 3..9 against 16-17 us
// for the quantizer launch followed by this kernel, so it was not kept.
constexpr int kQW = 4;    // waves per row tile (K split)
constexpr int kQT = 3;    // row tiles per workgroup, at most
constexpr int kQXP = 4;   // staged 16-byte activation pieces per thread

__host__ __device__ __forceinline__ int rows_q_pitch(int K) { return K + 16; }

template <int CPW, int XT>  // 64-k chunks per wave (K = 256 * CPW); XT as i8_rows_kernel
__global__ __launch_bounds__(64 * kQW * kQT) void i8_rows_q_kernel(I8Args args) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ float sred[16];
  __shared__ int sflag;
  if constexpr (XT >= 0) {
    if ((int)blockIdx.x < args.np) {
      a8_producer<XT>(args, sred);
      a8_done(args);
      return;
    }
  }
  const int bx = XT >= 0 ? (int)blockIdx.x - args.np : (int)blockIdx.x;
  constexpr int NT = 64 * kQW * kQT;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15, grp = lane >> 4;
  const int K = args.K, N = args.N, M = args.M;
  const int T = (N + 15) >> 4;
  const int t0 = (int)((int64_t)bx * T / args.wgs);
  const int nt = (int)((int64_t)(bx + 1) * T / args.wgs) - t0;
  const int pitch = rows_q_pitch(K);
  int8_t* xs = reinterpret_cast<int8_t*>(smem);                                  // [16][pitch]
  i32x4_t* red = reinterpret_cast<i32x4_t*>(smem + 16 * pitch);                 // [kQT][kQW-1][64]

  // 1. staging loads: piece p = row p / npr, 16 bytes at 16 * (p % npr) of
  // the 16-row activation tile (rows past M read zeros). Issued on every
  // path: a branch around a load would make the compiler wait for it where
  // the paths join.
  const int npr = K >> 4, np = 16 * npr;
  const rsrc_t ra = make_rsrc(args.a, (uint32_t)M * (uint32_t)K);
  u32x4_t xr[kQXP];
  if constexpr (XT < 0) {
#pragma unroll
    for (int i = 0; i < kQXP; ++i) {
      const int p = tid + i * NT;
      const int row = p / npr, pc = p - row * npr;
      xr[i] = buf_load16(ra, p < np && row < M ? (uint32_t)(row * K + 16 * pc) : kOob);
    }
  }
  // 2. the wave's weights: tile w/4, chunks [q*CPW, (q+1)*CPW) of quarter q
  const int tt = wave / kQW, q = wave - tt * kQW;
  const bool has_tile = tt < nt;
  const int n0 = (t0 + tt) * 16;
  const int nrows = has_tile ? min(16, N - n0) : 0;
  const rsrc_t rb = make_rsrc(args.b + (int64_t)(has_tile ? n0 : 0) * K, (uint32_t)nrows * (uint32_t)K);
  const uint32_t off = (uint32_t)(n16 * K + 16 * grp + 64 * q * CPW);
  u32x4_t bv[CPW];
#pragma unroll
  for (int u = 0; u < CPW; ++u) bv[u] = buf_load16(rb, has_tile ? off + 64u * u : kOob);
  __builtin_amdgcn_sched_barrier(0);  // every load above ahead of the arithmetic
  if constexpr (XT >= 0) {
    // one launch: the activation tile once the rows are written
    a8_wait_rows<XT>(args, &sflag, sred);
#pragma unroll
    for (int i = 0; i < kQXP; ++i) {
      const int p = tid + i * NT;
      const int row = p / npr, pc = p - row * npr;
      xr[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                              ra, (int)(p < np && row < M ? (uint32_t)(row * K + 16 * pc) : kOob),
                                              0, kSc1));
    }
  }

  // 3. activations to LDS
#pragma unroll
  for (int i = 0; i < kQXP; ++i) {
    const int p = tid + i * NT;
    if (p < np) {
      const int row = p / npr, pc = p - row * npr;
      *reinterpret_cast<u32x4_t*>(xs + row * pitch + 16 * pc) = xr[i];
    }
  }
  __syncthreads();

  // 4. the quarter's MFMAs: A = activation row n16 (k 16*grp.. of the chunk)
  i32x4_t acc = {0, 0, 0, 0};
  const int8_t* xa = xs + n16 * pitch + 16 * grp + 64 * q * CPW;
#pragma unroll
  for (int u = 0; u < CPW; ++u) {
    const u32x4_t av = *reinterpret_cast<const u32x4_t*>(xa + 64 * u);
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4_t, av),
                                                __builtin_bit_cast(i32x4_t, bv[u]), acc, 0, 0, 0);
  }
  // 5. quarters 1..3 to LDS, quarter 0 adds them and writes the tile
  if (has_tile && q > 0) red[(tt * (kQW - 1) + q - 1) * 64 + lane] = acc;
  __syncthreads();
  if (has_tile && q == 0) {
#pragma unroll
    for (int w = 0; w < kQW - 1; ++w) acc += red[(tt * (kQW - 1) + w) * 64 + lane];
    // lane (grp, n16) holds token rows 4grp .. 4grp+3 of weight row n0 + n16
    const int nn = n0 + n16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * grp + r;
      if (m < M && nn < N) {
        if constexpr (XT < 0)
          i8_store(args, m, nn, acc[r]);
        else
          i8_store_sync(args, m, nn, acc[r]);
      }
    }
  }
  if constexpr (XT >= 0) a8_done(args);
}

struct RowsQPlan {
  bool ok;
  int wgs, cpw;
  size_t lds;
};

// At least two row tiles per workgroup slot (2 per CU), whole 256-k quarter
// chunks of 4..12 64-k chunks (K = 1024 .. 3072 in steps of 512), the
// activation tile within the staging budget.
static RowsQPlan plan_rows_q(int64_t M, int64_t N, int64_t K, int np = 0) {
  RowsQPlan p{};
  if (env_int("SPARKQ_I8_NO_ROWSQ", 0) || M < 1 || M > 16 || K % 256 != 0) return p;
  const int64_t cpw = K / 256;
  if (cpw < 4 || cpw > 12 || cpw % 2 != 0) return p;
  const int64_t T = cdiv(N, 16), P = 2 * device_cus();
  if (T < 2 * P || K > kQXP * 64 * kQW * kQT) return p;  // one staging pass: K pieces
  if (N * K >= (int64_t)kOob || M * K >= (int64_t)kOob) return p;
  // (with producer workgroups in the grid, as many fewer tile workgroups)
  p.wgs = (int)std::max<int64_t>(P - np, cdiv(T, kQT));
  p.cpw = (int)cpw;
  p.lds = (size_t)16 * rows_q_pitch((int)K) + (size_t)kQT * (kQW - 1) * 64 * 16;
  p.ok = p.lds <= 65536;
  return p;
}

template <int XT>
static void launch_rows_q_x(const I8Args& args, const RowsQPlan& p, hipStream_t st) {
  const dim3 grid((unsigned)(p.wgs + args.np)), block(64 * kQW * kQT);
  switch (p.cpw) {
    case 4: hipLaunchKernelGGL((i8_rows_q_kernel<4, XT>), grid, block, p.lds, st, args); break;
    case 6: hipLaunchKernelGGL((i8_rows_q_kernel<6, XT>), grid, block, p.lds, st, args); break;
    case 8: hipLaunchKernelGGL((i8_rows_q_kernel<8, XT>), grid, block, p.lds, st, args); break;
    case 10: hipLaunchKernelGGL((i8_rows_q_kernel<10, XT>), grid, block, p.lds, st, args); break;
    default: hipLaunchKernelGGL((i8_rows_q_kernel<12, XT>), grid, block, p.lds, st, args); break;
  }
}

// 3..16 rows (1..16 with the decode GEMV switched off), whole 64-k chunks
static bool use_rows(int64_t M, int64_t N, int64_t K) {
  return M >= 1 && M <= 16 && K % 64 == 0 && N * K < (int64_t)kOob && M * K < (int64_t)kOob &&
         !env_int("SPARKQ_I8_NO_ROWS", 0);
}

template <int RW, int XT>
static void launch_rows_w(int rpd, const I8Args& args, hipStream_t st) {
  const dim3 grid((unsigned)(cdiv(args.N, 16) + args.np)), block(64 * RW);
  if (rpd == 10)
    hipLaunchKernelGGL((i8_rows_kernel<RW, 10, XT>), grid, block, 0, st, args);
  else
    hipLaunchKernelGGL((i8_rows_kernel<RW, 8, XT>), grid, block, 0, st, args);
}

template <int XT>
static void launch_rows_x(const I8Args& args, hipStream_t st) {
  const bool long_rows = args.K / 64 > 64;
  const int rw = env_int("SPARKQ_I8_ROWS_RW", long_rows ? 16 : 8);
  const int rpd = env_int("SPARKQ_I8_ROWS_RPD", long_rows ? 10 : 8);
  if (rw == 4)
    launch_rows_w<4, XT>(rpd, args, st);
  else if (rw == 16)
    launch_rows_w<16, XT>(rpd, args, st);
  else
    launch_rows_w<8, XT>(rpd, args, st);
}

// Rows of more than 64 chunks (K > 4096) take 16 waves with ten chunks in
// flight each, so that a wave's share of K is one batch of loads (down
// 2560 x 9728: 16.0 -> 15.0 us at M = 8, 18.2 -> 17.2 at M = 16); shorter
// rows keep 8 waves of up to eight chunks (4 waves of ten, 16 of eight or
// ten measured slower on QKV and gate+up). xt: -1 = the int8 rows are in
// args.a, 0 / 1 = one launch quantizing bf16 / fp16 args.x (args.np
// producer workgroups, counters and int8 buffer in args).
static int launch_rows(const I8Args& args, int xt, hipStream_t st) {
  const RowsQPlan qp = plan_rows_q(args.M, args.N, args.K, args.np);
  if (qp.ok) {
    I8Args a = args;
    a.wgs = qp.wgs;
    if (xt == 0)
      launch_rows_q_x<0>(a, qp, st);
    else if (xt == 1)
      launch_rows_q_x<1>(a, qp, st);
    else
      launch_rows_q_x<-1>(a, qp, st);
    return check_launch("i8_rows_q_kernel");
  }
  if (xt == 0)
    launch_rows_x<0>(args, st);
  else if (xt == 1)
    launch_rows_x<1>(args, st);
  else
    launch_rows_x<-1>(args, st);
  return check_launch("i8_rows_kernel");
}

// One launch with the quantizer for 16-bit activations whose rows fit one
// producer pass (K/8 16-byte pieces over the smallest rows workgroup of 512
// threads), for rows longer than 4096 k. Measured against the quantizer
// launch followed by the int8 kernel (36 weight sets per graph replay):
// down 2560 x 9728 at M = 3 / 8 / 16 14.4 -> 12.2, 15.7 -> 14.2, 17.3 ->
// 17.4 us; QKV 3584 x 2560 8.2 -> 9.2, 8.9 -> 10.4, 9.5 -> 11.7 us and
// gate+up 17.0 -> 17.6, 17.8 -> 18.5, 18.8 -> 19.9 us, where the wait for
// the rows (a poll after the wave's weight loads, then the activation loads)
// costs more than the launch it saves.
static bool use_rows_sync(int64_t M, int64_t K, int xdt) {
  return (xdt == SPARKQ_BF16 || xdt == SPARKQ_F16) && M >= 1 && K / 8 <= (int64_t)kA8PP * 512 &&
         (K > 4096 || env_int("SPARKQ_I8_SYNCQ_ALL", 0)) && !env_int("SPARKQ_I8_NO_SYNCQ", 0);
}

// ---------------------------------------------------------------------------
// Tiled int8 GEMM for prefill sizes (i8_gemm_kernel)
// ---------------------------------------------------------------------------
// The reference serves out_proj at any M with a BM128 x BN128 x BK512
// tensor-op GEMM (X/src/spark_w8a8.cpp:120-150). Here: a 128 x 128 tile per
// workgroup of four waves in a 2 x 2 arrangement, each wave 64 x 64 (two
// 32-row by two 32-column fragments of v_mfma_i32_32x32x32_i8). A k step is
// 128 bytes of every row of both operands, staged through LDS (double
// buffered; 128-byte rows whose 16-byte chunks are swizzled by the row, so
// the 32 rows a fragment read touches at one chunk index fall on distinct
// banks); the loads of step s+1 go out before the MFMAs of step s. Lane
// (l % 32, l / 32) of a fragment holds bytes 16 * (l / 32) .. +15 of row
// l % 32 of a 32-k sub-step, for activations and weights alike. Grids with
// fewer tiles than CUs split K into S pieces: each piece stores
// its int32 tile (16-byte stores at the device coherence level), the last
// to arrive adds them (int32 addition is exact, so the result is the
// unsplit one bit for bit) and writes the output, raw or through the
// epilogue fmaf(float(acc) * sa[m], sw[n], bias[n]); grids of one to two
// tiles per CU keep one whole tile per CU and split only the tiles past
// them. Work item i runs on XCD i % 8 (round-robin dispatch): the tile
// order gives each XCD a contiguous chunk of tiles walked in groups of four
// tile rows, so the tiles an XCD runs together share their A rows and B
// columns in its L2. Rows and columns past M and N read zeros and are not
// stored; K % 128 == 0.
constexpr int kI8GK = 128;  // bytes of k per step

__device__ __forceinline__ uint32_t i8_tile_off(int row, int kc) {
  const int t = row & 31;
  return (uint32_t)(row * 128 + ((kc ^ ((t ^ (t >> 3)) & 7)) << 4));
}

__global__ __launch_bounds__(256, 2) void i8_gemm_kernel(I8Args a) {
  constexpr int BM = 128, BN = 128, TB = (BM + BN) * kI8GK;  // bytes per stage
  __shared__ __attribute__((aligned(16))) unsigned char lds[2 * TB];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int l32 = lane & 31, j = lane >> 5;
  const int M = a.M, N = a.N, K = a.K;
  // work item -> (tile, piece): items [0, full) are whole tiles; tile full + i
  // of the rest is split in S pieces, piece p at item full + p * nsplit + i
  // (piece-major, so that the workgroups running together read one k range)
  const int item = blockIdx.x, nsplit = a.tiles - a.full;
  const bool split = item >= a.full;
  const int si = split ? (item - a.full) % nsplit : 0;  // split tile index
  const int tile = split ? a.full + si : item;
  const int piece = split ? (item - a.full) / nsplit : 0;
  const int S = split ? a.S : 1;
  int tm = tile / a.tiles_n, tn = tile - tm * a.tiles_n;
  if (a.gm > 0) {
    // XCD-contiguous chunks of the tile order (workgroups go to the XCDs
    // round-robin, so item i runs on XCD i % 8), each chunk walking groups of
    // gm tile rows column by column
    const int T = a.tiles;
    const int v = (T & 7) == 0 ? (tile & 7) * (T >> 3) + (tile >> 3) : tile;
    const int tiles_m = T / a.tiles_n, width = a.gm * a.tiles_n;
    const int g = v / width, fm = g * a.gm, gs = min(tiles_m - fm, a.gm), r = v - g * width;
    tm = fm + r % gs;
    tn = r / gs;
  }
  const int m0 = tm * BM, n0 = tn * BN;
  const int nst = K / kI8GK;
  const int s_begin = (int)((int64_t)piece * nst / S), s_end = (int)((int64_t)(piece + 1) * nst / S);
  const int mr = min(BM, M - m0), nr = min(BN, N - n0);
  const rsrc_t ra = make_rsrc(a.a + (int64_t)m0 * K, (uint32_t)mr * (uint32_t)K);
  const rsrc_t rb = make_rsrc(a.b + (int64_t)n0 * K, (uint32_t)nr * (uint32_t)K);

  // staging: chunk p = tid + 256 i of each operand, row p / 8, chunk p % 8
  constexpr int CH = BM * 8 / 256;  // chunks per thread and operand (4)
  uint32_t goff[CH], loff[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int p = tid + 256 * i, row = p >> 3, kc = p & 7;
    goff[i] = (uint32_t)(row * K + kc * 16);
    loff[i] = i8_tile_off(row, kc);
  }
  u32x4_t va[CH], vb[CH];
  auto load = [&](int step) {
    const int k0 = step * kI8GK;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      va[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(ra, (int)goff[i], k0, 0));
      vb[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rb, (int)goff[i], k0, 0));
    }
  };
  auto stage = [&](int buf) {
    unsigned char* base = lds + buf * TB;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      *reinterpret_cast<u32x4_t*>(base + loff[i]) = va[i];
      *reinterpret_cast<u32x4_t*>(base + BM * kI8GK + loff[i]) = vb[i];
    }
  };

  i32x16_t acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) acc[x][y] = i32x16_t{};
  // fragment rows (a multiple of 32 plus l32: the swizzle's t is l32)
  const int ar0 = wm * 64 + l32, br0 = wn * 64 + l32;

  if (s_begin < s_end) {
    load(s_begin);
    stage(0);
    __syncthreads();
  }
  for (int step = s_begin; step < s_end; ++step) {
    const int cur = (step - s_begin) & 1;
    const bool more = step + 1 < s_end;
    if (more) load(step + 1);
    const unsigned char* base = lds + cur * TB;
#pragma unroll
    for (int ss = 0; ss < 4; ++ss) {
      const int kc = 2 * ss + j;
      u32x4_t af[2], bf[2];
#pragma unroll
      for (int x = 0; x < 2; ++x)
        af[x] = *reinterpret_cast<const u32x4_t*>(base + i8_tile_off(ar0 + 32 * x, kc));
#pragma unroll
      for (int y = 0; y < 2; ++y)
        bf[y] = *reinterpret_cast<const u32x4_t*>(base + BM * kI8GK + i8_tile_off(br0 + 32 * y, kc));
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y) acc[x][y] = mfma_i8(af[x], bf[y], acc[x][y]);
    }
    if (more) stage(cur ^ 1);
    __syncthreads();
  }

  if (S > 1) {
    // this piece's tile: chunk c (16 bytes) of every thread at (c * 256 + tid) * 16
    constexpr uint32_t PB = 4 * 16 * 4 * 256;  // bytes per piece
    const rsrc_t rp = make_rsrc(a.part + (size_t)si * S * (PB / 4), (uint32_t)S * PB);
#pragma unroll
    for (int xy = 0; xy < 4; ++xy)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const i32x16_t& v = acc[xy >> 1][xy & 1];
        const u32x4_t w = {(uint32_t)v[4 * q], (uint32_t)v[4 * q + 1], (uint32_t)v[4 * q + 2],
                           (uint32_t)v[4 * q + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(w, rp, (uint32_t)tid * 16u,
                                               piece * PB + (xy * 4 + q) * 256 * 16, kSc1);
      }
    if (!splitk_arrive(a.counters + si, S, &s_last)) return;
#pragma unroll
    for (int xy = 0; xy < 4; ++xy) {
      i32x16_t t = acc[xy >> 1][xy & 1];
      for (int z = 0; z < S; ++z) {
        if (z == piece) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4_t w = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                            rp, (uint32_t)tid * 16u, z * PB + (xy * 4 + q) * 256 * 16, kSc1));
#pragma unroll
          for (int e = 0; e < 4; ++e) t[4 * q + e] += (int32_t)w[e];
        }
      }
      acc[xy >> 1][xy & 1] = t;
    }
    splitk_reset(a.counters + si);
  }

#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int gn = n0 + wn * 64 + 32 * y + l32;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int gm = m0 + wm * 64 + 32 * x + mfma32_row(lane, v);
        if (gm < M && gn < N) i8_store(a, gm, gn, acc[x][y][v]);
      }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
// Decode GEMV plan: a row has U = ceil(K/256) spans; a wave keeps at most 10
// spans of weights in flight, so rows of up to 40 spans (K <= 10240) split
// into SG = 1, 2 or 4 span groups; workgroups of 4 waves (8 when SG = 4)
// cover R = 4 * waves / SG rows. The staged activations must fit the fixed
// per-thread budget and the tensors the buffer loads' offset range.
//
// v_dot4 here against the 16x16x64 int8 MFMA of i8_rows_kernel (after its
// own quantizer launch), measured on the MI355X with 36 distinct weight
// sets per graph replay: at M = 1 and 2 the GEMV is faster (M = 1: QKV
// 3584 x 2560 5.3 vs 12.4 us, gate+up 19456 x 2560 12.0 vs 16.2, down
// 2560 x 9728 11.5 vs 15.0; M = 2: QKV 7.0 vs 12.5, gate+up 14.5 vs 16.7),
// from M = 3 the MFMA path is (M = 3: QKV 8.6 vs 8.4, gate+up 18.3 vs
// 17.1, down 15.9 vs 14.8; M = 4: QKV 9.0 vs 8.7, gate+up 18.6 vs 17.6,
// down 16.4 vs 14.9). The GEMV re-stages M x K activations in every
// workgroup and its dot products grow with M on the VALU.
struct I8GemvPlan {
  bool ok;
  int SG, USr, US, NW, MQ, R;
  size_t lds;
  int64_t wgs;
};

static I8GemvPlan plan_i8_gemv(int64_t M, int64_t N, int64_t K, int esize) {
  I8GemvPlan p{};
  const int64_t maxm = K % 64 == 0 ? std::min<int64_t>(env_int("SPARKQ_I8_GEMV_MAXM", 2), 4) : 4;
  if (M > maxm || env_int("SPARKQ_I8_NO_GEMV", 0)) return p;
  if (N * K >= (int64_t)kOob || M * K * esize >= (int64_t)kOob) return p;
  // 16-bit activations over rows longer than 4096 k take the rows kernel
  // with its producer workgroups instead (down 2560 x 9728 at M = 1: 11.5
  // -> 11.1 us; the same at M = 2), where every workgroup here would
  // quantize the whole long row itself
  if (esize == 2 && K > 4096 && K % 64 == 0 && K / 8 <= (int64_t)kA8PP * 512 &&
      !env_int("SPARKQ_I8_NO_SYNCQ", 0))
    return p;
  const int64_t U = cdiv(K, 256);
  if (U <= 10)
    p.SG = 1;
  else if (U <= 20)
    p.SG = 2;
  else if (U <= 40)
    p.SG = 4;
  else
    return p;
  p.USr = (int)cdiv(U, p.SG);
  p.US = p.USr <= 2 ? 2 : (p.USr <= 5 ? 5 : 10);
  p.NW = p.SG == 4 ? 8 : 4;
  p.MQ = M == 1 ? 1 : 4;
  p.R = 4 * (p.NW / p.SG);
  if (M * K * esize > (int64_t)kI8XP * 16 * 64 * p.NW) return p;
  p.lds = round_up((size_t)M * K, 16) + 16 + (size_t)p.NW * 64;
  p.wgs = cdiv(N, p.R);
  p.ok = true;
  return p;
}

template <int MQ, int US, int NW>
static void launch_i8_gemv_x(const I8GemvPlan& p, const I8GemvArgs& a, int xt, hipStream_t st) {
  dim3 grid((unsigned)p.wgs), block(64 * NW);
  switch (xt) {
    case 0: hipLaunchKernelGGL((i8_gemv_kernel<MQ, US, NW, 0>), grid, block, p.lds, st, a); break;
    case 1: hipLaunchKernelGGL((i8_gemv_kernel<MQ, US, NW, 1>), grid, block, p.lds, st, a); break;
    case 2: hipLaunchKernelGGL((i8_gemv_kernel<MQ, US, NW, 2>), grid, block, p.lds, st, a); break;
    default: hipLaunchKernelGGL((i8_gemv_kernel<MQ, US, NW, 3>), grid, block, p.lds, st, a); break;
  }
}
template <int MQ, int US>
static void launch_i8_gemv_w(const I8GemvPlan& p, const I8GemvArgs& a, int xt, hipStream_t st) {
  if (p.NW == 4)
    launch_i8_gemv_x<MQ, US, 4>(p, a, xt, st);
  else
    launch_i8_gemv_x<MQ, US, 8>(p, a, xt, st);
}
template <int MQ>
static void launch_i8_gemv_u(const I8GemvPlan& p, const I8GemvArgs& a, int xt, hipStream_t st) {
  if (p.US == 2)
    launch_i8_gemv_w<MQ, 2>(p, a, xt, st);
  else if (p.US == 5)
    launch_i8_gemv_w<MQ, 5>(p, a, xt, st);
  else
    launch_i8_gemv_w<MQ, 10>(p, a, xt, st);
}
static int launch_i8_gemv(const I8GemvPlan& p, const I8GemvArgs& a, int xt, hipStream_t st) {
  if (p.MQ == 1)
    launch_i8_gemv_u<1>(p, a, xt, st);
  else
    launch_i8_gemv_u<4>(p, a, xt, st);
  return check_launch("i8_gemv_kernel");
}

// Streaming int8 GEMV plan (M <= 2, 16-bit or fp32 activations): one
// workgroup per CU, equal row ranges, at most 12 items of 1 KB per wave; the
// activation rows must fit the staging registers and the run's byte offsets
// the float quotient. Taken where it measured faster (MI355X, 36 distinct
// weight sets per graph replay, bf16): one row over more than 4096 k (down
// 2560 x 9728: 10.7 us against 11.1 on the rows kernel with its producer
// workgroups and 10.85 on i8_gemv_kernel) and two rows over runs of at most
// 48 KB a CU (QKV 3584 x 2560: 6.7 against 7.3 us). One row over short rows
// (QKV 5.7 against 5.1 us) and runs of 97-194 KB at two rows (down 14.1
// against 11.6, gate+up 20.5 against 15.3) stay on the other kernels, whose
// several workgroups per CU overlap their staging chains.
struct I8StreamPlan {
  bool ok;
  int P, NI;
  size_t lds;
};

static I8StreamPlan plan_i8_stream(int64_t M, int64_t N, int64_t K, int esize) {
  I8StreamPlan p{};
  if (M < 1 || M > 2 || env_int("SPARKQ_I8_NO_STREAM", 0)) return p;
  if (K < 1024 || K % 16 != 0 || N * K >= (int64_t)kOob) return p;
  if (M * K * esize > (int64_t)kI8SXP * 16 * 1024) return p;
  p.P = (int)std::min<int64_t>(N, device_cus());
  const int64_t rows = cdiv(N, p.P), bytes = rows * K;
  if (bytes >= (int64_t)1 << 24) return p;
  const bool measured = M == 1 ? K > 4096 : bytes <= 48 * 1024;
  if (!measured && !env_int("SPARKQ_I8_STREAM", 0)) return p;
  const int64_t ni = cdiv(cdiv(bytes, 1024), 16);
  if (ni > 12) return p;
  p.NI = ni <= 4 ? 4 : (ni <= 6 ? 6 : (ni <= 8 ? 8 : 12));
  p.lds = round_up((size_t)M * K, 16) + 16 + (size_t)rows * M * 4;
  p.ok = p.lds <= 65536;
  return p;
}

template <int MQ, int NI>
static void launch_i8_stream_x(const I8StreamPlan& p, const I8GemvArgs& a, int xt,
                               hipStream_t st) {
  const dim3 grid((unsigned)p.P), block(1024);
  switch (xt) {
    case 0: hipLaunchKernelGGL((i8_gemv_stream_kernel<MQ, NI, 0>), grid, block, p.lds, st, a); break;
    case 1: hipLaunchKernelGGL((i8_gemv_stream_kernel<MQ, NI, 1>), grid, block, p.lds, st, a); break;
    default: hipLaunchKernelGGL((i8_gemv_stream_kernel<MQ, NI, 2>), grid, block, p.lds, st, a); break;
  }
}
template <int MQ>
static void launch_i8_stream_n(const I8StreamPlan& p, const I8GemvArgs& a, int xt,
                               hipStream_t st) {
  switch (p.NI) {
    case 4: launch_i8_stream_x<MQ, 4>(p, a, xt, st); break;
    case 6: launch_i8_stream_x<MQ, 6>(p, a, xt, st); break;
    case 8: launch_i8_stream_x<MQ, 8>(p, a, xt, st); break;
    default: launch_i8_stream_x<MQ, 12>(p, a, xt, st); break;
  }
}
static int launch_i8_stream(const I8StreamPlan& p, const I8GemvArgs& a, int xt, hipStream_t st) {
  if (a.M == 1)
    launch_i8_stream_n<1>(p, a, xt, st);
  else
    launch_i8_stream_n<2>(p, a, xt, st);
  return check_launch("i8_gemv_stream_kernel");
}

// One-round int8 GEMV plan (M <= 2, K % 256 == 0, K <= 2560): the W4
// one-round grid (twice the CUs workgroups when that gives at least 8 quads
// per CU, else one per CU, at most 16 row-quad waves each), with at least the
// waves that stage the activations; two spans in flight per wave where a CU
// holds 12 or more row-quad waves, every span on smaller grids. Taken at two
// rows, where it measured faster (MI355X, 36 distinct weight sets per graph
// replay, bf16): QKV 3584 x 2560 6.8 -> 6.0 us against the streaming int8
// GEMV, gate+up 19456 x 2560 15.4 -> 13.6 us (13.9 at one span in flight,
// 16.8 at all) against i8_gemv_kernel. At one row i8_gemv_kernel's 1216
// four-wave workgroups stay faster on gate+up (12.0 against 12.9-14.4 us)
// and QKV is even (5.1 / 5.0 us).
struct I8QPlan {
  bool ok;
  int P, NWQ, U, D;
  size_t lds;
};

static I8QPlan plan_i8q(int64_t M, int64_t N, int64_t K, int esize) {
  I8QPlan p{};
  if (M < 1 || M > 2 || K % 256 != 0 || K > 2560 || env_int("SPARKQ_I8_NO_Q", 0)) return p;
  if (M != 2 && !env_int("SPARKQ_I8_Q", 0)) return p;
  if (N * K >= (int64_t)kOob) return p;
  const int64_t nq = cdiv(N, 4), cus = device_cus();
  int64_t P = std::min<int64_t>(nq, cus * (nq >= 8 * cus ? 2 : 1));
  if (cdiv(nq, P) > 16) P = cdiv(nq, 16);
  p.P = (int)P;
  const int64_t wpc = cdiv(nq, cus);
  p.NWQ = (int)std::max<int64_t>(cdiv(nq, P), cdiv(M * K * esize / 16, 64 * kI8QXP));
  if (p.NWQ > 16) return p;
  p.U = K <= 1024 ? 4 : 10;
  const int64_t d = env_int("SPARKQ_I8_Q_DEPTH", wpc >= 12 ? 2 : 8);
  p.D = d == 1 || d == 2 ? (int)d : p.U;
  p.lds = round_up((size_t)M * K, 16) + 16;
  p.ok = true;
  return p;
}

template <int MQ, int U, int D>
static void launch_i8q_x(const I8QPlan& p, const I8GemvArgs& a, int xt, hipStream_t st) {
  const dim3 grid((unsigned)p.P), block(64 * p.NWQ);
  switch (xt) {
    case 0: hipLaunchKernelGGL((i8_gemvq_kernel<MQ, U, D, 0>), grid, block, p.lds, st, a); break;
    case 1: hipLaunchKernelGGL((i8_gemvq_kernel<MQ, U, D, 1>), grid, block, p.lds, st, a); break;
    default: hipLaunchKernelGGL((i8_gemvq_kernel<MQ, U, D, 2>), grid, block, p.lds, st, a); break;
  }
}
template <int MQ, int U>
static void launch_i8q_u(const I8QPlan& p, const I8GemvArgs& a, int xt, hipStream_t st) {
  if (p.D == 1)
    launch_i8q_x<MQ, U, 1>(p, a, xt, st);
  else if (p.D == 2)
    launch_i8q_x<MQ, U, 2>(p, a, xt, st);
  else
    launch_i8q_x<MQ, U, U>(p, a, xt, st);
}
template <int MQ>
static void launch_i8q_m(const I8QPlan& p, const I8GemvArgs& a, int xt, hipStream_t st) {
  if (p.U == 4)
    launch_i8q_u<MQ, 4>(p, a, xt, st);
  else
    launch_i8q_u<MQ, 10>(p, a, xt, st);
}
static int launch_i8q(const I8QPlan& p, const I8GemvArgs& a, int xt, hipStream_t st) {
  if (a.M == 1)
    launch_i8q_m<1>(p, a, xt, st);
  else
    launch_i8q_m<2>(p, a, xt, st);
  return check_launch("i8_gemvq_kernel");
}

// activation type code of the GEMV kernel (3 = int8) and its element size
static int i8_xt(int xdt) { return xdt == SPARKQ_BF16 ? 0 : (xdt == SPARKQ_F16 ? 1 : 2); }
static int esize_of(int xdt) { return xdt == SPARKQ_F32 ? 4 : 2; }

struct I8Plan {
  int S, cps, slab;
  size_t lds;
  size_t counter_bytes, part_bytes;
};

static I8Plan plan_i8(int64_t M, int64_t N, int64_t K) {
  I8Plan p;
  const int64_t mrows = M < 32 ? M : 32;
  const int64_t tiles = cdiv(N, 32) * cdiv(M, 32);
  const int64_t nchunks = K / 32;
  // activation slab in LDS <= 32 KB
  int64_t slab = (32768 / mrows - 16) / 32;
  if (slab < 1) slab = 1;
  // about four workgroups per CU; SPARKQ_I8_TARGET_WGS overrides it for tuning
  int64_t S = tiles > kMaxCounterTiles ? 1 : cdiv(env_int("SPARKQ_I8_TARGET_WGS", 1024), tiles);
  const int64_t s_cap = nchunks / 8 > 0 ? nchunks / 8 : 1;
  if (S > s_cap) S = s_cap;
  if (S < 1) S = 1;
  const int64_t cps = cdiv(nchunks, S);
  S = cdiv(nchunks, cps);
  p.S = (int)S;
  p.cps = (int)cps;
  p.slab = (int)(slab < cps ? slab : cps);
  p.lds = (size_t)mrows * (size_t)(p.slab * 32 + 16);
  p.counter_bytes = S > 1 ? kCounterBytes : 0;
  p.part_bytes = S > 1 ? round_up((size_t)S * M * N * 4, 256) : 0;
  return p;
}

// Plan of the tiled GEMM: at least 64 rows (SPARKQ_I8_GEMM_FROM; the
// weight-streaming kernel below that), K % 128 == 0. Grids of fewer tiles
// than twice the CUs split K into S = min(4, 2*CUs / tiles) pieces of at
// least eight steps (tiles within the counter block).
struct I8GemmPlan {
  bool ok;
  int tiles_n, tiles, S, full;
  size_t part_bytes;
};

static I8GemmPlan plan_i8_gemm(int64_t M, int64_t N, int64_t K) {
  I8GemmPlan p{};
  if (M < env_int("SPARKQ_I8_GEMM_FROM", 64) || env_int("SPARKQ_I8_NO_GEMM", 0)) return p;
  if (K % kI8GK != 0 || (int64_t)kI8GK * K >= (int64_t)kOob) return p;
  const int64_t tn = cdiv(N, 128), tiles = cdiv(M, 128) * tn, cus = device_cus();
  if (tiles * 4 > (int64_t)0x7FFFFFFF) return p;
  // Fewer tiles than CUs: every tile split in S pieces. Between one and two
  // tiles per CU (M=2048 out_proj: 320 tiles on 256 CUs), one whole tile per
  // CU and the tiles past them split in S pieces, so that every CU runs one
  // whole tile and at most one piece instead of a quarter of the CUs running
  // two whole tiles (the whole call at M=2048, N=2560, K=4096: 64.0-64.1 ->
  // 57.7-59.3 us; SPARKQ_I8_GEMM_NO_CU1 keeps the unsplit grid).
  int64_t S = 1, full = 0;
  if (tiles < cus && tiles <= kMaxCounterTiles) {
    S = std::min<int64_t>(std::min<int64_t>(4, 2 * cus / tiles), std::max<int64_t>(1, (K / kI8GK) / 8));
  } else if (tiles < 2 * cus && !env_int("SPARKQ_I8_GEMM_NO_CU1", 0)) {
    const int64_t rest = tiles - cus;
    const int64_t s = std::min<int64_t>(std::min<int64_t>(4, cus / rest), std::max<int64_t>(1, (K / kI8GK) / 8));
    if (s > 1 && rest <= kMaxCounterTiles) {
      S = s;
      full = cus;
    }
  }
  if (env_int("SPARKQ_I8_GEMM_SPLITS", 0) > 0 && tiles <= kMaxCounterTiles) {
    S = std::min<int64_t>(env_int("SPARKQ_I8_GEMM_SPLITS", 1), K / kI8GK);
    full = 0;
  }
  p.tiles_n = (int)tn;
  p.tiles = (int)tiles;
  p.S = (int)std::max<int64_t>(S, 1);
  p.full = p.S > 1 ? (int)full : (int)tiles;
  p.part_bytes = p.S > 1 ? round_up((size_t)(tiles - p.full) * p.S * 65536, 256) : 0;
  p.ok = true;
  return p;
}

size_t w8a8_workspace(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  // the fused decode GEMV needs no workspace for any activation dtype
  if (plan_i8_gemv(M, N, K, 4).ok && plan_i8_gemv(M, N, K, 2).ok) return 0;
  const I8GemmPlan gp = plan_i8_gemm(M, N, K);
  const size_t part = use_rows(M, N, K) ? 0 : gp.ok ? gp.part_bytes : plan_i8(M, N, K).part_bytes;
  // counters, int8 activations, fp32 scales, int32 partials
  return kCounterBytes + round_up((size_t)M * K, 256) + round_up((size_t)M * 4, 256) + part;
}

size_t i8_matmul_workspace(int64_t M, int64_t N, int64_t K) {
  if (plan_i8_gemv(M, N, K, 1).ok || use_rows(M, N, K)) return 0;
  const I8GemmPlan gp = plan_i8_gemm(M, N, K);
  if (gp.ok) return gp.S > 1 ? kCounterBytes + gp.part_bytes : 0;
  const I8Plan p = plan_i8(M, N, K);
  return p.counter_bytes + p.part_bytes;
}

static int launch_i8_gemm(I8Args args, const I8GemmPlan& p, hipStream_t st) {
  args.tiles_n = p.tiles_n;
  // XCD-grouped tile order, groups of four tile rows (M = 2048 / 4096 out_proj
  // 780 -> 800 / 844 -> 868 TOP/s; M = 512 unchanged); SPARKQ_I8_GEMM_ROWMAJOR
  // keeps the row-major order
  args.gm = env_int("SPARKQ_I8_GEMM_ROWMAJOR", 0) ? 0 : (int)env_int("SPARKQ_I8_GEMM_GM", 4);
  args.tiles = p.tiles;
  args.S = p.S;
  args.full = p.full;
  hipLaunchKernelGGL(i8_gemm_kernel, dim3((unsigned)(p.full + (p.tiles - p.full) * p.S)), dim3(256), 0, st,
                     args);
  return check_launch("i8_gemm_kernel");
}

static int launch_i8(const I8Args& args, const I8Plan& p, hipStream_t st) {
  dim3 grid((unsigned)cdiv(args.N, 32), (unsigned)p.S, (unsigned)cdiv(args.M, 32));
  hipLaunchKernelGGL(i8_skinny_kernel, grid, dim3(256), p.lds, st, args);
  return check_launch("i8_skinny_kernel");
}

int a8_quantize(const void* x, int8_t* q, float* scales, int64_t M, int64_t K, int xdt,
                hipStream_t st) {
  const int64_t bytes = K * esize_of(xdt);
  if (bytes % 16 == 0 && bytes <= 16 * 256 * kQPieces && M <= 65535) {
    const dim3 grid((unsigned)M), block(256);
    if (xdt == SPARKQ_BF16)
      hipLaunchKernelGGL(a8_quantize_reg_kernel<0>, grid, block, 0, st, x, q, scales, (int)K);
    else if (xdt == SPARKQ_F16)
      hipLaunchKernelGGL(a8_quantize_reg_kernel<1>, grid, block, 0, st, x, q, scales, (int)K);
    else
      hipLaunchKernelGGL(a8_quantize_reg_kernel<2>, grid, block, 0, st, x, q, scales, (int)K);
    return check_launch("a8_quantize_reg_kernel");
  }
  hipLaunchKernelGGL(a8_quantize_kernel, dim3((unsigned)M), dim3(256), 0, st, x, q, scales,
                     K, xdt);
  return check_launch("a8_quantize_kernel");
}

int int8_matmul_i32(const int8_t* a, const int8_t* b, int32_t* c, int64_t M, int64_t N,
                    int64_t K, void* ws, size_t wsb, hipStream_t st) {
  const I8GemvPlan gp = plan_i8_gemv(M, N, K, 1);
  if (gp.ok) {
    I8GemvArgs g{};
    g.x = a;
    g.w = b;
    g.c_raw = c;
    g.M = (int)M;
    g.N = (int)N;
    g.K = (int)K;
    g.SG = gp.SG;
    g.USr = gp.USr;
    g.R = gp.R;
    g.mode = kOutRaw;
    return launch_i8_gemv(gp, g, 3, st);
  }
  if (use_rows(M, N, K)) {
    I8Args r{};
    r.a = a;
    r.b = b;
    r.c_raw = c;
    r.M = (int)M;
    r.N = (int)N;
    r.K = (int)K;
    r.mode = kOutRaw;
    return launch_rows(r, -1, st);
  }
  const I8GemmPlan tp = plan_i8_gemm(M, N, K);
  if (tp.ok) {
    const size_t need = tp.S > 1 ? kCounterBytes + tp.part_bytes : 0;
    if (need > 0 && (ws == nullptr || wsb < need))
      return set_error(SPARKQ_ERR_WORKSPACE,
                       "int8_matmul_i32 needs a workspace of %zu bytes (got %zu)", need, wsb);
    I8Args args{};
    args.a = a;
    args.b = b;
    args.c_raw = c;
    args.M = (int)M;
    args.N = (int)N;
    args.K = (int)K;
    args.mode = kOutRaw;
    if (tp.S > 1) {
      args.counters = reinterpret_cast<unsigned*>(ws);
      args.part = reinterpret_cast<int32_t*>(reinterpret_cast<unsigned char*>(ws) + kCounterBytes);
    }
    return launch_i8_gemm(args, tp, st);
  }
  const I8Plan p = plan_i8(M, N, K);
  const size_t need = p.counter_bytes + p.part_bytes;
  if (need > 0 && (ws == nullptr || wsb < need))
    return set_error(SPARKQ_ERR_WORKSPACE,
                     "int8_matmul_i32 needs a workspace of %zu bytes (got %zu)", need, wsb);
  I8Args args{};
  args.a = a;
  args.b = b;
  args.c_raw = c;
  args.M = (int)M;
  args.N = (int)N;
  args.K = (int)K;
  args.cps = p.cps;
  args.slab = p.slab;
  args.S = p.S;
  args.mode = kOutRaw;
  if (p.S > 1) {
    args.counters = reinterpret_cast<unsigned*>(ws);
    args.part = reinterpret_cast<int32_t*>(reinterpret_cast<unsigned char*>(ws) + kCounterBytes);
  }
  return launch_i8(args, p, st);
}

int w8a8_linear(const void* x, const int8_t* w, const float* wsc, const void* bias,
                int bias_dtype, void* y, int64_t M, int64_t N, int64_t K, int xdt, int ydt,
                void* ws, size_t wsb, hipStream_t st) {
  const I8QPlan qp = plan_i8q(M, N, K, esize_of(xdt));
  if (qp.ok) {
    I8GemvArgs g{};
    g.x = x;
    g.w = w;
    g.sw = wsc;
    g.bias = bias;
    g.bias_dtype = bias_dtype;
    g.y = y;
    g.y_dtype = ydt;
    g.x_dtype = xdt;
    g.M = (int)M;
    g.N = (int)N;
    g.K = (int)K;
    g.mode = kOutEpilogue;
    g.nq = (int)cdiv(N, 4);
    g.P = qp.P;
    return launch_i8q(qp, g, i8_xt(xdt), st);
  }
  const I8StreamPlan sp = plan_i8_stream(M, N, K, esize_of(xdt));
  if (sp.ok) {
    I8GemvArgs g{};
    g.x = x;
    g.w = w;
    g.sw = wsc;
    g.bias = bias;
    g.bias_dtype = bias_dtype;
    g.y = y;
    g.y_dtype = ydt;
    g.x_dtype = xdt;
    g.M = (int)M;
    g.N = (int)N;
    g.K = (int)K;
    g.mode = kOutEpilogue;
    return launch_i8_stream(sp, g, i8_xt(xdt), st);
  }
  const I8GemvPlan gp = plan_i8_gemv(M, N, K, esize_of(xdt));
  if (gp.ok) {
    I8GemvArgs g{};
    g.x = x;
    g.w = w;
    g.sw = wsc;
    g.bias = bias;
    g.bias_dtype = bias_dtype;
    g.y = y;
    g.y_dtype = ydt;
    g.x_dtype = xdt;
    g.M = (int)M;
    g.N = (int)N;
    g.K = (int)K;
    g.SG = gp.SG;
    g.USr = gp.USr;
    g.R = gp.R;
    g.mode = kOutEpilogue;
    return launch_i8_gemv(gp, g, i8_xt(xdt), st);
  }
  const size_t need = w8a8_workspace(M, N, K);
  if (ws == nullptr || wsb < need)
    return set_error(SPARKQ_ERR_WORKSPACE,
                     "w8a8_linear needs a workspace of %zu bytes (got %zu)", need, wsb);
  unsigned char* base = reinterpret_cast<unsigned char*>(ws);
  int8_t* q = reinterpret_cast<int8_t*>(base + kCounterBytes);
  float* sa = reinterpret_cast<float*>(base + kCounterBytes + round_up((size_t)M * K, 256));
  int32_t* part = reinterpret_cast<int32_t*>(base + kCounterBytes + round_up((size_t)M * K, 256) +
                                             round_up((size_t)M * 4, 256));
  if (use_rows(M, N, K) && use_rows_sync(M, K, xdt)) {
    I8Args r{};
    r.a = q;
    r.b = w;
    r.sa = sa;
    r.sw = wsc;
    r.bias = bias;
    r.bias_dtype = bias_dtype;
    r.y = y;
    r.y_dtype = ydt;
    r.M = (int)M;
    r.N = (int)N;
    r.K = (int)K;
    r.mode = kOutEpilogue;
    r.counters = reinterpret_cast<unsigned*>(base);
    r.x = x;
    r.xt = xdt == SPARKQ_BF16 ? 0 : 1;
    r.np = (int)M;
    r.spin = env_int("SPARKQ_I8_SELF_QUANTIZE", 0) ? 0 : 4000;
    return launch_rows(r, r.xt, st);
  }
  if (int rc = a8_quantize(x, q, sa, M, K, xdt, st)) return rc;
  if (use_rows(M, N, K)) {
    I8Args r{};
    r.a = q;
    r.b = w;
    r.sa = sa;
    r.sw = wsc;
    r.bias = bias;
    r.bias_dtype = bias_dtype;
    r.y = y;
    r.y_dtype = ydt;
    r.M = (int)M;
    r.N = (int)N;
    r.K = (int)K;
    r.mode = kOutEpilogue;
    return launch_rows(r, -1, st);
  }
  const I8GemmPlan tp = plan_i8_gemm(M, N, K);
  if (tp.ok) {
    I8Args args{};
    args.a = q;
    args.b = w;
    args.sa = sa;
    args.sw = wsc;
    args.bias = bias;
    args.bias_dtype = bias_dtype;
    args.y = y;
    args.y_dtype = ydt;
    args.M = (int)M;
    args.N = (int)N;
    args.K = (int)K;
    args.mode = kOutEpilogue;
    if (tp.S > 1) {
      args.counters = reinterpret_cast<unsigned*>(base);
      args.part = part;
    }
    return launch_i8_gemm(args, tp, st);
  }
  const I8Plan p = plan_i8(M, N, K);
  I8Args args{};
  args.a = q;
  args.b = w;
  args.sa = sa;
  args.sw = wsc;
  args.bias = bias;
  args.bias_dtype = bias_dtype;
  args.y = y;
  args.y_dtype = ydt;
  args.M = (int)M;
  args.N = (int)N;
  args.K = (int)K;
  args.cps = p.cps;
  args.slab = p.slab;
  args.S = p.S;
  args.mode = kOutEpilogue;
  if (p.S > 1) {
    args.counters = reinterpret_cast<unsigned*>(base);
    args.part = part;
  }
  return launch_i8(args, p, st);
}

}  // namespace sparkq
