// w8a16.hip -- W8A16 per-channel decode GEMV on gfx950:
// y[m,n] = to_dtype(scale[n] * sum_k x[m,k] * w[n,k]) with signed int8
// weights [N,K], an fp32 scale per output channel and 16-bit activations
// (X/src/spark_w8a16.cpp:74-110, X/src/kernels/w8a16_matvec.metal:12-31:
// the fp32 dot, then one multiply by the channel scale, then the cast).
//
// Kernel w8a16_gemvq_kernel (M = 1, K % 256 == 0, K <= 2560): the W4
// one-round layout, one row quad per wave over its whole row, the decode
// below.
//
// Kernel w8a16_gemv_kernel (M <= 4, every other shape): the streaming decode layout of the
// W4A16 GEMV. One workgroup of 16 waves per CU owns a contiguous range of row
// quads; its work items are (row quad, 256-byte span) pairs in quad-major
// order, and each wave takes a contiguous run of them. Lane l = 4b + j loads
// the 16 bytes at byte 16b of a span of weight row 4q+j (4 rows x 256
// contiguous bytes per load instruction) and DEPTH items' loads stay in
// flight ahead of the arithmetic.
//
// Decode. An int8 weight v is read as the byte u = v ^ 0x80 = v + 128 =
// 16h + l. The strided 4-bit decode of the W4A16 kernels turns each word of
// four bytes into the exact 16-bit pairs OFFSET+l and OFFSET+h of bytes
// (0, 2) and (1, 3); with the activations staged as the pairs (x0, x2) and
// (x1, x3) of each 4-k word, two 4x4x4 MFMAs per word (low nibbles, high
// nibbles, same activation operand) accumulate D_l = sum x*(OFFSET+l) and
// D_h = sum x*(OFFSET+h), and sum x*v = 16*D_h + D_l - (17*OFFSET+128)*sum x.
// A load past a row's end reads zeros, which decode as v = 0.
// While the row quad stays the same the lanes keep D_l, D_h and the
// activation sums in registers; at the end of a run the sixteen blocks are
// added (DPP and permlane swaps) and the quad's sums go to the LDS slot of
// the run's first span (the other slots of the run stay zero). Each output
// is the sum of its quad's slots in span order times the channel scale.
#include <algorithm>

#include "common.h"

namespace sparkq {

struct W8a16Args {
  const uint16_t* x;
  const int8_t* w;
  const float* scales;
  void* y;
  int y_dtype;
  int M, N, K;
  int nq;  // row quads
  int P;   // workgroups
  int QW;  // row quads of the largest workgroup
};

constexpr int kW8NW = 16;  // waves per workgroup
constexpr int kW8XP = 2;   // staged activation pieces (16 k, 32 B) per thread, at most

// LDS layout (byte offsets)
struct W8Lds {
  int xp;    // activations [M][K/16 pieces][8 dwords], pair order
  int xs;    // piece sums [K/16][4] fp32
  int part;  // quad sums [QW][U][4][MR] fp32 (MR = 1, or 4 for M > 1)
  int bytes;
};
__host__ __device__ __forceinline__ W8Lds w8_lds(int M, int K, int QW) {
  const int U = (K + 255) >> 8, MR = M == 1 ? 1 : 4;
  W8Lds l;
  l.xp = 0;
  l.xs = (M * K * 2 + 15) & ~15;
  l.part = l.xs + (K / 16) * 16;
  l.bytes = l.part + QW * U * 4 * MR * 4;
  return l;
}

constexpr int kW8MaxLds = 160 * 1024;

template <typename T, int MQ, int DEPTH>
__global__ __launch_bounds__(64 * kW8NW) void w8a16_gemv_kernel(W8a16Args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int NT = 64 * kW8NW;
  constexpr int MR = MQ == 1 ? 1 : 4;   // activation rows per slot
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = lane >> 2, j = lane & 3;
  const int M = a.M, N = a.N, K = a.K;
  const int U = (K + 255) >> 8;   // spans per row
  const int np = K >> 4;          // 16-k pieces per row
  const int qa = (int)((int64_t)blockIdx.x * a.nq / a.P);
  const int nql = (int)((int64_t)(blockIdx.x + 1) * a.nq / a.P) - qa;
  const int nitems = nql * U;
  const int i0 = (int)((int64_t)wave * nitems / kW8NW);
  const int nmy = (int)((int64_t)(wave + 1) * nitems / kW8NW) - i0;
  const W8Lds L = w8_lds(M, K, a.QW);

  const rsrc_t rx = make_rsrc(a.x, (uint32_t)M * K * 2);
  const rsrc_t rw = make_rsrc(a.w, (uint32_t)N * K);

  // weight offset of this lane's piece of item it (wave-uniform it); pieces
  // past the row end or past N read nothing (zeros)
  auto item_off = [&](int it) -> uint32_t {
    if (it >= i0 + nmy) return kOob;
    const int ql = it / U, s = it - ql * U;
    const int row = 4 * (qa + ql) + j, p = 256 * s + 16 * b;
    return row < N && p + 16 <= K ? (uint32_t)row * K + p : kOob;
  };

  // 1. staging loads of the activations (32-byte pieces); a wave with no
  // piece to fetch skips the instruction
  const int nxp = M * np;
  u32x4_t xr[kW8XP][2];
#pragma unroll
  for (int i = 0; i < kW8XP; ++i) {
    const int pi = tid + i * NT;
    if (i * NT + 64 * wave < nxp) {
      const uint32_t off = pi < nxp ? 32u * pi : kOob;
      xr[i][0] = buf_load16(rx, off);
      xr[i][1] = buf_load16(rx, off + 16);
    }
  }
  // 2. the first DEPTH items' weights
  u32x4_t wb[DEPTH];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) wb[d] = buf_load16(rw, item_off(i0 + d));
  __builtin_amdgcn_sched_barrier(0);

  // 3. LDS: activations in pair order, piece sums, cleared quad slots
  {
    float* part = reinterpret_cast<float*>(smem + L.part);
    for (int e = tid; e < nql * U * 4 * MR; e += NT) part[e] = 0.0f;
    uint32_t* xp = reinterpret_cast<uint32_t*>(smem + L.xp);
    float* xs = reinterpret_cast<float*>(smem + L.xs);
#pragma unroll
    for (int i = 0; i < kW8XP; ++i) {
      const int pi = tid + i * NT;
      if (pi < nxp) {
        uint32_t r[8] = {xr[i][0].x, xr[i][0].y, xr[i][0].z, xr[i][0].w,
                         xr[i][1].x, xr[i][1].y, xr[i][1].z, xr[i][1].w};
        uint32_t o[8];
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          o[2 * w] = __builtin_amdgcn_perm(r[2 * w + 1], r[2 * w], 0x05040100u);      // (x0, x2)
          o[2 * w + 1] = __builtin_amdgcn_perm(r[2 * w + 1], r[2 * w], 0x07060302u);  // (x1, x3)
          sum = pair_sum<T>(r[2 * w], sum);
          sum = pair_sum<T>(r[2 * w + 1], sum);
        }
        *reinterpret_cast<u32x4_t*>(xp + 8 * pi) = u32x4_t{o[0], o[1], o[2], o[3]};
        *reinterpret_cast<u32x4_t*>(xp + 8 * pi + 4) = u32x4_t{o[4], o[5], o[6], o[7]};
        const int m = pi / np, piece = pi - m * np;
        xs[4 * piece + m] = sum;
      }
    }
  }
  __syncthreads();

  // 4. the wave's items, DEPTH loads ahead
  const unsigned char* xp = smem + L.xp;
  const float* xs = reinterpret_cast<const float*>(smem + L.xs);
  float* part = reinterpret_cast<float*>(smem + L.part);
  const DecodeConsts dc = decode_consts<T>();
  constexpr float C = 17.0f * T::OFFSET + 128.0f;
  f32x4_t dl = {0.0f, 0.0f, 0.0f, 0.0f}, dh = dl, xsum = dl;
  int first = nmy > 0 ? (i0 - (i0 / U) * U) : 0;  // first span of the current run
  for (int base = 0; base < nmy; base += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int i = base + d;
      if (i < nmy) {
        const u32x4_t cur = wb[d];
        const int it = i0 + i;
        const int ql = it / U, s = it - ql * U;
        const int piece = min(16 * s + b, np - 1);
        const int pi = min(j, M - 1) * np + piece;
        const u32x4_t x0 = *reinterpret_cast<const u32x4_t*>(xp + 32 * pi);
        const u32x4_t x1 = *reinterpret_cast<const u32x4_t*>(xp + 32 * pi + 16);
        const uint32_t xa[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          uint32_t pr[4];
          decode_w4_strided<T>(cur[w] ^ 0x80808080u, dc, pr);
          dl = mfma4x4<T>(xa[2 * w], xa[2 * w + 1], pr[0], pr[2], dl);
          dh = mfma4x4<T>(xa[2 * w], xa[2 * w + 1], pr[1], pr[3], dh);
        }
        // a piece past the row end reads zeros, which decode as v = 0: its
        // D terms are exactly (17*OFFSET+128) times its activation sum, which
        // the correction removes again
        if constexpr (MQ == 1) {
          xsum[0] += xs[4 * piece];
        } else {
          xsum += *reinterpret_cast<const f32x4_t*>(xs + 4 * piece);
        }
        // end of a run: the next item is in another row quad, or none
        const bool last = i + 1 >= nmy || (it + 1) / U != ql;
        if (last) {
          float* dst = part + ((ql * U + first) * 4) * MR;
#pragma unroll
          for (int m = 0; m < MQ; ++m) {
            const float t = fmaf(16.0f, dh[m], dl[m]) - C * xsum[m];
            const float v = sum_blocks(t);
            if (lane < 4) dst[lane * MR + m] = v;
          }
          dl = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
          dh = dl;
          xsum = dl;
          first = s + 1 < U ? s + 1 : 0;
        }
      }
      // the next load into this slot goes after the decode has read it, on
      // every path, so each slot keeps its registers and the wait before an
      // item counts exactly the DEPTH - 1 loads issued after it
      __builtin_amdgcn_sched_barrier(0);
      wb[d] = buf_load16(rw, item_off(i0 + i + DEPTH));
    }
  }
  __syncthreads();

  // 5. each output: its quad's slots in span order, times the channel scale
  for (int t = tid; t < 4 * nql * M; t += NT) {
    const int rl = t / M, m = t - rl * M;
    const int row = 4 * qa + rl;
    if (row < N) {
      const float* src = part + ((rl >> 2) * U * 4 + (rl & 3)) * MR + m;
      float v = 0.0f;
      for (int s = 0; s < U; ++s) v += src[s * 4 * MR];
      store_out(a.y, (int64_t)m * N + row, v * a.scales[row], a.y_dtype);
    }
  }
}

// ---------------------------------------------------------------------------
// one-round W8A16 GEMV, M = 1, rows of up to 2560 k (w8a16_gemvq_kernel)
// ---------------------------------------------------------------------------
// The W4 one-round layout: every workgroup owns a contiguous range of row
// quads, one quad per wave, and the grid holds every quad at once. A wave
// walks its quad's 256-byte spans in order (lane 4b+j: bytes 256s + 16b of
// row 4q+j) with D spans' loads in flight (the first D ahead of the staging
// loads, each later one issued as the span D before it is taken up; with
// D = U all of them right after the staging loads), decodes each span as
// w8a16_gemv_kernel does and keeps D_l, D_h and the activation sum in
// registers over the whole row; the activations are staged in LDS once per
// workgroup (pair order, 16-k piece sums). Whole spans only (K % 256 == 0).
template <typename T, int U, int D>
__global__ __launch_bounds__(1024) void w8a16_gemvq_kernel(W8a16Args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = lane >> 2, j = lane & 3;
  const int N = a.N, K = a.K;
  const int ns = K >> 8;   // spans per row (<= U)
  const int np = K >> 4;   // 16-k pieces per row
  const int qa = (int)((int64_t)blockIdx.x * a.nq / a.P);
  const int nql = (int)((int64_t)(blockIdx.x + 1) * a.nq / a.P) - qa;

  const rsrc_t rx = make_rsrc(a.x, (uint32_t)K * 2);
  const rsrc_t rw = make_rsrc(a.w, (uint32_t)N * K);

  const bool has_quad = wave < nql;
  const int row = 4 * (qa + wave) + j;
  const uint32_t wbase = has_quad && row < N ? (uint32_t)row * K + 16u * b : kOob;
  u32x4_t wv[U];
  if constexpr (D < U) {
#pragma unroll
    for (int s = 0; s < D; ++s) wv[s] = buf_load16(rw, s < ns ? wbase + 256u * s : kOob);
  }
  // staging loads: one 32-byte piece per thread; a wave with none skips them
  u32x4_t xr0, xr1;
  if (64 * wave < np) {
    const uint32_t off = tid < np ? 32u * tid : kOob;
    xr0 = buf_load16(rx, off);
    xr1 = buf_load16(rx, off + 16);
  }
  if constexpr (D == U) {
#pragma unroll
    for (int s = 0; s < U; ++s) wv[s] = buf_load16(rw, s < ns ? wbase + 256u * s : kOob);
  }
  // keep every load above ahead of the arithmetic below
  __builtin_amdgcn_sched_barrier(0);

  uint32_t* xp = reinterpret_cast<uint32_t*>(smem);          // [K/16][8] dwords, pair order
  float* xs = reinterpret_cast<float*>(smem + 2 * K);        // [K/16] piece sums
  if (tid < np) {
    const uint32_t r[8] = {xr0.x, xr0.y, xr0.z, xr0.w, xr1.x, xr1.y, xr1.z, xr1.w};
    uint32_t o[8];
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      o[2 * w] = __builtin_amdgcn_perm(r[2 * w + 1], r[2 * w], 0x05040100u);      // (x0, x2)
      o[2 * w + 1] = __builtin_amdgcn_perm(r[2 * w + 1], r[2 * w], 0x07060302u);  // (x1, x3)
      sum = pair_sum<T>(r[2 * w], sum);
      sum = pair_sum<T>(r[2 * w + 1], sum);
    }
    *reinterpret_cast<u32x4_t*>(xp + 8 * tid) = u32x4_t{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<u32x4_t*>(xp + 8 * tid + 4) = u32x4_t{o[4], o[5], o[6], o[7]};
    xs[tid] = sum;
  }
  __syncthreads();
  if (!has_quad) return;

  const DecodeConsts dc = decode_consts<T>();
  constexpr float C = 17.0f * T::OFFSET + 128.0f;
  f32x4_t dl = {0.0f, 0.0f, 0.0f, 0.0f}, dh = dl;
  float xsum = 0.0f;
#pragma unroll
  for (int s = 0; s < U; ++s) {
    // span s + D's load goes out as span s is taken up
    if (s + D < U) wv[s + D] = buf_load16(rw, s + D < ns ? wbase + 256u * (s + D) : kOob);
    if (s < ns) {
      const int piece = 16 * s + b;
      const u32x4_t x0 = *reinterpret_cast<const u32x4_t*>(xp + 8 * piece);
      const u32x4_t x1 = *reinterpret_cast<const u32x4_t*>(xp + 8 * piece + 4);
      const uint32_t xa[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        uint32_t pr[4];
        decode_w4_strided<T>(wv[s][w] ^ 0x80808080u, dc, pr);
        dl = mfma4x4<T>(xa[2 * w], xa[2 * w + 1], pr[0], pr[2], dl);
        dh = mfma4x4<T>(xa[2 * w], xa[2 * w + 1], pr[1], pr[3], dh);
      }
      xsum += xs[piece];
    }
  }
  const float v = sum_blocks(fmaf(16.0f, dh[0], dl[0]) - C * xsum);
  const int orow = 4 * (qa + wave) + lane;
  if (lane < 4 && orow < N) store_out(a.y, orow, v * a.scales[orow], a.y_dtype);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
// One-round plan (M = 1, K % 256 == 0, K <= 2560): twice the CUs
// workgroups when that gives at least 8 quads per CU, else one per CU, at
// most 16 row-quad waves each (more workgroups past that), with at least
// the waves that stage the activations (one 32-byte piece per thread). One
// span in flight per wave where a CU holds 12 or more row-quad waves, every
// span on smaller grids. Measured on the MI355X (36 distinct weight sets per
// graph replay; the W8 lm_head 3): QKV 3584 x 2560 6.2 -> 4.4 us (all spans
// in flight; 5.7 at two, 6.2 at one), gate+up 19456 x 2560 13.7 -> 11.6 us
// (one in flight; 12.0 at two, 12.7 at all), lm_head 131072 x 2560 69 ->
// 58.7 us (5.7 TB/s) against the streaming kernel.
struct W8qPlan {
  bool ok;
  int P, NWQ, U, D;
  size_t lds;
};

static W8qPlan plan_w8q(int64_t M, int64_t N, int64_t K) {
  W8qPlan p{};
  if (M != 1 || K % 256 != 0 || K > 2560 || env_int("SPARKQ_W8A16_NO_Q", 0)) return p;
  if (N * K >= (int64_t)kOob) return p;
  const int64_t nq = cdiv(N, 4), cus = device_cus();
  int64_t P = std::min<int64_t>(nq, cus * (nq >= 8 * cus ? 2 : 1));
  if (cdiv(nq, P) > 16) P = cdiv(nq, 16);
  p.P = (int)P;
  const int64_t wpc = cdiv(nq, cus);
  p.NWQ = (int)std::max<int64_t>(cdiv(nq, P), cdiv(K / 16, 64));
  p.U = K <= 1024 ? 4 : 10;
  const int64_t d = env_int("SPARKQ_W8A16_Q_DEPTH", wpc >= 12 ? 1 : 8);
  p.D = d == 1 || d == 2 ? (int)d : p.U;
  p.lds = (size_t)K * 2 + (size_t)(K / 16) * 4;
  p.ok = true;
  return p;
}

template <typename T, int U>
static void launch_w8q_u(const W8qPlan& p, const W8a16Args& a, hipStream_t st) {
  const dim3 grid((unsigned)p.P), block(64 * p.NWQ);
  if (p.D == 1)
    hipLaunchKernelGGL((w8a16_gemvq_kernel<T, U, 1>), grid, block, p.lds, st, a);
  else if (p.D == 2)
    hipLaunchKernelGGL((w8a16_gemvq_kernel<T, U, 2>), grid, block, p.lds, st, a);
  else
    hipLaunchKernelGGL((w8a16_gemvq_kernel<T, U, U>), grid, block, p.lds, st, a);
}
template <typename T>
static void launch_w8q(const W8qPlan& p, const W8a16Args& a, hipStream_t st) {
  if (p.U == 4)
    launch_w8q_u<T, 4>(p, a, st);
  else
    launch_w8q_u<T, 10>(p, a, st);
}

struct W8a16Plan {
  bool ok;
  int P, QW, MQ, DEPTH;
  size_t lds;
};

static W8a16Plan plan_w8a16(int64_t M, int64_t N, int64_t K) {
  W8a16Plan p{};
  if (M < 1 || M > 4 || K % 16 != 0) return p;
  if (N * K >= (int64_t)kOob || M * K * 2 >= (int64_t)kOob) return p;
  const int64_t nq = cdiv(N, 4);
  p.P = (int)std::min<int64_t>(nq, device_cus());
  p.QW = (int)cdiv(nq, p.P);
  p.MQ = M == 1 ? 1 : 4;
  if (M * (K / 16) > kW8XP * 64 * kW8NW) return p;
  const W8Lds l = w8_lds((int)M, (int)K, p.QW);
  if (l.bytes > kW8MaxLds) return p;
  p.lds = (size_t)l.bytes;
  const int64_t dep = env_int("SPARKQ_W8A16_DEPTH", 4);
  p.DEPTH = dep >= 8 ? 8 : (dep >= 4 ? 4 : 2);
  p.ok = true;
  return p;
}

template <typename T, int MQ, int DEPTH>
static void launch_w8a16_d(const W8a16Plan& p, const W8a16Args& a, hipStream_t st) {
  auto* k = w8a16_gemv_kernel<T, MQ, DEPTH>;
  // dynamic LDS above 64 KB must be enabled per kernel
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, kW8MaxLds);
  (void)attr;
  hipLaunchKernelGGL(k, dim3((unsigned)p.P), dim3(64 * kW8NW), p.lds, st, a);
}
template <typename T, int MQ>
static void launch_w8a16_m(const W8a16Plan& p, const W8a16Args& a, hipStream_t st) {
  if (p.DEPTH == 2)
    launch_w8a16_d<T, MQ, 2>(p, a, st);
  else if (p.DEPTH == 4)
    launch_w8a16_d<T, MQ, 4>(p, a, st);
  else
    launch_w8a16_d<T, MQ, 8>(p, a, st);
}

int w8a16_linear(const void* x, const int8_t* w, const float* scales, void* y, int64_t M,
                 int64_t N, int64_t K, int xdt, int ydt, hipStream_t st) {
  const W8qPlan q = plan_w8q(M, N, K);
  if (q.ok) {
    W8a16Args a{};
    a.x = (const uint16_t*)x;
    a.w = w;
    a.scales = scales;
    a.y = y;
    a.y_dtype = ydt;
    a.M = 1;
    a.N = (int)N;
    a.K = (int)K;
    a.nq = (int)cdiv(N, 4);
    a.P = q.P;
    if (xdt == SPARKQ_BF16)
      launch_w8q<BF16>(q, a, st);
    else
      launch_w8q<F16>(q, a, st);
    return check_launch("w8a16_gemvq_kernel");
  }
  const W8a16Plan p = plan_w8a16(M, N, K);
  if (!p.ok)
    return set_error(SPARKQ_ERR_UNSUPPORTED,
                     "w8a16_linear: M=%lld N=%lld K=%lld is outside the kernel's range "
                     "(M <= 4, K %% 16 == 0, M*K <= 32768)",
                     (long long)M, (long long)N, (long long)K);
  W8a16Args a{};
  a.x = (const uint16_t*)x;
  a.w = w;
  a.scales = scales;
  a.y = y;
  a.y_dtype = ydt;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.nq = (int)cdiv(N, 4);
  a.P = p.P;
  a.QW = p.QW;
  if (xdt == SPARKQ_BF16) {
    if (p.MQ == 1)
      launch_w8a16_m<BF16, 1>(p, a, st);
    else
      launch_w8a16_m<BF16, 4>(p, a, st);
  } else {
    if (p.MQ == 1)
      launch_w8a16_m<F16, 1>(p, a, st);
    else
      launch_w8a16_m<F16, 4>(p, a, st);
  }
  return check_launch("w8a16_gemv_kernel");
}

}  // namespace sparkq
