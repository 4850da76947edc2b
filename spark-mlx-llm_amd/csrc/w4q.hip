// w4q.hip -- W4A16 decode GEMV for up to four activation rows, one row quad
// per wave.
//
// The M = 1 projection is HBM-bound, and its time is set by how the weight
// stream is spread over the CUs: measured on the gate+up weights (19456 x
// 2560, G64), a grid whose workgroups do not divide evenly over the CUs
// leaves the CUs with one workgroup more ~1.8 us behind the others, and a
// grid larger than what fits at once runs a second round that starts only
// when the first retires. This kernel runs every row quad in one round,
// with the same number of quads on every CU to within one:
//  * P workgroups (twice the CUs when there are at least 8 quads per CU,
//    else one per CU), workgroup i owning the contiguous quads
//    [i*nq/P, (i+1)*nq/P), one wave per quad; the workgroups of a CU hold
//    all its quads at once (occupancy: the activations are read from LDS per
//    span, not held for the whole row, so a wave needs 66-78 VGPRs);
//  * the activations (in the pair order of the strided decode) with their
//    32-k piece sums, and the (scale, bias) pairs of the workgroup's rows,
//    are staged once per workgroup in LDS;
//  * a wave loads its row quad one 16-byte load per lane and 256-byte span
//    (lane 4b+j reads bytes 16b.. of row 4q+j): all spans up front on small
//    grids, two spans ahead of the arithmetic when the CU holds 12 or more
//    row-quad waves (gate+up 7.8-8.2 -> 7.5 us: the CU's memory queue then
//    interleaves its waves' spans, so the arithmetic runs under the stream
//    instead of after it); per span it reads its activation piece from LDS,
//    decodes the codes to OFFSET + q 16-bit pairs and runs eight 4x4x4
//    MFMAs, and adds s*D + (b - OFFSET*s)*X for its group;
//  * the sixteen 4-lane blocks are added by DPP and permlane swaps and
//    lanes 0..3 write the quad's four outputs (plus an optional 16-bit
//    residual, rounded as the reference's hidden + mlp_output).
// K % 512 == 0 (whole spans), N % 4 == 0, rows of at most 8 spans, at most
// four activation rows.
#include <algorithm>

#include "common.h"

namespace sparkq {

struct GemvQArgs {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* sc;
  const uint16_t* bi;
  void* y;
  const uint16_t* res;  // 16-bit residual added to the rounded output (or null)
  int y_dtype;
  int M, N, K;
  int nq;  // row quads
  int P;   // workgroups
};

// LDS slot (dword index) of 16-byte chunk w of activation piece pi, the
// chunk-major span layout of the decode GEMVs: the 16 lane blocks of a wave
// read 16 consecutive pieces, 256 contiguous bytes per read.
__device__ __forceinline__ int q_xslot(int pi, int w) {
  return 256 * (pi >> 4) + 64 * w + 4 * (pi & 15);
}

struct GemvQLds {
  int xp;  // activations [M][K] in pair order (2 B each)
  int xs;  // piece sums [K/32] fp32, or [K/32][4] for several rows
  int sb;  // (scale, bias) of the workgroup's rows [4*NWQ][K/G] dwords
  int bytes;
};
__host__ __device__ __forceinline__ GemvQLds gemvq_lds(int M, int K, int NWQ, int G) {
  GemvQLds l;
  l.xp = 0;
  l.xs = (M * K * 2 + 1023) & ~1023;
  l.sb = l.xs + (((K / 32) * 4 * (M > 1 ? 4 : 1) + 15) & ~15);
  l.bytes = l.sb + 4 * NWQ * (K / G) * 4;
  return l;
}

// Staging of the one-round kernels: activation piece pc (64 B, 32 k, in
// r[0..3]) to LDS row xrow in the pair order of the strided decode, returning
// the piece's sum; and 16-byte (scale, bias) pieces t to (s, b) pairs.
template <typename T>
__device__ __forceinline__ float stage_x_piece(uint32_t* xrow, int pc, const u32x4_t (&r)[4]) {
  float sum = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const u32x4_t o = {__builtin_amdgcn_perm(r[w].z, r[w].x, 0x05040100u),   // (x0, x4)
                       __builtin_amdgcn_perm(r[w].z, r[w].x, 0x07060302u),   // (x1, x5)
                       __builtin_amdgcn_perm(r[w].w, r[w].y, 0x05040100u),   // (x2, x6)
                       __builtin_amdgcn_perm(r[w].w, r[w].y, 0x07060302u)};  // (x3, x7)
    *reinterpret_cast<u32x4_t*>(xrow + q_xslot(pc, w)) = o;
#pragma unroll
    for (int e = 0; e < 4; ++e) sum = pair_sum<T>(r[w][e], sum);
  }
  return sum;
}
__device__ __forceinline__ void stage_sb_piece(uint32_t* sb, int t, u32x4_t s, u32x4_t b) {
  u32x4_t lo, hi;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    lo[e] = __builtin_amdgcn_perm(b[e], s[e], 0x05040100u);  // (s0, b0)
    hi[e] = __builtin_amdgcn_perm(b[e], s[e], 0x07060302u);  // (s1, b1)
  }
  *reinterpret_cast<u32x4_t*>(sb + 8 * t) = u32x4_t{lo[0], hi[0], lo[1], hi[1]};
  *reinterpret_cast<u32x4_t*>(sb + 8 * t + 4) = u32x4_t{lo[2], hi[2], lo[3], hi[3]};
}

// Steps 4 and 5 of the one-round kernels: per span, the activation piece
// from LDS, the decode, eight 4x4x4 MFMAs and the group epilogue; then the
// sixteen lane blocks (lanes j, j+4, ..., j+60) summed and lanes 0..3
// storing row 4q+j of each activation row. wave indexes the row quad's
// (scale, bias) rows in LDS.
template <typename T, int G, int U, int MQ, int D>
__device__ __forceinline__ void gemvq_spans(const GemvQArgs& a, u32x4_t (&wv)[U], rsrc_t rw,
                                            uint32_t wbase, const unsigned char* smem,
                                            const GemvQLds& L, int ns, int wave, int M, int row) {
  const int lane = threadIdx.x & 63, b = lane >> 2, j = lane & 3;
  const int K = a.K, N = a.N, ng = K / G;
  const unsigned char* xp = smem + L.xp;
  const float* xs = reinterpret_cast<const float*>(smem + L.xs);
  const uint32_t* sb = reinterpret_cast<const uint32_t*>(smem + L.sb);
  const DecodeConsts dc = decode_consts<T>();
  // with several rows, lane 4b+j feeds activation row min(j, M-1) as the A
  // operand's row j, and its result D[i] is row i's (the row quad's row j)
  const int xrow = MQ == 1 ? 0 : min(j, M - 1);
  float acc[MQ];
#pragma unroll
  for (int m = 0; m < MQ; ++m) acc[m] = 0.0f;
#pragma unroll
  for (int s = 0; s < U; ++s) {
    // span s + D's load goes out as span s is taken up
    if (s + D < U) wv[s + D] = buf_load16(rw, s + D < ns ? wbase + 256u * (s + D) : kOob);
    if (s < ns) {
      const int piece = 16 * s + b;
      u32x4_t xa[4];
#pragma unroll
      for (int w = 0; w < 4; ++w)
        xa[w] = *reinterpret_cast<const u32x4_t*>(xp + 4 * (xrow * (K >> 1) + q_xslot(piece, w)));
      const uint32_t pair = sb[(4 * wave + j) * ng + (512 * s + 32 * b) / G];
      // one chain of eight MFMAs per span for rows of three or more spans,
      // two chains of four below: the summation order of w4_gemv_kernel, so
      // that the fused FFN and QKV launches (built on that kernel) and this
      // plain projection give identical bits
      f32x4_t d0 = {0.0f, 0.0f, 0.0f, 0.0f}, d1 = d0;
      if (ns >= 3) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          uint32_t pr[4];
          decode_w4_strided<T>(wv[s][w], dc, pr);
          d0 = mfma4x4<T>(xa[w][0], xa[w][1], pr[0], pr[1], d0);
          d0 = mfma4x4<T>(xa[w][2], xa[w][3], pr[2], pr[3], d0);
        }
      } else {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          uint32_t pr[4];
          decode_w4_strided<T>(wv[s][w], dc, pr);
          d0 = mfma4x4<T>(xa[w][0], xa[w][1], pr[0], pr[1], d0);
          d1 = mfma4x4<T>(xa[w][2], xa[w][3], pr[2], pr[3], d1);
        }
#pragma unroll
        for (int m = 0; m < MQ; ++m) d0[m] += d1[m];
      }
      const float sf = T::to_f32((uint16_t)(pair & 0xFFFFu));
      const float bf = fmaf(-T::OFFSET, sf, T::to_f32((uint16_t)(pair >> 16)));
      if constexpr (MQ == 1) {
        acc[0] = fmaf(sf, d0[0], fmaf(bf, xs[piece], acc[0]));
      } else {
        const f32x4_t xm = *reinterpret_cast<const f32x4_t*>(xs + 4 * piece);
#pragma unroll
        for (int m = 0; m < MQ; ++m) acc[m] = fmaf(sf, d0[m], fmaf(bf, xm[m], acc[m]));
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MQ; ++m) {
    const float v = sum_blocks(acc[m]);
    if (lane < 4 && row < N && m < M) {
      const int64_t idx = (int64_t)m * N + row;
      store_out(a.y, idx, a.res ? add_rounded<T>(v, a.res[idx]) : v, a.y_dtype);
    }
  }
}

// MQ: 1, or 4 for 2..4 activation rows; D: weight loads of a wave in flight
// (the first D spans' go out right after the staging loads)
template <typename T, int G, int U, int MQ, int D>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(5)))
void w4_gemv_q_kernel(GemvQArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int nt = blockDim.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = lane >> 2, j = lane & 3;
  const int M = MQ == 1 ? 1 : a.M, N = a.N, K = a.K;
  const int RB = K >> 1;     // bytes per weight row
  const int ns = RB >> 8;    // spans per row (<= U)
  const int ng = K / G;      // groups per row
  const int qa = (int)((int64_t)blockIdx.x * a.nq / a.P);
  const int nql = (int)((int64_t)(blockIdx.x + 1) * a.nq / a.P) - qa;
  const GemvQLds L = gemvq_lds(M, K, nt >> 6, G);

  const rsrc_t rx = make_rsrc(a.x, (uint32_t)(M * K) * 2);
  const rsrc_t rw = make_rsrc(a.w, (uint32_t)N * RB);
  const rsrc_t rs = make_rsrc(a.sc, (uint32_t)N * ng * 2);
  const rsrc_t rb = make_rsrc(a.bi, (uint32_t)N * ng * 2);

  // 1. the wave's row quad, lane 4b+j reading bytes 256s + 16b of row 4q+j
  // for span s. With D < U spans in flight, the loads of the first D go out
  // right after the staging loads and each later one as the span D before
  // it is taken up, so that the CU's memory queue serves all its waves'
  // early spans before their late ones and every wave computes while the
  // stream lasts (with all spans in flight at once, the waves issued last
  // got their whole row last and computed it after the stream ended). The
  // staging loads go first: the workgroup's barrier waits for them, not for
  // the weights (gate+up 7.67 -> 7.53 us, 4 rows 9.22 -> 9.03 us against the
  // first D weight loads ahead of them). With D = U all spans go out there.
  const bool has_quad = wave < nql;
  const int row = 4 * (qa + wave) + j;
  const uint32_t wbase = has_quad ? (uint32_t)row * RB + 16u * b : kOob;
  u32x4_t wv[U];

  // 2. staging loads: activation pieces (64 B: 32 k; piece i of the M rows
  // in order) and 16-byte (scale, bias) pieces of the workgroup's 4*nql
  // rows. A thread takes at most one activation piece and at most two scale
  // pieces (the plan gives the workgroup the waves for both); a wave with
  // nothing to fetch skips the instruction.
  const int nxp = M * (K >> 5);
  const int nsp = (4 * nql * ng) >> 3;
  u32x4_t xr[4], sr[2] = {}, br[2] = {};
  if (64 * wave < nxp) {
    const uint32_t off = tid < nxp ? 64u * tid : kOob;
#pragma unroll
    for (int w = 0; w < 4; ++w) xr[w] = buf_load16(rx, off + 16 * w);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int t = tid + h * nt;
    if (64 * wave + h * nt < nsp) {
      const uint32_t off = t < nsp ? 8u * (uint32_t)qa * ng + 16u * t : kOob;
      sr[h] = buf_load16(rs, off);
      br[h] = buf_load16(rb, off);
    }
  }

  // the first D spans' weights (all of them when D = U)
#pragma unroll
  for (int s = 0; s < D; ++s)
    wv[s] = buf_load16(rw, has_quad && s < ns ? wbase + 256u * s : kOob);

  // keep every load above ahead of the arithmetic below
  __builtin_amdgcn_sched_barrier(0);

  // 3. staged data to LDS
  {
    uint32_t* xp = reinterpret_cast<uint32_t*>(smem + L.xp);
    float* xs = reinterpret_cast<float*>(smem + L.xs);
    if (tid < nxp) {
      // piece tid is piece `pc` of activation row m (rows of K/2 dwords)
      const int m = MQ == 1 ? 0 : tid / (K >> 5), pc = tid - m * (K >> 5);
      xs[MQ == 1 ? pc : 4 * pc + m] = stage_x_piece<T>(xp + m * (K >> 1), pc, xr);
    }
    uint32_t* sb = reinterpret_cast<uint32_t*>(smem + L.sb);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int t = tid + h * nt;
      if (t < nsp) stage_sb_piece(sb, t, sr[h], br[h]);
    }
  }
  __syncthreads();
  if (!has_quad) return;

  // 4. per span: activations from LDS, decode, eight 4x4x4 MFMAs, group
  // epilogue; 5. the row quad's outputs
  gemvq_spans<T, G, U, MQ, D>(a, wv, rw, wbase, smem, L, ns, wave, M, row);
}

// Plan: M <= 4, K % 512 == 0 with at most 8 spans per row, N % 4 == 0, the
// scale tensors ending on a 16-byte boundary (2..4 rows: the 4x4x4 blocks'
// four A rows carry the activation rows, and every workgroup stages all of
// them, one 32-k piece per thread). Workgroups: twice the CUs when
// that gives at least 8 quads per CU (two workgroups of ~nq/(2*CUs) waves
// each), else one per CU, else one quad each; at most 16 waves. Measured
// alternatives that ran slower on the gate+up weights: two or four quads per
// wave (9.1-10 us against 7.8-8.1), one workgroup per CU (10.2 us). At 2, 3
// and 4 rows gate+up takes 8.5 / 8.8 / 9.6 us here against 9.4 / 10.1 / 10.9
// on the whole-row kernel (w4_gemv_kernel), QKV the same within 0.2 us. Rows of
// up to 20 spans (the down projection, 2560 x 9728: 19 spans, five waves per
// workgroup to stage its activations) ran 7.3 us here against 6.1 us in the
// streaming kernel, so longer rows stay there. Five to eight rows as two row
// quartets per 4x4x4 block (two MFMA chains on each decoded piece) ran
// gate+up at 5 / 6 / 8 rows in 12.8 / 13.6 / 16.9 us against 12.6 / 13.0 /
// 14.1 on the multi-row streaming kernel, so they stay there.
struct GemvQPlan {
  bool ok;
  int P, NWQ, U, MQ, D;
  size_t lds;
};

static GemvQPlan plan_gemvq(int64_t M, int64_t N, int64_t K, int G) {
  GemvQPlan p{};
  if (M < 1 || M > env_int("SPARKQ_W4_GEMVQ_MAXM", 4) || M > 4 || env_int("SPARKQ_W4_NO_GEMVQ", 0)) return p;
  if (K % 512 != 0 || N % 4 != 0 || K / 512 > 8) return p;
  if (N * (K / 2) >= (int64_t)kOob || M * K * 2 >= (int64_t)kOob) return p;
  const int64_t ng = K / G;
  if ((N * ng * 2) % 16 != 0 || ng % 2 != 0) return p;
  const int64_t nq = N / 4, cus = device_cus();
  const int64_t wgpc = env_int("SPARKQ_W4_GEMVQ_WGPC", nq >= 8 * cus ? 2 : 1);
  int64_t P = std::min<int64_t>(nq, cus * wgpc);
  if (cdiv(nq, P) > 16) P = cdiv(nq, 16);
  p.P = (int)P;
  p.NWQ = (int)cdiv(nq, P);
  p.U = K / 512 <= 5 ? 5 : 8;
  // weight loads in flight per wave: two when the CU holds at least 12 row-quad
  // waves (gate+up: 19), all spans for smaller grids, whose few waves need
  // every load in flight to keep the CU's stream going (QKV 3584 x 2560: 3.5
  // waves per CU ran 3.68 -> 3.83 us at two)
  const int64_t wpc = cdiv(P * p.NWQ, cus);
  p.D = (int)env_int("SPARKQ_W4_GEMVQ_DEPTH", wpc >= 12 ? 2 : 8);
  if (p.D != 1 && p.D != 2) p.D = 8;
  // threads enough to stage the activations, one 32-k piece each
  p.NWQ = (int)std::max<int64_t>(std::max<int64_t>(p.NWQ, 4), cdiv(M * K / 32, 64));
  if (p.NWQ > 16) return p;
  if (4 * p.NWQ * ng / 8 > 2 * 64 * p.NWQ) return p;  // two scale pieces per thread
  p.MQ = M == 1 ? 1 : 4;
  const GemvQLds l = gemvq_lds((int)M, (int)K, p.NWQ, G);
  if (l.bytes > 65536) return p;
  p.lds = (size_t)l.bytes;
  p.ok = true;
  return p;
}

template <typename T, int G, int MQ, int U>
static void launch_gemvq_u(const GemvQPlan& p, const GemvQArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)p.P), block(64 * p.NWQ);
  if (p.D == 1)
    hipLaunchKernelGGL((w4_gemv_q_kernel<T, G, U, MQ, 1>), grid, block, p.lds, st, a);
  else if (p.D == 2)
    hipLaunchKernelGGL((w4_gemv_q_kernel<T, G, U, MQ, 2>), grid, block, p.lds, st, a);
  else
    hipLaunchKernelGGL((w4_gemv_q_kernel<T, G, U, MQ, U>), grid, block, p.lds, st, a);
}
template <typename T, int G, int MQ>
static void launch_gemvq_m(const GemvQPlan& p, const GemvQArgs& a, hipStream_t st) {
  if (p.U == 5)
    launch_gemvq_u<T, G, MQ, 5>(p, a, st);
  else
    launch_gemvq_u<T, G, MQ, 8>(p, a, st);
}
template <typename T, int G>
static void launch_gemvq_g(const GemvQPlan& p, const GemvQArgs& a, hipStream_t st) {
  if (p.MQ == 1)
    launch_gemvq_m<T, G, 1>(p, a, st);
  else
    launch_gemvq_m<T, G, 4>(p, a, st);
}

// Returns 1 when the shape is not this kernel's (the caller picks another).
int w4_gemvq_linear(const void* x, const uint32_t* w, const void* s, const void* b, void* y,
                    int64_t M, int64_t N, int64_t K, int G, int xdt, int ydt, hipStream_t st,
                    const void* res) {
  const GemvQPlan p = plan_gemvq(M, N, K, G);
  if (!p.ok) return 1;
  GemvQArgs a{};
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
  a.nq = (int)(N / 4);
  a.P = p.P;
  if (xdt == SPARKQ_BF16) {
    if (G == 32) launch_gemvq_g<BF16, 32>(p, a, st);
    else if (G == 64) launch_gemvq_g<BF16, 64>(p, a, st);
    else launch_gemvq_g<BF16, 128>(p, a, st);
  } else {
    if (G == 32) launch_gemvq_g<F16, 32>(p, a, st);
    else if (G == 64) launch_gemvq_g<F16, 64>(p, a, st);
    else launch_gemvq_g<F16, 128>(p, a, st);
  }
  return check_launch("w4_gemv_q_kernel");
}

}  // namespace sparkq
