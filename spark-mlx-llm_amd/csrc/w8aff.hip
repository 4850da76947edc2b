// w8aff.hip -- MLX affine 8-bit quantized matmul on gfx950:
// y[m,n] = sum_k x[m,k] * (u[n,k] * s[n,k/G] + b[n,k/G])
// with u the unsigned byte k%4 of word k/4 of row n (packed uint32 [N,K/4]),
// groupwise scales and biases [N,K/G] and 16-bit activations. This is
// mx.quantized_matmul(x, w, scales, biases, transpose=True, group_size,
// bits=8) as the reference's W8 layers call it when no per-channel adapter
// takes the input (spark_mlx_llm/ops/linear.py:413-476 falls back to the
// affine nn.QuantizedLinear for prefill and verify rows, and 'native'/'auto'
// W8 checkpoints use it for every input, :651-711).
//
// Kernel w8_affine_kernel. A workgroup of 4 waves owns a 32 x 128 output
// tile, each wave 32 activation rows x 32 weight rows as 2 x 2 blocks of the
// 16x16x32 MFMA:
//  * every code 0..255 is an exact 16-bit operand (bf16 and fp16 hold 8
//    significant bits), so D = sum_k x*u is formed from exact products in
//    fp32 per quantization group;
//  * the activation group sums X = sum_k x come from one more MFMA per
//    activation block against an operand of ones, which leaves them in the
//    accumulator layout of D;
//  * at each group's end y += s*D + b*X (two fp32 FMAs per output).
// A step covers 64 k (16-byte code loads) when G >= 64 and 32 k (8-byte code
// loads) when G = 32, so that one MFMA never straddles a group: within a step
// lane group g (lanes 16g..16g+15) owns the k range [KS/4*g, KS/4*(g+1)),
// for the activation operand and the code operand alike. The next step's
// loads are issued before the current step's MFMAs. Rows past M and columns
// past N read zeros (out-of-range buffer offsets) and are not stored.
#include "common.h"

namespace sparkq {

struct W8AffArgs {
  const uint16_t* x;    // [M][K] 16-bit
  const uint32_t* w;    // [N][K/4] packed codes
  const void* sc;       // [N][K/G] in the scale dtype
  const void* bi;       // [N][K/G]
  void* y;              // [M][N]
  int y_dtype, s_dtype;
  int M, N, K;
};

template <typename T>
__device__ __forceinline__ f32x4_t mfma_16x16x32(u32x4_t a, u32x4_t b, f32x4_t c);
template <>
__device__ __forceinline__ f32x4_t mfma_16x16x32<BF16>(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4_t mfma_16x16x32<F16>(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// Eight codes (two words, byte j of word w = code 4w+j) as eight exact 16-bit
// values in k order.
template <typename T>
__device__ __forceinline__ u32x4_t codes_to_16(uint32_t w0, uint32_t w1) {
  u32x4_t r;
  r.x = pack_round<T>((float)(w0 & 0xFFu), (float)((w0 >> 8) & 0xFFu));
  r.y = pack_round<T>((float)((w0 >> 16) & 0xFFu), (float)(w0 >> 24));
  r.z = pack_round<T>((float)(w1 & 0xFFu), (float)((w1 >> 8) & 0xFFu));
  r.w = pack_round<T>((float)((w1 >> 16) & 0xFFu), (float)(w1 >> 24));
  return r;
}

__device__ __forceinline__ float load_scale(const void* p, int64_t i, int dt) {
  return load_in(p, i, dt);
}

template <typename T, int KS>
__global__ __launch_bounds__(256) void w8_affine_kernel(W8AffArgs a, int G) {
  constexpr int NSUB = KS / 32;  // MFMAs per operand block and step
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int M = a.M, N = a.N, K = a.K;
  const int m0 = blockIdx.y * 32;
  const int n0 = blockIdx.x * 128 + wave * 32;
  const int ng = K / G;
  const int steps_per_group = G / KS;
  const rsrc_t rx = make_rsrc(a.x, (uint32_t)M * (uint32_t)K * 2u);
  const rsrc_t rw = make_rsrc(a.w, (uint32_t)N * (uint32_t)K);

  // per-lane row bases; rows past M / N read zeros
  uint32_t xoff[2], woff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = m0 + 16 * i + r16;
    const int n = n0 + 16 * i + r16;
    xoff[i] = m < M ? ((uint32_t)m * K + (uint32_t)(KS / 4) * g) * 2u : kOob;
    woff[i] = n < N ? (uint32_t)n * K + (uint32_t)(KS / 4) * g : kOob;
  }
  auto load_x = [&](int i, int k0, u32x4_t* dst) {
#pragma unroll
    for (int s = 0; s < NSUB; ++s)
      dst[s] = buf_load16(rx, xoff[i] == kOob ? kOob : xoff[i] + 2u * (uint32_t)k0 + 16u * s);
  };
  auto load_w = [&](int i, int k0, uint32_t* dst) {
    if constexpr (KS == 64) {
      const u32x4_t v = buf_load16(rw, woff[i] == kOob ? kOob : woff[i] + (uint32_t)k0);
      dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
    } else {
      const uint32_t o = woff[i] == kOob ? kOob : woff[i] + (uint32_t)k0;
      dst[0] = __builtin_amdgcn_raw_buffer_load_b32(rw, (int)o, 0, 0);
      dst[1] = __builtin_amdgcn_raw_buffer_load_b32(rw, (int)(o == kOob ? kOob : o + 4u), 0, 0);
    }
  };

  const uint32_t one = T::code == SPARKQ_BF16 ? 0x3F803F80u : 0x3C003C00u;
  const u32x4_t ones = {one, one, one, one};
  f32x4_t acc[2][2], d[2][2], xs[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    xs[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      d[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  }

  // scale and bias of this lane's two columns for the group of step st
  auto load_sb = [&](int st, float* sv, float* bv) {
    const int gq = st / steps_per_group;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t si = (int64_t)min(n0 + 16 * j + r16, N - 1) * ng + gq;
      sv[j] = load_scale(a.sc, si, a.s_dtype);
      bv[j] = load_scale(a.bi, si, a.s_dtype);
    }
  };

  u32x4_t xa[2][NSUB], xb[2][NSUB];
  uint32_t wa[2][2 * NSUB], wb[2][2 * NSUB];
  float sa[2], ba[2], sb[2], bb[2];
  const int nsteps = K / KS;
  load_x(0, 0, xa[0]);
  load_x(1, 0, xa[1]);
  load_w(0, 0, wa[0]);
  load_w(1, 0, wa[1]);
  load_sb(0, sa, ba);
  int step_in_group = 0;
  for (int st = 0; st < nsteps; ++st) {
    // the next step's loads first (after the last step they repeat step 0's
    // addresses and are unused)
    const int sn = st + 1 < nsteps ? st + 1 : 0;
    load_x(0, sn * KS, xb[0]);
    load_x(1, sn * KS, xb[1]);
    load_w(0, sn * KS, wb[0]);
    load_w(1, sn * KS, wb[1]);
    load_sb(sn, sb, bb);
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
      u32x4_t bop[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) bop[j] = codes_to_16<T>(wa[j][2 * s], wa[j][2 * s + 1]);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        xs[i] = mfma_16x16x32<T>(xa[i][s], ones, xs[i]);
#pragma unroll
        for (int j = 0; j < 2; ++j) d[i][j] = mfma_16x16x32<T>(xa[i][s], bop[j], d[i][j]);
      }
    }
    if (++step_in_group == steps_per_group) {
      // group epilogue: y += s*D + b*X for this lane's columns
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[i][j][r] = fmaf(ba[j], xs[i][r], fmaf(sa[j], d[i][j][r], acc[i][j][r]));
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        xs[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; ++j) d[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
      step_in_group = 0;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int s = 0; s < NSUB; ++s) xa[i][s] = xb[i][s];
#pragma unroll
      for (int e = 0; e < 2 * NSUB; ++e) wa[i][e] = wb[i][e];
      sa[i] = sb[i];
      ba[i] = bb[i];
    }
  }

  // C layout of the 16x16 MFMA: lane (g, r16) holds rows 4g..4g+3 of the
  // activation block and column r16 of the weight block
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + 16 * j + r16;
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + 16 * i + 4 * g + r;
        if (m < M) store_out(a.y, (int64_t)m * N + n, acc[i][j][r], a.y_dtype);
      }
    }
}

int w8_affine_linear(const void* x, const uint32_t* w, const void* s, const void* b, void* y,
                     int64_t M, int64_t N, int64_t K, int G, int xdt, int sdt, int ydt,
                     hipStream_t st) {
  W8AffArgs a{};
  a.x = (const uint16_t*)x;
  a.w = w;
  a.sc = s;
  a.bi = b;
  a.y = y;
  a.y_dtype = ydt;
  a.s_dtype = sdt;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  const dim3 grid((unsigned)cdiv(N, 128), (unsigned)cdiv(M, 32));
  if (G >= 64) {
    if (xdt == SPARKQ_BF16)
      hipLaunchKernelGGL((w8_affine_kernel<BF16, 64>), grid, dim3(256), 0, st, a, G);
    else
      hipLaunchKernelGGL((w8_affine_kernel<F16, 64>), grid, dim3(256), 0, st, a, G);
  } else {
    if (xdt == SPARKQ_BF16)
      hipLaunchKernelGGL((w8_affine_kernel<BF16, 32>), grid, dim3(256), 0, st, a, G);
    else
      hipLaunchKernelGGL((w8_affine_kernel<F16, 32>), grid, dim3(256), 0, st, a, G);
  }
  return check_launch("w8_affine_kernel");
}

}  // namespace sparkq
