// common.h -- device helpers shared by the gfx950 kernels of libsparkq.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "sparkq.h"

namespace sparkq {

// ---------------------------------------------------------------------------
// vector types used as MFMA operands (gfx950, wave64)
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// 16-bit float <-> fp32 (bit-level, round-to-nearest-even)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float((uint32_t)h << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Element traits of the 16-bit activation types. MAGIC is the exponent
// pattern under which a 4-bit code q placed in the low mantissa bits reads as
// exactly MAGIC_VALUE + q; OFFSET is what remains in the decoded operand.
// fp16 removes its 1024 exactly with a packed fp16 subtract (OFFSET 0);
// bf16 has no packed subtract and keeps 128 + q, which the per-group epilogue
// corrects with b' = b - 128*s.
struct BF16 {
  static constexpr int code = SPARKQ_BF16;
  static constexpr uint32_t MAGIC = 0x43004300u;  // bf16 128.0 in each half
  static constexpr bool kExactDecode = false;
  static constexpr float OFFSET = 128.0f;
  __device__ static __forceinline__ float to_f32(uint16_t h) { return bf16_to_f32(h); }
  __device__ static __forceinline__ uint16_t from_f32(float f) { return f32_to_bf16(f); }
};
struct F16 {
  static constexpr int code = SPARKQ_F16;
  static constexpr uint32_t MAGIC = 0x64006400u;  // fp16 1024.0 in each half
  static constexpr bool kExactDecode = true;
  static constexpr float OFFSET = 0.0f;
  __device__ static __forceinline__ float to_f32(uint16_t h) { return f16_to_f32(h); }
  __device__ static __forceinline__ uint16_t from_f32(float f) { return f32_to_f16(f); }
};

// 32x32x16 MFMA on 16-bit operands held as four packed uint32 registers.
template <typename T>
__device__ __forceinline__ f32x16_t mfma32x32x16(u32x4_t a, u32x4_t b, f32x16_t c);
template <>
__device__ __forceinline__ f32x16_t mfma32x32x16<BF16>(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16_t mfma32x32x16<F16>(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Decode one uint32 of eight 4-bit codes (code j at bits 4j) into the four
// packed 16-bit pairs (OFFSET+q[2i], OFFSET+q[2i+1]), i = 0..3, in natural k
// order: a byte permute pulls code 2i from w and code 2i+1 from w>>4 into the
// low nibble of each half, and one and-or masks the nibble under MAGIC.
__device__ __forceinline__ uint32_t exact_f16_pair(uint32_t r) {
  const f16x2_t v = __builtin_bit_cast(f16x2_t, r) - f16x2_t{(_Float16)1024.0f, (_Float16)1024.0f};
  return __builtin_bit_cast(uint32_t, v);
}

// A 32-bit constant held in a VGPR. gfx9 VALU instructions read at most one
// SGPR or literal, so (x & mask) | magic with both constants as literals
// splits into two instructions; with them in VGPRs it is one v_bitop3.
__device__ __forceinline__ uint32_t vgpr_const(uint32_t v) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(v));
  return r;
}

// The two decode constants, materialised once per kernel.
struct DecodeConsts {
  uint32_t mask, magic;
};
template <typename T>
__device__ __forceinline__ DecodeConsts decode_consts() {
  return DecodeConsts{vgpr_const(0x000F000Fu), vgpr_const(T::MAGIC)};
}

template <typename T>
__device__ __forceinline__ u32x4_t decode_w4(uint32_t w, DecodeConsts c) {
  const uint32_t ws = w >> 4;
  u32x4_t r;
  r.x = (__builtin_amdgcn_perm(ws, w, 0x0C040C00u) & c.mask) | c.magic;
  r.y = (__builtin_amdgcn_perm(ws, w, 0x0C050C01u) & c.mask) | c.magic;
  r.z = (__builtin_amdgcn_perm(ws, w, 0x0C060C02u) & c.mask) | c.magic;
  r.w = (__builtin_amdgcn_perm(ws, w, 0x0C070C03u) & c.mask) | c.magic;
  if constexpr (T::kExactDecode) {
    r.x = exact_f16_pair(r.x);
    r.y = exact_f16_pair(r.y);
    r.z = exact_f16_pair(r.z);
    r.w = exact_f16_pair(r.w);
  }
  return r;
}

// ---------------------------------------------------------------------------
// reductions over the 16 lanes of each 16-lane row (DPP row rotations by 1,
// 2, 4 and 8, each doubling the window; every lane ends with the result).
// All lanes of the wave must be active.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_row(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float sum_row16(float v) {
  v += dpp_row<0x121>(v);
  v += dpp_row<0x122>(v);
  v += dpp_row<0x124>(v);
  v += dpp_row<0x128>(v);
  return v;
}
__device__ __forceinline__ float max_row16(float v) {
  v = fmaxf(v, dpp_row<0x121>(v));
  v = fmaxf(v, dpp_row<0x122>(v));
  v = fmaxf(v, dpp_row<0x124>(v));
  v = fmaxf(v, dpp_row<0x128>(v));
  return v;
}

// ---------------------------------------------------------------------------
// 4x4x4 MFMA blocks, pair sums and the strided 4-bit decode shared by the
// decode GEMVs
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ f32x4_t mfma4x4(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1,
                                           f32x4_t c);
template <>
__device__ __forceinline__ f32x4_t mfma4x4<BF16>(uint32_t a0, uint32_t a1, uint32_t b0,
                                                 uint32_t b1, f32x4_t c) {
  typedef short s16x4_t __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4_t, u32x2_t{a0, a1}),
                                                __builtin_bit_cast(s16x4_t, u32x2_t{b0, b1}), c,
                                                0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4_t mfma4x4<F16>(uint32_t a0, uint32_t a1, uint32_t b0,
                                                uint32_t b1, f32x4_t c) {
  typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4_t, u32x2_t{a0, a1}),
                                            __builtin_bit_cast(f16x4_t, u32x2_t{b0, b1}), c, 0,
                                            0, 0);
}

// sum of the two 16-bit values of a packed pair, in fp32
template <typename T>
__device__ __forceinline__ float pair_sum(uint32_t p, float acc);
template <>
__device__ __forceinline__ float pair_sum<BF16>(uint32_t p, float acc) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, p),
                                         __builtin_bit_cast(bf16x2_t, 0x3F803F80u), acc, false);
}
template <>
__device__ __forceinline__ float pair_sum<F16>(uint32_t p, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, p),
                                __builtin_bit_cast(f16x2_t, 0x3C003C00u), acc, false);
}

// Decode one word of eight codes into the pairs (q[j], q[j+4]), j = 0..3, as
// OFFSET+q 16-bit values: pair j is ((w >> 4j) & 0x000F000F) | MAGIC.
template <typename T>
__device__ __forceinline__ void decode_w4_strided(uint32_t w, DecodeConsts c, uint32_t p[4]) {
  p[0] = (w & c.mask) | c.magic;
  p[1] = ((w >> 4) & c.mask) | c.magic;
  p[2] = ((w >> 8) & c.mask) | c.magic;
  p[3] = ((w >> 12) & c.mask) | c.magic;
  if constexpr (T::kExactDecode) {
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = exact_f16_pair(p[i]);
  }
}

// Sum over the sixteen 4-lane blocks of a wave (lanes j, j+4, ..., j+60):
// two row rotations inside each 16-lane row (DPP), then the row pairs and the
// wave halves exchanged with v_permlane16/32_swap (a swap of v with itself
// leaves each lane's value and its partner's in the two results). Every lane
// ends with the sum of its j.
__device__ __forceinline__ float sum_blocks(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// ---------------------------------------------------------------------------
// buffer loads: a load whose offset lies outside the buffer returns zero and
// touches no memory, so a lane that has nothing to read gets zeros without a
// branch (a branch around a load makes the compiler wait for the load where
// the branch rejoins). Buffers must be smaller than kOob bytes.
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOob = 0x80000000u;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // dword 3 = 0x00020000: 32-bit data format, as raw loads require on gfx9
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4_t buf_load16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
__device__ __forceinline__ uint32_t buf_load2(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}

// Output row of accumulator v held by lane l for a 32x32 MFMA tile.
__device__ __forceinline__ int mfma32_row(int lane, int v) {
  return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
}

// Store one fp32 as the requested output dtype.
__device__ __forceinline__ void store_out(void* y, int64_t idx, float v, int dtype) {
  if (dtype == SPARKQ_F32) {
    reinterpret_cast<float*>(y)[idx] = v;
  } else if (dtype == SPARKQ_BF16) {
    reinterpret_cast<uint16_t*>(y)[idx] = f32_to_bf16(v);
  } else {
    reinterpret_cast<uint16_t*>(y)[idx] = f32_to_f16(v);
  }
}

// ---------------------------------------------------------------------------
// elementwise steps of the decoder layer around the projections, each with
// the rounding points of the reference's 16-bit graph: every operation of the
// bf16/fp16 graph computes in fp32 and rounds to the 16-bit type.
// ---------------------------------------------------------------------------
// Round v to T, then add a 16-bit residual (hidden + mlp_output,
// spark_mlx_llm/ops/ffn.py:105). The caller rounds the sum when it stores.
template <typename T>
__device__ __forceinline__ float add_rounded(float v, uint16_t res) {
  return T::to_f32(T::from_f32(v)) + T::to_f32(res);
}

// The two 16-bit values of a packed pair as fp32, and two fp32 values rounded
// (to nearest even) into a packed pair: one v_cvt_pk_bf16_f32 on gfx950.
template <typename T> __device__ __forceinline__ float lo16(uint32_t p);
template <typename T> __device__ __forceinline__ float hi16(uint32_t p);
template <typename T> __device__ __forceinline__ uint32_t pack_round(float a, float b);
template <> __device__ __forceinline__ float lo16<BF16>(uint32_t p) { return __uint_as_float(p << 16); }
template <> __device__ __forceinline__ float hi16<BF16>(uint32_t p) {
  return __uint_as_float(p & 0xFFFF0000u);
}
template <> __device__ __forceinline__ uint32_t pack_round<BF16>(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}
template <> __device__ __forceinline__ float lo16<F16>(uint32_t p) { return f16_to_f32((uint16_t)p); }
template <> __device__ __forceinline__ float hi16<F16>(uint32_t p) {
  return f16_to_f32((uint16_t)(p >> 16));
}
template <> __device__ __forceinline__ uint32_t pack_round<F16>(float a, float b) {
  return (uint32_t)f32_to_f16(a) | ((uint32_t)f32_to_f16(b) << 16);
}

// Sum over the 64 lanes of a wave, the same value in every lane: pairs and
// quads by DPP, the sixteen quads by sum_blocks, then lane 0's value.
__device__ __forceinline__ float wave_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v = sum_blocks(v);
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// erf(t) as it rounds to T: the fp32 erff (error of a few units of fp32)
// decides the 16-bit result unless it lies within 16 fp32 units of a
// rounding tie of T (or in fp16's subnormal range); those few are redone in
// double and rounded to fp32, as a correctly rounded float erf would give.
template <typename T>
__device__ __forceinline__ float erf_for16(float t) {
  float e = erff(t);
  const uint32_t u = __float_as_uint(e);
  bool redo;
  if constexpr (T::code == SPARKQ_BF16) {
    const int low = (int)(u & 0xFFFFu) - 0x8000;
    redo = low > -16 && low < 16;
  } else {
    const int low = (int)(u & 0x1FFFu) - 0x1000;
    redo = (low > -16 && low < 16) || fabsf(e) < 6.2e-5f;
  }
  if (redo) e = (float)erf((double)t);
  return e;
}

// gelu(gate) * up as mlx.nn.gelu computes it on a 16-bit array,
// x * (1 + erf(x / sqrt(2))) / 2 (spark_mlx_llm/ops/ffn.py:102): the constant
// sqrt(2) is rounded to T (1.4140625 for both types) and each operation's
// result is rounded to T. erf runs in double and is rounded to fp32 first,
// as a float erf would deliver it. g and u are the projections' fp32 sums;
// the result is the product's fp32 value, which the caller rounds to T.
template <typename T>
__device__ __forceinline__ float gelu_mul(float g, float u) {
  auto r = [](float v) { return T::to_f32(T::from_f32(v)); };
  const float gate = r(g), up = r(u);
  const float c = r(1.41421356237309515f);
  const float t1 = r(gate / c);
  const float e = r(erf_for16<T>(t1));
  const float t3 = r(1.0f + e);
  const float t5 = r(r(gate * t3) / 2.0f);
  return t5 * up;
}

// Inverse frequency of rotary pair i of mx.fast.rope: 2^(-(i / half) *
// log2(base)), d and the exponent in fp32, the power correctly rounded to
// fp32 (through double: a unit of fp32 in the frequency is a position-sized
// error in the angle).
__device__ __forceinline__ float rope_inv_freq(int i, int half, float log2_base) {
  const float d = (float)i / (float)half;
  return (float)exp2((double)(-d * log2_base));
}

__device__ __forceinline__ float load_in(const void* p, int64_t idx, int dtype) {
  if (dtype == SPARKQ_F32) return reinterpret_cast<const float*>(p)[idx];
  uint16_t h = reinterpret_cast<const uint16_t*>(p)[idx];
  return dtype == SPARKQ_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

// ---------------------------------------------------------------------------
// split-K handshake: combine per-workgroup partials in the same launch
// ---------------------------------------------------------------------------
// Partials are written and read with device-scope relaxed atomics, which take
// the coherent path between the XCDs' L2 caches without the L2 writeback and
// invalidate that a device-scope fence costs. A workgroup waits until its own
// partial stores are performed (s_waitcnt 0) before bumping the tile counter,
// so the workgroup that sees the count reach S-1 finds every partial in
// place; it resets the counter to zero for the next launch.
//
// Why relaxed atomics suffice here (the ordering argument). On gfx942/gfx950
// the LLVM AMDGPU memory model implements an agent-scope release as
// "buffer_wbl2 sc1; s_waitcnt vmcnt(0)" before the flag access and an
// acquire as "s_waitcnt vmcnt(0); buffer_inv sc1" after it, and a relaxed
// agent-scope load or store as the plain access with the sc1 cache policy,
// which is coherent at the device coherence point by itself. The L2
// writeback and invalidate exist only for data accessed WITHOUT sc1 (dirty
// or stale lines in one XCD's L2). Here every access to the exchanged data
// is an sc1 access: the partial stores (splitk_store, or raw buffer stores
// with the sc1 policy bit) and the partial loads (splitk_load, or raw
// buffer loads with sc1). What remains of release/acquire is the ordering,
// and the hardware gives it as follows:
//  * writer: s_waitcnt vmcnt(0) returns only after every store of the
//    thread has been acknowledged, and an sc1 store is acknowledged once it
//    is performed at the coherence point; the barrier then orders all
//    threads' completed stores before thread 0 issues the counter RMW;
//  * reader: the partial loads are issued only after the RMW has returned
//    its value (the branch on it, broadcast through LDS and a barrier), so
//    they are performed after it, and being sc1 they read the coherence
//    point, not a stale L2 line.
// The same holds for the producer/consumer counters of the W8A8 one-launch
// quantizer. A full acq_rel RMW would add an L2 writeback and invalidate of
// the whole XCD L2 per arrival, which the protocol does not need.
template <typename V>
__device__ __forceinline__ void splitk_store(V* p, V v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename V>
__device__ __forceinline__ V splitk_load(const V* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Returns true in the last workgroup to arrive at *counter (all threads).
__device__ __forceinline__ bool splitk_arrive(unsigned* counter, int S, int* s_last) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0)
    *s_last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              (unsigned)(S - 1);
  __syncthreads();
  return *s_last != 0;
}

__device__ __forceinline__ void splitk_reset(unsigned* counter) {
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sum of S partials p[0], p[stride], ... in split order, loads issued in
// batches of eight so that they overlap.
template <typename V>
__device__ __forceinline__ V splitk_sum(const V* p, int64_t stride, int S) {
  V s = 0;
  int k = 0;
  for (; k + 8 <= S; k += 8) {
    V v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = splitk_load(p + (k + u) * stride);
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; k < S; ++k) s += splitk_load(p + k * stride);
  return s;
}

}  // namespace sparkq

// ---------------------------------------------------------------------------
// host-side helpers shared by the launchers (defined in abi.cpp)
// ---------------------------------------------------------------------------
namespace sparkq {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
int device_check();
// CUs of the current device (256 when it cannot be queried)
int device_cus();
inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
// positive integer from the environment, or dflt
inline int64_t env_int(const char* name, int64_t dflt) {
  const char* e = getenv(name);
  const long long v = e ? atoll(e) : 0;
  return v > 0 ? (int64_t)v : dflt;
}
inline size_t round_up(size_t a, size_t b) { return (a + b - 1) / b * b; }

// Split-K workspaces start with a fixed block of tile counters: zero before
// the first call, and every call leaves them zero. The block has the same
// size for every shape so that one call's partials never overlap another
// call's counters; shapes with more tiles than it holds do not split K.
constexpr size_t kCounterBytes = 16384;
constexpr int64_t kMaxCounterTiles = (int64_t)(kCounterBytes / 4);
}  // namespace sparkq
