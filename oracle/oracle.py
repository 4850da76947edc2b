"""ctypes binding of the C oracle (oracle/sparkq_oracle.c) plus numpy helpers.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Every function restates a
reference algorithm; the C source cites the reference file:line for each.
16-bit floats travel as their uint16 bit patterns.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

__all__ = [
    "F32", "F16", "BF16",
    "bf16_bits", "bits_to_f32", "f16_bits", "round16",
    "randn", "randn16",
    "pack4", "unpack4", "w4_quantize", "w4_quantize_converter",
    "w4_dequantize", "w4a16_matmul", "w8a16_matmul", "unpack8", "w8_affine_matmul",
    "a8_quantize", "w8_quantize_channel", "w8_unpack_affine",
    "int8_matmul", "w8a8_epilogue",
    "kv_quantize_s8", "kv_quantize_affine_u8", "kv_dequantize_s8",
    "kv_dequantize_affine_u8", "sdpa_decode", "sdpa_prefill", "sdpa_prefill_rounded",
    "kv_quantize_affine", "kv_dequantize_affine", "sdpa_staged",
    "cpu_w4a16_gemv", "cpu_w8a8_linear", "cpu_int8kv_sdpa", "cpu_isa", "scalar_f32_to_bf16", "scalar_f32_to_f16",
    "scalar_f16_to_f32",
    "attention_gate16", "add16", "rms_norm16", "gelu16", "gelu_mul16", "rope16", "ffn_block", "qkv_rope",
]

F32, F16, BF16 = 0, 1, 2
_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_CPU = None


def _build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "libsparkq_oracle.so")
        if not os.path.exists(path):
            _build()
        _LIB = ctypes.CDLL(path)
        _declare(_LIB)
    return _LIB


def _cpu_flags():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("flags"):
                return set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return set()


def cpu_isa() -> str:
    """The instruction set of the CPU legs this host runs: 'avx512' when the
    CPU has AVX-512 F/BW/VL/VNNI, else 'avx2'."""
    return "avx512" if {"avx512f", "avx512bw", "avx512vl", "avx512_vnni"} <= _cpu_flags() else "avx2"


def _cpu():
    global _CPU
    if _CPU is None:
        name = "libsparkq_cpubase_avx512.so" if cpu_isa() == "avx512" else "libsparkq_cpubase.so"
        path = os.path.join(_HERE, name)
        if not os.path.exists(path):
            _build()
        _CPU = ctypes.CDLL(path)
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        for fn in ("sq_cpu_w4a16_gemv", "sq_cpu_w4a16_matmul"):
            getattr(_CPU, fn).restype = I
            getattr(_CPU, fn).argtypes = [P] * 4 + [I64, I64, I64, I, P, I]
        _CPU.sq_cpu_w8a8_linear.restype = I
        _CPU.sq_cpu_w8a8_linear.argtypes = [P, P, P, I64, I64, I64, P, I]
        _CPU.sq_cpu_int8kv_sdpa.restype = I
        _CPU.sq_cpu_int8kv_sdpa.argtypes = [P] * 5 + [I64] * 5 + [ctypes.c_float, P, I]
    return _CPU


def _declare(lib):
    P, I64, I, F, D, U64 = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                            ctypes.c_float, ctypes.c_double, ctypes.c_uint64)
    sig = {
        "sq_f32_to_bf16": (ctypes.c_uint16, [F]),
        "sq_f32_to_f16": (ctypes.c_uint16, [F]),
        "sq_f16_to_f32": (F, [ctypes.c_uint16]),
        "sq_randn": (None, [U64, U64, F, P, I64]),
        "sq_randn16": (None, [U64, U64, F, I, P, I64]),
        "sq_pack4": (None, [P, P, I64, I64]),
        "sq_unpack4": (None, [P, P, I64, I64]),
        "sq_w4_quantize": (None, [P, I64, I64, I, I, P, P, P]),
        "sq_w4_quantize_converter": (None, [P, I64, I64, I, P, P, P]),
        "sq_w4_dequantize": (None, [P, P, P, I64, I64, I, I, P]),
        "sq_w4a16_matmul": (None, [P, I, P, P, P, I64, I64, I64, I, P]),
        "sq_w8a16_matmul": (None, [P, I, P, P, I64, I64, I64, P]),
        "sq_a8_quantize": (None, [P, I64, I64, P, P]),
        "sq_w8_quantize_channel": (None, [P, I64, I64, P, P]),
        "sq_w8_unpack_affine": (None, [P, I64, I64, P]),
        "sq_int8_matmul": (I, [P, P, I64, I64, I64, P]),
        "sq_w8a8_epilogue": (None, [P, P, P, P, I64, I64, P]),
        "sq_kv_quantize_s8": (None, [P, I64, I64, P, P]),
        "sq_kv_quantize_affine_u8": (None, [P, I64, I64, I, I, P, P, P]),
        "sq_kv_dequantize_s8": (None, [P, P, I64, I64, P]),
        "sq_kv_dequantize_affine_u8": (None, [P, P, P, I64, I64, I, I, P]),
        "sq_sdpa_decode": (None, [P, P, P, I64, I64, I64, I64, I64, D, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------------------
# vectorised 16-bit conversions (same rules as the C scalars; pinned in tests)
# ---------------------------------------------------------------------------

def bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 bits, round-to-nearest-even (conversion.py:154-159)."""
    w = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (w & 0x7FFFFFFF) > 0x7F800000
    r = ((w.astype(np.uint64) + 0x7FFF + ((w >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((w >> 16) | 0x40).astype(np.uint16), r)


def f16_bits(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def bits_to_f32(h, dtype) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    if dtype == F16:
        return h.view(np.float16).astype(np.float32)
    return (h.astype(np.uint32) << 16).view(np.float32)


def round16(x, dtype) -> np.ndarray:
    return f16_bits(x) if dtype == F16 else bf16_bits(x)


def scalar_f32_to_bf16(f: float) -> int:
    return int(_lib().sq_f32_to_bf16(f))


def scalar_f32_to_f16(f: float) -> int:
    return int(_lib().sq_f32_to_f16(f))


def scalar_f16_to_f32(h: int) -> float:
    return float(_lib().sq_f16_to_f32(h))


# ---------------------------------------------------------------------------
# generator
# ---------------------------------------------------------------------------

def randn(seed: int, stream: int, n: int, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    _lib().sq_randn(seed, stream, std, _p(out), n)
    return out


def randn16(seed: int, stream: int, n: int, std: float = 1.0,
            dtype: int = BF16) -> np.ndarray:
    out = np.empty(n, np.uint16)
    _lib().sq_randn16(seed, stream, std, dtype, _p(out), n)
    return out


# ---------------------------------------------------------------------------
# W4 affine
# ---------------------------------------------------------------------------

def pack4(codes) -> np.ndarray:
    codes = _c(codes, np.uint8)
    n, k = codes.shape
    out = np.empty((n, k // 8), np.uint32)
    _lib().sq_pack4(_p(codes), _p(out), n, k)
    return out


def unpack4(words, k: int) -> np.ndarray:
    words = _c(words, np.uint32)
    n = words.shape[0]
    out = np.empty((n, k), np.uint8)
    _lib().sq_unpack4(_p(words), _p(out), n, k)
    return out


def w4_quantize(w, group_size: int, dtype: int = BF16):
    w = _c(w, np.float32)
    n, k = w.shape
    wq = np.empty((n, k // 8), np.uint32)
    s = np.empty((n, k // group_size), np.uint16)
    b = np.empty_like(s)
    _lib().sq_w4_quantize(_p(w), n, k, group_size, dtype, _p(wq), _p(s), _p(b))
    return wq, s, b


def w4_quantize_converter(w, group_size: int = 32):
    w = _c(w, np.float32)
    n, k = w.shape
    wq = np.empty((n, k // 8), np.uint32)
    s = np.empty((n, k // group_size), np.uint16)
    b = np.empty_like(s)
    _lib().sq_w4_quantize_converter(_p(w), n, k, group_size, _p(wq), _p(s), _p(b))
    return wq, s, b


def w4_dequantize(wq, s, b, group_size: int, dtype: int = BF16) -> np.ndarray:
    wq, s, b = _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    n = wq.shape[0]
    k = wq.shape[1] * 8
    out = np.empty((n, k), np.float32)
    _lib().sq_w4_dequantize(_p(wq), _p(s), _p(b), n, k, group_size, dtype, _p(out))
    return out


def w4a16_matmul(x16, wq, s, b, group_size: int, dtype: int = BF16) -> np.ndarray:
    x16 = _c(x16, np.uint16)
    wq, s, b = _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    m, k = x16.shape
    n = wq.shape[0]
    y = np.empty((m, n), np.float64)
    _lib().sq_w4a16_matmul(_p(x16), dtype, _p(wq), _p(s), _p(b), m, n, k,
                           group_size, _p(y))
    return y


def unpack8(words) -> np.ndarray:
    """MLX affine 8-bit layout: byte j of word w (little endian) is the
    unsigned code of k = 4w + j (spark_mlx_llm/conversion.py:429-433 packs
    32/bits codes per uint32 from the least significant bits up)."""
    words = np.ascontiguousarray(words, np.uint32)
    return words.view(np.uint8).reshape(*words.shape[:-1], words.shape[-1] * 4)


def w8_affine_matmul(x16, words, s, b, group_size: int, dtype: int = BF16,
                     scale_dtype: int | None = None) -> np.ndarray:
    """mx.quantized_matmul(x, w, scales, biases, transpose=True, group_size,
    bits=8) in float64: y[m,n] = sum_k x[m,k] * (u[n,k]*s[n,k/G] + b[n,k/G])
    (the affine dequantize of spark_mlx_llm/ops/linear.py:181-191, 299-324
    with 8-bit codes). x16 holds 16-bit patterns of dtype; s and b are 16-bit
    patterns of scale_dtype (default dtype) or float32 arrays."""
    x = bits_to_f32(x16, dtype).astype(np.float64)
    sd = dtype if scale_dtype is None else scale_dtype
    sf = (np.asarray(s, np.float64) if sd == F32 else bits_to_f32(s, sd).astype(np.float64))
    bf = (np.asarray(b, np.float64) if sd == F32 else bits_to_f32(b, sd).astype(np.float64))
    u = unpack8(words).astype(np.float64)
    w = u * np.repeat(sf, group_size, axis=1) + np.repeat(bf, group_size, axis=1)
    return x @ w.T


def w8a16_matmul(x16, w8, scales, dtype: int = BF16) -> np.ndarray:
    """scale[n] * sum_k x[m,k] * w[n,k] in float64 (w8a16_per_channel)."""
    x16, w8, sc = _c(x16, np.uint16), _c(w8, np.int8), _c(scales, np.float32)
    m, k = x16.shape
    n = w8.shape[0]
    y = np.empty((m, n), np.float64)
    _lib().sq_w8a16_matmul(_p(x16), dtype, _p(w8), _p(sc), m, n, k, _p(y))
    return y


# ---------------------------------------------------------------------------
# W8A8
# ---------------------------------------------------------------------------

def a8_quantize(x):
    x = _c(x, np.float32)
    m, k = x.shape
    q = np.empty((m, k), np.int8)
    sc = np.empty(m, np.float32)
    _lib().sq_a8_quantize(_p(x), m, k, _p(q), _p(sc))
    return q, sc


def w8_quantize_channel(w):
    w = _c(w, np.float32)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    sc = np.empty(n, np.float32)
    _lib().sq_w8_quantize_channel(_p(w), n, k, _p(q), _p(sc))
    return q, sc


def w8_unpack_affine(words) -> np.ndarray:
    words = _c(words, np.uint32)
    n, k4 = words.shape
    out = np.empty((n, k4 * 4), np.int8)
    _lib().sq_w8_unpack_affine(_p(words), n, k4 * 4, _p(out))
    return out


def int8_matmul(a, b) -> np.ndarray:
    a, b = _c(a, np.int8), _c(b, np.int8)
    m, k = a.shape
    n = b.shape[0]
    c = np.empty((m, n), np.int32)
    if _lib().sq_int8_matmul(_p(a), _p(b), m, n, k, _p(c)) != 0:
        raise OverflowError("int8 matmul sum leaves int32")
    return c


def w8a8_epilogue(acc, sa, sw, bias=None) -> np.ndarray:
    acc = _c(acc, np.int32)
    sa, sw = _c(sa, np.float32), _c(sw, np.float32)
    m, n = acc.shape
    y = np.empty((m, n), np.float32)
    bias_p = None if bias is None else _p(_c(bias, np.float32))
    if bias is not None:
        bias = _c(bias, np.float32)
        bias_p = _p(bias)
    _lib().sq_w8a8_epilogue(_p(acc), _p(sa), _p(sw), bias_p, m, n, _p(y))
    return y


# ---------------------------------------------------------------------------
# INT8 KV and decode attention
# ---------------------------------------------------------------------------

def kv_quantize_s8(x):
    x = _c(x, np.float32)
    d = x.shape[-1]
    r = x.size // d
    codes = np.empty(x.shape, np.int8)
    sc = np.empty(x.shape[:-1], np.uint16)
    _lib().sq_kv_quantize_s8(_p(x), r, d, _p(codes), _p(sc))
    return codes, sc


def kv_quantize_affine_u8(x, group_size: int, dtype: int = BF16):
    x = _c(x, np.float32)
    d = x.shape[-1]
    r = x.size // d
    packed = np.empty((*x.shape[:-1], d // 4), np.uint32)
    s = np.empty((*x.shape[:-1], d // group_size), np.uint16)
    b = np.empty_like(s)
    _lib().sq_kv_quantize_affine_u8(_p(x), r, d, group_size, dtype, _p(packed),
                                    _p(s), _p(b))
    return packed, s, b


def kv_dequantize_s8(codes, scales) -> np.ndarray:
    codes, scales = _c(codes, np.int8), _c(scales, np.uint16)
    d = codes.shape[-1]
    r = codes.size // d
    out = np.empty(codes.shape, np.float32)
    _lib().sq_kv_dequantize_s8(_p(codes), _p(scales), r, d, _p(out))
    return out


def kv_dequantize_affine_u8(packed, s, b, group_size: int,
                            dtype: int = BF16) -> np.ndarray:
    packed, s, b = _c(packed, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    d = packed.shape[-1] * 4
    r = packed.size // packed.shape[-1]
    out = np.empty((*packed.shape[:-1], d), np.float32)
    _lib().sq_kv_dequantize_affine_u8(_p(packed), _p(s), _p(b), r, d,
                                      group_size, dtype, _p(out))
    return out


def sdpa_decode(q, kdq, vdq, scale: float) -> np.ndarray:
    """q [B,Hq,D]; kdq/vdq [B,Hkv,N,D] dequantized -> out [B,Hq,D] fp64."""
    q, kdq, vdq = _c(q, np.float32), _c(kdq, np.float32), _c(vdq, np.float32)
    bsz, hq, d = q.shape
    hkv, n = kdq.shape[1], kdq.shape[2]
    out = np.empty((bsz, hq, d), np.float64)
    _lib().sq_sdpa_decode(_p(q), _p(kdq), _p(vdq), bsz, hq, hkv, n, d,
                          float(scale), _p(out))
    return out


def sdpa_prefill(q, kdq, vdq, scale: float, causal: bool) -> np.ndarray:
    """Staged attention in float64 over dequantized K/V, the reference's
    _fallback (X/spark_mlx_ext/int8_quantized_sdpa.py:122-153): q*scale,
    scores = q K^T, the bottom-right causal mask arange(N-L, N)[:, None] >=
    arange(N)[None, :] when causal, softmax, probs V. q [B,Hq,L,D]; kdq/vdq
    [B,Hkv,N,D] -> out [B,Hq,L,D]."""
    q = np.asarray(q, np.float64)
    kdq, vdq = np.asarray(kdq, np.float64), np.asarray(vdq, np.float64)
    bsz, hq, length, d = q.shape
    hkv, n = kdq.shape[1], kdq.shape[2]
    rep = hq // hkv
    k = np.repeat(kdq, rep, axis=1)
    v = np.repeat(vdq, rep, axis=1)
    scores = (q * scale) @ np.swapaxes(k, -1, -2)
    if causal:
        vis = np.arange(n - length, n)[:, None] >= np.arange(n)[None, :]
        scores = np.where(vis, scores, -np.inf)
    scores -= scores.max(axis=-1, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(axis=-1, keepdims=True)
    return p @ v


def kv_quantize_affine(x, group_size: int, bits: int, dtype: int = BF16):
    """The build's affine KV quantizer at 8, 4 or 2 bits (the min/max rule of
    sq_kv_quantize_affine_u8 with 2^bits - 1 bins): per group of G values,
    scale = T((max-min)/nbins), bias = T(min), code = clamp(rint((x - bias) /
    scale), 0, nbins) with the rounded scale and bias (0 when the scale is 0),
    32/bits codes per uint32 from the lowest bits up. numpy; x [..., D]."""
    x = np.asarray(x, np.float32)
    nb = (1 << bits) - 1
    d = x.shape[-1]
    g = x.reshape(*x.shape[:-1], d // group_size, group_size)
    lo, hi = g.min(-1), g.max(-1)
    s16 = round16(((hi - lo) / np.float32(nb)).astype(np.float32), dtype)
    b16 = round16(lo, dtype)
    sf = bits_to_f32(s16, dtype)[..., None]
    bf = bits_to_f32(b16, dtype)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(sf != 0, np.clip(np.rint((g - bf) / sf), 0, nb), 0).astype(np.uint32)
    q = q.reshape(*x.shape[:-1], d // (32 // bits), 32 // bits)
    words = np.zeros(q.shape[:-1], np.uint32)
    for j in range(32 // bits):
        words |= q[..., j] << np.uint32(bits * j)
    return words, s16, b16


def kv_dequantize_affine(packed, s16, b16, group_size: int, bits: int,
                         dtype: int = BF16) -> np.ndarray:
    """code * scale + bias, rounded once to float32, of an affine tuple of
    `bits` bits (code j of word w is dim (32/bits)*w + j)."""
    packed = np.asarray(packed, np.uint32)
    cpw = 32 // bits
    codes = ((packed[..., None] >> (np.arange(cpw, dtype=np.uint32) * np.uint32(bits)))
             & np.uint32((1 << bits) - 1)).reshape(*packed.shape[:-1], packed.shape[-1] * cpw)
    sf = np.repeat(bits_to_f32(s16, dtype).astype(np.float64), group_size, axis=-1)
    bf = np.repeat(bits_to_f32(b16, dtype).astype(np.float64), group_size, axis=-1)
    return (codes.astype(np.float64) * sf + bf).astype(np.float32)


_LOWEST = {BF16: -3.3895313892515355e38, F16: -65504.0, F32: -3.4028234663852886e38}


def sdpa_staged(q, kdq, vdq, scale: float, mask=None, dtype: int = BF16) -> np.ndarray:
    """The reference's staged quantized attention
    (X/spark_mlx_ext/int8_quantized_sdpa.py:122-153) in float64 over
    dequantized K [B,Hkv,N,D] and V [B,Hkv,N,Dv]: scores = (q*scale) K^T;
    mask "causal" is arange(N-L, N)[:, None] >= arange(N) (:141-142), a
    boolean array keeps True entries and replaces the others by the lowest
    finite value of the query dtype (mx.where with finfo.min, :147-150), a
    floating array is added; softmax; weights V. Returns [B,Hq,L,Dv]."""
    q = np.asarray(q, np.float64)
    kd, vd = np.asarray(kdq, np.float64), np.asarray(vdq, np.float64)
    bsz, hq, length, _ = q.shape
    hkv, n = kd.shape[1], kd.shape[2]
    k = np.repeat(kd, hq // hkv, axis=1)
    v = np.repeat(vd, hq // hkv, axis=1)
    scores = (q * scale) @ np.swapaxes(k, -1, -2)
    if isinstance(mask, str):
        mask = np.arange(n - length, n)[:, None] >= np.arange(n)[None, :]
    if mask is not None:
        mask = np.broadcast_to(np.asarray(mask), scores.shape)
        if mask.dtype == np.bool_:
            scores = np.where(mask, scores, _LOWEST[dtype])
        else:
            scores = scores + mask.astype(np.float64)
    scores = scores - scores.max(axis=-1, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(axis=-1, keepdims=True)
    return p @ v


def sdpa_prefill_rounded(q16, kdq, vdq, scale: float, causal: bool,
                         dtype: int = BF16) -> np.ndarray:
    """Multi-token attention with the rounding points of the reference's
    prefill kernel spark_affine_u8_sdpa_prefill
    (X/spark_mlx_ext/_int8_prefill_sources.py:60-146): K and V dequantize to
    the query dtype T (:73, :115), the softmax weights are rounded to T for
    the PV product while the normalizer sums the unrounded weights (:99-103),
    and scores, normalizer and output stay wide. Scores are
    (q . k) * scale * log2(e) in float64 with q exact (the reference also
    rounds q * scale to T, :38-39, a loss this oracle does not restate); a
    row's weights are 2^(s - c) with the integer c = ceil(max_row s), and
    since rounding to T commutes with powers of two, T(2^(s-c)) * 2^c does
    not depend on the integer chosen. q16 [B,Hq,L,D] 16-bit patterns of
    dtype; kdq/vdq [B,Hkv,N,D] dequantized values, rounded to T here. Returns
    float64 [B,Hq,L,D]."""
    q = bits_to_f32(q16, dtype).astype(np.float64)
    kt = bits_to_f32(round16(np.asarray(kdq, np.float32), dtype), dtype).astype(np.float64)
    vt = bits_to_f32(round16(np.asarray(vdq, np.float32), dtype), dtype).astype(np.float64)
    bsz, hq, length, d = q.shape
    hkv, n = kt.shape[1], kt.shape[2]
    rep = hq // hkv
    k = np.repeat(kt, rep, axis=1)
    v = np.repeat(vt, rep, axis=1)
    s2 = (q @ np.swapaxes(k, -1, -2)) * (scale * np.log2(np.e))
    if causal:
        vis = np.arange(n - length, n)[:, None] >= np.arange(n)[None, :]
        s2 = np.where(vis, s2, -np.inf)
    c = np.ceil(s2.max(axis=-1, keepdims=True))
    p = np.exp2(s2 - c)
    pt = bits_to_f32(round16(p.astype(np.float32), dtype), dtype).astype(np.float64)
    return (pt @ v) / p.sum(axis=-1, keepdims=True)


# ---------------------------------------------------------------------------
# Decoder-layer steps around the projections, in the 16-bit graph's rounding.
# MLX 0.32.4 (un-vendored; pinned by X/spark_mlx_ext/__init__.py:6-7) runs
# each operation of a bf16/f16 graph in fp32 and rounds its result to the
# array dtype; under mx.compile the intermediates keep their dtype. The
# functions below restate that arithmetic; the 16-bit inputs and outputs are
# bit patterns.
# ---------------------------------------------------------------------------

def add16(a16, b16, dtype: int = BF16) -> np.ndarray:
    """a + b of two 16-bit arrays: the fp32 sum rounded to the dtype
    (hidden = x + attention_output and hidden + mlp_output,
    spark_mlx_llm/ops/ffn.py:98,105)."""
    return round16(bits_to_f32(a16, dtype) + bits_to_f32(b16, dtype), dtype)


def rms_norm16(h16, w16, eps: float, dtype: int = BF16) -> np.ndarray:
    """mx.fast.rms_norm(h, w, eps) over the last axis (spark_mlx_llm/ops/
    ffn.py:99): inv = rsqrt(mean(h^2) + eps) (float64 here, rounded to fp32),
    out = w * T(h * inv), each product rounded to the dtype."""
    h = bits_to_f32(h16, dtype)
    w = bits_to_f32(w16, dtype)
    h64 = h.astype(np.float64)
    ms = (h64 * h64).mean(axis=-1, keepdims=True)
    inv = (1.0 / np.sqrt(ms + np.float64(np.float32(eps)))).astype(np.float32)
    n = bits_to_f32(round16(h * inv, dtype), dtype)
    return round16(w * n, dtype)


def gelu16(g16, dtype: int = BF16) -> np.ndarray:
    """mlx.nn.gelu on a 16-bit array, x * (1 + erf(x / sqrt(2))) / 2
    (spark_mlx_llm/ops/ffn.py:102): the Python constant sqrt(2) takes the
    array dtype; every operation rounds to the dtype; erf of the 16-bit value
    is rounded to fp32 before the dtype."""
    from scipy.special import erf

    def r(v):
        return bits_to_f32(round16(np.asarray(v, np.float32), dtype), dtype)

    g = bits_to_f32(g16, dtype)
    c = r(np.float32(np.sqrt(2.0)))
    t1 = r(g / c)
    e = r(erf(t1.astype(np.float64)).astype(np.float32))
    t3 = r(np.float32(1.0) + e)
    t4 = r(g * t3)
    return round16(t4 / np.float32(2.0), dtype)


def gelu_mul16(g16, u16, dtype: int = BF16) -> np.ndarray:
    """gelu(gate) * up, the product rounded to the dtype (ffn.py:102)."""
    return round16(bits_to_f32(gelu16(g16, dtype), dtype) * bits_to_f32(u16, dtype), dtype)


def rope16(x16, dims: int, base: float, offset: int, dtype: int = BF16,
           traditional: bool = False, scale: float = 1.0) -> np.ndarray:
    """mx.fast.rope on x [..., L, D] (X/src/spark_qkv_rope.cpp:99-100;
    spark_mlx_llm/ops/qkv.py:176-177). Token l sits at position offset + l.
    For pair i < dims/2: d = fp32(i) / fp32(dims/2), inv_freq = 2^(-d *
    log2(base)) (fp32 exponent, the power correctly rounded to fp32), theta =
    fp32(scale * position) * inv_freq in fp32; x1 = x[i], x2 = x[i + dims/2]
    (x[2i], x[2i+1] when traditional); out1 = x1 cos - x2 sin, out2 = x1 sin
    + x2 cos (float64 here), rounded to the dtype; dims past `dims` unchanged."""
    x = bits_to_f32(x16, dtype).astype(np.float64)
    length = x.shape[-2]
    half = dims // 2
    l2b = np.float32(np.log2(np.float64(np.float32(base))))
    d = np.arange(half, dtype=np.float32) / np.float32(half)
    inv = np.exp2((-d * l2b).astype(np.float64)).astype(np.float32)
    pos = (np.float32(scale) * (np.float32(offset) + np.arange(length, dtype=np.float32)))
    theta = (pos[:, None] * inv[None, :]).astype(np.float32).astype(np.float64)
    c, s = np.cos(theta), np.sin(theta)
    if traditional:
        i1, i2 = np.arange(0, dims, 2), np.arange(1, dims, 2)
    else:
        i1, i2 = np.arange(half), np.arange(half, dims)
    x1, x2 = x[..., i1], x[..., i2]
    out = np.array(bits_to_f32(x16, dtype), np.float64)
    out[..., i1] = x1 * c - x2 * s
    out[..., i2] = x1 * s + x2 * c
    res = round16(out.astype(np.float32), dtype)
    return np.where(np.arange(x.shape[-1]) < dims, res, np.asarray(x16, np.uint16))


def ffn_block(x16, attn16, norm16, eps, gate, up, down, group_size: int,
              dtype: int = BF16) -> dict:
    """compiled_ffn (spark_mlx_llm/ops/ffn.py:96-105) in stages: hidden =
    x + attn; normed = rms_norm(hidden); gate/up = the W4 projections of
    normed (float64, rounded to the dtype as mx.quantized_matmul returns
    them); act = gelu(gate) * up; mlp = down(act); out = hidden + mlp.
    gate, up, down are (packed weight, scales, biases)."""
    hidden = add16(x16, attn16, dtype)
    normed = rms_norm16(hidden, norm16, eps, dtype)
    g = w4a16_matmul(normed, *gate, group_size, dtype)
    u = w4a16_matmul(normed, *up, group_size, dtype)
    act = gelu_mul16(round16(g, dtype), round16(u, dtype), dtype)
    mlp = w4a16_matmul(act, *down, group_size, dtype)
    out = add16(hidden, round16(mlp, dtype), dtype)
    return {"hidden": hidden, "normed": normed, "gate": g, "up": u, "act": act, "mlp": mlp,
            "out": out}


def qkv_rope(x16, wq, s, b, group_size: int, n_heads: int, n_kv: int, head_dim: int,
             rope_dims: int, base: float, offset: int, dtype: int = BF16):
    """spark_qkv_rope (X/src/spark_qkv_rope.cpp:83-101) for one token x [K]:
    qkv = the W4 projection rounded to the dtype; split into q, k, v
    [heads, head_dim]; q and k through rope16 at position offset. Returns
    (q, k, v, qkv) with qkv the float64 projection."""
    qkv = w4a16_matmul(np.asarray(x16, np.uint16).reshape(1, -1), wq, s, b, group_size, dtype)[0]
    r = round16(qkv, dtype)
    qs, ks = n_heads * head_dim, n_kv * head_dim
    q = r[:qs].reshape(n_heads, 1, head_dim)
    k = r[qs:qs + ks].reshape(n_kv, 1, head_dim)
    v = r[qs + ks:].reshape(n_kv, head_dim)
    return (rope16(q, rope_dims, base, offset, dtype)[:, 0],
            rope16(k, rope_dims, base, offset, dtype)[:, 0], v, qkv)


# ---------------------------------------------------------------------------
# CPU baseline (bench.py only)
# ---------------------------------------------------------------------------

def cpu_w4a16_gemv(x16, wq, s, b, group_size: int, threads: int = 0):
    """Multi-threaded fp32 dequantize-then-matmul (any M); returns (y fp32,
    threads used)."""
    x16 = _c(x16, np.uint16)
    wq, s, b = _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    m, k = x16.shape
    n = wq.shape[0]
    y = np.empty((m, n), np.float32)
    used = _cpu().sq_cpu_w4a16_matmul(_p(x16), _p(wq), _p(s), _p(b), m, n, k,
                                      group_size, _p(y), threads)
    if used < 0:
        raise ValueError("unsupported CPU baseline shape")
    return y, used


def cpu_w8a8_linear(x16, wq, sw, threads: int = 0):
    """Multi-threaded per-token int8 quantization, int8 dots into int32 and
    the fp32 scale epilogue; x16 bf16 bits [M,K], wq int8 [N,K], sw fp32 [N].
    Returns (y fp32 [M,N], threads used)."""
    x16 = _c(x16, np.uint16)
    wq, sw = _c(wq, np.int8), _c(sw, np.float32)
    m, k = x16.shape
    n = wq.shape[0]
    y = np.empty((m, n), np.float32)
    used = _cpu().sq_cpu_w8a8_linear(_p(x16), _p(wq), _p(sw), m, n, k, _p(y), threads)
    if used < 0:
        raise ValueError("unsupported CPU baseline shape")
    return y, used


def cpu_int8kv_sdpa(q16, kc, ks16, vc, vs16, scale: float, threads: int = 0):
    """Multi-threaded INT8-KV GQA decode attention: q16 bf16 bits [B,Hq,D],
    kc/vc int8 [B,Hkv,N,D], ks16/vs16 fp16 bits [B,Hkv,N]. Returns (out fp32
    [B,Hq,D], threads used)."""
    q16 = _c(q16, np.uint16)
    kc, vc = _c(kc, np.int8), _c(vc, np.int8)
    ks16, vs16 = _c(ks16, np.uint16), _c(vs16, np.uint16)
    bq, hq, d = q16.shape
    _, hkv, n, _ = kc.shape
    out = np.empty((bq, hq, d), np.float32)
    used = _cpu().sq_cpu_int8kv_sdpa(_p(q16), _p(kc), _p(ks16), _p(vc), _p(vs16), bq, hq, hkv, n,
                                     d, scale, _p(out), threads)
    if used < 0:
        raise ValueError("unsupported CPU baseline shape")
    return out, used


def attention_gate16(x16, attn16, gw16, dtype: int = BF16):
    """The head-wise gate of spark_mlx_llm/ops/attention_output.py:69-95 in
    the 16-bit graph's roundings: gate = T(sigmoid(T(x . g_proj[h]))) with the
    dot and the sigmoid exact (float64) before each rounding, and
    out[b,l,h*D+d] = T(attn[b,h,l,d] * gate[b,l,h]). x16 [B,L,hidden],
    attn16 [B,H,L,D], gw16 [H,hidden] as 16-bit patterns; returns the gate
    [B,L,H] and out [B,L,H*D] as 16-bit patterns."""
    x = bits_to_f32(x16, dtype).astype(np.float64)
    a = bits_to_f32(attn16, dtype).astype(np.float64)
    w = bits_to_f32(gw16, dtype).astype(np.float64)
    dot = bits_to_f32(round16((x @ w.T).astype(np.float32), dtype), dtype).astype(np.float64)
    gate = round16((1.0 / (1.0 + np.exp(-dot))).astype(np.float32), dtype)
    g = bits_to_f32(gate, dtype).astype(np.float64)
    b, h, length, d = a.shape
    prod_ = np.swapaxes(a, 1, 2) * g[..., None]
    out = round16(prod_.astype(np.float32), dtype).reshape(b, length, h * d)
    return gate, out
