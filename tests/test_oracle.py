"""Pins the CPU oracle (oracle/sparkq_oracle.c) with checks that do not retype
its formulas: library conversions (torch, numpy), closed forms, invariants,
extremes and brute force on tiny inputs. The reference ships no golden
vectors or tests for this path (its tests/ directory is excluded from the
repository), so these checks are the oracle's anchor.
"""

import math
import os

import numpy as np
import pytest
import torch

import oracle as o
from helpers import rel_l2, ulp_distance16


# ---------------------------------------------------------------------------
# 16-bit conversions
# ---------------------------------------------------------------------------

def _specials():
    v = [0.0, -0.0, 1.0, -1.0, 1.00390625, 1.01171875, 3.0e38, -3.0e38, 1e-40, -1e-40,
         65504.0, 65519.0, 65520.0, 6.1e-5, 5.96e-8, 2.98e-8, 1e-8, float("inf"),
         float("-inf"), 0.1, 1.0 / 3.0]
    rng = np.random.default_rng(0)
    v += list(rng.standard_normal(2000).astype(np.float32) * 10 ** rng.uniform(-8, 8, 2000))
    # exact bf16 ties: halfway between two bf16 values
    ties = (np.arange(1, 200, dtype=np.uint32) << 16) | 0x8000
    v += list(ties.view(np.float32))
    # exact f16 ties
    h = np.arange(0x3C00, 0x3D00, dtype=np.uint16).view(np.float16).astype(np.float32)
    v += list((h[:-1] + (h[1:] - h[:-1]) / 2).astype(np.float32))
    return np.array(v, dtype=np.float32)


def test_bf16_rounding_matches_torch():
    x = _specials()
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(o.bf16_bits(x), ref)
    for f in x[:300]:
        assert o.scalar_f32_to_bf16(float(f)) == int(o.bf16_bits(np.float32(f)).reshape(-1)[0])


def test_f16_rounding_matches_numpy():
    x = _specials()
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    ours = np.array([o.scalar_f32_to_f16(float(f)) for f in x], dtype=np.uint16)
    assert np.array_equal(ours, ref)
    back = np.array([o.scalar_f16_to_f32(int(h)) for h in ref[np.isfinite(x)]], np.float32)
    assert np.array_equal(back, ref[np.isfinite(x)].view(np.float16).astype(np.float32))


def test_generator_deterministic_and_normal():
    a = o.randn(0, 7, 200001)
    assert np.array_equal(a, o.randn(0, 7, 200001))
    assert not np.array_equal(a[:100], o.randn(0, 8, 100))
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    assert np.array_equal(o.randn16(0, 7, 1001, 0.02, o.BF16), o.bf16_bits(o.randn(0, 7, 1001, 0.02)))
    assert np.array_equal(o.randn16(0, 7, 999, 1.0, o.F16), o.f16_bits(o.randn(0, 7, 999)))


# ---------------------------------------------------------------------------
# W4 layout, quantizers, dequantization, matmul
# ---------------------------------------------------------------------------

def test_pack4_layout_known_answer():
    # code k of a word sits at bits 4*(k%8): codes 1..8 -> 0x87654321
    codes = np.array([[1, 2, 3, 4, 5, 6, 7, 8, 15, 0, 0, 0, 0, 0, 0, 9]], np.uint8)
    w = o.pack4(codes)
    assert w.tolist() == [[0x87654321, 0x9000000F]]
    # little-endian byte view: byte k/2, even k in the low nibble
    b = w.view(np.uint8)[0]
    assert b[0] == 0x21 and b[4] == 0x0F and b[7] == 0x90


def test_pack4_round_trip():
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 16, (7, 64), dtype=np.uint8)
    assert np.array_equal(o.unpack4(o.pack4(codes), 64), codes)


def _w(shape, seed=0, std=0.02):
    return o.bits_to_f32(o.randn16(seed, 11, int(np.prod(shape)), std, o.BF16), o.BF16).reshape(shape)


@pytest.mark.parametrize("g", [32, 64, 128])
@pytest.mark.parametrize("dt", [o.BF16, o.F16])
def test_w4_quantize_properties(g, dt):
    w = _w((16, 256), seed=g)
    if dt == o.F16:
        w = o.bits_to_f32(o.f16_bits(w), o.F16).reshape(w.shape)
    wq, s16, b16 = o.w4_quantize(w, g, dt)
    codes = o.unpack4(wq, 256).reshape(16, -1, g).astype(np.int64)
    s = o.bits_to_f32(s16, dt)[..., None]
    b = o.bits_to_f32(b16, dt)[..., None]
    grp = w.reshape(16, -1, g)
    # scale and bias are the stated statistics rounded to the storage dtype
    assert np.array_equal(s16, o.round16((grp.max(-1) - grp.min(-1)) / np.float32(15), dt))
    assert np.array_equal(b16, o.round16(grp.min(-1), dt))
    assert codes.min() >= 0 and codes.max() <= 15
    # codes are monotone in w within a group
    order = np.argsort(grp, axis=-1, kind="stable")
    assert np.all(np.diff(np.take_along_axis(codes, order, -1), axis=-1) >= 0)
    # reconstruction error is at most half a step (plus the bias rounding)
    err = np.abs(codes * s + b - grp)
    assert np.all(err <= s / 2 + np.abs(b - grp.min(-1, keepdims=True)) + 1e-7)
    # the group minimum is code 0
    assert np.all(np.take_along_axis(codes, grp.argmin(-1)[..., None], -1) == 0)


def test_w4_quantize_constant_group():
    w = np.full((1, 64), 0.25, np.float32)
    wq, s, b = o.w4_quantize(w, 64, o.BF16)
    assert wq.max() == 0 and s[0, 0] == 0 and o.bits_to_f32(b, o.BF16)[0, 0] == 0.25


def test_converter_quantizer_properties():
    w = _w((8, 128), seed=3, std=0.05)
    w[0, :32] = 0.0
    wq, s16, b16 = o.w4_quantize_converter(w, 32)
    codes = o.unpack4(wq, 128).reshape(8, 4, 32).astype(np.float64)
    s = o.bits_to_f32(s16, o.BF16)[..., None].astype(np.float64)
    b = o.bits_to_f32(b16, o.BF16)[..., None].astype(np.float64)
    grp = w.reshape(8, 4, 32).astype(np.float64)
    # an all-zero group has scale 1, zero point 0 and reconstructs to 0
    assert o.bits_to_f32(s16, o.BF16)[0, 0] == 1.0 and np.all(codes[0, 0] == 0)
    assert np.all(codes[0, 0] * s[0, 0] + b[0, 0] == 0)
    # zero lies in the representable range and values reconstruct to <= s/2
    # (+ the bf16 rounding of the scale and of the offset -zero*s)
    err = np.abs(codes * s + b - grp)
    slack = s * (2.0 ** -8) * 16 + np.abs(b) * 2.0 ** -8
    assert np.all(err <= s / 2 + slack)


@pytest.mark.parametrize("dt", [o.BF16, o.F16])
def test_w4_dequantize_is_single_rounding(dt):
    rng = np.random.default_rng(5)
    n, k, g = 6, 128, 32
    codes = rng.integers(0, 16, (n, k), dtype=np.uint8)
    codes[0, :16] = np.arange(16)
    wq = o.pack4(codes)
    sv = (rng.standard_normal((n, k // g)) * 10 ** rng.uniform(-6, 3, (n, k // g))).astype(np.float32)
    bv = (rng.standard_normal((n, k // g)) * 10 ** rng.uniform(-6, 3, (n, k // g))).astype(np.float32)
    sv[1, 0], bv[1, 0], sv[1, 1], bv[1, 1] = 0.0, -0.0, -0.0, 0.0
    s16, b16 = o.round16(sv, dt), o.round16(bv, dt)
    if dt == o.BF16:
        s16[2, 0], b16[2, 0] = 0x0001, 0x8001  # subnormal bf16
        # 2*2^127 overflows as a product, but 2^128 - 2^125 is finite: the
        # dequantization rounds the exact q*s+b once
        s16[3, 0], b16[3, 0] = 0x7F00, 0xFE00
        codes[3, :8] = 2
        wq = o.pack4(codes)
    out = o.w4_dequantize(wq, s16, b16, g, dt)
    s = np.repeat(o.bits_to_f32(s16, dt).astype(np.float64), g, axis=1)
    b = np.repeat(o.bits_to_f32(b16, dt).astype(np.float64), g, axis=1)
    exact = codes.astype(np.float64) * s + b  # exact product, one rounding below
    with np.errstate(over="ignore"):
        assert np.array_equal(out, exact.astype(np.float32))
    if dt == o.BF16:
        assert np.isfinite(out[3, :8]).all() and out[3, 0] == np.float32(2.0 ** 128 - 2.0 ** 125)


def test_w4a16_matmul_against_numpy_and_special_cases():
    m, n, k, g = 3, 5, 128, 64
    w = _w((n, k), seed=9)
    wq, s, b = o.w4_quantize(w, g)
    deq = o.w4_dequantize(wq, s, b, g).astype(np.float64)
    x16 = o.randn16(0, 21, m * k).reshape(m, k)
    xf = o.bits_to_f32(x16, o.BF16).astype(np.float64)
    y = o.w4a16_matmul(x16, wq, s, b, g)
    assert np.allclose(y, xf @ deq.T, rtol=1e-12, atol=1e-12)
    # one-hot rows select dequantized weight columns exactly
    onehot = np.zeros((2, k), np.float32)
    onehot[0, 7] = 1.0
    onehot[1, 100] = 1.0
    yh = o.w4a16_matmul(o.bf16_bits(onehot), wq, s, b, g)
    assert np.array_equal(yh[0], deq[:, 7]) and np.array_equal(yh[1], deq[:, 100])
    # zero scales: y = b * sum(x) per group
    s0 = np.zeros_like(s)
    y0 = o.w4a16_matmul(x16, wq, s0, b, g)
    bf = o.bits_to_f32(b, o.BF16).astype(np.float64)
    xs = xf.reshape(m, k // g, g).sum(-1)
    assert np.allclose(y0, xs @ bf.T, rtol=1e-12)


# ---------------------------------------------------------------------------
# W8A8
# ---------------------------------------------------------------------------

def test_a8_quantize_known_answers():
    x = np.zeros((4, 32), np.float32)
    x[1] = 1.0                                   # amax 1 -> scale 1/127 -> 127
    x[2, 0], x[2, 1], x[2, 2] = 2.54, -2.54, 0.01  # exact +-amax -> +-127
    x[3, :3] = [2.5, 1.5, -127.0]                # ties at .5 go to even
    q, sc = o.a8_quantize(x)
    assert sc[0] == 1.0 and np.all(q[0] == 0)    # all-zero row: scale 1
    assert sc[1] == np.float32(1.0) / np.float32(127) and np.all(q[1] == 127)
    assert q[2, 0] == 127 and q[2, 1] == -127 and q[2, 2] == 0
    assert sc[3] == np.float32(127.0) / np.float32(127.0)
    assert q[3, 0] == 2 and q[3, 1] == 2 and q[3, 2] == -127


def test_a8_quantize_properties():
    x = o.randn(3, 1, 4 * 2560).reshape(4, 2560)
    q, sc = o.a8_quantize(x)
    assert np.all(np.abs(q) <= 127)
    assert np.all(np.abs(q).max(1) == 127)
    err = np.abs(q.astype(np.float64) * sc[:, None] - x)
    assert np.all(err <= sc[:, None] * (0.5 + 1e-6))


def test_int8_matmul_exact_and_extremes():
    rng = np.random.default_rng(2)
    a = rng.integers(-128, 128, (5, 96), dtype=np.int8)
    b = rng.integers(-128, 128, (7, 96), dtype=np.int8)
    assert np.array_equal(o.int8_matmul(a, b), a.astype(np.int64) @ b.astype(np.int64).T)
    # K = 131040 at (-128)*(-128) is the largest sum that still fits int32
    k = 131040
    big = np.full((1, k), -128, np.int8)
    c = o.int8_matmul(big, big)
    assert int(c[0, 0]) == 16384 * k
    with pytest.raises(OverflowError):
        o.int8_matmul(np.full((1, k + 32), -128, np.int8), np.full((1, k + 32), -128, np.int8))


def test_w8a8_epilogue_is_fused():
    rng = np.random.default_rng(4)
    acc = rng.integers(-2 ** 30, 2 ** 30, (3, 9)).astype(np.int32)
    sa = rng.random(3).astype(np.float32) * 0.02
    sw = rng.random(9).astype(np.float32) * 0.01
    bias = rng.standard_normal(9).astype(np.float32)
    y = o.w8a8_epilogue(acc, sa, sw, bias)
    t = (acc.astype(np.float32) * sa[:, None]).astype(np.float64)
    exact = t * sw.astype(np.float64)[None] + bias[None]  # t*sw exact in fp64
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(y - exact) <= 0.5 * ulp + 1e-30)
    # README known answer adapted to W8A8: ones(32) x ones(4,32), scale 1 -> 32
    q, sc = o.a8_quantize(np.ones((1, 32), np.float32))
    acc1 = o.int8_matmul(q, np.ones((4, 32), np.int8))
    y1 = o.w8a8_epilogue(acc1, sc, np.ones(4, np.float32))
    assert np.all(o.bf16_bits(y1) == o.bf16_bits(np.float32(32.0)))


def test_w8_unpack_affine():
    codes = np.array([[0, 1, 127, 128, 129, 255, 200, 55]], np.uint8)  # unsigned storage
    words = codes.view(np.uint32).reshape(1, 2)
    assert o.w8_unpack_affine(words).tolist() == [[-128, -127, -1, 0, 1, 127, 72, -73]]


# ---------------------------------------------------------------------------
# INT8 KV and decode attention
# ---------------------------------------------------------------------------

def test_kv_quantize_s8_properties():
    x = o.randn(5, 2, 64 * 128).reshape(64, 128)
    x[3] = 0.0
    codes, sc = o.kv_quantize_s8(x)
    s = sc.view(np.float16).astype(np.float32)
    assert s[3] == 1.0 and np.all(codes[3] == 0)
    live = np.arange(64) != 3
    assert np.array_equal(sc[live], (np.abs(x[live]).max(1) / np.float32(127)).astype(np.float16).view(np.uint16))
    assert np.all(np.abs(codes) <= 127)
    err = np.abs(codes[live] * s[live, None] - x[live])
    assert np.all(err <= s[live, None] * 0.5 + np.abs(x[live]).max(1, keepdims=True) * 2 ** -10)


def test_kv_affine_u8_round_trip():
    x = o.randn(6, 2, 16 * 128).reshape(16, 128)
    packed, s, b = o.kv_quantize_affine_u8(x, 32, o.BF16)
    deq = o.kv_dequantize_affine_u8(packed, s, b, 32, o.BF16)
    sf = np.repeat(o.bits_to_f32(s, o.BF16), 32, axis=1)
    assert np.all(np.abs(deq - x) <= sf * 0.5 + np.abs(x) * 2 ** -7 + 1e-6)


def _sdpa_np(q, k, v, scale):
    rep = q.shape[1] // k.shape[1]
    k = np.repeat(k.astype(np.float64), rep, axis=1)
    v = np.repeat(v.astype(np.float64), rep, axis=1)
    s = np.einsum("bhd,bhnd->bhn", q.astype(np.float64), k) * scale
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhn,bhnd->bhd", p, v)


def test_sdpa_decode_against_numpy_and_invariants():
    b, hq, hkv, n, d = 2, 8, 2, 37, 64
    q = o.randn(1, 1, b * hq * d).reshape(b, hq, d)
    k = o.randn(1, 2, b * hkv * n * d).reshape(b, hkv, n, d)
    v = o.randn(1, 3, b * hkv * n * d).reshape(b, hkv, n, d)
    scale = 1 / math.sqrt(d)
    out = o.sdpa_decode(q, k, v, scale)
    assert np.allclose(out, _sdpa_np(q, k, v, scale), rtol=1e-12, atol=1e-12)
    # a single token returns its value row
    o1 = o.sdpa_decode(q, k[:, :, :1].copy(), v[:, :, :1].copy(), scale)
    assert np.allclose(o1, np.repeat(v[:, :, 0], hq // hkv, axis=1), atol=1e-7)
    # identical keys average the values
    kk = np.repeat(k[:, :, :1], n, axis=2)
    om = o.sdpa_decode(q, kk, v, scale)
    assert np.allclose(om, np.repeat(v.mean(2), hq // hkv, axis=1), atol=1e-6)
    # token order does not matter
    perm = np.random.default_rng(0).permutation(n)
    op = o.sdpa_decode(q, k[:, :, perm].copy(), v[:, :, perm].copy(), scale)
    assert np.allclose(op, out, atol=1e-12)


@pytest.mark.parametrize("m,n,k", [(1, 96, 256), (2, 96, 256), (9, 37, 512), (37, 40, 1536)])
def test_cpu_baseline_matches_oracle(m, n, k):
    g = 64
    w = _w((n, k), seed=12)
    wq, s, b = o.w4_quantize(w, g)
    x16 = o.randn16(0, 13, m * k).reshape(m, k)
    y, used = o.cpu_w4a16_gemv(x16, wq, s, b, g)
    assert used >= 1
    ref = o.w4a16_matmul(x16, wq, s, b, g)
    assert np.abs(y - ref).max() < 1e-4 * max(1.0, np.abs(ref).max())


def test_cpu_baseline_w8a8_is_bit_exact():
    """The CPU W8A8 leg: per-token quantizer, int32 dots and the fp32 scale
    product give the oracle's bits."""
    m, n, k = 5, 70, 640
    xf = o.bits_to_f32(o.randn16(0, 31, m * k), o.BF16).reshape(m, k)
    xf[3] = 0.0  # an all-zero token
    wq, sw = o.w8_quantize_channel(o.randn(0, 32, n * k, 0.02).reshape(n, k))
    y, used = o.cpu_w8a8_linear(o.bf16_bits(xf), wq, sw)
    qa, sa = o.a8_quantize(xf)
    ref = o.w8a8_epilogue(o.int8_matmul(qa, wq), sa, sw)
    assert used >= 1
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("b,n", [(1, 1), (1, 300), (2, 77)])
def test_cpu_baseline_int8kv_sdpa_matches_oracle(b, n):
    hq, hkv, d = 8, 2, 128
    q16 = o.randn16(0, 40, b * hq * d).reshape(b, hq, d)
    kc, ks = o.kv_quantize_s8(o.randn(0, 41, b * hkv * n * d).reshape(b, hkv, n, d))
    vc, vs = o.kv_quantize_s8(o.randn(0, 42, b * hkv * n * d).reshape(b, hkv, n, d))
    out, used = o.cpu_int8kv_sdpa(q16, kc, ks, vc, vs, 1 / math.sqrt(d))
    ref = o.sdpa_decode(o.bits_to_f32(q16, o.BF16), o.kv_dequantize_s8(kc, ks),
                        o.kv_dequantize_s8(vc, vs), 1 / math.sqrt(d))
    assert used >= 1
    assert np.abs(out - ref).max() < 1e-5


# ---------------------------------------------------------------------------
# golden vectors written by the reference converter (tests/golden/)
# ---------------------------------------------------------------------------
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "converter_vectors.npz")


def _golden():
    return np.load(GOLDEN)  # plain arrays, no pickle


def test_converter_w4_quantizer_matches_reference_vectors():
    """The oracle's G32 converter quantizer against `_rows` (scheme
    bf16-int4, conversion.py:551-608) on 34 rows of edge cases: codes,
    scales and biases bit for bit."""
    g = _golden()
    wq, s, b = o.w4_quantize_converter(o.bits_to_f32(g["w16"], o.BF16), 32)
    assert np.array_equal(wq, g["w4_words"])
    assert np.array_equal(s, g["w4_scales"])
    assert np.array_equal(b, g["w4_biases"])


def test_converter_w8_format_unpacks_to_symmetric_codes():
    """The converter's W8 rows (scheme bf16-int8) unpack, through the oracle
    and through the operator layer's unpack (ops/linear.py:299-324), to
    rint(w / scale) clipped to +-127 with one repeated per-row scale and
    biases -128 * scale."""
    from sparkq.ops.linear import unpack_affine_w8

    g = _golden()
    w = o.bits_to_f32(g["w16"], o.BF16).astype(np.float64)
    sc = o.bits_to_f32(g["w8_scales"], o.BF16)
    assert np.all(sc == sc[:, :1])
    expect = np.clip(np.rint(w / sc[:, :1].astype(np.float64)), -127, 127).astype(np.int8)
    assert np.array_equal(o.w8_unpack_affine(g["w8_words"]), expect)
    assert np.array_equal(g["w8_biases"], o.bf16_bits(-128.0 * sc))
    w8, ch = unpack_affine_w8(torch.from_numpy(g["w8_words"].view(np.int32)),
                              torch.from_numpy(g["w8_scales"].view(np.int16)).view(torch.bfloat16),
                              torch.from_numpy(g["w8_biases"].view(np.int16)).view(torch.bfloat16),
                              group_size=32)
    assert np.array_equal(w8.numpy(), expect)
    assert np.array_equal(ch.numpy(), sc[:, 0])


def test_bf16_rounding_matches_reference_vectors():
    g = _golden()
    assert np.array_equal(o.bf16_bits(g["bf16_in"]), g["bf16_out"])


def test_w8a16_oracle_matches_numpy():
    """sq_w8a16_matmul against a float64 numpy matmul (random and extreme
    codes), and one-hot activations picking w[:, k] * scale."""
    rng = np.random.default_rng(8)
    m, n, k = 3, 17, 96
    x = o.randn16(8, 1, m * k).reshape(m, k)
    w8 = rng.integers(-128, 128, (n, k), dtype=np.int8)
    w8[0] = -128
    sc = rng.random(n).astype(np.float32)
    y = o.w8a16_matmul(x, w8, sc)
    ref = (o.bits_to_f32(x, o.BF16).astype(np.float64) @ w8.T.astype(np.float64)) * sc
    assert np.allclose(y, ref, rtol=1e-14, atol=0)
    e = np.zeros((1, k), np.float32)
    e[0, 5] = 1.0
    assert np.array_equal(o.w8a16_matmul(o.bf16_bits(e), w8, sc)[0],
                          w8[:, 5].astype(np.float64) * sc.astype(np.float64))


# ---------------------------------------------------------------------------
# decoder-layer steps: residual add, RMSNorm, GELU, RoPE, FFN block, QKV+RoPE
# ---------------------------------------------------------------------------

def _b(vals):
    return o.round16(np.asarray(vals, np.float32), o.BF16)


def test_add16_rounding_and_identities():
    x = o.randn16(1, 70, 4096)
    y = o.randn16(1, 71, 4096)
    zero = np.zeros_like(x)
    assert np.array_equal(o.add16(x, zero), x & 0x7FFF | (x & 0x8000) * (x != 0x8000))
    assert np.array_equal(o.add16(x, y), o.add16(y, x))
    assert not o.bits_to_f32(o.add16(x, x ^ 0x8000), o.BF16).any()
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: even wins; 1 + 3*2^-9 rounds up
    one = _b([1.0, 1.0])
    assert o.bits_to_f32(o.add16(one, _b([2.0 ** -8, 3 * 2.0 ** -9])), o.BF16).tolist() == \
        [1.0, 1.0078125]
    # fp16: 1 + 2^-11 ties to 1, 1 + 3*2^-12 rounds up to 1 + 2^-10
    one16 = o.round16(np.ones(2, np.float32), o.F16)
    t = o.round16(np.array([2.0 ** -11, 3 * 2.0 ** -12], np.float32), o.F16)
    assert o.bits_to_f32(o.add16(one16, t, o.F16), o.F16).tolist() == [1.0, 1.0 + 2.0 ** -10]


def test_rms_norm16_known_answer_and_invariants():
    # h = [3, 4]: mean(h^2) = 12.5, 3/sqrt(12.5) = 0.84853 -> 0.84765625,
    # 4/sqrt(12.5) = 1.13137 -> 1.1328125 (bf16 nearest)
    out = o.rms_norm16(_b([[3.0, 4.0]]), _b([1.0, 1.0]), 0.0)
    assert o.bits_to_f32(out, o.BF16).tolist() == [[0.84765625, 1.1328125]]
    # a weight of 2 doubles exactly; the weight multiplies per feature
    h = o.randn16(2, 72, 4 * 2560).reshape(4, 2560)
    one = _b(np.ones(2560))
    n1 = o.bits_to_f32(o.rms_norm16(h, one, 1e-6), o.BF16)
    n2 = o.bits_to_f32(o.rms_norm16(h, _b(np.full(2560, 2.0)), 1e-6), o.BF16)
    assert np.array_equal(n2, 2 * n1)
    # scale invariance with eps = 0: scaling h by 2 is exact, so is the norm
    h2 = o.round16(2 * o.bits_to_f32(h, o.BF16), o.BF16)
    assert np.array_equal(o.rms_norm16(h2, one, 0.0), o.rms_norm16(h, one, 0.0))
    # unit mean square within the rounding of each element
    assert np.allclose((n1.astype(np.float64) ** 2).mean(axis=-1), 1.0, atol=5e-3)
    # eps enters under the root: a zero row stays zero, a tiny row is damped
    z = o.rms_norm16(_b(np.zeros((1, 64))), _b(np.ones(64)), 1e-6)
    assert not o.bits_to_f32(z, o.BF16).any()
    small = o.rms_norm16(_b(np.full((1, 64), 1e-3)), _b(np.ones(64)), 1e-6)
    assert np.allclose(o.bits_to_f32(small, o.BF16), 1e-3 / np.sqrt(1e-6 + 1e-6), rtol=8e-3)


def test_gelu16_against_the_erf_definition():
    from scipy.special import erf

    x = np.linspace(-6, 6, 4001, dtype=np.float32)
    for dt, eps in ((o.BF16, 2.0 ** -8), (o.F16, 2.0 ** -11)):
        g = o.round16(x, dt)
        xv = o.bits_to_f32(g, dt).astype(np.float64)
        exact = 0.5 * xv * (1.0 + erf(xv / np.sqrt(2.0)))
        got = o.bits_to_f32(o.gelu16(g, dt), dt)
        # the 16-bit 1 + erf(.) loses up to one unit of 1 to cancellation, so
        # the error is bounded by |x| units of the format (and the result's
        # own rounding), not by the result's units
        assert np.all(np.abs(got - exact) <= 1.5 * eps * np.abs(xv) + eps * np.abs(exact) + 1e-30)
    # hand-derived at the rounding points, x = -3 in bf16: x / 1.4140625 =
    # -2.1215 -> -2.125; erf(-2.125) = -0.99730 -> -0.99609375; 1 + that =
    # 2^-8; times x = -0.01171875; halved = -0.005859375 (one fp32 rounding at
    # the end would give -0.00405)
    assert o.bits_to_f32(o.gelu16(_b([-3.0])), o.BF16).tolist() == [-0.005859375]
    assert o.bits_to_f32(o.gelu16(_b([0.0, 8.0, 100.0])), o.BF16).tolist() == [0.0, 8.0, 100.0]
    assert o.bits_to_f32(o.gelu16(_b([-8.0, -100.0])), o.BF16).tolist() == [0.0, 0.0]
    gm = o.gelu_mul16(_b([8.0, 8.0]), _b([0.5, -3.0]))
    assert o.bits_to_f32(gm, o.BF16).tolist() == [4.0, -24.0]


def test_rope16_geometry():
    d, length = 128, 6
    x = o.randn16(3, 73, 2 * 4 * length * d).reshape(2, 4, length, d)
    y = o.rope16(x, d, 10000.0, 0)
    assert np.array_equal(y[:, :, 0], x[:, :, 0])           # position 0 is the identity
    # one-hot inputs land on cos/sin of the textbook angle p * base^(-2i/d)
    for i, p in ((0, 1), (5, 7), (63, 4095), (17, 30000)):
        e = np.zeros((1, 1, d), np.float32)
        e[0, 0, i] = 1.0
        r = o.bits_to_f32(o.rope16(o.round16(e, o.BF16), d, 10000.0, p), o.BF16)[0, 0]
        th = p * 10000.0 ** (-2 * i / d)
        assert abs(r[i] - np.cos(th)) <= 2 ** -8 and abs(r[i + d // 2] - np.sin(th)) <= 2 ** -8
        assert np.count_nonzero(r) <= 2
    # each pair keeps its length
    xf = o.bits_to_f32(x, o.BF16).astype(np.float64)
    yf = o.bits_to_f32(o.rope16(x, d, 10000.0, 123), o.BF16).astype(np.float64)
    n0 = xf[..., :64] ** 2 + xf[..., 64:] ** 2
    n1 = yf[..., :64] ** 2 + yf[..., 64:] ** 2
    assert np.allclose(n1, n0, rtol=2e-2, atol=1e-3)
    # partial rotation: the dims past rope_dims pass through bit for bit
    yp = o.rope16(x, 32, 10000.0, 5)
    assert np.array_equal(yp[..., 32:], x[..., 32:])
    # traditional pairs (2i, 2i+1) are the non-traditional pairs after an
    # interleaving permutation of the features
    perm = np.concatenate([np.arange(0, d, 2), np.arange(1, d, 2)])
    yt = o.rope16(x, d, 10000.0, 9, traditional=True)
    yn = o.rope16(x[..., perm], d, 10000.0, 9)
    assert np.array_equal(yt[..., perm], yn)
    # consecutive tokens: token l at offset a equals token 0 at offset a + l
    ya = o.rope16(x, d, 500000.0, 40)
    yb = o.rope16(x[:, :, 3:4], d, 500000.0, 43)
    assert np.array_equal(ya[:, :, 3:4], yb)


def test_ffn_block_against_textbook_float64():
    """The staged 16-bit FFN against the same formulas in float64 without
    intermediate rounding: close (bf16 noise), and the known-wrong orders
    (residual on the normed rows, GELU on up) are far."""
    from scipy.special import erf

    k, inter, g = 256, 512, 64
    x = o.randn16(4, 74, 2 * k).reshape(2, k)
    a = o.randn16(4, 75, 2 * k).reshape(2, k)
    nw = o.round16(1.0 + 0.1 * o.randn(4, 76, k), o.BF16)
    mats = []
    for n, kk, st in ((inter, k, 77), (inter, k, 78), (k, inter, 79)):
        w = o.bits_to_f32(o.randn16(4, st, n * kk, 0.05), o.BF16).reshape(n, kk)
        mats.append(o.w4_quantize(w, g, o.BF16))
    st = o.ffn_block(x, a, nw, 1e-6, *mats, g)
    wd = [o.w4_dequantize(*m, g).astype(np.float64) for m in mats]
    h = o.bits_to_f32(x, o.BF16).astype(np.float64) + o.bits_to_f32(a, o.BF16)
    n = h / np.sqrt((h * h).mean(-1, keepdims=True) + 1e-6) * o.bits_to_f32(nw, o.BF16)
    gate, up = n @ wd[0].T, n @ wd[1].T
    act = 0.5 * gate * (1 + erf(gate / np.sqrt(2))) * up
    out = h + act @ wd[2].T
    got = o.bits_to_f32(st["out"], o.BF16)
    assert rel_l2(got, out) < 4e-3
    assert np.array_equal(st["hidden"], o.add16(x, a))
    wrong = n + (0.5 * up * (1 + erf(up / np.sqrt(2))) * gate) @ wd[2].T
    assert rel_l2(got, wrong) > 0.05


def test_qkv_rope_split_and_rotation():
    k, nh, nkv, hd, g = 256, 4, 2, 64, 32
    w = o.bits_to_f32(o.randn16(5, 80, (nh + 2 * nkv) * hd * k, 0.05), o.BF16).reshape(-1, k)
    wq, s, b = o.w4_quantize(w, g, o.BF16)
    x = o.randn16(5, 81, k)
    q, kk, v, qkv = o.qkv_rope(x, wq, s, b, g, nh, nkv, hd, hd, 10000.0, 0)
    r = o.round16(qkv, o.BF16)
    # position 0 rotates nothing: the split alone, queries, keys, values in order
    assert np.array_equal(q.reshape(-1), r[:nh * hd])
    assert np.array_equal(kk.reshape(-1), r[nh * hd:(nh + nkv) * hd])
    assert np.array_equal(v.reshape(-1), r[(nh + nkv) * hd:])
    q7, k7, v7, _ = o.qkv_rope(x, wq, s, b, g, nh, nkv, hd, 32, 10000.0, 7)
    assert np.array_equal(v7, v)
    assert np.array_equal(q7[:, 32:], q[:, 32:]) and not np.array_equal(q7[:, :32], q[:, :32])
    assert np.array_equal(k7, o.rope16(kk[:, None], 32, 10000.0, 7)[:, 0])


# ---------------------------------------------------------------------------
# W8 affine (groupwise) quantized matmul
# ---------------------------------------------------------------------------

def test_w8_affine_oracle_against_brute_force_and_special_cases():
    """w8_affine_matmul: pure-Python loops over the packed bytes on a tiny
    case; one-hot activations pick u*s+b; a zero scale leaves b * group sum
    of x; per-channel symmetric W8 (biases -128*s, the converter's layout)
    equals the independent W8A16 oracle s * sum x*(u-128)."""
    rng = np.random.default_rng(21)
    m, n, k, g = 2, 3, 64, 32
    words = rng.integers(0, 2 ** 32, (n, k // 4), dtype=np.uint64).astype(np.uint32)
    s = o.bf16_bits(rng.standard_normal((n, k // g)).astype(np.float32) * 0.01)
    b = o.bf16_bits(rng.standard_normal((n, k // g)).astype(np.float32) * 0.1)
    x = o.randn16(21, 1, m * k).reshape(m, k)
    y = o.w8_affine_matmul(x, words, s, b, g)
    xf, sf, bf = (o.bits_to_f32(a, o.BF16) for a in (x, s, b))
    for i in range(m):
        for j in range(n):
            acc = 0.0
            for kk in range(k):
                code = (int(words[j, kk // 4]) >> (8 * (kk % 4))) & 0xFF
                acc += float(xf[i, kk]) * (code * float(sf[j, kk // g]) + float(bf[j, kk // g]))
            assert abs(y[i, j] - acc) <= 1e-12 * max(1.0, abs(acc))
    # one-hot rows
    e = np.zeros((1, k), np.float32)
    e[0, 37] = 1.0
    code = (words[:, 37 // 4] >> np.uint32(8 * (37 % 4))) & 0xFF
    assert np.array_equal(o.w8_affine_matmul(o.bf16_bits(e), words, s, b, g)[0],
                          code * sf[:, 1].astype(np.float64) + bf[:, 1].astype(np.float64))
    # zero scales: b times the group sums of x
    z = np.zeros_like(s)
    yz = o.w8_affine_matmul(x, words, z, b, g)
    gs = xf.astype(np.float64).reshape(m, k // g, g).sum(-1)
    assert np.allclose(yz, gs @ bf.astype(np.float64).T, rtol=1e-13, atol=1e-13)
    # converter W8 rows against the W8A16 oracle (fp32 scale per channel)
    gold = _golden()
    x8 = o.randn16(22, 1, 3 * 256).reshape(3, 256)
    sc = o.bits_to_f32(gold["w8_scales"], o.BF16)[:, 0].copy()
    ya = o.w8_affine_matmul(x8, gold["w8_words"], gold["w8_scales"], gold["w8_biases"], 32)
    yb = o.w8a16_matmul(x8, o.w8_unpack_affine(gold["w8_words"]), sc)
    assert np.allclose(ya, yb, rtol=1e-12, atol=1e-9)
    # fp32 scales (the converter's lm_head coefficients) are taken as is
    sf32 = rng.random((n, k // g)).astype(np.float32)
    bf32 = rng.random((n, k // g)).astype(np.float32)
    y32 = o.w8_affine_matmul(x, words, sf32, bf32, g, o.BF16, o.F32)
    u = o.unpack8(words).astype(np.float64)
    w = u * np.repeat(sf32.astype(np.float64), g, 1) + np.repeat(bf32.astype(np.float64), g, 1)
    assert np.allclose(y32, xf.astype(np.float64) @ w.T, rtol=1e-13)
    assert np.array_equal(o.unpack8(np.array([[0x04030201]], np.uint32))[0], [1, 2, 3, 4])


# ---------------------------------------------------------------------------
# multi-token (prefill) attention oracle
# ---------------------------------------------------------------------------

def test_sdpa_prefill_oracle_pins():
    """oracle.sdpa_prefill against the independent C decode oracle and
    textbook invariants: each causal row i (of L) equals decode of that query
    over the first N-L+i+1 tokens, so the last row is decode over all N; an
    unmasked L-row call equals decode row by row; identical keys give the
    mean of the visible values; a wrong (top-left) mask alignment fails."""
    b, hq, hkv, length, n, d = 1, 4, 2, 5, 9, 16
    q = o.randn(5, 1, b * hq * length * d).reshape(b, hq, length, d)
    k = o.randn(5, 2, b * hkv * n * d).reshape(b, hkv, n, d)
    v = o.randn(5, 3, b * hkv * n * d).reshape(b, hkv, n, d)
    scale = 0.3
    causal = o.sdpa_prefill(q, k, v, scale, causal=True)
    full = o.sdpa_prefill(q, k, v, scale, causal=False)
    for i in range(length):
        vis = n - length + i + 1
        dec = o.sdpa_decode(q[:, :, i].copy(), k[:, :, :vis].copy(), v[:, :, :vis].copy(), scale)
        assert np.allclose(causal[:, :, i], dec, atol=1e-6), i
        decf = o.sdpa_decode(q[:, :, i].copy(), k, v, scale)
        assert np.allclose(full[:, :, i], decf, atol=1e-6), i
    assert np.allclose(causal[:, :, -1], full[:, :, -1], atol=1e-12)
    # identical keys: uniform weights over each row's visible tokens
    kk = np.repeat(k[:, :, :1], n, axis=2)
    same = o.sdpa_prefill(q, kk, v, scale, causal=True)
    vr = np.repeat(v.astype(np.float64), hq // hkv, axis=1)
    for i in range(length):
        vis = n - length + i + 1
        assert np.allclose(same[:, :, i], vr[:, :, :vis].mean(2), atol=1e-6)
    # a top-left alignment (query i sees tokens 0..i) would differ
    vis_tl = np.arange(length)[:, None] >= np.arange(n)[None, :]
    kr = np.repeat(k.astype(np.float64), hq // hkv, axis=1)
    sc = (q.astype(np.float64) * scale) @ np.swapaxes(kr, -1, -2)
    sc = np.where(vis_tl, sc, -np.inf)
    p = np.exp(sc - sc.max(-1, keepdims=True))
    wrong = (p / p.sum(-1, keepdims=True)) @ vr
    assert not np.allclose(wrong, causal, atol=1e-3)


def test_sdpa_prefill_rounded_pins():
    """sdpa_prefill_rounded (the reference prefill kernel's rounding points)
    against an independent loop that rounds through numpy's float16 on a tiny
    case; with values exact in T and weights that are powers of two it is
    the unrounded oracle; identical keys give the mean of the rounded V over
    each row's visible tokens; its weights' rounding does not depend on the
    integer offset; and it stays within the bf16 bound of the exact oracle."""
    b, hq, hkv, length, n, d = 1, 2, 1, 3, 6, 8
    q = o.randn(6, 1, b * hq * length * d).reshape(b, hq, length, d)
    k = o.randn(6, 2, b * hkv * n * d).reshape(b, hkv, n, d)
    v = o.randn(6, 3, b * hkv * n * d).reshape(b, hkv, n, d)
    q16 = o.f16_bits(q)
    y = o.sdpa_prefill_rounded(q16, k, v, 0.4, True, o.F16)
    # independent loop with numpy float16
    qf = q16.view(np.float16).astype(np.float64)
    kf = k.astype(np.float16).astype(np.float64)
    vf = v.astype(np.float16).astype(np.float64)
    ref = np.zeros_like(y)
    for h in range(hq):
        for i in range(length):
            vis = n - length + i + 1
            s = np.array([qf[0, h, i] @ kf[0, 0, t] for t in range(vis)]) * 0.4 / math.log(2)
            c = math.ceil(s.max())
            p = [2.0 ** (st - c) for st in s]
            pt = [float(np.float16(np.float32(pp))) for pp in p]
            ref[0, h, i] = sum(pt[t] * vf[0, 0, t] for t in range(vis)) / sum(p)
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-12)
    # zero keys: every weight is exactly 1, so each row is the mean of the
    # T-rounded values it sees (with other identical keys the rounded weight
    # over the unrounded normalizer scales that mean by T(p)/p, as in the
    # reference kernel)
    same = o.sdpa_prefill_rounded(q16, np.zeros_like(k), v, 0.4, True, o.F16)
    for i in range(length):
        vis = n - length + i + 1
        assert np.allclose(same[0, :, i], vf[0, 0, :vis].mean(0), atol=1e-12)
    # against the exact oracle: values already in T and integer log2 scores
    # leave nothing to round
    kk = np.zeros_like(k)
    kk[..., 0] = np.arange(n)[None, None, :]
    qq = np.zeros((b, hq, length, d), np.float32)
    qq[..., 0] = 1.0
    vv = vf.astype(np.float32)
    y0 = o.sdpa_prefill_rounded(o.f16_bits(qq), kk, vv, math.log(2), True, o.F16)
    y1 = o.sdpa_prefill(qq, kk, vv, math.log(2), True)
    assert np.allclose(y0, y1, rtol=1e-12, atol=1e-12)
    # bf16 rounding of K, V and the weights moves a N(0,1) problem by ~1e-3
    bq, l2, n2, d2 = 1, 16, 40, 64
    q2 = o.randn(7, 1, bq * 4 * l2 * d2).reshape(bq, 4, l2, d2)
    k2 = o.randn(7, 2, bq * 2 * n2 * d2).reshape(bq, 2, n2, d2)
    v2 = o.randn(7, 3, bq * 2 * n2 * d2).reshape(bq, 2, n2, d2)
    q2b = o.bf16_bits(q2)
    yr = o.sdpa_prefill_rounded(q2b, k2, v2, 0.125, True, o.BF16)
    ye = o.sdpa_prefill(o.bits_to_f32(q2b, o.BF16), k2, v2, 0.125, True)
    assert 3e-4 < rel_l2(yr, ye) < 1e-2


def test_attention_gate16_against_torch_and_known_answers():
    """attention_gate16 against the same graph written with torch's own
    float64 ops and 16-bit casts; a zero dot gives the gate 0.5 exactly (the
    output halves exactly); a large dot gives 1 (the output passes through);
    out[b, l, h*D:(h+1)*D] is head h of position l, scaled."""
    b, h, length, d, hid = 2, 3, 4, 8, 32
    x16 = o.randn16(31, 1, b * length * hid).reshape(b, length, hid)
    a16 = o.randn16(31, 2, b * h * length * d).reshape(b, h, length, d)
    w16 = o.randn16(31, 3, h * hid, 0.3).reshape(h, hid)
    gate, out = o.attention_gate16(x16, a16, w16, o.BF16)
    t = lambda u: torch.from_numpy(u.view(np.int16)).view(torch.bfloat16)  # noqa: E731
    xt, at, wt = t(x16), t(a16), t(w16)
    dot = (xt.double() @ wt.double().T).float().to(torch.bfloat16)
    gt = torch.sigmoid(dot.double()).float().to(torch.bfloat16)
    ot = (at.transpose(1, 2).double() * gt.double()[..., None]).float().to(torch.bfloat16)
    assert np.array_equal(gate, gt.view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(out, ot.reshape(b, length, h * d).view(torch.int16).numpy()
                          .view(np.uint16))
    g0, o0 = o.attention_gate16(np.zeros_like(x16), a16, w16, o.BF16)
    assert np.all(o.bits_to_f32(g0, o.BF16) == 0.5)
    half = o.bits_to_f32(a16, o.BF16).transpose(0, 2, 1, 3).reshape(b, length, h * d) / 2
    assert np.array_equal(o.bits_to_f32(o0, o.BF16), half)
    big = o.bf16_bits(np.full((h, hid), 4.0, np.float32))
    ones = o.bf16_bits(np.ones((b, length, hid), np.float32))
    g1, o1 = o.attention_gate16(ones, a16, big, o.BF16)
    assert np.all(o.bits_to_f32(g1, o.BF16) == 1.0)
    assert np.array_equal(o1, a16.transpose(0, 2, 1, 3).reshape(b, length, h * d))


# ---------------------------------------------------------------------------
# affine KV caches of 8, 4 and 2 bits and the staged attention over them
# ---------------------------------------------------------------------------

def test_kv_quantize_affine_matches_c_and_packing():
    """The numpy affine KV quantizer equals the C one at 8 bits bit for bit;
    at 4 bits its words are the W4 packing (pack4, pinned by a known answer)
    of its codes; at 2 bits sixteen codes fill a word from the low bits; and
    every width dequantizes within half a step of the input."""
    x = o.randn(41, 1, 3 * 5 * 128).reshape(3, 5, 128)
    x[0, 0, :32] = 1.5                                  # a constant group: scale 0
    for g in (32, 64, 128):
        p8, s8, b8 = o.kv_quantize_affine(x, g, 8, o.BF16)
        c8, cs, cb = o.kv_quantize_affine_u8(x, g, o.BF16)
        assert np.array_equal(p8, c8) and np.array_equal(s8, cs) and np.array_equal(b8, cb)
        assert np.array_equal(o.kv_dequantize_affine(p8, s8, b8, g, 8, o.BF16),
                              o.kv_dequantize_affine_u8(c8, cs, cb, g, o.BF16))
    p4, s4, b4 = o.kv_quantize_affine(x, 32, 4, o.BF16)
    sf = np.repeat(o.bits_to_f32(s4, o.BF16), 32, -1)
    bf = np.repeat(o.bits_to_f32(b4, o.BF16), 32, -1)
    with np.errstate(divide="ignore", invalid="ignore"):
        codes = np.where(sf != 0, np.clip(np.rint((x - bf) / sf), 0, 15), 0).astype(np.uint8)
    assert np.array_equal(p4.reshape(-1, 16), o.pack4(codes.reshape(-1, 128)))
    y = np.tile(np.array([0, 1, 2, 3], np.float32), 8)[None]      # one group of 32
    p2, s2, b2 = o.kv_quantize_affine(y, 32, 2, o.F16)
    assert o.bits_to_f32(s2, o.F16)[0, 0] == 1.0 and o.bits_to_f32(b2, o.F16)[0, 0] == 0.0
    assert p2.tolist() == [[0xE4E4E4E4, 0xE4E4E4E4]]  # codes 0,1,2,3 from the low bits
    for bits in (8, 4, 2):
        p, s, b = o.kv_quantize_affine(x, 64, bits, o.F16)
        back = o.kv_dequantize_affine(p, s, b, 64, bits, o.F16)
        step = np.repeat(o.bits_to_f32(s, o.F16), 64, -1)
        assert np.all(np.abs(back - x) <= step / 2 + 1e-3 * np.abs(x) + 1e-6), bits


def test_sdpa_staged_oracle_pins():
    """sdpa_staged against sdpa_prefill (no mask, causal), and the mask
    semantics of the reference's fallback: an all-True boolean mask and an
    all-zero additive one change nothing; an -inf additive entry hides a
    token like a False; a row with nothing visible averages every value (the
    finfo.min fill); a mask broadcast from [L,N] equals the full one; values
    may have a head dim of their own."""
    b, hq, hkv, length, n, d, dv = 1, 4, 2, 3, 7, 8, 16
    q = o.randn(42, 1, b * hq * length * d).reshape(b, hq, length, d)
    k = o.randn(42, 2, b * hkv * n * d).reshape(b, hkv, n, d)
    v = o.randn(42, 3, b * hkv * n * d).reshape(b, hkv, n, d)
    assert np.allclose(o.sdpa_staged(q, k, v, 0.3), o.sdpa_prefill(q, k, v, 0.3, False))
    assert np.allclose(o.sdpa_staged(q, k, v, 0.3, "causal"), o.sdpa_prefill(q, k, v, 0.3, True))
    ones = np.ones((length, n), bool)
    assert np.allclose(o.sdpa_staged(q, k, v, 0.3, ones), o.sdpa_staged(q, k, v, 0.3))
    assert np.allclose(o.sdpa_staged(q, k, v, 0.3, np.zeros((length, n))),
                       o.sdpa_staged(q, k, v, 0.3))
    hide = ones.copy()
    hide[:, 2] = False
    add = np.where(hide, 0.0, -np.inf)
    assert np.allclose(o.sdpa_staged(q, k, v, 0.3, hide), o.sdpa_staged(q, k, v, 0.3, add))
    none = ones.copy()
    none[1] = False
    out = o.sdpa_staged(q, k, v, 0.3, none)
    vr = np.repeat(v.astype(np.float64), hq // hkv, axis=1)
    assert np.allclose(out[:, :, 1], vr.mean(2))
    full = np.broadcast_to(hide, (b, hq, length, n))
    assert np.allclose(o.sdpa_staged(q, k, v, 0.3, full), o.sdpa_staged(q, k, v, 0.3, hide))
    v2 = o.randn(42, 4, b * hkv * n * dv).reshape(b, hkv, n, dv)
    out2 = o.sdpa_staged(q, k, v2, 0.3, "causal")
    assert out2.shape == (b, hq, length, dv)
    # the last causal row sees every token: the weights of the unmasked call
    assert np.allclose(out2[:, :, -1], o.sdpa_staged(q, k, v2, 0.3)[:, :, -1])
