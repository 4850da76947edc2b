"""GPU parity of the matrix-core decode attention over the MLX affine KV
caches (8-, 4- and 2-bit codes, group sizes 32/64/128, head dims 64/128/256,
1..8 query heads per KV head, bf16 and fp16 queries) against the fp64 oracle
over the dequantized cache, against the vector decode kernel it replaces,
and its fallbacks."""

import math

import numpy as np
import pytest
import torch

import oracle as o
from helpers import check_fp32, up16

pytestmark = pytest.mark.gpu


def _cache(dev, b, hkv, n, d, g, bits, dtype, seed):
    x = o.randn(seed, 71, b * hkv * n * d).reshape(b, hkv, n, d)
    p, s, bb = o.kv_quantize_affine(x, g, bits, dtype)
    dq = o.kv_dequantize_affine(p, s, bb, g, bits, dtype)
    return (torch.from_numpy(p.view(np.int32)).to(dev), up16(s, dtype, dev), up16(bb, dtype, dev)), dq


def _query(dev, b, hq, d, qdtype, seed):
    q16 = o.round16(o.randn(seed, 73, b * hq * d).reshape(b, hq, 1, d), qdtype)
    return up16(q16, qdtype, dev), o.bits_to_f32(q16, qdtype)


CASES = [
    # bits, b, hq, hkv, n, d, g, qdtype
    (8, 1, 32, 8, 4096, 128, 32, o.BF16),   # the reference's cache format, split context
    (8, 2, 8, 8, 300, 64, 32, o.F16),       # one query head per KV head
    (8, 1, 16, 8, 33, 256, 64, o.BF16),     # two heads per KV head, one partial block
    (8, 3, 64, 8, 1, 128, 128, o.F16),      # eight heads per KV head, a single token
    (8, 8, 32, 8, 2048, 128, 64, o.BF16),   # batch 8
    (4, 1, 32, 8, 4100, 128, 32, o.BF16),
    (4, 2, 8, 2, 777, 64, 64, o.F16),
    (4, 1, 16, 2, 200, 256, 128, o.BF16),
    (2, 1, 32, 8, 5000, 128, 32, o.BF16),   # 2-bit G32: column blocks span two groups
    (2, 2, 16, 4, 129, 64, 32, o.F16),      # 8-byte value pieces
    (2, 1, 8, 1, 70, 256, 64, o.BF16),
    # rows as heads with one PV pass per group (heads x groups > 16)
    (8, 1, 64, 8, 500, 128, 32, o.BF16),    # 8 heads x 4 groups
    (4, 1, 32, 4, 300, 256, 32, o.F16),     # 8 x 8
    (2, 1, 32, 4, 200, 256, 32, o.BF16),    # 8 x 8, 2-bit column blocks spanning two groups
    (8, 2, 16, 2, 650, 256, 64, o.BF16),    # 8 x 4
    # (head, group) rows at the widest group count and at 16 rows
    (8, 1, 8, 4, 300, 256, 32, o.F16),      # 2 x 8: the row's group depends on the lane group
    (2, 1, 16, 4, 333, 256, 64, o.BF16),    # 4 x 4
]


@pytest.mark.parametrize("bits,b,hq,hkv,n,d,g,qdtype", CASES)
def test_affine_mfma_decode_matches_oracle(gpu, bits, b, hq, hkv, n, d, g, qdtype):
    """fp32 output within the north-star tolerance of the fp64 attention over
    the dequantized cache; the 16-bit output is its rounding."""
    import sparkq

    print(f"[case] affine mfma decode bits={bits} b={b} hq={hq} hkv={hkv} N={n} D={d} G={g}",
          flush=True)
    keys, kd = _cache(gpu, b, hkv, n, d, g, bits, qdtype, 3 * n + bits)
    vals, vd = _cache(gpu, b, hkv, n, d, g, bits, qdtype, 3 * n + bits + 1)
    qt, qref = _query(gpu, b, hq, d, qdtype, n + d)
    scale = 1.0 / math.sqrt(d)
    y = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=scale, group_size=g, bits=bits,
                                   out_dtype=torch.float32).cpu().numpy()
    ref = o.sdpa_decode(qref[:, :, 0], kd, vd, scale)
    check_fp32(y.reshape(b, hq, d), ref)
    if n == 1:
        vrow = np.repeat(vd[:, :, 0], hq // hkv, axis=1)
        assert np.allclose(y.reshape(b, hq, d), vrow, rtol=1e-5, atol=1e-5)
    y16 = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=scale, group_size=g, bits=bits)
    assert np.array_equal(y16.float().cpu().numpy(), torch.from_numpy(y).to(qt.dtype).float().numpy())


@pytest.mark.parametrize("bits,d,g", [(8, 128, 32), (4, 128, 64), (2, 64, 32)])
def test_affine_mfma_against_vector_kernel(gpu, monkeypatch, bits, d, g):
    """The matrix-core kernel and the vector kernel (SPARKQ_SDPA_NO_MFMA=1)
    agree to fp32 accumulation error, and they are distinct code paths (the
    outputs are not bit-identical)."""
    import sparkq

    b, hq, hkv, n = 1, 32, 8, 3000
    keys, _ = _cache(gpu, b, hkv, n, d, g, bits, o.BF16, 11 + bits)
    vals, _ = _cache(gpu, b, hkv, n, d, g, bits, o.BF16, 12 + bits)
    qt, _ = _query(gpu, b, hq, d, o.BF16, 5)
    scale = 1.0 / math.sqrt(d)
    y = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=scale, group_size=g, bits=bits,
                                   out_dtype=torch.float32).cpu().numpy()
    monkeypatch.setenv("SPARKQ_SDPA_NO_MFMA", "1")
    yv = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=scale, group_size=g, bits=bits,
                                    out_dtype=torch.float32).cpu().numpy()
    assert np.abs(y - yv).max() <= 1e-4 * max(1.0, np.abs(yv).max())
    assert not np.array_equal(y, yv)


def test_affine_mfma_strided_cache_view(gpu):
    """A cache allocated for 512 tokens holding 300 (a view along tokens):
    the matrix-core kernel reads the strided view."""
    import sparkq

    b, hq, hkv, n, cap, d, g = 2, 16, 4, 300, 512, 128, 32
    keys, kd = _cache(gpu, b, hkv, cap, d, g, 8, o.BF16, 21)
    vals, vd = _cache(gpu, b, hkv, cap, d, g, 8, o.BF16, 22)
    keys = tuple(t[:, :, :n] for t in keys)
    vals = tuple(t[:, :, :n] for t in vals)
    qt, qref = _query(gpu, b, hq, d, o.BF16, 23)
    scale = 1.0 / math.sqrt(d)
    y = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=scale, group_size=g,
                                   out_dtype=torch.float32).cpu().numpy()
    ref = o.sdpa_decode(qref[:, :, 0], kd[:, :, :n], vd[:, :, :n], scale)
    check_fp32(y.reshape(b, hq, d), ref)


def test_affine_mfma_unaligned_scales_fall_back(gpu):
    """Scale and bias vectors whose token stride is not a multiple of their
    width (a padded last axis) take the vector kernel, with the same result
    bar accumulation order."""
    import sparkq

    b, hq, hkv, n, d, g = 1, 8, 2, 400, 128, 32
    (kc, ks, kb), kd = _cache(gpu, b, hkv, n, d, g, 8, o.BF16, 31)
    (vc, vs, vb), vd = _cache(gpu, b, hkv, n, d, g, 8, o.BF16, 32)

    def pad(t):
        p = torch.zeros(*t.shape[:-1], t.shape[-1] + 1, dtype=t.dtype, device=t.device)
        p[..., :-1] = t
        return p[..., :-1]

    qt, qref = _query(gpu, b, hq, d, o.BF16, 33)
    scale = 1.0 / math.sqrt(d)
    y = sparkq.int8_quantized_sdpa(qt, (kc, pad(ks), pad(kb)), (vc, pad(vs), pad(vb)),
                                   scale=scale, group_size=g, out_dtype=torch.float32)
    ref = o.sdpa_decode(qref[:, :, 0], kd, vd, scale)
    check_fp32(y.cpu().numpy().reshape(b, hq, d), ref)


@pytest.mark.parametrize("shift", [-60, 40])
def test_affine_mfma_value_scale_range(gpu, shift):
    """bf16 value scales and biases far outside the fp16 range (scaled by
    2^shift): the weights p * scale stay in bf16's exponent range, so the
    output is 2^shift times the unscaled one to the same tolerance."""
    import sparkq

    b, hq, hkv, n, d, g = 1, 16, 4, 1500, 128, 64
    keys, kd = _cache(gpu, b, hkv, n, d, g, 8, o.BF16, 41)
    (vc, vs, vb), vd = _cache(gpu, b, hkv, n, d, g, 8, o.BF16, 42)
    f = 2.0 ** shift
    vals = (vc, vs * f, vb * f)
    qt, qref = _query(gpu, b, hq, d, o.BF16, 43)
    scale = 1.0 / math.sqrt(d)
    y = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=scale, group_size=g,
                                   out_dtype=torch.float32).cpu().numpy()
    assert np.isfinite(y).all()
    ref = o.sdpa_decode(qref[:, :, 0], kd, vd, scale)
    check_fp32(y.reshape(b, hq, d) / f, ref)
