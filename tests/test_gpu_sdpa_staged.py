"""GPU parity of the staged quantized attention (sparkq_quantized_sdpa, the
reference's _fallback, X/spark_mlx_ext/int8_quantized_sdpa.py:122-153):
2-, 4- and 8-bit affine caches, group sizes 32/64/128, head dims outside the
fused kernels' (and value dims of their own), head ratios outside 1/2/4/8,
and None / causal / boolean / additive masks, against the float64 oracle;
plus the 4- and 2-bit quantize-on-append and the routing of dispatch_sdpa."""

import math

import numpy as np
import pytest
import torch

import oracle as o
from helpers import TORCH16, check_fp32, up16

pytestmark = pytest.mark.gpu


def _cache(dev, b, hkv, n, d, g, bits, dtype, seed, tensor_dtype=None):
    x = o.randn(seed, 71, b * hkv * n * d).reshape(b, hkv, n, d)
    p, s, bb = o.kv_quantize_affine(x, g, bits, dtype)
    dq = o.kv_dequantize_affine(p, s, bb, g, bits, dtype)
    if tensor_dtype == torch.float32:
        dev_t = (torch.from_numpy(p.view(np.int32)).to(dev),
                 torch.from_numpy(o.bits_to_f32(s, dtype)).to(dev),
                 torch.from_numpy(o.bits_to_f32(bb, dtype)).to(dev))
    else:
        dev_t = (torch.from_numpy(p.view(np.int32)).to(dev), up16(s, dtype, dev),
                 up16(bb, dtype, dev))
    return dev_t, dq


CASES = [
    # b, hq, hkv, L, n, d, dv, g, bits, qdtype, mask
    (1, 32, 8, 1, 4096, 128, 128, 64, 4, o.BF16, None),     # 4-bit decode, split context
    (1, 16, 4, 1, 1000, 256, 256, 32, 2, o.BF16, "causal"),  # 2-bit
    (2, 12, 4, 1, 777, 96, 96, 32, 8, o.F16, None),         # head dim 96, ratio 3
    (1, 16, 1, 5, 300, 80 + 16, 64, 32, 4, o.BF16, "causal"),  # ratio 16, Dv != D
    (1, 8, 8, 37, 100, 128, 128, 128, 8, o.BF16, "bool"),   # boolean mask array
    (1, 4, 2, 9, 50, 64, 64, 64, 4, o.F16, "add"),          # additive mask array
    (1, 4, 2, 6, 4, 64, 64, 32, 8, o.BF16, "causal"),       # L > N: early rows see nothing
    (1, 8, 2, 1, 5000, 64, 64, 32, 4, o.F32, None),         # fp32 queries and metadata
    (1, 8, 8, 3, 20, 512, 512, 128, 2, o.BF16, "bool"),     # the widest head dims
    (1, 32, 8, 1, 20000, 128, 128, 64, 4, o.BF16, "bool"),  # 128 context splits merged
    (2, 12, 4, 3, 9000, 96, 96, 32, 8, o.F16, "causal"),    # many splits, three rows, ratio 3
]


@pytest.mark.parametrize("b,hq,hkv,length,n,d,dv,g,bits,qdtype,mask", CASES)
def test_staged_attention_matches_oracle(gpu, b, hq, hkv, length, n, d, dv, g, bits, qdtype,
                                         mask):
    import sparkq

    print(f"[case] staged b={b} hq={hq} hkv={hkv} L={length} N={n} D={d} Dv={dv} G={g} "
          f"bits={bits} q={qdtype} mask={mask}", flush=True)
    seed = n + d + bits
    mdt = o.BF16 if qdtype == o.F32 else qdtype
    tdt = torch.float32 if qdtype == o.F32 else None
    keys, kd = _cache(gpu, b, hkv, n, d, g, bits, mdt, seed, tdt)
    vals, vd = _cache(gpu, b, hkv, n, dv, g, bits, mdt, seed + 1, tdt)
    qf = o.randn(seed, 72, b * hq * length * d).reshape(b, hq, length, d)
    if qdtype == o.F32:
        qt = torch.from_numpy(qf).to(gpu)
        qref = qf
    else:
        q16 = o.round16(qf, qdtype)
        qt = up16(q16, qdtype, gpu)
        qref = o.bits_to_f32(q16, qdtype)
    rng = np.random.default_rng(seed)
    if mask == "bool":
        m = rng.random((length, n)) > 0.4
        if length > 1:
            m[0] = False                 # a row that sees nothing: the mean of V
        mask_t, mask_ref = torch.from_numpy(m).to(gpu), m
    elif mask == "add":
        m = (rng.standard_normal((1, hq, length, n)) * 2).astype(np.float32)
        m[..., 3] = -np.inf
        mask_t = torch.from_numpy(m).to(TORCH16[qdtype]).to(gpu)
        mask_ref = o.bits_to_f32(o.round16(m, qdtype), qdtype)
    else:
        mask_t = mask_ref = mask
    scale = 1.0 / math.sqrt(d)
    y = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=scale, group_size=g, bits=bits,
                                   mask=mask_t, out_dtype=torch.float32).cpu().numpy()
    ref = o.sdpa_staged(qref, kd, vd, scale, mask_ref, mdt if qdtype != o.F32 else o.F32)
    assert y.shape == (b, hq, length, dv)
    check_fp32(y, ref)
    y16 = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=scale, group_size=g, bits=bits,
                                     mask=mask_t)
    assert y16.dtype == qt.dtype
    assert np.array_equal(y16.float().cpu().numpy(),
                          torch.from_numpy(y).to(qt.dtype).float().numpy())


@pytest.mark.parametrize("bits", [4, 2])
def test_low_bit_cache_append_and_dispatch(gpu, bits):
    """QuantizedKVCache(bits) appends bit for bit with the oracle's quantizer
    across the growth step, and dispatch_sdpa takes the resulting cache (the
    reference's mlx-lm quantized path) to the staged kernel."""
    import sparkq
    from sparkq.ops import dispatch_sdpa

    b, hkv, hq, d, g = 1, 4, 16, 128, 64
    cache = sparkq.QuantizedKVCache(group_size=g, bits=bits)
    chunks = [200, 100, 1]
    xs = []
    for i, length in enumerate(chunks):
        kx = o.randn16(bits, 80 + i, b * hkv * length * d).reshape(b, hkv, length, d)
        vx = o.randn16(bits, 90 + i, b * hkv * length * d).reshape(b, hkv, length, d)
        xs.append((kx, vx))
        keys, vals = cache.update_and_fetch(up16(kx, o.BF16, gpu), up16(vx, o.BF16, gpu))
    n = sum(chunks)
    kall = np.concatenate([k for k, _ in xs], axis=2)
    vall = np.concatenate([v for _, v in xs], axis=2)
    kp, ks, kb = o.kv_quantize_affine(o.bits_to_f32(kall, o.BF16), g, bits, o.BF16)
    assert keys[0].shape == (b, hkv, n, d * bits // 32)
    assert np.array_equal(keys[0].cpu().numpy().view(np.uint32), kp)
    assert np.array_equal(keys[1].view(torch.int16).cpu().numpy().view(np.uint16), ks)
    assert np.array_equal(keys[2].view(torch.int16).cpu().numpy().view(np.uint16), kb)
    vp, vs, vb = o.kv_quantize_affine(o.bits_to_f32(vall, o.BF16), g, bits, o.BF16)

    class Cache:
        pass

    Cache.bits, Cache.group_size = bits, g
    q16 = o.randn16(bits, 99, b * hq * d).reshape(b, hq, 1, d)
    y = dispatch_sdpa(up16(q16, o.BF16, gpu), keys, vals, cache=Cache(), scale=d ** -0.5,
                      mask=None)
    ref = o.sdpa_staged(o.bits_to_f32(q16, o.BF16),
                        o.kv_dequantize_affine(kp, ks, kb, g, bits, o.BF16),
                        o.kv_dequantize_affine(vp, vs, vb, g, bits, o.BF16), d ** -0.5)
    assert np.abs(y.float().cpu().numpy() - ref).max() <= 2e-2


@pytest.mark.parametrize("qdtype", [o.BF16, o.F16])
def test_staged_additive_mask_hides_leading_chunks(gpu, qdtype):
    """Additive masks that hide the first 256-token chunk and the whole first
    context split (N = 1300 runs in three splits) with -inf and with the
    dtype's lowest finite value: those tokens weigh nothing and the row stays
    finite, as in the reference's scores + mask softmax; a row masked
    everywhere with the lowest finite bf16 value averages every value."""
    import sparkq

    b, hq, hkv, length, n, d, g, bits = 1, 4, 2, 3, 1300, 64, 64, 4
    print(f"[case] staged masked lead q={qdtype} N={n}", flush=True)
    keys, kd = _cache(gpu, b, hkv, n, d, g, bits, qdtype, 5)
    vals, vd = _cache(gpu, b, hkv, n, d, g, bits, qdtype, 6)
    q16 = o.round16(o.randn(7, 72, b * hq * length * d).reshape(b, hq, length, d), qdtype)
    lowest = float(torch.finfo(TORCH16[qdtype]).min)
    m = (np.random.default_rng(3).standard_normal((1, hq, length, n)) * 2).astype(np.float32)
    m[:, :, 0, :600] = -np.inf
    m[:, :, 1, :600] = lowest
    if qdtype == o.BF16:
        m[:, :, 2, :] = lowest
    else:
        m[:, :, 2, 100:700] = -np.inf
    mask_t = torch.from_numpy(m).to(TORCH16[qdtype]).to(gpu)
    mask_ref = o.bits_to_f32(o.round16(m, qdtype), qdtype)
    scale = 1.0 / math.sqrt(d)
    y = sparkq.int8_quantized_sdpa(up16(q16, qdtype, gpu), keys, vals, scale=scale,
                                   group_size=g, bits=bits, mask=mask_t,
                                   out_dtype=torch.float32).cpu().numpy()
    assert np.isfinite(y).all()
    ref = o.sdpa_staged(o.bits_to_f32(q16, qdtype), kd, vd, scale, mask_ref, qdtype)
    check_fp32(y, ref)
    if qdtype == o.BF16:
        mean_v = np.repeat(vd, hq // hkv, axis=1).mean(axis=2)
        assert np.abs(y[:, :, 2] - mean_v).max() <= 1e-4


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("b,hq,hkv,n,d,g,qdtype", [
    (1, 32, 8, 4096, 128, 64, o.BF16),    # the 4-bit decode bench geometry (split context)
    (2, 16, 4, 777, 64, 32, o.F16),
    (1, 8, 1, 300, 256, 128, o.BF16),     # eight query heads per KV head
    (3, 4, 4, 1, 128, 32, o.BF16),        # one token: the value row itself
    (1, 16, 8, 5000, 128, 64, o.F32)])
def test_low_bit_decode_matches_oracle(gpu, bits, b, hq, hkv, n, d, g, qdtype):
    """One query token over a 4- or 2-bit MLX affine cache takes the decode
    entry on the codes (the matrix-core kernel for 16-bit queries, the
    vector kernel for fp32 ones): the fp32 output within the north-star
    tolerance of the fp64 attention over the dequantized cache, the 16-bit
    output equal to its rounding, for head dims 64/128/256, groups
    32/64/128, head ratios 1..8, split contexts and a single token."""
    import sparkq

    print(f"[case] low-bit decode bits={bits} b={b} hq={hq} hkv={hkv} N={n} D={d} G={g}",
          flush=True)
    mdt = o.BF16 if qdtype == o.F32 else qdtype
    tdt = torch.float32 if qdtype == o.F32 else None
    keys, kd = _cache(gpu, b, hkv, n, d, g, bits, mdt, n + bits, tdt)
    vals, vd = _cache(gpu, b, hkv, n, d, g, bits, mdt, n + bits + 1, tdt)
    qf = o.randn(n, 73, b * hq * d).reshape(b, hq, 1, d)
    if qdtype == o.F32:
        qt, qref = torch.from_numpy(qf).to(gpu), qf
    else:
        q16 = o.round16(qf, qdtype)
        qt, qref = up16(q16, qdtype, gpu), o.bits_to_f32(q16, qdtype)
    scale = 1.0 / math.sqrt(d)
    y = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=scale, group_size=g, bits=bits,
                                   out_dtype=torch.float32).cpu().numpy()
    ref = o.sdpa_decode(qref[:, :, 0], kd, vd, scale)
    check_fp32(y.reshape(b, hq, d), ref)
    if n == 1:
        vrow = np.repeat(vd[:, :, 0], hq // hkv, axis=1)
        assert np.allclose(y.reshape(b, hq, d), vrow, rtol=1e-6, atol=1e-6)
    y16 = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=scale, group_size=g, bits=bits)
    assert np.array_equal(y16.float().cpu().numpy(), torch.from_numpy(y).to(qt.dtype).float().numpy())
