"""GPU parity of the INT8 KV cache producer and of multi-token attention:
quantize-on-append (QuantizedKVCache / kv_append) bit-exact with the oracle's
quantizers for both formats across appends that cross the cache's 256-token
growth steps, decode attention on the fetched views, and the prefill
attention (L > 1, bottom-right causal or unmasked) for both formats against
the fp64 staged attention of the reference's _fallback."""

import math

import numpy as np
import pytest
import torch

import oracle as o
from helpers import check_fp32, check_rounded16, down16, max_abs, rel_l2, up16

pytestmark = pytest.mark.gpu


def _x16(seed, stream, shape, dtype=o.BF16):
    return o.randn16(seed, stream, int(np.prod(shape)), 1.0, dtype).reshape(shape)


@pytest.mark.parametrize("fmt,d,g", [("s8", 128, 32), ("s8", 64, 32), ("affine_u8", 128, 32),
                                     ("affine_u8", 256, 64), ("affine_u8", 128, 128),
                                     ("affine_u8", 64, 32), ("affine_u8", 64, 64),
                                     ("affine_u8", 256, 32)])
def test_append_matches_oracle(gpu, fmt, d, g):
    import sparkq

    b, h = 2, 4
    cache = sparkq.QuantizedKVCache(group_size=g, kv_format=fmt)
    chunks = [5, 1, 300, 2]
    ks, vs = [], []
    for i, length in enumerate(chunks):
        k16 = _x16(i, 10, (b, h, length, d))
        v16 = _x16(i, 20, (b, h, length, d))
        ks.append(k16)
        vs.append(v16)
        keys, values = cache.update_and_fetch(up16(k16, o.BF16, gpu), up16(v16, o.BF16, gpu))
    n = sum(chunks)
    assert cache.offset == n and keys[0].shape[2] == n
    assert cache.keys[0].shape[2] == 512          # grown in steps of 256
    kf = o.bits_to_f32(np.concatenate(ks, axis=2), o.BF16)
    vf = o.bits_to_f32(np.concatenate(vs, axis=2), o.BF16)
    for got, want in ((keys, kf), (values, vf)):
        if fmt == "s8":
            codes, sc = o.kv_quantize_s8(want)
            assert np.array_equal(got[0].cpu().numpy(), codes)
            assert np.array_equal(got[1].cpu().numpy().view(np.uint16), sc)
        else:
            packed, s, bb = o.kv_quantize_affine_u8(want, g, o.BF16)
            assert np.array_equal(got[0].cpu().numpy().view(np.uint32), packed)
            assert np.array_equal(down16(got[1]), s)
            assert np.array_equal(down16(got[2]), bb)
    # decode attention straight on the fetched views
    q16 = _x16(7, 30, (b, 2 * h, d))
    y = sparkq.int8_quantized_sdpa(up16(q16[:, :, None], o.BF16, gpu), keys, values,
                                   scale=1.0 / math.sqrt(d), group_size=g,
                                   out_dtype=torch.float32)
    if fmt == "s8":
        kd = o.kv_dequantize_s8(*o.kv_quantize_s8(kf))
        vd = o.kv_dequantize_s8(*o.kv_quantize_s8(vf))
    else:
        kd = o.kv_dequantize_affine_u8(*o.kv_quantize_affine_u8(kf, g, o.BF16), g, o.BF16)
        vd = o.kv_dequantize_affine_u8(*o.kv_quantize_affine_u8(vf, g, o.BF16), g, o.BF16)
    ref = o.sdpa_decode(o.bits_to_f32(q16, o.BF16), kd, vd, 1.0 / math.sqrt(d))
    check_fp32(y.cpu().numpy().reshape(ref.shape), ref)


def _prefill(dev, b, hq, hkv, length, n, d, causal, seed, qdtype=o.BF16, out_dtype=None):
    import sparkq

    q16 = _x16(seed, 40, (b, hq, length, d), qdtype)
    k = o.randn(seed, 41, b * hkv * n * d).reshape(b, hkv, n, d)
    v = o.randn(seed, 42, b * hkv * n * d).reshape(b, hkv, n, d)
    kc, ks = o.kv_quantize_s8(k)
    vc, vs = o.kv_quantize_s8(v)
    keys = (torch.from_numpy(kc).to(dev), torch.from_numpy(ks.view(np.float16)).to(dev))
    vals = (torch.from_numpy(vc).to(dev), torch.from_numpy(vs.view(np.float16)).to(dev))
    scale = 1.0 / math.sqrt(d)
    y = sparkq.int8_quantized_sdpa(up16(q16, qdtype, dev), keys, vals, scale=scale,
                                   mask="causal" if causal else None, out_dtype=out_dtype)
    ref = o.sdpa_prefill(o.bits_to_f32(q16, qdtype), o.kv_dequantize_s8(kc, ks),
                         o.kv_dequantize_s8(vc, vs), scale, causal)
    return y, ref


@pytest.mark.parametrize("b,hq,hkv,length,n,d,causal", [
    (1, 32, 8, 16, 16, 128, True), (1, 32, 8, 100, 300, 128, True),
    (2, 32, 8, 257, 257, 128, True), (1, 32, 8, 64, 200, 128, False),
    (1, 8, 8, 33, 90, 64, True), (1, 16, 2, 40, 129, 256, True), (2, 16, 8, 7, 7, 64, True),
    (1, 4, 2, 1000, 1000, 128, True)])
def test_prefill_matches_oracle(gpu, b, hq, hkv, length, n, d, causal):
    y32, ref = _prefill(gpu, b, hq, hkv, length, n, d, causal, seed=length + n,
                        out_dtype=torch.float32)
    check_fp32(y32.cpu().numpy(), ref)
    y16, _ = _prefill(gpu, b, hq, hkv, length, n, d, causal, seed=length + n)
    # the fp32 result is within ~2e-5 absolute (the 1152 code offset costs
    # ~1152 * 2^-24 of the value scale); that is several bf16 units of the
    # smallest outputs, so the one-unit bound applies from rms/16 up
    check_rounded16(down16(y16), ref, o.BF16, near_zero=2.0 ** -4)


def test_prefill_f16_queries(gpu):
    y32, ref = _prefill(gpu, 1, 32, 8, 48, 80, 128, True, seed=3, qdtype=o.F16,
                        out_dtype=torch.float32)
    check_fp32(y32.cpu().numpy(), ref)


def test_prefill_last_row_is_decode(gpu):
    """Under the causal mask the last query position sees all N tokens, so its
    output must equal single-token decode of that query."""
    import sparkq

    b, hq, hkv, length, n, d = 1, 32, 8, 20, 150, 128
    q16 = _x16(5, 50, (b, hq, length, d))
    k = o.randn(5, 51, b * hkv * n * d).reshape(b, hkv, n, d)
    v = o.randn(5, 52, b * hkv * n * d).reshape(b, hkv, n, d)
    kc, ks = o.kv_quantize_s8(k)
    vc, vs = o.kv_quantize_s8(v)
    keys = (torch.from_numpy(kc).to(gpu), torch.from_numpy(ks.view(np.float16)).to(gpu))
    vals = (torch.from_numpy(vc).to(gpu), torch.from_numpy(vs.view(np.float16)).to(gpu))
    qt = up16(q16, o.BF16, gpu)
    yp = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=0.1, mask="causal",
                                    out_dtype=torch.float32)
    yd = sparkq.int8_quantized_sdpa(qt[:, :, -1:].contiguous(), keys, vals, scale=0.1,
                                    out_dtype=torch.float32)
    # different summation orders (decode splits the context over waves and
    # workgroups), each within ~2e-5 of the exact value
    assert torch.allclose(yp[:, :, -1], yd[:, :, 0], rtol=1e-4, atol=1e-4)
    # identical keys: every visible token has the same score, so position i
    # returns the mean of V over its N-L+i+1 visible tokens
    kc1 = np.repeat(kc[:, :, :1], n, axis=2)
    ks1 = np.repeat(ks[:, :, :1], n, axis=2)
    keys1 = (torch.from_numpy(kc1).to(gpu), torch.from_numpy(ks1.view(np.float16)).to(gpu))
    y = sparkq.int8_quantized_sdpa(qt, keys1, vals, scale=0.1, mask="causal",
                                   out_dtype=torch.float32).cpu().numpy()
    vd = o.kv_dequantize_s8(vc, vs).astype(np.float64)
    for i in (0, length // 2, length - 1):
        mean = vd[:, :, : n - length + i + 1].mean(axis=2)
        assert np.allclose(y[:, :, i], np.repeat(mean, hq // hkv, axis=1), rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------------------
# prefill over the MLX affine 8-bit cache
# ---------------------------------------------------------------------------
def _affine_cache(dev, b, hkv, n, d, g, seed, qdtype):
    k = o.randn(seed, 61, b * hkv * n * d).reshape(b, hkv, n, d)
    v = o.randn(seed, 62, b * hkv * n * d).reshape(b, hkv, n, d)
    kq = o.kv_quantize_affine_u8(k, g, qdtype)
    vq = o.kv_quantize_affine_u8(v, g, qdtype)

    def dev_tuple(t):
        packed, s, bias = t
        return (torch.from_numpy(packed.view(np.int32)).to(dev), up16(s, qdtype, dev),
                up16(bias, qdtype, dev))

    kd = o.kv_dequantize_affine_u8(*kq, g, qdtype)
    vd = o.kv_dequantize_affine_u8(*vq, g, qdtype)
    return dev_tuple(kq), dev_tuple(vq), kd, vd


def _row_rel(out, ref):
    num = np.linalg.norm((out - ref).reshape(-1, ref.shape[-1]), axis=1)
    den = np.maximum(np.linalg.norm(ref.reshape(-1, ref.shape[-1]), axis=1), 1e-30)
    return float(np.max(num / den))


# K and V dequantized to the query dtype and the weights rounded to it for
# PV (the reference kernel's rounding points): with bf16 that is ~2^-9 per
# element, ~2.5e-3 relative L2 on N(0,1) data; fp16 ~2^-12
_AFF_TOL = {o.BF16: (5e-3, 3e-2), o.F16: (8e-4, 5e-3)}


@pytest.mark.parametrize("b,hq,hkv,length,n,d,g,causal,qdtype", [
    (1, 16, 4, 64, 64, 256, 32, True, o.BF16),
    (1, 16, 4, 200, 333, 256, 32, True, o.BF16),
    (2, 8, 2, 37, 100, 128, 64, True, o.F16),
    (1, 32, 8, 130, 300, 128, 32, False, o.BF16),
    (1, 4, 4, 45, 45, 64, 32, True, o.BF16),
    (1, 6, 2, 70, 96, 128, 128, True, o.F16),
    (2, 8, 1, 300, 300, 256, 64, True, o.F16),
    # 512 row tiles: paired causal tiles, and the unsplit unmasked grid
    (4, 32, 8, 512, 512, 64, 32, True, o.BF16),
    (4, 32, 8, 512, 600, 64, 64, False, o.BF16),
])
def test_prefill_affine_matches_oracle(gpu, b, hq, hkv, length, n, d, g, causal, qdtype):
    import sparkq

    seed = length + n + d
    keys, vals, kd, vd = _affine_cache(gpu, b, hkv, n, d, g, seed, qdtype)
    q16 = _x16(seed, 60, (b, hq, length, d), qdtype)
    qt = up16(q16, qdtype, gpu)
    scale = 1.0 / math.sqrt(d)
    mask = "causal" if causal else None
    print(f"[prefill_affine] b={b} hq={hq} hkv={hkv} L={length} N={n} D={d} G={g} "
          f"causal={causal} q={'bf16' if qdtype == o.BF16 else 'f16'}", flush=True)
    y32 = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=scale, group_size=g, mask=mask,
                                     out_dtype=torch.float32)
    y16 = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=scale, group_size=g, mask=mask)
    torch.cuda.synchronize()
    out = y32.cpu().numpy().astype(np.float64)
    # the oracle with the reference kernel's rounding points (K, V and the
    # softmax weights rounded to the query dtype)
    refr = o.sdpa_prefill_rounded(q16, kd, vd, scale, causal, qdtype)
    rl, rr, ma = rel_l2(out, refr), _row_rel(out, refr), max_abs(out, refr)
    print(f"  vs rounding-faithful oracle: rel_l2={rl:.3e} worst_row={rr:.3e} max_abs={ma:.3e}")
    assert rl <= 1e-3 and ma <= 2e-2
    # and against exact float64 attention, where the roundings themselves show
    ref = o.sdpa_prefill(o.bits_to_f32(q16, qdtype), kd, vd, scale, causal)
    rl, rr, ma = rel_l2(out, ref), _row_rel(out, ref), max_abs(out, ref)
    print(f"  vs exact oracle: rel_l2={rl:.3e} worst_row={rr:.3e} max_abs={ma:.3e}")
    tol_l2, tol_row = _AFF_TOL[qdtype]
    assert rl <= tol_l2 and rr <= tol_row and ma <= 2e-2
    # the 16-bit output is the fp32 result rounded once
    assert np.array_equal(down16(y16), o.round16(y32.cpu().numpy(), qdtype))


@pytest.mark.parametrize("d,g,qdtype", [(256, 32, o.BF16), (128, 64, o.F16), (64, 32, o.BF16)])
def test_prefill_affine_identical_keys_mean_of_values(gpu, d, g, qdtype):
    """Zero keys (scales and biases 0) give every visible token the score 0
    and the weight 1 exactly, so row i returns the mean of the dequantized
    (query-dtype) V over its N-L+i+1 visible tokens: pins the V operand
    layout and the causal limits."""
    import sparkq

    b, hq, hkv, length, n = 1, 8, 2, 40, 77
    keys, vals, kd, vd = _affine_cache(gpu, b, hkv, n, d, g, 7, qdtype)
    keys1 = (keys[0], torch.zeros_like(keys[1]), torch.zeros_like(keys[2]))
    q16 = _x16(7, 63, (b, hq, length, d), qdtype)
    y = sparkq.int8_quantized_sdpa(up16(q16, qdtype, gpu), keys1, vals, scale=0.1, group_size=g,
                                   mask="causal", out_dtype=torch.float32).cpu().numpy()
    v16 = o.bits_to_f32(o.round16(vd, qdtype), qdtype).astype(np.float64)
    for i in range(length):
        mean = v16[:, :, : n - length + i + 1].mean(axis=2)
        assert np.allclose(y[:, :, i], np.repeat(mean, hq // hkv, axis=1), rtol=1e-5, atol=1e-6), i


@pytest.mark.parametrize("b,hq,hkv,length,n,d", [(1, 16, 4, 300, 900, 256), (1, 32, 8, 70, 2000, 128)])
def test_prefill_affine_split_repeats(gpu, b, hq, hkv, length, n, d):
    """Short prompts over long caches split each row tile's context over
    several workgroups, merged in the same launch by the last to finish: the
    result matches the oracle and repeats bit for bit (the tile counters are
    left zero for the next call)."""
    import sparkq

    lib = sparkq._lib.lib()
    assert lib.sparkq_int8kv_sdpa_prefill_affine_workspace_bytes(b, hq, hkv, length, n, d, 1) > 0
    keys, vals, kd, vd = _affine_cache(gpu, b, hkv, n, d, 32, 11, o.BF16)
    q16 = _x16(11, 65, (b, hq, length, d))
    qt = up16(q16, o.BF16, gpu)
    y1 = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=0.08, mask="causal", out_dtype=torch.float32)
    y2 = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=0.08, mask="causal", out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    out = y1.cpu().numpy().astype(np.float64)
    # the splits' partials merge exactly (integer offsets, power-of-two
    # factors), so the split result meets the rounding-faithful oracle too
    refr = o.sdpa_prefill_rounded(q16, kd, vd, 0.08, True, o.BF16)
    assert rel_l2(out, refr) <= 1e-3 and max_abs(out, refr) <= 2e-2
    ref = o.sdpa_prefill(o.bits_to_f32(q16, o.BF16), kd, vd, 0.08, True)
    assert rel_l2(out, ref) <= _AFF_TOL[o.BF16][0] and _row_rel(out, ref) <= _AFF_TOL[o.BF16][1]


@pytest.mark.parametrize("fmt,b,hq,hkv,length,n,d", [
    ("s8", 2, 32, 8, 257, 257, 128), ("s8", 1, 32, 8, 100, 300, 128), ("s8", 1, 16, 2, 40, 129, 256),
    ("affine_u8", 4, 32, 8, 512, 512, 64), ("affine_u8", 1, 32, 8, 70, 2000, 128),
    ("affine_u8", 2, 8, 2, 37, 100, 128)])
def test_prefill_xcd_order_identical(gpu, fmt, b, hq, hkv, length, n, d, monkeypatch):
    """The XCD-grouped work order of both prefill kernels (the row tiles of
    one (sequence, KV head) dispatched to one XCD) changes no row's
    arithmetic: identical outputs with and without it, for grids whose size
    is and is not a multiple of eight, paired causal tiles and context
    splits."""
    import sparkq

    print(f"[prefill xcd] {fmt} b={b} hq={hq} hkv={hkv} L={length} N={n} D={d}", flush=True)
    q = up16(_x16(n + d, 70, (b, hq, length, d)), o.BF16, gpu)
    if fmt == "s8":
        kc, ks = o.kv_quantize_s8(o.randn(n, 71, b * hkv * n * d).reshape(b, hkv, n, d))
        vc, vs = o.kv_quantize_s8(o.randn(n, 72, b * hkv * n * d).reshape(b, hkv, n, d))
        keys = (torch.from_numpy(kc).to(gpu), torch.from_numpy(ks.view(np.float16)).to(gpu))
        vals = (torch.from_numpy(vc).to(gpu), torch.from_numpy(vs.view(np.float16)).to(gpu))
        group = {}
    else:
        keys, vals, _, _ = _affine_cache(gpu, b, hkv, n, d, 32, n + d, o.BF16)
        group = {"group_size": 32}
    run = lambda: sparkq.int8_quantized_sdpa(q, keys, vals, scale=0.09, mask="causal",  # noqa: E731
                                             out_dtype=torch.float32, **group)
    y = run()
    monkeypatch.setenv("SPARKQ_PREFILL_NO_XCD", "1")
    assert torch.equal(y, run())


def test_prefill_affine_dispatch(gpu):
    """dispatch_sdpa routes multi-token queries over the affine tuple to the
    fused kernel when fused_quantized_sdpa_prefill is set."""
    import sparkq
    from sparkq.ops import SDPAConfig, dispatch_sdpa

    class Cache:
        bits, group_size = 8, 32

    keys, vals, _, _ = _affine_cache(gpu, 1, 4, 96, 256, 32, 9, o.BF16)
    qt = up16(_x16(9, 64, (1, 16, 50, 256)), o.BF16, gpu)
    y = dispatch_sdpa(qt, keys, vals, cache=Cache(), scale=0.0625, mask="causal",
                      config=SDPAConfig(fused_quantized_sdpa_prefill=True))
    ref = sparkq.int8_quantized_sdpa(qt, keys, vals, scale=0.0625, mask="causal")
    assert torch.equal(y, ref)
