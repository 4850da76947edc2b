"""GPU parity of the INT8-KV decode attention against the fp64 oracle, for
both KV formats (symmetric s8 + fp16 scale, MLX affine u8 tuple), plus the
device KV quantizer bit-exact."""

import math

import numpy as np
import pytest
import torch

import oracle as o
from helpers import TORCH16, check_fp32, check_rounded16, down16, up16, up32

pytestmark = pytest.mark.gpu


def _problem(b, hq, hkv, n, d, seed=0, qdtype=o.BF16):
    q16 = o.randn16(seed, 1, b * hq * d, 1.0, qdtype).reshape(b, hq, d)
    k = o.randn(seed, 2, b * hkv * n * d).reshape(b, hkv, n, d)
    v = o.randn(seed, 3, b * hkv * n * d).reshape(b, hkv, n, d)
    return q16, k, v


def _run_s8(dev, q16, kc, ks, vc, vs, scale, qdtype=o.BF16, out_dtype=None):
    import sparkq

    q = up16(q16[:, :, None, :], qdtype, dev)
    keys = (torch.from_numpy(kc).to(dev), torch.from_numpy(ks.view(np.float16)).to(dev))
    vals = (torch.from_numpy(vc).to(dev), torch.from_numpy(vs.view(np.float16)).to(dev))
    return sparkq.int8_quantized_sdpa(q, keys, vals, scale=scale, out_dtype=out_dtype)


@pytest.mark.parametrize("b,hq,hkv,n,d", [
    (1, 32, 8, 1, 128), (1, 32, 8, 5, 128), (1, 32, 8, 63, 128), (1, 32, 8, 64, 128),
    (1, 32, 8, 65, 128), (2, 32, 8, 1000, 128), (1, 32, 8, 4096, 128), (3, 8, 8, 300, 64),
    (1, 16, 2, 777, 256), (2, 16, 8, 129, 128)])
def test_s8_decode(gpu, b, hq, hkv, n, d):
    q16, k, v = _problem(b, hq, hkv, n, d, seed=n)
    kc, ks = o.kv_quantize_s8(k)
    vc, vs = o.kv_quantize_s8(v)
    scale = 1.0 / math.sqrt(d)
    ref = o.sdpa_decode(o.bits_to_f32(q16, o.BF16), o.kv_dequantize_s8(kc, ks),
                        o.kv_dequantize_s8(vc, vs), scale)
    y32 = _run_s8(gpu, q16, kc, ks, vc, vs, scale, out_dtype=torch.float32)
    check_fp32(y32.cpu().numpy().reshape(b, hq, d), ref)
    y16 = _run_s8(gpu, q16, kc, ks, vc, vs, scale)
    check_rounded16(down16(y16).reshape(b, hq, d), ref, o.BF16)


def test_s8_single_token_returns_value_row(gpu):
    b, hq, hkv, n, d = 2, 32, 8, 1, 128
    q16, k, v = _problem(b, hq, hkv, n, d, seed=4)
    kc, ks = o.kv_quantize_s8(k)
    vc, vs = o.kv_quantize_s8(v)
    y = _run_s8(gpu, q16, kc, ks, vc, vs, 0.088, out_dtype=torch.float32).cpu().numpy()
    vrow = np.repeat(o.kv_dequantize_s8(vc, vs)[:, :, 0], hq // hkv, axis=1)
    assert np.allclose(y.reshape(b, hq, d), vrow, rtol=1e-6, atol=1e-6)


def test_s8_strided_cache_view(gpu):
    """A cache allocated for 512 tokens holding 300: the kernel reads the view."""
    import sparkq

    b, hq, hkv, n, cap, d = 2, 32, 8, 300, 512, 128
    q16, k, v = _problem(b, hq, hkv, cap, d, seed=8)
    kc, ks = o.kv_quantize_s8(k)
    vc, vs = o.kv_quantize_s8(v)
    scale = 1.0 / math.sqrt(d)
    kt = torch.from_numpy(kc).to(gpu)[:, :, :n]
    vt = torch.from_numpy(vc).to(gpu)[:, :, :n]
    kst = torch.from_numpy(ks.view(np.float16)).to(gpu)[:, :, :n]
    vst = torch.from_numpy(vs.view(np.float16)).to(gpu)[:, :, :n]
    y = sparkq.int8_quantized_sdpa(up16(q16[:, :, None], o.BF16, gpu), (kt, kst), (vt, vst),
                                   scale=scale, out_dtype=torch.float32)
    ref = o.sdpa_decode(o.bits_to_f32(q16, o.BF16), o.kv_dequantize_s8(kc, ks)[:, :, :n],
                        o.kv_dequantize_s8(vc, vs)[:, :, :n], scale)
    check_fp32(y.cpu().numpy().reshape(b, hq, d), ref)


@pytest.mark.parametrize("qdtype", [o.BF16, o.F16])
@pytest.mark.parametrize("d,g,hq,hkv,n", [(256, 32, 16, 4, 1500), (128, 64, 32, 8, 200),
                                          (128, 128, 8, 1, 70), (64, 32, 4, 2, 33)])
def test_affine_u8_decode(gpu, d, g, hq, hkv, n, qdtype):
    import sparkq

    b = 2
    q16, k, v = _problem(b, hq, hkv, n, d, seed=d + g, qdtype=qdtype)
    kp, ks, kb = o.kv_quantize_affine_u8(k, g, qdtype)
    vp, vs, vb = o.kv_quantize_affine_u8(v, g, qdtype)
    scale = 1.0 / math.sqrt(d)
    ref = o.sdpa_decode(o.bits_to_f32(q16, qdtype),
                        o.kv_dequantize_affine_u8(kp, ks, kb, g, qdtype),
                        o.kv_dequantize_affine_u8(vp, vs, vb, g, qdtype), scale)
    keys = (up32(kp, gpu), up16(ks, qdtype, gpu), up16(kb, qdtype, gpu))
    vals = (up32(vp, gpu), up16(vs, qdtype, gpu), up16(vb, qdtype, gpu))
    q = up16(q16[:, :, None, :], qdtype, gpu)
    y = sparkq.int8_quantized_sdpa(q, keys, vals, scale=scale, group_size=g,
                                   out_dtype=torch.float32)
    check_fp32(y.cpu().numpy().reshape(b, hq, d), ref)
    y16 = sparkq.int8_quantized_sdpa(q, keys, vals, scale=scale, group_size=g)
    assert y16.dtype == TORCH16[qdtype]
    check_rounded16(down16(y16).reshape(b, hq, d), ref, qdtype)


def test_kv_quantizer_bit_exact(gpu):
    import sparkq

    x16 = o.randn16(9, 9, 64 * 128, 1.0, o.BF16).reshape(64, 128)
    x16[5] = 0
    codes, sc = sparkq.kv_quantize_s8(up16(x16, o.BF16, gpu))
    rc, rs = o.kv_quantize_s8(o.bits_to_f32(x16, o.BF16))
    assert np.array_equal(codes.cpu().numpy(), rc)
    assert np.array_equal(sc.cpu().numpy().view(np.uint16), rs)


@pytest.mark.parametrize("b,n", [(1, 4096), (1, 32768), (8, 4096), (8, 32768)])
def test_benchmark_shapes_sampled_heads(gpu, b, n):
    """Full kernels at benchmark sizes; oracle on two KV heads."""
    hq, hkv, d = 32, 8, 128
    g = torch.Generator(device="cpu").manual_seed(n)
    k = torch.randn((b, hkv, n, d), generator=g)
    v = torch.randn((b, hkv, n, d), generator=g)
    q = torch.randn((b, hq, 1, d), generator=g).to(torch.bfloat16)
    kc, ks = o.kv_quantize_s8(k.numpy())
    vc, vs = o.kv_quantize_s8(v.numpy())
    scale = 1.0 / math.sqrt(d)
    q16 = q.view(torch.int16).numpy().view(np.uint16).reshape(b, hq, d)
    y = _run_s8(gpu, q16, kc, ks, vc, vs, scale, out_dtype=torch.float32).cpu().numpy()
    y = y.reshape(b, hq, d)
    for kh in (0, hkv - 1):
        sl = slice(kh * 4, kh * 4 + 4)
        ref = o.sdpa_decode(o.bits_to_f32(q16[:, sl], o.BF16),
                            o.kv_dequantize_s8(kc[:, kh:kh + 1], ks[:, kh:kh + 1]),
                            o.kv_dequantize_s8(vc[:, kh:kh + 1], vs[:, kh:kh + 1]), scale)
        check_fp32(y[:, sl], ref)


def test_host_cache_tensors_raise_before_launch(gpu):
    """Every cache tensor (codes, scales, biases) and the mask must live on the
    device: a host scales tensor raises ValueError instead of reaching a
    kernel as a host pointer."""
    import sparkq

    b, hq, hkv, n, d, g = 1, 8, 2, 40, 128, 32
    q16, k, v = _problem(b, hq, hkv, n, d, seed=1)
    kc, ks = o.kv_quantize_s8(k)
    vc, vs = o.kv_quantize_s8(v)
    q = up16(q16[:, :, None, :], o.BF16, gpu)
    kt, vt = torch.from_numpy(kc).to(gpu), torch.from_numpy(vc).to(gpu)
    kst = torch.from_numpy(ks.view(np.float16))
    vst = torch.from_numpy(vs.view(np.float16)).to(gpu)
    with pytest.raises(ValueError, match="GPU"):
        sparkq.int8_quantized_sdpa(q, (kt, kst), (vt, vst), scale=0.1)
    kp, aks, akb = o.kv_quantize_affine_u8(k, g, o.BF16)
    vp, avs, avb = o.kv_quantize_affine_u8(v, g, o.BF16)
    keys = (up32(kp, gpu), up16(aks, o.BF16, gpu), torch.from_numpy(akb.view(np.int16)).view(
        torch.bfloat16))
    vals = (up32(vp, gpu), up16(avs, o.BF16, gpu), up16(avb, o.BF16, gpu))
    with pytest.raises(ValueError, match="GPU"):    # fused decode
        sparkq.int8_quantized_sdpa(q, keys, vals, scale=0.1, group_size=g)
    keys = (keys[0], keys[1], up16(akb, o.BF16, gpu))
    mask = torch.ones((1, n), dtype=torch.bool)      # staged path, host mask is moved
    y = sparkq.int8_quantized_sdpa(q, keys, vals, scale=0.1, group_size=g, mask=mask)
    assert y.device.type == "cuda"
