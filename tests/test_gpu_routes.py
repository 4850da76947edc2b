"""GPU execution of the dispatch routes that select a kernel by configuration
and shape: the W4 projection backends of LinearConfig.w4_qmv_backend
(spark_mlx_llm/ops/linear.py:84-94, 116-257), the direct multirow entry
point (X/spark_mlx_ext/w4a16_multirow.py:238-437), the derived prefill
buffer with its identity-keyed cache (ops/linear.py:260-268), and the L=1
fused route of dispatch_sdpa over both INT8 cache formats
(spark_mlx_llm/ops/sdpa.py:39-103). Each test asserts which callable the
route selected (a broken predicate would otherwise fall back to the native
projection unnoticed) and checks the result against the oracle."""

import math

import numpy as np
import pytest
import torch

import oracle as o
from helpers import check_fp32, check_rounded16, down16, up16, up32

pytestmark = pytest.mark.gpu

G = 64
PROJ = {"qkv": (3584, 2560), "down": (2560, 9728)}


@pytest.fixture(scope="module")
def layers(gpu):
    """The benchmark's QKV and down projections: N(0,0.02) bf16 weights
    quantized on the device (G64), as QuantizedLinear modules."""
    import sparkq
    from sparkq.ops import QuantizedLinear

    out = {}
    for name, (n, k) in PROJ.items():
        w16 = o.randn16(5, n, n * k, 0.02, o.BF16).reshape(n, k)
        wq, s, b = sparkq.affine_quantize(up16(w16, o.BF16, gpu), group_size=G)
        out[name] = QuantizedLinear(wq, s, b, group_size=G, bits=4)
    return out


def _sampled_oracle(layer, x16, cols):
    wq = layer.weight.cpu().numpy().view(np.uint32)[cols]
    s, b = down16(layer.scales)[cols], down16(layer.biases)[cols]
    return o.w4a16_matmul(x16, wq, s, b, G)


def _spy(monkeypatch, module, name, calls):
    orig = getattr(module, name)

    def wrapped(*args, **kwargs):
        calls.append(name)
        return orig(*args, **kwargs)

    monkeypatch.setattr(module, name, wrapped)


ROUTES = [("splitk", 1, "splitk", "w4a16_qmv"),
          ("multirow", 2, "multirow", "w4a16_multirow"),
          ("multirow", 8, "multirow", "w4a16_multirow"),
          ("multirow", 16, "multirow", "w4a16_multirow"),
          ("multirow_packed", 8, "multirow_packed", "w4a16_multirow"),
          # outside a backend's geometry the reference falls back to native
          ("splitk", 4, "native", "affine_quantized_matmul"),
          ("multirow", 1, "native", "affine_quantized_matmul")]


@pytest.mark.parametrize("proj", list(PROJ))
@pytest.mark.parametrize("backend,m,selected,entry", ROUTES)
def test_dispatch_linear_backend_routes(gpu, layers, monkeypatch, proj, backend, m, selected,
                                        entry):
    from sparkq import ext
    from sparkq.ops import AffineParameters, LinearConfig, dispatch_linear

    print(f"[case] route {backend} M={m} {proj}", flush=True)
    layer = layers[proj]
    n, k = PROJ[proj]
    x16 = o.randn16(0, 300 + m, m * k).reshape(m, k)
    x = up16(x16, o.BF16, gpu).reshape(1, m, k)
    config = LinearConfig(w4_qmv_backend=backend)
    project, params = AffineParameters.resolve(layer, x.shape, x.dtype, config)
    assert project is getattr(AffineParameters, selected)
    assert params.prepared is None
    calls = []
    _spy(monkeypatch, ext, entry, calls)
    y = dispatch_linear(x, layer, config=config)
    assert calls == [entry], calls
    assert y.shape == (1, m, n) and y.dtype == torch.bfloat16
    # every route reaches the same kernel as the native projection
    native = AffineParameters.native(x, *AffineParameters.from_module(layer))
    assert torch.equal(y, native)
    cols = np.sort(np.random.default_rng(m).choice(n, size=192, replace=False))
    ref = _sampled_oracle(layer, x16, cols)
    check_rounded16(down16(y.reshape(m, n))[:, cols], ref, o.BF16)


@pytest.mark.parametrize("algorithm", ["wide", "nax4", "p2"])
def test_w4a16_multirow_direct(gpu, layers, algorithm):
    """ext.w4a16_multirow at 8 rows (the reference's verify geometry) with
    its tuning keywords, against the oracle."""
    import sparkq

    layer = layers["qkv"]
    n, k = PROJ["qkv"]
    m = 8
    x16 = o.randn16(1, 400, m * k).reshape(m, k)
    y = sparkq.w4a16_multirow(up16(x16, o.BF16, gpu), layer.weight, layer.scales,
                              layer.biases, algorithm=algorithm, k_lanes=8, simdgroups=8)
    assert y.shape == (m, n)
    cols = np.sort(np.random.default_rng(8).choice(n, size=256, replace=False))
    check_rounded16(down16(y)[:, cols], _sampled_oracle(layer, x16, cols), o.BF16)


@pytest.mark.parametrize("proj", list(PROJ))
def test_prefill_route_uses_prepared_buffer(gpu, layers, monkeypatch, proj):
    """More than 32 rows: resolve attaches the layer's derived buffer, made
    once per weight set and reused; the prepared GEMM call equals the
    unprepared one bit for bit; replacing or modifying a source tensor
    rebuilds it."""
    import sparkq
    from sparkq import ext
    from sparkq.ops import AffineParameters, LinearConfig, dispatch_linear, prepare_w4_layers

    layer = layers[proj]
    n, k = PROJ[proj]
    m = 64
    x16 = o.randn16(2, 500, m * k).reshape(m, k)
    x = up16(x16, o.BF16, gpu)
    calls = []
    _spy(monkeypatch, ext, "prepare_w4a16", calls)
    config = LinearConfig(w4_qmv_backend="splitk")
    project, params = AffineParameters.resolve(layer, x.shape, x.dtype, config)
    assert project is AffineParameters.native and params.prepared is not None
    again = AffineParameters.resolve(layer, x.shape, x.dtype, config)[1].prepared
    assert again is params.prepared and calls == ["prepare_w4a16"]
    y = dispatch_linear(x, layer, config=config)
    y_module = layer(x)                            # QuantizedLinear.forward, native backend
    plain = sparkq.affine_quantized_matmul(x, layer.weight, layer.scales, layer.biases,
                                           group_size=G)
    assert torch.equal(y, plain) and torch.equal(y_module, plain)
    assert calls == ["prepare_w4a16"]
    y32 = sparkq.affine_quantized_matmul(x, layer.weight, layer.scales, layer.biases,
                                         group_size=G, out_dtype=torch.float32,
                                         prepared=params.prepared)
    cols = np.sort(np.random.default_rng(3).choice(n, size=128, replace=False))
    check_fp32(y32.cpu().numpy()[:, cols], _sampled_oracle(layer, x16, cols))
    # in-place change of the scales: the cache notices and rebuilds
    old = params.prepared
    layer.scales.mul_(2)
    try:
        fresh = AffineParameters.resolve(layer, x.shape, x.dtype, config)[1].prepared
        assert fresh is not old and calls == ["prepare_w4a16"] * 2
        y2 = layer(x)
        plain2 = sparkq.affine_quantized_matmul(x, layer.weight, layer.scales, layer.biases,
                                                group_size=G)
        assert torch.equal(y2, plain2)
    finally:
        layer.scales.div_(2)
    assert prepare_w4_layers(torch.nn.ModuleList([layer])) == 1


def test_prepared_buffer_validation(gpu, layers):
    import sparkq

    layer = layers["qkv"]
    n, k = PROJ["qkv"]
    prep = sparkq.prepare_w4a16(layer.weight, layer.scales, layer.biases)
    x = torch.zeros((40, k), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="prepared"):
        sparkq.affine_quantized_matmul(x, layer.weight, layer.scales, layer.biases,
                                       group_size=G, prepared=prep[:100])
    # fp16 scales have no prepared form
    assert sparkq.prepare_w4a16(layer.weight, layer.scales.half(), layer.biases.half()) is None


# ---------------------------------------------------------------------------
# dispatch_sdpa at L = 1: the fused decode route over both cache formats
# ---------------------------------------------------------------------------

class _Cache:
    def __init__(self, bits, group_size):
        self.bits, self.group_size = bits, group_size


@pytest.mark.parametrize("fmt", ["s8", "affine_u8"])
@pytest.mark.parametrize("n", [1000, 4096])
def test_dispatch_sdpa_fused_decode_route(gpu, monkeypatch, fmt, n):
    """The decode benchmark's geometry (B=1, 32 query / 8 KV heads, D=128)
    through dispatch_sdpa: the fused predicate holds, the fused decode runs
    (not the staged kernel), and the result matches the fp64 oracle."""
    from sparkq import ext
    from sparkq.ops import SDPAConfig, dispatch_sdpa
    from sparkq.ops import sdpa as sdpa_mod

    b, hq, hkv, d, g = 1, 32, 8, 128, 32
    print(f"[case] dispatch_sdpa L=1 {fmt} N={n}", flush=True)
    q16 = o.randn16(n, 1, b * hq * d, 1.0, o.BF16).reshape(b, hq, 1, d)
    k = o.randn(n, 2, b * hkv * n * d).reshape(b, hkv, n, d)
    v = o.randn(n, 3, b * hkv * n * d).reshape(b, hkv, n, d)
    if fmt == "s8":
        kc, ks = o.kv_quantize_s8(k)
        vc, vs = o.kv_quantize_s8(v)
        keys = (torch.from_numpy(kc).to(gpu), torch.from_numpy(ks.view(np.float16)).to(gpu))
        vals = (torch.from_numpy(vc).to(gpu), torch.from_numpy(vs.view(np.float16)).to(gpu))
        kd, vd = o.kv_dequantize_s8(kc, ks), o.kv_dequantize_s8(vc, vs)
    else:
        kp, ks, kb = o.kv_quantize_affine_u8(k, g, o.BF16)
        vp, vs, vb = o.kv_quantize_affine_u8(v, g, o.BF16)
        keys = (up32(kp, gpu), up16(ks, o.BF16, gpu), up16(kb, o.BF16, gpu))
        vals = (up32(vp, gpu), up16(vs, o.BF16, gpu), up16(vb, o.BF16, gpu))
        kd = o.kv_dequantize_affine_u8(kp, ks, kb, g, o.BF16)
        vd = o.kv_dequantize_affine_u8(vp, vs, vb, g, o.BF16)
    q = up16(q16, o.BF16, gpu)
    cache = _Cache(8, g)
    scale = 1.0 / math.sqrt(d)
    assert sdpa_mod._supports_int8(q, keys, vals, cache=cache, mask=None)
    calls = []
    for mod, name in ((sdpa_mod, "_int8_attention"), (sdpa_mod, "_quantized_attention"),
                      (ext, "_decode"), (ext, "_staged_attention")):
        _spy(monkeypatch, mod, name, calls)
    y = dispatch_sdpa(q, keys, vals, cache=cache, scale=scale, mask=None, config=SDPAConfig())
    assert calls == ["_int8_attention", "_decode"], calls
    ref = o.sdpa_decode(o.bits_to_f32(q16[:, :, 0], o.BF16), kd, vd, scale)
    check_rounded16(down16(y).reshape(b, hq, d), ref, o.BF16)
    # the causal mask string keeps the fused route; disabling it in the
    # config sends the tuple to the staged kernel (the reference's mlx-lm path)
    calls.clear()
    yc = dispatch_sdpa(q, keys, vals, cache=cache, scale=scale, mask="causal")
    assert calls == ["_int8_attention", "_decode"] and torch.equal(yc, y)
    if fmt == "affine_u8":
        calls.clear()
        ys = dispatch_sdpa(q, keys, vals, cache=cache, scale=scale, mask=None,
                           config=SDPAConfig(fused_quantized_sdpa=False))
        assert calls == ["_quantized_attention", "_staged_attention"], calls
        check_fp32(ys.float().cpu().numpy().reshape(b, hq, d), ref, atol=2e-2, rtol_l2=5e-3)


def test_dispatch_sdpa_prefill_flag_routes(gpu, monkeypatch):
    """Multi-token queries over the affine tuple: the fused prefill kernel
    only with fused_quantized_sdpa_prefill (opt-in, as in the reference),
    the staged kernel otherwise; both match the fp64 staged oracle."""
    from sparkq import ext
    from sparkq.ops import SDPAConfig, dispatch_sdpa
    from sparkq.ops import sdpa as sdpa_mod

    b, hq, hkv, length, n, d, g = 1, 16, 4, 8, 300, 128, 32
    k = o.randn(11, 2, b * hkv * n * d).reshape(b, hkv, n, d)
    v = o.randn(11, 3, b * hkv * n * d).reshape(b, hkv, n, d)
    kp, ks, kb = o.kv_quantize_affine_u8(k, g, o.BF16)
    vp, vs, vb = o.kv_quantize_affine_u8(v, g, o.BF16)
    keys = (up32(kp, gpu), up16(ks, o.BF16, gpu), up16(kb, o.BF16, gpu))
    vals = (up32(vp, gpu), up16(vs, o.BF16, gpu), up16(vb, o.BF16, gpu))
    q16 = o.randn16(11, 1, b * hq * length * d, 1.0, o.BF16).reshape(b, hq, length, d)
    q = up16(q16, o.BF16, gpu)
    scale = d ** -0.5
    ref = o.sdpa_staged(o.bits_to_f32(q16, o.BF16),
                        o.kv_dequantize_affine_u8(kp, ks, kb, g, o.BF16),
                        o.kv_dequantize_affine_u8(vp, vs, vb, g, o.BF16), scale, "causal")
    calls = []
    for mod, name in ((sdpa_mod, "_int8_attention"), (sdpa_mod, "_quantized_attention"),
                      (ext, "_int8_prefill_affine"), (ext, "_staged_attention")):
        _spy(monkeypatch, mod, name, calls)
    cache = _Cache(8, g)
    y = dispatch_sdpa(q, keys, vals, cache=cache, scale=scale, mask="causal")
    assert calls == ["_quantized_attention", "_staged_attention"], calls
    check_fp32(y.float().cpu().numpy(), ref, atol=2e-2, rtol_l2=5e-3)
    calls.clear()
    yf = dispatch_sdpa(q, keys, vals, cache=cache, scale=scale, mask="causal",
                       config=SDPAConfig(fused_quantized_sdpa_prefill=True))
    assert calls == ["_int8_attention", "_int8_prefill_affine"], calls
    check_fp32(yf.float().cpu().numpy(), ref, atol=2e-2, rtol_l2=5e-3)
