"""CPU tests of the host layer: configuration contracts, dispatch predicates
and the validation the operators perform before any device call."""

import pytest
import torch

import sparkq
from sparkq import ext
from sparkq.ops import (AffineParameters, LinearConfig, QuantizedLinear, SDPAConfig,
                        dispatch_linear, dispatch_sdpa)
from sparkq.ops.linear import unpack_affine_w8


def test_linear_config_contract():
    assert LinearConfig().w4_qmv_backend == "native"
    assert LinearConfig.choices("w4_qmv_backend") == ("native", "splitk", "multirow",
                                                       "multirow_packed")
    assert LinearConfig.choices("w8_qmv_backend") == ("auto", "native", "w8a16", "w8a8",
                                                       "multirow")
    with pytest.raises(ValueError, match="must be one of"):
        LinearConfig(w4_qmv_backend="fast")
    with pytest.raises(ValueError, match="renamed"):
        LinearConfig.validate_values({"qmv_backend": "native"})
    cfg = LinearConfig.from_dict({"w4_qmv_backend": "splitk", "hidden_size": 2560})
    assert cfg.w4_qmv_backend == "splitk"


def test_sdpa_config_contract():
    with pytest.raises(ValueError, match="boolean"):
        SDPAConfig.validate_values({"fused_quantized_sdpa": 1})
    assert SDPAConfig().fused_quantized_sdpa is True


def _layer(n=64, k=256, g=64):
    wq = torch.zeros((n, k // 8), dtype=torch.int32)
    s = torch.ones((n, k // g), dtype=torch.bfloat16)
    b = torch.zeros((n, k // g), dtype=torch.bfloat16)
    return QuantizedLinear(wq, s, b, group_size=g, bits=4)


def test_affine_predicates_on_cpu_tensors_are_false():
    layer = _layer()
    p = AffineParameters.from_module(layer)
    assert AffineParameters.accepts(layer)
    assert not AffineParameters.supports_splitk((1, 256), torch.bfloat16, *p)
    assert not AffineParameters.supports_multirow((1, 8, 256), torch.bfloat16, *p)
    # the native projection runs only on the device: no CPU fallback
    with pytest.raises(ValueError, match="GPU"):
        dispatch_linear(torch.zeros((1, 256), dtype=torch.bfloat16), layer,
                        config=LinearConfig(w4_qmv_backend="splitk"))


def test_affine_validation_errors():
    wq = torch.zeros((64, 32), dtype=torch.int32)
    s = torch.ones((64, 4), dtype=torch.bfloat16)
    x = torch.zeros((2, 256), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="exactly one activation row"):
        ext.w4a16_qmv(x, wq, s, s)
    with pytest.raises(ValueError, match="BF16 or F16"):
        ext.affine_quantized_matmul(x.float(), wq, s, s, group_size=64)
    with pytest.raises(ValueError, match="UINT32"):
        ext.affine_quantized_matmul(x, wq.float(), s, s, group_size=64)
    with pytest.raises(ValueError, match="shape"):
        ext.affine_quantized_matmul(x, wq, s[:, :2], s[:, :2], group_size=64)
    with pytest.raises(TypeError):
        ext.w4a16_qmv(x[:1], None, s, s)
    with pytest.raises(ValueError, match="algorithm"):
        ext.w4a16_multirow(x, wq, s, s, algorithm="nope")


def test_w8a8_validation_errors():
    w = torch.zeros((16, 64), dtype=torch.int8)
    sc = torch.ones(16)
    with pytest.raises(ValueError, match="matching K"):
        ext.w8a8_linear(torch.zeros((1, 32)), w, sc)
    with pytest.raises(ValueError, match="multiple of 32"):
        ext.w8a8_linear(torch.zeros((1, 48)), torch.zeros((16, 48), dtype=torch.int8), sc)
    with pytest.raises(ValueError, match="scales"):
        ext.w8a8_linear(torch.zeros((1, 64)), w, sc.double())
    with pytest.raises(ValueError, match="INT8"):
        ext.W8A8Linear(w.float(), sc)
    with pytest.raises(ValueError, match="int8"):
        ext.int8_matmul_int32(torch.zeros((1, 64)), w)


def test_unpack_affine_w8_on_host():
    # unsigned codes 0,128,255,1 -> signed -128,0,127,-127; scale repeated, bias -128*s
    words = torch.tensor([[0x01FF8000]], dtype=torch.int32)
    s = torch.full((1, 1), 0.5, dtype=torch.bfloat16)
    b = torch.full((1, 1), -64.0, dtype=torch.bfloat16)
    w8, sc = unpack_affine_w8(words, s, b, group_size=4)
    assert w8.tolist() == [[-128, 0, 127, -127]] and sc.tolist() == [0.5]
    with pytest.raises(ValueError, match="biases=-128"):
        unpack_affine_w8(words, s, torch.zeros_like(b), group_size=4)
    assert unpack_affine_w8(words, s, torch.zeros_like(b), group_size=4,
                            allow_fallback=True) is None


def test_sdpa_dispatch_validation():
    class Cache:
        bits, group_size = 8, 32

    q = torch.zeros((1, 8, 1, 128))
    keys = (torch.zeros((1, 2, 16, 128), dtype=torch.int8), torch.ones((1, 2, 16), dtype=torch.float16))
    # CPU tensors never take the fused route; a quantized cache then goes to
    # the staged kernel, which (like every sparkq operator) runs only on the GPU
    with pytest.raises(ValueError, match="GPU"):
        dispatch_sdpa(q, keys, keys, cache=Cache(), scale=0.1, mask=None)
    with pytest.raises(ValueError, match="single_pass_max_length"):
        ext.int8_quantized_sdpa(q, keys, keys, scale=0.1, single_pass_max_length=-1)
    with pytest.raises(ValueError, match="finite"):
        ext.int8_quantized_sdpa(q, keys, keys, scale=float("nan"))
    # multi-token queries: 16-bit queries, L <= N under a causal mask; the
    # affine tuple needs bits 8, G in 32/64/128 and metadata in the query dtype
    with pytest.raises(ValueError, match="float16 or bfloat16 queries"):
        ext.int8_quantized_sdpa(torch.zeros((1, 8, 2, 128)), keys, keys, scale=0.1)
    q2 = torch.zeros((1, 8, 32, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="L <= N"):
        ext.int8_quantized_sdpa(q2, keys, keys, scale=0.1, mask="causal")
    aff = (torch.zeros((1, 2, 16, 32), dtype=torch.int32), torch.ones((1, 2, 16, 4), dtype=torch.bfloat16),
           torch.zeros((1, 2, 16, 4), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="group size"):
        ext.int8_quantized_sdpa(q2[:, :, :2], aff, aff, scale=0.1, group_size=16)
    with pytest.raises(ValueError, match="Incompatible key packed"):
        ext.int8_quantized_sdpa(q2[:, :, :2], aff, aff, scale=0.1, group_size=64)
    # a head dim outside 64/128/256 is a staged-kernel shape, not an error
    aff96 = (torch.zeros((1, 2, 16, 24), dtype=torch.int32),
             torch.ones((1, 2, 16, 3), dtype=torch.bfloat16),
             torch.zeros((1, 2, 16, 3), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="GPU"):
        ext.int8_quantized_sdpa(torch.zeros((1, 8, 2, 96), dtype=torch.bfloat16),
                                aff96, aff96, scale=0.1)
    # 4-bit tuples: the packed width is D/8; bits 3 is not an MLX KV format
    aff4 = (torch.zeros((1, 2, 16, 16), dtype=torch.int32),
            torch.ones((1, 2, 16, 4), dtype=torch.bfloat16),
            torch.zeros((1, 2, 16, 4), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="GPU"):
        ext.int8_quantized_sdpa(q2[:, :, :2], aff4, aff4, scale=0.1, bits=4)
    with pytest.raises(ValueError, match="bits 2/4/8"):
        ext.int8_quantized_sdpa(q2[:, :, :2], aff4, aff4, scale=0.1, bits=3)
    with pytest.raises(ValueError, match="Incompatible key"):
        ext.int8_quantized_sdpa(q2[:, :, :2], aff4, aff4, scale=0.1, bits=8)
    with pytest.raises(ValueError, match="does not broadcast"):
        ext.int8_quantized_sdpa(q2[:, :, :2], aff4, aff4, scale=0.1, bits=4,
                                mask=torch.ones((3, 16), dtype=torch.bool))
    with pytest.raises(ValueError, match="GPU"):
        ext.int8_quantized_sdpa(q2[:, :, :2], aff, aff, scale=0.1)
    # unquantized caches take torch's attention
    out = dispatch_sdpa(torch.ones((1, 8, 1, 64)), torch.ones((1, 2, 5, 64)),
                        torch.ones((1, 2, 5, 64)), cache=None, scale=0.125, mask=None)
    assert torch.allclose(out, torch.ones_like(out))


def test_native_causal_mask_is_bottom_right():
    """mask='causal' over an unquantized cache that already holds tokens
    (L < S): query i sees tokens 0 .. S-L+i, as MLX aligns it, not torch's
    top-left is_causal."""
    from sparkq.ops.sdpa import causal_mask

    g = torch.Generator().manual_seed(0)
    b, hq, hkv, length, s, d = 1, 4, 2, 3, 7, 16
    q = torch.randn((b, hq, length, d), generator=g, dtype=torch.float64)
    k = torch.randn((b, hkv, s, d), generator=g, dtype=torch.float64)
    v = torch.randn((b, hkv, s, d), generator=g, dtype=torch.float64)
    out = dispatch_sdpa(q, k, v, cache=None, scale=0.25, mask="causal")
    # textbook: explicit loops over the visible tokens of each query
    kk, vv = k.repeat_interleave(2, dim=1), v.repeat_interleave(2, dim=1)
    ref = torch.empty_like(out)
    for h in range(hq):
        for i in range(length):
            visible = s - length + i + 1
            w = torch.softmax(0.25 * kk[0, h, :visible] @ q[0, h, i], dim=0)
            ref[0, h, i] = w @ vv[0, h, :visible]
    assert torch.allclose(out, ref, atol=1e-12)
    # the mask itself: last row sees everything, first row sees S-L+1 tokens
    m = causal_mask(length, s)
    assert m[-1].all() and int(m[0].sum()) == s - length + 1
    assert torch.equal(causal_mask(s, s), torch.ones((s, s), dtype=torch.bool).tril())
    # an explicit boolean mask array is passed through unchanged
    keep = torch.rand((length, s), generator=g) > 0.3
    keep[:, 0] = True
    out2 = dispatch_sdpa(q, k, v, cache=None, scale=0.25, mask=keep)
    sc = 0.25 * (q @ kk.transpose(-1, -2))
    ref2 = torch.softmax(sc.masked_fill(~keep, float("-inf")), -1) @ vv
    assert torch.allclose(out2, ref2, atol=1e-12)


def test_package_surface():
    for name in sparkq.__all__:
        assert callable(getattr(sparkq, name))
    assert sparkq.prepare_w4a16_nax4(1, 2, 3) == (1, 2, 3)


def test_w8a16_layer_contract():
    """W8A16PerChannelLinear (spark_mlx_llm/ops/linear.py:413-476): needs a
    bias-free affine W8 fallback and matching int8 [N,K] / fp32 [N] inputs;
    serves single 16-bit rows on the device only."""
    from sparkq.ops import W8A16PerChannelLinear

    n, k = 16, 64
    fb = QuantizedLinear(torch.zeros((n, k // 4), dtype=torch.int32),
                         torch.ones((n, k // 32), dtype=torch.bfloat16),
                         torch.full((n, k // 32), -128.0, dtype=torch.bfloat16),
                         group_size=32, bits=8)
    w8 = torch.zeros((n, k), dtype=torch.int8)
    sc = torch.ones(n, dtype=torch.float32)
    layer = W8A16PerChannelLinear(fb, w8, sc)
    assert layer.scales.shape == (n,)
    with pytest.raises(ValueError, match="matching signed INT8"):
        W8A16PerChannelLinear(fb, w8.to(torch.int16), sc)
    with pytest.raises(ValueError, match="matching signed INT8"):
        W8A16PerChannelLinear(fb, torch.zeros((n, k + 4), dtype=torch.int8), sc)
    with pytest.raises(ValueError, match="bias-free affine W8"):
        W8A16PerChannelLinear(_layer(), w8, sc)
    assert W8A16PerChannelLinear.supports_rows(1, torch.bfloat16)
    assert not W8A16PerChannelLinear.supports_rows(2, torch.bfloat16)
    assert not W8A16PerChannelLinear.supports_rows(1, torch.float32)
    assert not W8A16PerChannelLinear.supports_rows(1, torch.bfloat16,
                                                   torch.zeros(1, k, dtype=torch.bfloat16))


def test_quantized_kv_cache_contract():
    """QuantizedKVCache mirrors mlx-lm's interface: affine caches of 8, 4 or 2
    bits (mlx-lm's kv_bits) and the symmetric s8 format, capacity in steps of
    256; appends run on the device only."""
    with pytest.raises(ValueError, match="bits 2, 4 or 8"):
        sparkq.QuantizedKVCache(bits=3)
    with pytest.raises(ValueError, match="s8 format 8"):
        sparkq.QuantizedKVCache(bits=4, kv_format="s8")
    c4 = sparkq.QuantizedKVCache(bits=4, group_size=32)
    with pytest.raises(ValueError, match="GPU"):
        c4.update_and_fetch(torch.zeros((1, 2, 3, 96), dtype=torch.bfloat16),
                            torch.zeros((1, 2, 3, 96), dtype=torch.bfloat16))
    assert c4.keys[0].shape == (1, 2, 256, 12)  # 96 dims * 4 bits / 32
    with pytest.raises(ValueError, match="kv_format"):
        sparkq.QuantizedKVCache(kv_format="fp8")
    cache = sparkq.QuantizedKVCache(group_size=64)
    assert cache.offset == 0 and cache.step == 256 and cache.state == (None, None)
    x = torch.zeros((1, 2, 3, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        cache.update_and_fetch(x, x)
    with pytest.raises(ValueError, match="capacity"):
        ext.kv_append(x, (torch.zeros((1, 2, 2, 128), dtype=torch.int8),
                          torch.zeros((1, 2, 2), dtype=torch.float16)), 0)


def test_layer_dispatch_contract_on_host():
    """The FFN/QKV dispatchers keep the reference's module fallback for
    non-standard modules, and the kernels never run on CPU tensors."""
    from sparkq import ext
    from sparkq.ops import RMSNorm, RoPE, dispatch_ffn, dispatch_qkv

    calls = []

    class Custom(torch.nn.Module):
        def forward(self, h):
            calls.append(h.shape)
            return 2 * h

    x = torch.ones(1, 1, 8)
    a = torch.full((1, 1, 8), 0.5)
    # custom norm and MLP: module calls, hidden + mlp(norm(hidden))
    y = dispatch_ffn(x, a, lambda h: h + 1, Custom(), mlp_type=torch.nn.Linear)
    assert torch.equal(y, 1.5 + 2 * 2.5 * torch.ones(1, 1, 8)) and calls == [(1, 1, 8)]
    # the kernels refuse host tensors instead of computing elsewhere
    with pytest.raises(ValueError, match="GPU"):
        ext.rope(torch.zeros(1, 2, 3, 8, dtype=torch.bfloat16), 8)
    norm = RMSNorm(8, 1e-6, weight=torch.ones(8, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="GPU"):
        norm(torch.zeros(2, 8, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="x must have shape"):
        ext.spark_qkv_rope(torch.zeros(1, 2, 64, dtype=torch.bfloat16), None, None, None,
                           64, 16, 4, 1, 16, 16, 10000.0, 0, 64, 4)
    with pytest.raises(ValueError, match="Invalid head counts"):
        ext.spark_qkv_rope(torch.zeros(1, 1, 64, dtype=torch.bfloat16), None, None, None,
                           64, 16, 4, 3, 16, 16, 10000.0, 0, 64, 4)
    # a projection that is not an affine W4 module is called as a module
    proj = Custom()
    rope = RoPE(8)
    with pytest.raises(ValueError, match="GPU"):
        dispatch_qkv(torch.zeros(1, 2, 24, dtype=torch.bfloat16), proj, rope, q_size=8,
                     kv_size=8, n_heads=1, n_kv_heads=1, head_dim=8, offset=0)
    assert calls[-1] == (1, 2, 24)


def test_prepared_buffer_host_rules():
    """The derived prefill buffer: routed only for more than 32 bf16 rows on
    the device (never on host tensors), fp16 scales have no prepared form,
    and the operators reject a malformed buffer before any device call."""
    layer = _layer()
    p = AffineParameters.from_module(layer)
    assert p.prepared is None and len(p) == 6
    assert not AffineParameters.supports_prepared((64, 256), torch.bfloat16, *p)
    assert ext.prepare_w4a16(layer.weight, layer.scales.half(), layer.biases.half()) is None
    with pytest.raises(ValueError, match="GPU"):
        ext.prepare_w4a16(layer.weight, layer.scales, layer.biases)
    with pytest.raises(ValueError, match="group_size"):
        ext.prepare_w4a16(layer.weight, layer.scales, layer.biases, group_size=48)
    x = torch.zeros((64, 256), dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        ext.affine_quantized_matmul(x, layer.weight, layer.scales, layer.biases, group_size=64,
                                    prepared=torch.zeros(8, dtype=torch.uint8))
