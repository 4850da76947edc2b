"""The torch.library registration of the sparkq operators (host side): every
hot-path operator is a torch.ops.sparkq custom op whose fake kernel gives the
eager function's output shapes and dtypes, so that a decoder layer built from
them traces (here in fake mode on meta tensors; the real kernels run in
tests/test_gpu_torch_ops.py)."""

import pytest
import torch
from torch.fx.experimental.proxy_tensor import make_fx

import sparkq  # noqa: F401  (registers torch.ops.sparkq.*)

OPS = ["affine_quantized_matmul", "w8a8_linear", "w8a16_per_channel", "quantize_per_token",
       "int8_matmul_int32", "int8_sdpa_s8", "int8_sdpa_affine", "rms_norm", "rope", "qkv_rope",
       "fused_ffn", "attention_gate"]
M = "meta"
BF = torch.bfloat16


def t(*shape, dtype=BF):
    return torch.empty(shape, device=M, dtype=dtype)


def test_every_operator_is_registered():
    for name in OPS:
        assert hasattr(torch.ops.sparkq, name), name


@pytest.mark.parametrize("lead", [(1,), (4,), (2, 3), (2048,)])
def test_linear_fakes(lead):
    x = t(*lead, 2560)
    w4, s = t(3584, 320, dtype=torch.int32), t(3584, 40)
    assert torch.ops.sparkq.affine_quantized_matmul(x, w4, s, s, 64, 4, None).shape == (*lead, 3584)
    y = torch.ops.sparkq.affine_quantized_matmul(x, w4, s, s, 64, 4, torch.float32)
    assert y.dtype == torch.float32
    # bits=8 promotes x with the scales: fp32 scales (the W8 lm_head) give fp32
    w8p, s8 = t(3584, 640, dtype=torch.uint32), t(3584, 80, dtype=torch.float32)
    y8 = torch.ops.sparkq.affine_quantized_matmul(x, w8p, s8, s8, 32, 8, None)
    assert y8.shape == (*lead, 3584) and y8.dtype == torch.float32
    y8 = torch.ops.sparkq.affine_quantized_matmul(x, w8p, t(3584, 80), t(3584, 80), 32, 8, None)
    assert y8.dtype == BF
    w8, sw = t(512, 2560, dtype=torch.int8), t(512, dtype=torch.float32)
    assert torch.ops.sparkq.w8a8_linear(x, w8, sw, None, None).shape == (*lead, 512)
    q, sa = torch.ops.sparkq.quantize_per_token(x)
    m = 1
    for d in lead:
        m *= d
    assert q.shape == (m, 2560) and q.dtype == torch.int8 and sa.shape == (m,)
    assert torch.ops.sparkq.int8_matmul_int32(q, w8).dtype == torch.int32


def test_attention_fakes():
    q = t(2, 32, 1, 128)
    kc, ks = t(2, 8, 300, 128, dtype=torch.int8), t(2, 8, 300, dtype=torch.float16)
    out = torch.ops.sparkq.int8_sdpa_s8(q, kc, ks, kc, ks, 0.088, False, None)
    assert out.shape == (2, 32, 1, 128) and out.dtype == BF
    kp, sc = t(2, 8, 300, 32, dtype=torch.uint32), t(2, 8, 300, 4)
    out = torch.ops.sparkq.int8_sdpa_affine(q, kp, sc, sc, kp, sc, sc, 0.088, 32, 8, None, None,
                                            torch.float32)
    assert out.shape == (2, 32, 1, 128) and out.dtype == torch.float32
    # 4-bit values: 8 codes per word
    vp = t(2, 8, 300, 16, dtype=torch.uint32)
    out = torch.ops.sparkq.int8_sdpa_affine(q, kp, sc, sc, vp, sc, sc, 0.088, 32, 4, "causal", None,
                                            None)
    assert out.shape == (2, 32, 1, 128)


def test_layer_fakes_and_a_traced_layer():
    """A decoder-layer step sequence (QKV+RoPE, gate, FFN) traces in fake mode
    into a graph of sparkq ops."""
    hidden, inter, heads, kvh, hd = 256, 512, 2, 1, 128
    x = t(1, 1, hidden)
    wq, sq = t(hidden + 2 * hd, hidden // 8, dtype=torch.int32), t(hidden + 2 * hd, hidden // 64)
    gw, gs = t(inter, hidden // 8, dtype=torch.int32), t(inter, hidden // 64)
    dw, ds = t(hidden, inter // 8, dtype=torch.int32), t(hidden, inter // 64)
    nw = t(hidden)
    gate_w = t(heads, hidden)

    def layer(x, wq, sq, gw, gs, dw, ds, nw, gate_w):
        q, k, v = torch.ops.sparkq.qkv_rope(x, wq, sq, sq, heads * hd, kvh * hd, heads, kvh, hd,
                                           hd, 10000.0, 7, 64, 4)
        attn = torch.cat([v, v], dim=1)  # stands in for attention over the cache
        gated = torch.ops.sparkq.attention_gate(x, attn, gate_w)
        normed = torch.ops.sparkq.rms_norm(x, nw, 1e-6)
        return torch.ops.sparkq.fused_ffn(x, gated + normed, nw, 1e-6, gw, gs, gs, gw, gs, gs, dw,
                                          ds, ds, 64, 4), q, k

    gm = make_fx(layer, tracing_mode="fake")(x, wq, sq, gw, gs, dw, ds, nw, gate_w)
    targets = {str(n.target) for n in gm.graph.nodes if n.op == "call_function"}
    for name in ("qkv_rope", "attention_gate", "rms_norm", "fused_ffn"):
        assert f"sparkq.{name}.default" in targets, targets
    out, q, k = layer(x, wq, sq, gw, gs, dw, ds, nw, gate_w)
    assert out.shape == (1, 1, hidden) and q.shape == (1, heads, 1, hd) and k.shape == (1, kvh, 1, hd)
