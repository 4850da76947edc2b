"""The gated attention output (spark_mlx_llm/ops/attention_output.py):
the gate kernel stage by stage against the 16-bit-graph oracle, and
dispatch_attention_output through each out_proj type (W4 affine, W8A16 per
channel at one row and its affine W8 fallback at several, W8A8, a biased
g_proj on the module path) against the oracle's composition."""

import numpy as np
import pytest
import torch
from torch import nn

import oracle as o
from helpers import check_fp32, down16, up16, up32

pytestmark = pytest.mark.gpu


def _inputs(dev, b, h, length, d, hid, dtype, seed):
    x16 = o.randn16(seed, 1, b * length * hid, 1.0, dtype).reshape(b, length, hid)
    a16 = o.randn16(seed, 2, b * h * length * d, 1.0, dtype).reshape(b, h, length, d)
    w16 = o.randn16(seed, 3, h * hid, 0.02, dtype).reshape(h, hid)
    return x16, a16, w16


@pytest.mark.parametrize("b,h,length,d,hid,dtype", [
    (1, 32, 1, 128, 2560, o.BF16),     # one decode token
    (1, 16, 8, 256, 2560, o.BF16),     # verify rows
    (2, 6, 37, 64, 512, o.F16),
    (1, 32, 512, 128, 2560, o.BF16),   # prefill
])
def test_gate_kernel_stage_by_stage(gpu, b, h, length, d, hid, dtype):
    import sparkq

    print(f"[case] attention_gate b={b} h={h} L={length} d={d} hid={hid}", flush=True)
    x16, a16, w16 = _inputs(gpu, b, h, length, d, hid, dtype, seed=length + d)
    out, gate = sparkq.attention_gate(up16(x16, dtype, gpu), up16(a16, dtype, gpu),
                                      up16(w16, dtype, gpu), return_gate=True)
    g_ref, o_ref = o.attention_gate16(x16, a16, w16, dtype)
    g_dev = down16(gate)
    # the gate: the dot is summed in fp32 (the oracle's is exact), so its
    # 16-bit rounding may flip by one unit, which moves the gate by at most
    # one unit; count those
    dg = np.abs(g_dev.astype(np.int64) - g_ref.astype(np.int64))
    print(f"  gate flips {(dg > 0).mean():.4f}")
    assert dg.max() <= 1 and (dg > 0).mean() <= 0.02
    # the gated output: bit for bit the product with the device's own gate
    gf = o.bits_to_f32(g_dev, dtype).astype(np.float64)
    af = o.bits_to_f32(a16, dtype).astype(np.float64)
    expect = o.round16((np.swapaxes(af, 1, 2) * gf[..., None]).astype(np.float32), dtype)
    assert np.array_equal(down16(out), expect.reshape(b, length, h * d))
    same = dg == 0
    assert np.array_equal(down16(out).reshape(b, length, h, d)[same],
                          o_ref.reshape(b, length, h, d)[same])


def _gate_linear(w16, dtype, dev, bias=False):
    h, hid = w16.shape
    lin = nn.Linear(hid, h, bias=bias, device=dev, dtype=torch.bfloat16 if dtype == o.BF16
                    else torch.float16)
    with torch.no_grad():
        lin.weight.copy_(up16(w16, dtype, dev))
        if bias:
            lin.bias.fill_(0.25)
    return lin


@pytest.mark.parametrize("rows", [1, 7])
def test_dispatch_affine_out_proj(gpu, rows):
    """W4 affine out_proj: the gate kernel then the affine projection, equal
    to the oracle's gate followed by the oracle projection of the device's
    gated rows."""
    import sparkq
    from sparkq.ops import QuantizedLinear, dispatch_attention_output

    b, h, d, hid, g = 1, 32, 128, 2560, 64
    x16, a16, w16 = _inputs(gpu, b, h, rows, d, hid, o.BF16, seed=rows)
    wo = o.bits_to_f32(o.randn16(5, 5, hid * h * d, 0.02), o.BF16).reshape(hid, h * d)
    wq, s, bb = o.w4_quantize(wo, g)
    proj = QuantizedLinear(up32(wq, gpu), up16(s, o.BF16, gpu), up16(bb, o.BF16, gpu),
                           group_size=g)
    gate = _gate_linear(w16, o.BF16, gpu)
    xt, at = up16(x16, o.BF16, gpu), up16(a16, o.BF16, gpu)
    y = dispatch_attention_output(xt, at, gate, proj)
    assert y.shape == (b, rows, hid)
    gated = down16(sparkq.attention_gate(xt, at, gate.weight)).reshape(b * rows, h * d)
    ref = o.w4a16_matmul(gated, wq, s, bb, g)
    y32 = sparkq.affine_quantized_matmul(
        up16(gated, o.BF16, gpu), proj.weight, proj.scales, proj.biases, group_size=g,
        out_dtype=torch.float32).cpu().numpy()
    check_fp32(y32, ref)
    assert np.array_equal(down16(y).reshape(b * rows, hid), o.round16(y32, o.BF16))


@pytest.mark.parametrize("rows", [1, 3])
def test_dispatch_w8_out_proj(gpu, tmp_path, rows):
    """W8 out_proj from a converter-format checkpoint: W8A16 per channel at one
    row, its affine W8 fallback at several rows, and W8A8."""
    from test_checkpoint import W8, _write_model

    import sparkq
    from sparkq.checkpoint import Checkpoint, load_projection
    from sparkq.ops import dispatch_attention_output

    tensors = _write_model(tmp_path, w8_backend="w8a16")
    ck = Checkpoint(str(tmp_path))
    words, sb, bb = tensors[W8 + ".weight"], tensors[W8 + ".scales"], tensors[W8 + ".biases"]
    n, k = words.shape[0], words.shape[1] * 4          # 34 x 256: 2 heads of 128
    h, d, hid = 2, 128, 512
    x16, a16, w16 = _inputs(gpu, 1, h, rows, d, hid, o.BF16, seed=9 + rows)
    xt, at = up16(x16, o.BF16, gpu), up16(a16, o.BF16, gpu)
    gate = _gate_linear(w16, o.BF16, gpu)
    gated = down16(sparkq.attention_gate(xt, at, gate.weight)).reshape(rows, k)
    w8 = o.w8_unpack_affine(words)
    sc = o.bits_to_f32(sb, o.BF16)[:, 0].copy()
    for backend in ("w8a16", "w8a8"):
        proj = load_projection(ck, W8, gpu, w8_backend=backend)
        y = dispatch_attention_output(xt, at, gate, proj).reshape(rows, n)
        yf = o.bits_to_f32(down16(y), o.BF16)
        if backend == "w8a8":
            q, sa = o.a8_quantize(o.bits_to_f32(gated, o.BF16))
            assert np.array_equal(down16(y), o.round16(
                o.w8a8_epilogue(o.int8_matmul(q, w8), sa, sc), o.BF16).reshape(rows, n))
        else:
            ref = (o.w8a16_matmul(gated, w8, sc) if rows == 1
                   else o.w8_affine_matmul(gated, words, sb, bb, 32))
            assert np.all(np.abs(yf - ref) <= 2 ** -7 * np.abs(ref) + 1e-3)


def test_dispatch_module_path_for_biased_gate(gpu):
    """A g_proj with a bias takes the reference's module path: the same
    arithmetic in separate steps."""
    from sparkq.ops import QuantizedLinear, dispatch_attention_output

    b, h, rows, d, hid, g = 1, 4, 2, 64, 256, 64
    x16, a16, w16 = _inputs(gpu, b, h, rows, d, hid, o.BF16, seed=3)
    wo = o.bits_to_f32(o.randn16(6, 6, hid * h * d, 0.02), o.BF16).reshape(hid, h * d)
    wq, s, bb = o.w4_quantize(wo, g)
    proj = QuantizedLinear(up32(wq, gpu), up16(s, o.BF16, gpu), up16(bb, o.BF16, gpu),
                           group_size=g)
    gate = _gate_linear(w16, o.BF16, gpu, bias=True)
    xt, at = up16(x16, o.BF16, gpu), up16(a16, o.BF16, gpu)
    y = dispatch_attention_output(xt, at, gate, proj)
    # oracle: the biased dot, then the same gate and projection
    xf = o.bits_to_f32(x16, o.BF16).astype(np.float64)
    dot = o.round16((xf @ o.bits_to_f32(w16, o.BF16).astype(np.float64).T + 0.25)
                    .astype(np.float32), o.BF16)
    gt = o.round16((1 / (1 + np.exp(-o.bits_to_f32(dot, o.BF16).astype(np.float64))))
                   .astype(np.float32), o.BF16)
    gated = o.round16((np.swapaxes(o.bits_to_f32(a16, o.BF16), 1, 2).astype(np.float64)
                       * o.bits_to_f32(gt, o.BF16)[..., None]).astype(np.float32), o.BF16)
    ref = o.w4a16_matmul(gated.reshape(rows, h * d), wq, s, bb, g)
    yf = o.bits_to_f32(down16(y), o.BF16).reshape(rows, hid)
    assert np.abs(yf - ref).max() <= 2e-2
