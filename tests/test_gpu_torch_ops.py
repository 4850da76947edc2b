"""torch.ops.sparkq on the GPU: torch.library.opcheck (schema, fake kernel
against the real outputs' shapes, dtypes and strides, autograd registration,
AOT dispatch) for the hot-path operators, and a decoder-layer function
compiled with torch.compile (aot_eager: traced through the fake kernels,
no code generation) giving the eager result bit for bit."""

import math

import numpy as np
import pytest
import torch

import oracle as o
from helpers import up16, up32, w4_problem

pytestmark = pytest.mark.gpu

UTILS = ("test_schema", "test_autograd_registration", "test_faketensor")


def _w4(gpu, m, n, k, g=64, seed=0):
    x, wq, s, b = w4_problem(m, n, k, g, seed=seed)
    return up16(x, o.BF16, gpu), up32(wq, gpu), up16(s, o.BF16, gpu), up16(b, o.BF16, gpu)


@pytest.mark.parametrize("m", [1, 4, 64])
def test_opcheck_affine_quantized_matmul(gpu, m):
    x, w, s, b = _w4(gpu, m, 512, 1024)
    for out_dtype in (None, torch.float32):
        torch.library.opcheck(torch.ops.sparkq.affine_quantized_matmul.default,
                              (x, w, s, b, 64, 4, out_dtype), test_utils=UTILS)


@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float32])
def test_opcheck_affine_w8(gpu, sdt):
    """bits=8: the result dtype is x's promoted with the scales' (fp32 for the
    converter's fp32-scaled W8 lm_head), and the fake kernel must say so."""
    n, k, g = 256, 512, 32
    x = torch.randn(2, k, device=gpu).to(torch.bfloat16)
    w = torch.randint(0, 2 ** 31 - 1, (n, k // 4), device=gpu, dtype=torch.int32)
    s = (torch.rand(n, k // g, device=gpu) * 1e-3 + 1e-4).to(sdt)
    bb = (-128 * s.float()).to(sdt)
    y = torch.ops.sparkq.affine_quantized_matmul(x, w, s, bb, g, 8, None)
    assert y.dtype == torch.promote_types(x.dtype, sdt)
    torch.library.opcheck(torch.ops.sparkq.affine_quantized_matmul.default,
                          (x, w, s, bb, g, 8, None), test_utils=UTILS)


def test_opcheck_w8a8_and_quantizer(gpu):
    xf = torch.randn(8, 512, device=gpu).to(torch.bfloat16)
    w = torch.randint(-127, 128, (256, 512), device=gpu, dtype=torch.int8)
    sw = torch.rand(256, device=gpu) * 1e-3
    torch.library.opcheck(torch.ops.sparkq.w8a8_linear.default, (xf, w, sw, None, None),
                          test_utils=UTILS)
    torch.library.opcheck(torch.ops.sparkq.quantize_per_token.default, (xf,), test_utils=UTILS)
    q, _ = torch.ops.sparkq.quantize_per_token(xf)
    torch.library.opcheck(torch.ops.sparkq.int8_matmul_int32.default, (q, w), test_utils=UTILS)
    torch.library.opcheck(torch.ops.sparkq.w8a16_per_channel.default, (xf[:1], w, sw, None),
                          test_utils=UTILS)


def test_opcheck_attention_and_norms(gpu):
    import sparkq

    b, hq, hkv, n, d = 1, 8, 2, 300, 128
    q = torch.randn(b, hq, 1, d, device=gpu).to(torch.bfloat16)
    kc, ks = sparkq.kv_quantize_s8(torch.randn(b, hkv, n, d, device=gpu, dtype=torch.bfloat16))
    vc, vs = sparkq.kv_quantize_s8(torch.randn(b, hkv, n, d, device=gpu, dtype=torch.bfloat16))
    torch.library.opcheck(torch.ops.sparkq.int8_sdpa_s8.default,
                          (q, kc, ks, vc, vs, 1 / math.sqrt(d), False, None), test_utils=UTILS)
    x = torch.randn(3, 256, device=gpu).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(256, device=gpu)).to(torch.bfloat16)
    torch.library.opcheck(torch.ops.sparkq.rms_norm.default, (x, nw, 1e-6), test_utils=UTILS)
    xr = torch.randn(1, 4, 5, 64, device=gpu).to(torch.bfloat16)
    torch.library.opcheck(torch.ops.sparkq.rope.default, (xr, 64, False, 10000.0, 1.0, 3),
                          test_utils=UTILS)


def test_compiled_layer_matches_eager(gpu):
    """rms_norm -> W4A16 projection -> W8A8 projection, compiled whole
    (fullgraph) through the custom ops, equals the eager ops bit for bit."""
    import sparkq  # noqa: F401

    x, w, s, b = _w4(gpu, 4, 512, 256, seed=3)
    nw = (1 + 0.1 * torch.randn(256, device=gpu)).to(torch.bfloat16)
    w8 = torch.randint(-127, 128, (256, 512), device=gpu, dtype=torch.int8)
    sw = torch.rand(256, device=gpu) * 1e-2

    def layer(x):
        h = torch.ops.sparkq.rms_norm(x, nw, 1e-6)
        y = torch.ops.sparkq.affine_quantized_matmul(h, w, s, b, 64, 4, None)
        return torch.ops.sparkq.w8a8_linear(y, w8, sw, None, None) + x

    eager = layer(x)
    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    for _ in range(2):
        got = compiled(x)
        torch.cuda.synchronize()
        assert torch.equal(got, eager)
    assert np.isfinite(eager.float().cpu().numpy()).all()
