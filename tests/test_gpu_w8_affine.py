"""GPU parity of the groupwise affine W8 matmul (sparkq_w8_affine_linear):
the bits=8 branch of affine_quantized_matmul that the reference's W8 layers
fall back to (spark_mlx_llm/ops/linear.py:413-476, 531-562, 651-711),
against the float64 oracle; and the W8 modules the checkpoint loader builds
for each w8_qmv_backend, run with several activation rows."""

import numpy as np
import pytest
import torch

import oracle as o
from helpers import check_fp32, check_rounded16, down16, up16, up32

pytestmark = pytest.mark.gpu

TORCH = {o.BF16: torch.bfloat16, o.F16: torch.float16}


def _problem(m, n, k, g, dtype, sdtype, seed):
    """Weights N(0, 0.02) quantized per group of g with 255 min/max bins
    (scale (max-min)/255, bias min, as stored; codes rint((w-b)/s)), so the
    outputs have the magnitudes of a real projection."""
    w = o.randn(seed, 11, n * k, 0.02).reshape(n, k // g, g).astype(np.float64)
    lo, hi = w.min(-1), w.max(-1)
    sf, bf = ((hi - lo) / 255).astype(np.float32), lo.astype(np.float32)
    if sdtype == o.F32:
        s, b = sf, bf
        s64, b64 = sf.astype(np.float64), bf.astype(np.float64)
    else:
        s, b = o.round16(sf, sdtype), o.round16(bf, sdtype)
        s64 = o.bits_to_f32(s, sdtype).astype(np.float64)
        b64 = o.bits_to_f32(b, sdtype).astype(np.float64)
    u = np.clip(np.rint((w - b64[..., None]) / s64[..., None]), 0, 255).astype(np.uint8)
    words = np.ascontiguousarray(u.reshape(n, k)).view(np.uint32)
    x = o.randn16(seed, 7, m * k, 1.0, dtype).reshape(m, k)
    return x, words, s, b


def _dev_scales(a, sdtype, dev):
    if sdtype == o.F32:
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return up16(a, sdtype, dev)


@pytest.mark.parametrize("m,n,k,g,dtype,sdtype", [
    (1, 2560, 4096, 32, o.BF16, o.BF16),     # out_proj decode, converter group size
    (8, 2560, 4096, 32, o.BF16, o.BF16),     # speculative verify rows
    (37, 300, 512, 64, o.BF16, o.BF16),      # ragged rows and columns
    (130, 1000, 1024, 128, o.F16, o.F16),
    (5, 4099, 2560, 32, o.BF16, o.F32),      # fp32 coefficients (the lm_head's)
    (256, 2560, 4096, 32, o.BF16, o.BF16),   # prefill rows
])
def test_w8_affine_matches_oracle(gpu, m, n, k, g, dtype, sdtype):
    import sparkq

    print(f"[case] w8_affine m={m} n={n} k={k} g={g} dtype={dtype} sdtype={sdtype}", flush=True)
    x, words, s, b = _problem(m, n, k, g, dtype, sdtype, seed=m + n)
    xt = up16(x, dtype, gpu)
    wt, st, bt = up32(words, gpu), _dev_scales(s, sdtype, gpu), _dev_scales(b, sdtype, gpu)
    ref = o.w8_affine_matmul(x, words, s, b, g, dtype, sdtype)
    y32 = sparkq.affine_quantized_matmul(xt, wt, st, bt, group_size=g, bits=8,
                                         out_dtype=torch.float32).cpu().numpy()
    check_fp32(y32, ref)
    y = sparkq.affine_quantized_matmul(xt, wt, st, bt, group_size=g, bits=8)
    if sdtype == o.F32:
        # MLX promotes the result to the scales' float32
        assert y.dtype == torch.float32
        assert np.array_equal(y.cpu().numpy(), y32)
    else:
        assert y.dtype == TORCH[dtype]
        # the 16-bit output is the fp32 epilogue rounded once
        assert np.array_equal(down16(y), o.round16(y32, dtype))
        check_rounded16(down16(y), ref, dtype)


def test_w8_affine_one_hot_columns_exact(gpu):
    """x = e_k picks u[:,k]*s + b exactly (products of codes and 16-bit
    scales are exact; one fp32 rounding of the sum)."""
    import sparkq

    m, n, k, g = 3, 640, 256, 32
    x, words, s, b = _problem(m, n, k, g, o.BF16, o.BF16, seed=3)
    e = np.zeros((m, k), np.float32)
    cols = [0, 131, 255]
    for i, c in enumerate(cols):
        e[i, c] = 1.0
    y = sparkq.affine_quantized_matmul(up16(o.bf16_bits(e), o.BF16, gpu), up32(words, gpu),
                                       up16(s, o.BF16, gpu), up16(b, o.BF16, gpu), group_size=g,
                                       bits=8, out_dtype=torch.float32).cpu().numpy()
    u = o.unpack8(words).astype(np.float32)
    sf, bf = o.bits_to_f32(s, o.BF16), o.bits_to_f32(b, o.BF16)
    for i, c in enumerate(cols):
        expect = (u[:, c] * sf[:, c // g] + bf[:, c // g]).astype(np.float32)
        assert np.array_equal(y[i], expect)


@pytest.mark.parametrize("backend", ["w8a16", "native", "auto", "w8a8"])
@pytest.mark.parametrize("rows", [1, 6])
def test_loaded_w8_projection_any_rows(gpu, tmp_path, backend, rows):
    """Every W8 module the loader builds runs at one row and at several rows
    (prefill / verify), where the per-channel adapters hand the input to the
    affine fallback; W8A8 modules quantize the activations per token."""
    from test_checkpoint import W8, _write_model

    from sparkq.checkpoint import Checkpoint, load_projection
    from sparkq.ops import (QuantizedLinear, W8A16PerChannelLinear, W8A8Projection,
                            W8A8QuantizedLinear)

    print(f"[case] loaded W8 backend={backend} rows={rows}", flush=True)
    tensors = _write_model(tmp_path, w8_backend=backend)
    ck = Checkpoint(str(tmp_path))
    if backend == "auto":
        # the converter's w8a8 checkpoints mark out_proj with input_activations
        ck.config["quantization_config"][W8]["input_activations"] = {
            "num_bits": 8, "type": "int", "strategy": "token", "symmetric": True,
            "dynamic": True}
    p8 = load_projection(ck, W8, gpu)
    expect_type = {"w8a16": W8A16PerChannelLinear, "native": QuantizedLinear,
                   "auto": W8A8QuantizedLinear, "w8a8": W8A8Projection}[backend]
    assert type(p8) is expect_type
    x = o.randn16(4, rows, rows * 256).reshape(rows, 256)
    xt = up16(x, o.BF16, gpu)
    y = p8(xt)
    words, sb, bb = tensors[W8 + ".weight"], tensors[W8 + ".scales"], tensors[W8 + ".biases"]
    assert y.shape == (rows, words.shape[0]) and y.dtype == torch.bfloat16
    w8 = o.w8_unpack_affine(words)
    sc = o.bits_to_f32(sb, o.BF16)[:, 0].copy()
    if backend in ("auto", "w8a8"):
        q, sa = o.a8_quantize(o.bits_to_f32(x, o.BF16))
        ref32 = o.w8a8_epilogue(o.int8_matmul(q, w8), sa, sc)
        assert np.array_equal(down16(y), o.round16(ref32, o.BF16))
    else:
        ref = o.w8_affine_matmul(x, words, sb, bb, 32)
        # the golden rows reach |y| ~ 4600: compare relative to magnitude
        yf = o.bits_to_f32(down16(y), o.BF16)
        assert np.all(np.abs(yf - ref) <= 2 ** -7 * np.abs(ref) + 1e-3), \
            float(np.max(np.abs(yf - ref)))
        # the affine fallback agrees with the per-channel identity
        alt = o.w8a16_matmul(x, w8, sc)
        assert np.allclose(ref, alt, rtol=1e-9, atol=1e-6)
