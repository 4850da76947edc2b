"""Gated attention-output dispatch on torch.

Mirrors spark_mlx_llm/ops/attention_output.py: there is no backend flag; the
output projection's type and the input's rows select the path
(dispatch_attention_output, :16-59). Every path computes
    out_proj(T(transpose(output) * T(sigmoid(float(g_proj(x))))))
and the compiled paths of the reference (_compiled_w8a16_output,
_compiled_affine_output, :69-89) become the gfx950 gate kernel
(ext.attention_gate: dot, sigmoid, per-head scale and transpose in one
launch) followed by the projection's kernel. The reference's
W8MultirowProjection route (Apple-measured shapes only) has no counterpart;
its fallback module is used, as the reference does for other shapes.
"""

from __future__ import annotations

import torch
from torch import nn

from .. import ext
from .linear import AffineParameters, W8A16PerChannelLinear

__all__ = ["dispatch_attention_output"]


def _plain_gate(gate_projection) -> bool:
    """The compiled paths need a bias-free unquantized g_proj (:20-24)."""
    return (type(gate_projection) is nn.Linear and gate_projection.bias is None
            and gate_projection.weight.dtype in (torch.bfloat16, torch.float16))


def dispatch_attention_output(x, output, gate_projection, output_projection):
    """x [B,L,hidden] (the attention block's input), output [B,H,L,D] (the
    attention result), gate_projection the g_proj Linear [H,hidden],
    output_projection the out_proj module -> [B,L,out_features]."""
    projection = output_projection
    fused = (_plain_gate(gate_projection) and output.device.type == "cuda"
             and x.dtype == output.dtype == gate_projection.weight.dtype
             and ext.is_w8a8_available())
    if fused and type(projection) is W8A16PerChannelLinear:
        if W8A16PerChannelLinear.supports_rows(x.shape[0] * x.shape[1], output.dtype, x):
            gated = ext.attention_gate(x, output, gate_projection.weight)
            return W8A16PerChannelLinear.matmul(gated, projection.weight, projection.scales)
        projection = projection.fallback
    if fused and AffineParameters.accepts(projection):
        gated = ext.attention_gate(x, output, gate_projection.weight)
        return AffineParameters.native(gated, *AffineParameters.from_module(projection))
    if fused:
        # any other out_proj module (W8A8, affine W8, linear with bias)
        return output_projection(ext.attention_gate(x, output, gate_projection.weight))
    return _module_output(x, output, gate_projection, output_projection)


def _module_output(x, output, gate_projection, output_projection):
    """The reference's module path (:92-95) for gates the kernel does not
    take (a biased or quantized g_proj): the same roundings, step by step."""
    b, h, length, d = output.shape
    output = output.transpose(1, 2).contiguous()
    gate = torch.sigmoid(gate_projection(x).to(torch.float32)).to(output.dtype)
    output = output * gate[..., None]
    return output_projection(output.reshape(b, length, h * d))
