"""Residual/RMSNorm/FFN dispatch on torch, mirroring spark_mlx_llm/ops/ffn.py.

dispatch_ffn (:17-80) keeps the reference's eligibility rules: the standard
MLP type, an RMSNorm, and affine W4 projections run the whole block,
compiled_ffn (:83-105), through sparkq.fused_ffn (one launch for the residual,
the norm, gate/up and gelu(gate)*up, one for down plus the residual); custom
modules keep their own calls (_module_ffn, :108-111).
"""

from __future__ import annotations

import torch
from torch import nn

from .. import ext
from .linear import AffineParameters, _on_gfx950

__all__ = ["RMSNorm", "dispatch_ffn"]


class RMSNorm(nn.Module):
    """torch counterpart of mlx.nn.RMSNorm: weight [dims], eps; computed by
    the gfx950 kernel with mx.fast.rms_norm's rounding."""

    def __init__(self, dims: int, eps: float = 1e-5, *, weight=None):
        super().__init__()
        self.register_buffer("weight", weight if weight is not None else torch.ones(dims))
        self.eps = eps

    def forward(self, x):
        return ext.rms_norm(x, self.weight, self.eps)


def dispatch_ffn(x, attention_output, norm, mlp, *, mlp_type):
    """hidden = x + attention_output; hidden + mlp(norm(hidden)) with the
    standard module set fused (spark_mlx_llm/ops/ffn.py:17-80)."""
    if type(mlp) is not mlp_type or type(norm) is not RMSNorm or not _on_gfx950(x):
        return _module_ffn(x, attention_output, norm, mlp)
    gate, up, down = mlp.gate_proj, mlp.up_proj, mlp.down_proj
    if not all(AffineParameters.accepts(layer) for layer in (gate, up, down)):
        return _module_ffn(x, attention_output, norm, mlp)
    groups = {layer.group_size for layer in (gate, up, down)}
    dtypes = {x.dtype, attention_output.dtype, norm.weight.dtype, gate.scales.dtype,
              up.scales.dtype, down.scales.dtype}
    if len(groups) != 1 or len(dtypes) != 1 or attention_output.shape != x.shape:
        return _module_ffn(x, attention_output, norm, mlp)

    def params(layer):
        return layer.weight, layer.scales, layer.biases

    return ext.fused_ffn(x, attention_output, norm.weight, norm.eps, params(gate), params(up),
                         params(down), group_size=groups.pop(), bits=gate.bits)


def _module_ffn(x, attention_output, norm, mlp):
    """Preserve module calls for biases, subclasses and adapters
    (spark_mlx_llm/ops/ffn.py:108-111)."""
    hidden_states = x + attention_output
    return hidden_states + mlp(norm(hidden_states))
