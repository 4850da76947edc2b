"""Operator dispatch mirroring spark_mlx_llm/ops on torch tensors."""

from .attention_output import dispatch_attention_output
from .base import OperatorConfig
from .ffn import RMSNorm, dispatch_ffn
from .linear import (
    AffineParameters,
    LinearConfig,
    QuantizedLinear,
    W8A16PerChannelLinear,
    W8A8Projection,
    W8A8QuantizedLinear,
    dispatch_linear,
    prepare_w4_layers,
)
from .qkv import RoPE, dispatch_qkv
from .sdpa import SDPAConfig, dispatch_sdpa

__all__ = [
    "AffineParameters",
    "LinearConfig",
    "OperatorConfig",
    "QuantizedLinear",
    "RMSNorm",
    "RoPE",
    "SDPAConfig",
    "W8A16PerChannelLinear",
    "W8A8Projection",
    "W8A8QuantizedLinear",
    "dispatch_attention_output",
    "dispatch_ffn",
    "dispatch_linear",
    "dispatch_qkv",
    "dispatch_sdpa",
    "prepare_w4_layers",
]
