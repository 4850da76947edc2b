"""Operator dispatch mirroring spark_mlx_llm/ops on torch tensors."""

from .base import OperatorConfig
from .linear import (
    AffineParameters,
    LinearConfig,
    QuantizedLinear,
    W8A16PerChannelLinear,
    W8A8Projection,
    W8A8QuantizedLinear,
    dispatch_linear,
)
from .sdpa import SDPAConfig, dispatch_sdpa

__all__ = [
    "AffineParameters",
    "LinearConfig",
    "OperatorConfig",
    "QuantizedLinear",
    "SDPAConfig",
    "W8A16PerChannelLinear",
    "W8A8Projection",
    "W8A8QuantizedLinear",
    "dispatch_linear",
    "dispatch_sdpa",
]
