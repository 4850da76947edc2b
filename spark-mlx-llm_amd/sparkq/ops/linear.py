"""Linear configuration, dispatch, implementations and W8 adapters on torch.

Mirrors spark_mlx_llm/ops/linear.py: LinearConfig and its backend choices
(:56-81), dispatch_linear (:84-94), AffineParameters with pure projection
callables and shape predicates (:97-257), the W8 unpack (:299-324) and the
W8A8 layers (:327-374, :531-562). Every projection callable routes to the
gfx950 kernels in libsparkq; the shape predicates are widened from the
reference's Apple-measured shapes to what those kernels accept.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from math import prod
from typing import NamedTuple, Optional

import torch
from torch import nn

from .. import ext
from .base import OperatorConfig

__all__ = [
    "AffineParameters",
    "LinearConfig",
    "QuantizedLinear",
    "W8A16PerChannelLinear",
    "W8A8Projection",
    "W8A8QuantizedLinear",
    "dispatch_linear",
    "prepare_w4_layers",
]

_GROUPS = (32, 64, 128)
_PACKED = (torch.uint32, torch.int32)
_HALF = (torch.bfloat16, torch.float16)


@dataclass(kw_only=True)
class LinearConfig(OperatorConfig):
    """Select implementations for existing W8/W4 layers (same fields and
    choices as the reference, spark_mlx_llm/ops/linear.py:56-81)."""

    w8_qmv_backend: str = field(
        default="w8a16",
        metadata={"choices": ("auto", "native", "w8a16", "w8a8", "multirow")},
    )
    w4_qmv_backend: str = field(
        default="native",
        metadata={"choices": ("native", "splitk", "multirow", "multirow_packed")},
    )

    @classmethod
    def validate_values(cls, values):
        if "qmv_backend" in values:
            raise ValueError("qmv_backend was renamed to w8_qmv_backend; update the configuration")
        super().validate_values(values)


class QuantizedLinear(nn.Module):
    """torch counterpart of mlx.nn.QuantizedLinear in affine mode: packed
    uint32 weight [N,K/8], scales and biases [N,K/G], optional linear bias."""

    def __init__(self, weight, scales, biases, *, group_size: int = 64, bits: int = 4,
                 bias: Optional[torch.Tensor] = None, mode: str = "affine"):
        super().__init__()
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)
        self.register_buffer("bias", bias)
        self.group_size = group_size
        self.bits = bits
        self.mode = mode

    @classmethod
    def from_linear(cls, linear_weight, group_size: int = 64, bits: int = 4, bias=None):
        wq, s, b = ext.affine_quantize(linear_weight, group_size=group_size, bits=bits)
        return cls(wq, s, b, group_size=group_size, bits=bits, bias=bias)

    def forward(self, x):
        prepared = None
        if AffineParameters.supports_prepared(x.shape, x.dtype, *AffineParameters.from_module(self)):
            prepared = _w4_prepared_parameters(self)
        y = AffineParameters.native(x, self.weight, self.scales, self.biases, self.group_size,
                                    self.bits, prepared)
        return y + self.bias if self.bias is not None else y


def _w4_prepared_parameters(layer):
    """The layer's derived GEMM buffer for its current source tensors
    (the identity-keyed cache of spark_mlx_llm/ops/linear.py:260-268). Kept
    outside the module's buffers, so checkpoints never hold it; rebuilt when
    a source tensor is replaced or modified in place (torch's version
    counter stands in for MLX's immutable arrays)."""
    sources = (layer.weight, layer.scales, layer.biases)
    versions = tuple(t._version for t in sources)
    cached = getattr(layer, "_sparkq_w4_prepared", None)
    if (cached is not None and cached[1] == versions
            and all(old is new for old, new in zip(cached[0], sources))):
        return cached[2]
    prepared = ext.prepare_w4a16(*sources, group_size=layer.group_size)
    object.__setattr__(layer, "_sparkq_w4_prepared", (sources, versions, prepared))
    return prepared


def prepare_w4_layers(model):
    """Derive the prefill buffers of every eligible W4 projection of a model
    up front, at load time (spark_mlx_llm/ops/linear.py:636-654 evaluates its
    prepared buffers the same way), instead of on each layer's first
    multi-token call. Returns the number of layers prepared."""
    count = 0
    for layer in model.modules():
        if (AffineParameters.accepts(layer) and layer.bits == 4
                and layer.scales.dtype == torch.bfloat16 and _on_gfx950(layer.weight)):
            if _w4_prepared_parameters(layer) is not None:
                count += 1
    return count


def dispatch_linear(x, projection, *, config: LinearConfig | None = None):
    """Select a W4 projection for eligible layers; otherwise call the module
    (spark_mlx_llm/ops/linear.py:84-94)."""
    config = config if config is not None else LinearConfig()
    if config.w4_qmv_backend != "native" and AffineParameters.accepts(projection):
        project, params = AffineParameters.resolve(projection, x.shape, x.dtype, config)
        return project(x, *params)
    return projection(x)


def _on_gfx950(t) -> bool:
    return t.device.type == "cuda" and ext.is_w8a8_available()


class AffineParameters(NamedTuple):
    """Affine tensors and metadata passed explicitly to pure projections
    (spark_mlx_llm/ops/linear.py:97-257)."""

    weight: torch.Tensor
    scales: torch.Tensor
    biases: Optional[torch.Tensor]
    group_size: int
    bits: int
    # derived prefill buffer (ext.prepare_w4a16), passed explicitly like the
    # reference's prepared arrays; None where the call needs none
    prepared: Optional[torch.Tensor] = None

    @classmethod
    def from_module(cls, layer):
        return cls(layer.weight, layer.scales, layer.biases, layer.group_size, layer.bits)

    @classmethod
    def resolve(cls, layer, shape, dtype, config):
        """Choose a pure projection and the current tensors. The gfx950 decode
        kernels read the native packed layout, so multirow_packed needs no
        repacked weights (prepare_w4a16_nax4 is the identity); shapes that
        reach the prefill GEMM get the layer's derived buffer, made once per
        weight set (_w4_prepared_parameters)."""
        params = cls.from_module(layer)
        if config.w4_qmv_backend == "multirow_packed" and params.supports_multirow(
                shape, dtype, *params):
            prepared = ext.prepare_w4a16_nax4(params.weight, params.scales, params.biases)
            return cls.multirow_packed, cls(*prepared, params.group_size, params.bits)
        project = params.select(shape, dtype, config)
        if project is cls.native and params.supports_prepared(shape, dtype, *params):
            params = params._replace(prepared=_w4_prepared_parameters(layer))
        return project, params

    def select(self, shape, dtype, config: LinearConfig):
        if config.w4_qmv_backend == "multirow" and self.supports_multirow(shape, dtype, *self):
            return self.multirow
        if config.w4_qmv_backend == "splitk" and self.supports_splitk(shape, dtype, *self):
            return self.splitk
        return self.native

    @staticmethod
    def accepts(layer):
        # Module call for linear biases, adapters and other quantization modes.
        return (
            type(layer) is QuantizedLinear
            and layer.mode == "affine"
            and layer.biases is not None
            and layer.bias is None
        )

    @staticmethod
    def _affine_ok(shape, dtype, weight, scales, biases, group_size, bits, prepared=None):
        return (
            bits == 4
            and group_size in _GROUPS
            and len(shape) >= 1
            and weight.ndim == 2
            and weight.dtype in _PACKED
            and weight.shape[1] * 8 == shape[-1]
            and shape[-1] % 64 == 0
            and scales.shape == (weight.shape[0], shape[-1] // group_size)
            and biases is not None
            and biases.shape == scales.shape
            and dtype in _HALF
            and scales.dtype == dtype
            and biases.dtype == dtype
            and _on_gfx950(weight)
        )

    @staticmethod
    def supports_splitk(shape, dtype, weight, scales, biases, group_size, bits, prepared=None):
        """One-row decode geometry (the reference's predicate, widened from its
        measured BF16/G32 shapes to every shape the gfx950 GEMV accepts)."""
        return prod(shape[:-1]) == 1 and AffineParameters._affine_ok(
            shape, dtype, weight, scales, biases, group_size, bits)

    @staticmethod
    def supports_multirow(shape, dtype, weight, scales, biases, group_size, bits,
                          prepared=None):
        """Verification geometries: 2..32 rows (reference: exactly 8)."""
        return (len(shape) >= 2 and 2 <= prod(shape[:-1]) <= 32
                and AffineParameters._affine_ok(shape, dtype, weight, scales, biases,
                                                group_size, bits))

    @staticmethod
    def supports_prepared(shape, dtype, weight, scales, biases, group_size, bits,
                          prepared=None):
        """Shapes that the bf16 prefill GEMM serves (more than 32 rows), where
        the derived buffer saves the weight half of its prologue."""
        return (len(shape) >= 2 and prod(shape[:-1]) > 32 and dtype == torch.bfloat16
                and AffineParameters._affine_ok(shape, dtype, weight, scales, biases,
                                                group_size, bits))

    @staticmethod
    def native(x, weight, scales, biases, group_size, bits, prepared=None):
        """mx.quantized_matmul(..., transpose=True, mode="affine") on gfx950."""
        return ext.affine_quantized_matmul(x, weight, scales, biases, group_size=group_size,
                                           bits=bits, prepared=prepared)

    @staticmethod
    def multirow(x, weight, scales, biases, group_size, bits, prepared=None):
        return ext.w4a16_multirow(x, weight, scales, biases, algorithm="wide")

    @staticmethod
    def multirow_packed(x, weight, scales, biases, group_size, bits, prepared=None):
        return ext.w4a16_multirow(x, weight, scales, biases, algorithm="nax4")

    @staticmethod
    def splitk(x, weight, scales, biases, group_size, bits, prepared=None):
        return ext.w4a16_qmv(x, weight, scales, biases)


# ---------------------------------------------------------------------------
# W8 adapters
# ---------------------------------------------------------------------------

_XOR80 = -2139062144  # 0x80808080 as a signed 32-bit value

_W8A8_ACTIVATIONS = {"num_bits": 8, "type": "int", "strategy": "token", "symmetric": True,
                     "dynamic": True}


def validate_w8a8_activations(activations):
    """A W8A8 module's input_activations must describe symmetric dynamic
    per-token int8 (spark_mlx_llm/ops/linear.py:280-296); absent keys take
    the expected values."""
    if not isinstance(activations, dict) or activations.get("num_bits") != 8 or any(
            activations.get(key, want) != want for key, want in _W8A8_ACTIVATIONS.items()):
        raise ValueError(
            "W8A8 out_proj requires symmetric dynamic per-token INT8 input_activations")


def unpack_affine_w8(weight, scales, biases, group_size: int, name: str = "layer",
                     *, allow_fallback: bool = False):
    """MLX affine W8 (uint32 [N,K/4], scales/biases [N,K/G]) -> signed int8
    [N,K] (bytes XOR 0x80) and fp32 channel scales [N]
    (spark_mlx_llm/ops/linear.py:299-324). Requires repeated positive
    per-channel scales and biases == -128*scales."""
    n, packed_k = weight.shape
    sc = scales.to(torch.float32)
    if (weight.dtype not in _PACKED or biases is None or sc.ndim != 2
            or sc.shape != (n, packed_k * 4 // group_size) or biases.shape != sc.shape):
        raise ValueError(f"{name}: QMV requires UINT32-packed affine W8 parameters")
    ok = bool(torch.all(torch.isfinite(sc) & (sc > 0)) & torch.all(sc == sc[:, :1])
              & torch.all(biases.to(torch.float32) == -128 * sc))
    if not ok:
        if allow_fallback:
            return None
        raise ValueError(
            f"{name}: QMV requires repeated positive per-channel scales and "
            "affine biases=-128*scales; groupwise/asymmetric W8 is unsupported")
    w8 = (weight.view(torch.int32) ^ _XOR80).contiguous().view(torch.int8)
    return w8, sc[:, 0].contiguous()


class W8A8QuantizedLinear(nn.Module):
    """Keeps MLX affine W8 checkpoint parameters and caches the unpacked int8
    kernel inputs (spark_mlx_llm/ops/linear.py:327-374)."""

    def __init__(self, weight, scales, biases, *, group_size: int = 32, bits: int = 8,
                 bias=None):
        super().__init__()
        if not ext.is_w8a8_available():
            raise RuntimeError("Cannot create a native W8A8 layer without W8A8 support")
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)
        self.register_buffer("bias", bias)
        self.group_size, self.bits, self.mode = group_size, bits, "affine"
        self._w8a8_cache = None

    def prepare_parameters(self):
        sources = (self.weight, self.scales, self.biases)
        cached = self._w8a8_cache
        if cached is not None and all(a is b for a, b in zip(cached[0], sources)):
            return cached[1:]
        if self.bits != 8 or self.weight.dtype not in _PACKED:
            raise ValueError("W8A8 out_proj requires UINT32-packed 8-bit affine weights")
        packed_k = self.weight.shape[1]
        if packed_k * 4 > 131040 or packed_k * 4 % 32:
            raise ValueError("W8A8 out_proj K must be a multiple of 32 in [32, 131040]")
        w8, sc = unpack_affine_w8(self.weight, self.scales, self.biases, self.group_size,
                                  "W8A8 out_proj")
        self._w8a8_cache = (sources, w8, sc)
        return w8, sc

    def forward(self, x):
        w8, sc = self.prepare_parameters()
        return ext.w8a8_linear(x, w8, sc, self.bias)


class W8A16PerChannelLinear(nn.Module):
    """Single-row W8A16 projection with the affine W8 layer kept as the
    fallback for other inputs (spark_mlx_llm/ops/linear.py:413-476): signed
    int8 weight [N,K] and fp32 channel scales [N] or [N,1] derived from the
    fallback's packed weights (unpack_affine_w8)."""

    def __init__(self, fallback, weight, scales):
        super().__init__()
        fb_w = getattr(fallback, "weight", None)
        if (getattr(fallback, "mode", None) != "affine" or getattr(fallback, "bits", None) != 8
                or getattr(fallback, "biases", None) is None
                or getattr(fallback, "bias", None) is not None):
            raise ValueError("W8A16 fallback must be a bias-free affine W8 QuantizedLinear")
        if (weight.ndim != 2 or weight.dtype != torch.int8 or fb_w is None
                or tuple(weight.shape) != (fb_w.shape[0], fb_w.shape[1] * 4)
                or scales.dtype != torch.float32
                or tuple(scales.shape) not in ((weight.shape[0],), (weight.shape[0], 1))):
            raise ValueError("W8A16 needs matching signed INT8 [N,K] and FP32 [N] scales")
        self.fallback = fallback
        self.register_buffer("weight", weight.contiguous())
        self.register_buffer("scales", scales.reshape(-1).contiguous())
        self.requires_grad_(False)

    def forward(self, x):
        if x.ndim >= 1 and x.shape[-1] > 0 and self.supports_rows(x.numel() // x.shape[-1],
                                                                    x.dtype, x):
            return self.matmul(x, self.weight, self.scales)
        return self.fallback(x)

    @staticmethod
    def supports_rows(num_rows, dtype, x=None):
        return num_rows == 1 and dtype in _HALF and (x is None or _on_gfx950(x))

    @staticmethod
    def matmul(x, weight, scales):
        return ext.w8a16_per_channel(x, weight, scales)


class W8A8Projection(nn.Module):
    """W8A8 arithmetic with the affine module kept as the fallback for inputs
    the kernel does not serve (spark_mlx_llm/ops/linear.py:531-562)."""

    def __init__(self, fallback, weight, scales):
        super().__init__()
        if not ext.is_w8a8_available():
            raise RuntimeError("w8_qmv_backend='w8a8' requires an MI355X (gfx950) device")
        self.fallback = fallback
        self.projection = ext.W8A8Linear(weight, scales, getattr(fallback, "bias", None))

    def forward(self, x):
        if x.dtype in (torch.bfloat16, torch.float16, torch.float32) and _on_gfx950(x):
            return self.projection(x)
        return self.fallback(x)
