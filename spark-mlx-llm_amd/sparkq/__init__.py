"""sparkq: MI355X (gfx950) kernels for Spark-MLX-LLM's quantized-linear hot path.

sparkq.ext mirrors the extension API (spark_mlx_ext); sparkq.ops mirrors the
operator dispatch layer (spark_mlx_llm/ops). Kernels live in libsparkq.so,
called over the C-ABI declared in include/sparkq.h.
"""

from .ext import (
    QuantizedKVCache,
    W8A8Linear,
    affine_dequantize,
    attention_gate,
    affine_quantize,
    affine_quantized_matmul,
    fused_ffn,
    int8_matmul_int32,
    int8_quantized_sdpa,
    is_w8a8_available,
    kv_append,
    kv_quantize_s8,
    prepare_w4a16,
    prepare_w4a16_nax4,
    quantize_per_token,
    rms_norm,
    rope,
    spark_qkv_rope,
    w4a16_multirow,
    w4a16_qmv,
    w8a16_per_channel,
    w8a8_linear,
)
from . import torch_ops  # registers torch.ops.sparkq.* (custom ops with fake kernels)

__all__ = [
    "QuantizedKVCache",
    "W8A8Linear",
    "affine_dequantize",
    "attention_gate",
    "affine_quantize",
    "affine_quantized_matmul",
    "fused_ffn",
    "int8_matmul_int32",
    "int8_quantized_sdpa",
    "is_w8a8_available",
    "kv_append",
    "kv_quantize_s8",
    "prepare_w4a16",
    "prepare_w4a16_nax4",
    "quantize_per_token",
    "rms_norm",
    "rope",
    "spark_qkv_rope",
    "w4a16_multirow",
    "w4a16_qmv",
    "w8a16_per_channel",
    "w8a8_linear",
]
