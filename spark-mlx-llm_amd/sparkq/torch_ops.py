"""torch.library registration of the sparkq operators (namespace ``sparkq``).

The reference composes its extension ops inside ``mx.compile``
(spark_mlx_llm/ops/ffn.py:83-105, spark_mlx_llm/ops/qkv.py:90-107). Here
each hot-path operator is also a PyTorch custom op, ``torch.ops.sparkq.*``,
with a fake kernel that gives the output's shape and dtype without running
the device code, so that ``torch.compile`` (and ``torch.export``) can trace
a decoder layer built from them; the compiled graph calls the same C-ABI
kernels as the eager functions of ``sparkq.ext``. Arguments are the eager
functions' own (tuples of cache or projection tensors are spelled out), and
the ops validate exactly as the eager functions do, raising ValueError.

Registered ops:
  affine_quantized_matmul(x, weight, scales, biases, group_size, bits, out_dtype)
  w8a8_linear(x, weight, scales, bias, out_dtype)
  w8a16_per_channel(x, weight, scales, out_dtype)
  quantize_per_token(x) -> (q, scales)
  int8_matmul_int32(x, weight)
  int8_sdpa_s8(queries, k_codes, k_scales, v_codes, v_scales, scale, causal, out_dtype)
  int8_sdpa_affine(queries, k_packed, k_scales, k_biases, v_packed, v_scales, v_biases,
                   scale, group_size, bits, mask, mask_array, out_dtype)
  rms_norm(x, weight, eps)
  rope(x, dims, traditional, base, scale, offset)
  qkv_rope(x, weight, scales, biases, q_size, kv_size, num_heads, num_key_value_heads,
           head_dim, rope_dims, rope_base, offset, group_size, bits) -> (q, k, v)
  fused_ffn(x, attention_output, norm_weight, eps, gate_w, gate_s, gate_b, up_w, up_s,
            up_b, down_w, down_s, down_b, group_size, bits)
  attention_gate(x, output, gate_weight)
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor
from torch.library import custom_op

from . import ext

_NS = "sparkq"


def _lead(x: Tensor) -> Tuple[int, ...]:
    return tuple(x.shape[:-1])


# --- W4A16 / W8 affine linear ----------------------------------------------

@custom_op(f"{_NS}::affine_quantized_matmul", mutates_args=())
def affine_quantized_matmul(x: Tensor, weight: Tensor, scales: Tensor, biases: Tensor,
                            group_size: int, bits: int, out_dtype: Optional[torch.dtype]) -> Tensor:
    return ext.affine_quantized_matmul(x, weight, scales, biases, group_size=group_size, bits=bits,
                                       out_dtype=out_dtype)


@affine_quantized_matmul.register_fake
def _(x, weight, scales, biases, group_size, bits, out_dtype):
    # bits=8 follows MLX's promotion of x with the scales (fp32 scales, as the
    # converter writes for the lm_head, give an fp32 result); bits=4 keeps x's
    result = torch.promote_types(x.dtype, scales.dtype) if bits == 8 else x.dtype
    return x.new_empty((*_lead(x), weight.shape[0]), dtype=out_dtype or result)


# --- W8A8 / W8A16 ------------------------------------------------------------

@custom_op(f"{_NS}::w8a8_linear", mutates_args=())
def w8a8_linear(x: Tensor, weight: Tensor, scales: Tensor, bias: Optional[Tensor],
                out_dtype: Optional[torch.dtype]) -> Tensor:
    return ext.w8a8_linear(x, weight, scales, bias, out_dtype=out_dtype)


@w8a8_linear.register_fake
def _(x, weight, scales, bias, out_dtype):
    return x.new_empty((*_lead(x), weight.shape[0]), dtype=out_dtype or x.dtype)


@custom_op(f"{_NS}::w8a16_per_channel", mutates_args=())
def w8a16_per_channel(x: Tensor, weight: Tensor, scales: Tensor,
                      out_dtype: Optional[torch.dtype]) -> Tensor:
    return ext.w8a16_per_channel(x, weight, scales, out_dtype=out_dtype)


@w8a16_per_channel.register_fake
def _(x, weight, scales, out_dtype):
    return x.new_empty((*_lead(x), weight.shape[0]), dtype=out_dtype or x.dtype)


@custom_op(f"{_NS}::quantize_per_token", mutates_args=())
def quantize_per_token(x: Tensor) -> Tuple[Tensor, Tensor]:
    return ext.quantize_per_token(x)


@quantize_per_token.register_fake
def _(x):
    k = x.shape[-1]
    m = x.numel() // k if k else 0
    return x.new_empty((m, k), dtype=torch.int8), x.new_empty((m,), dtype=torch.float32)


@custom_op(f"{_NS}::int8_matmul_int32", mutates_args=())
def int8_matmul_int32(x: Tensor, weight: Tensor) -> Tensor:
    return ext.int8_matmul_int32(x, weight)


@int8_matmul_int32.register_fake
def _(x, weight):
    return x.new_empty((x.shape[0], weight.shape[0]), dtype=torch.int32)


# --- INT8-KV attention ---------------------------------------------------------

def _sdpa_out(queries: Tensor, dv: int, out_dtype: Optional[torch.dtype]) -> Tensor:
    b, h, length, _ = queries.shape
    return queries.new_empty((b, h, length, dv), dtype=out_dtype or queries.dtype)


@custom_op(f"{_NS}::int8_sdpa_s8", mutates_args=())
def int8_sdpa_s8(queries: Tensor, k_codes: Tensor, k_scales: Tensor, v_codes: Tensor,
                 v_scales: Tensor, scale: float, causal: bool,
                 out_dtype: Optional[torch.dtype]) -> Tensor:
    return ext.int8_quantized_sdpa(queries, (k_codes, k_scales), (v_codes, v_scales), scale=scale,
                                   mask="causal" if causal else None, out_dtype=out_dtype)


@int8_sdpa_s8.register_fake
def _(queries, k_codes, k_scales, v_codes, v_scales, scale, causal, out_dtype):
    return _sdpa_out(queries, v_codes.shape[-1], out_dtype)


@custom_op(f"{_NS}::int8_sdpa_affine", mutates_args=())
def int8_sdpa_affine(queries: Tensor, k_packed: Tensor, k_scales: Tensor, k_biases: Tensor,
                     v_packed: Tensor, v_scales: Tensor, v_biases: Tensor, scale: float,
                     group_size: int, bits: int, mask: Optional[str],
                     mask_array: Optional[Tensor], out_dtype: Optional[torch.dtype]) -> Tensor:
    m = mask_array if mask_array is not None else mask
    return ext.int8_quantized_sdpa(queries, (k_packed, k_scales, k_biases),
                                   (v_packed, v_scales, v_biases), scale=scale,
                                   group_size=group_size, bits=bits, mask=m, out_dtype=out_dtype)


@int8_sdpa_affine.register_fake
def _(queries, k_packed, k_scales, k_biases, v_packed, v_scales, v_biases, scale, group_size,
      bits, mask, mask_array, out_dtype):
    return _sdpa_out(queries, v_packed.shape[-1] * (32 // bits), out_dtype)


# --- decoder-layer steps around the projections --------------------------------

@custom_op(f"{_NS}::rms_norm", mutates_args=())
def rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    return ext.rms_norm(x, weight, eps)


@rms_norm.register_fake
def _(x, weight, eps):
    return x.new_empty(x.shape)


@custom_op(f"{_NS}::rope", mutates_args=())
def rope(x: Tensor, dims: int, traditional: bool, base: float, scale: float, offset: int) -> Tensor:
    return ext.rope(x, dims, traditional=traditional, base=base, scale=scale, offset=offset)


@rope.register_fake
def _(x, dims, traditional, base, scale, offset):
    return x.new_empty(x.shape)


@custom_op(f"{_NS}::qkv_rope", mutates_args=())
def qkv_rope(x: Tensor, weight: Tensor, scales: Tensor, biases: Tensor, q_size: int,
             kv_size: int, num_heads: int, num_key_value_heads: int, head_dim: int,
             rope_dims: int, rope_base: float, offset: int, group_size: int,
             bits: int) -> Tuple[Tensor, Tensor, Tensor]:
    return ext.spark_qkv_rope(x, weight, scales, biases, q_size, kv_size, num_heads,
                              num_key_value_heads, head_dim, rope_dims, rope_base, offset,
                              group_size, bits)


@qkv_rope.register_fake
def _(x, weight, scales, biases, q_size, kv_size, num_heads, num_key_value_heads, head_dim,
      rope_dims, rope_base, offset, group_size, bits):
    q = x.new_empty((1, num_heads, 1, head_dim))
    k = x.new_empty((1, num_key_value_heads, 1, head_dim))
    return q, k, torch.empty_like(k)


@custom_op(f"{_NS}::fused_ffn", mutates_args=())
def fused_ffn(x: Tensor, attention_output: Tensor, norm_weight: Tensor, eps: float,
              gate_w: Tensor, gate_s: Tensor, gate_b: Tensor, up_w: Tensor, up_s: Tensor,
              up_b: Tensor, down_w: Tensor, down_s: Tensor, down_b: Tensor, group_size: int,
              bits: int) -> Tensor:
    return ext.fused_ffn(x, attention_output, norm_weight, eps, (gate_w, gate_s, gate_b),
                         (up_w, up_s, up_b), (down_w, down_s, down_b), group_size=group_size,
                         bits=bits)


@fused_ffn.register_fake
def _(x, attention_output, norm_weight, eps, gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w,
      down_s, down_b, group_size, bits):
    return x.new_empty(x.shape)


@custom_op(f"{_NS}::attention_gate", mutates_args=())
def attention_gate(x: Tensor, output: Tensor, gate_weight: Tensor) -> Tensor:
    return ext.attention_gate(x, output, gate_weight)


@attention_gate.register_fake
def _(x, output, gate_weight):
    b, h, length, d = output.shape
    return output.new_empty((b, length, h * d))


__all__ = [
    "affine_quantized_matmul", "w8a8_linear", "w8a16_per_channel", "quantize_per_token",
    "int8_matmul_int32", "int8_sdpa_s8", "int8_sdpa_affine", "rms_norm", "rope", "qkv_rope",
    "fused_ffn", "attention_gate",
]
