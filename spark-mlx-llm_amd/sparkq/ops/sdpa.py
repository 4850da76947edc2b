"""SDPA configuration and dispatch for INT8 KV caches on torch.

Mirrors spark_mlx_llm/ops/sdpa.py: SDPAConfig (:13-20), dispatch_sdpa
(:39-78), _supports_int8 (:81-103) and _int8_attention (:149-163). The
predicate is widened from the reference's D=256/G32 affine format to the
formats and head sizes the gfx950 decode kernel serves (D in 64/128/256,
affine G in 32/64/128, or symmetric s8 codes with fp16 per-token scales);
multi-token queries (the opt-in fused_quantized_sdpa_prefill) are served on
both formats with 16-bit queries. Other quantized caches (2- and 4-bit, other
head dims, mask arrays) take the staged-attention kernel, where the
reference's mlx-lm native path runs the same staged arithmetic.
Unquantized caches go to torch's scaled_dot_product_attention, the analogue
of the reference's mlx-lm native path.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import ext
from .base import OperatorConfig

__all__ = ["SDPAConfig", "dispatch_sdpa"]


@dataclass(kw_only=True)
class SDPAConfig(OperatorConfig):
    """Prefer available kernels; KV cache quantization is configured separately."""

    fused_quantized_sdpa: bool = True
    fused_quantized_sdpa_prefill: bool = False
    tuned_bf16_sdpa: bool = False
    verification_bf16_sdpa: bool = False


def dispatch_sdpa(queries, keys, values, *, cache, scale, mask, config: SDPAConfig | None = None,
                  is_sliding=False):
    config = config if config is not None else SDPAConfig()
    if config.fused_quantized_sdpa and _supports_int8(queries, keys, values, cache=cache,
                                                      mask=mask,
                                                      prefill=config.fused_quantized_sdpa_prefill):
        return _int8_attention(queries, keys, values, cache=cache, scale=scale, mask=mask)
    if isinstance(keys, (tuple, list)):
        return _quantized_attention(queries, keys, values, cache=cache, scale=scale, mask=mask)
    return _native_attention(queries, keys, values, scale=scale, mask=mask)


def _supports_int8(queries, keys, values, *, cache, mask, prefill=False):
    if not (isinstance(keys, (tuple, list)) and isinstance(values, (tuple, list))
            and len(keys) == len(values) and len(keys) in (2, 3)):
        return False
    if getattr(cache, "bits", None) != 8:
        return False
    affine = len(keys) == 3
    dim = queries.shape[-1] if queries.ndim == 4 else -1
    length = queries.shape[-2] if queries.ndim == 4 else 0
    # multi-token queries (prefill, opt-in as in the reference) run on either
    # cache format with 16-bit queries and L <= N under a causal mask
    multi_ok = (prefill and queries.dtype in (torch.float16, torch.bfloat16)
                and (mask is None or length <= keys[0].shape[2]))
    return (
        queries.ndim == 4
        and (length == 1 or (length > 1 and multi_ok))
        and dim in (64, 128, 256)
        and keys[0].ndim == values[0].ndim == 4
        and keys[0].shape[1] > 0
        and queries.shape[1] % keys[0].shape[1] == 0
        and queries.shape[1] // keys[0].shape[1] in (1, 2, 4, 8)
        and queries.dtype in (torch.float16, torch.bfloat16, torch.float32)
        and (
            (affine and getattr(cache, "group_size", None) in (32, 64, 128)
             and keys[0].shape[-1] * 4 == dim
             and all(t.dtype == queries.dtype for t in (*keys[1:], *values[1:])))
            or (not affine and keys[0].dtype == torch.int8 and keys[0].shape[-1] == dim
                and keys[1].dtype == values[1].dtype == torch.float16)
        )
        and (mask is None or (isinstance(mask, str) and mask == "causal"))
        and queries.device.type == "cuda"
        and ext.is_w8a8_available()
    )


def _quantized_attention(queries, keys, values, *, cache, scale, mask):
    """Quantized caches the fused route does not take (or all of them when
    fused_quantized_sdpa is off): the reference hands them to mlx-lm's
    scaled_dot_product_attention, whose quantized branch is the staged
    quantized_matmul / softmax / quantized_matmul form (the same arithmetic
    as X/spark_mlx_ext/int8_quantized_sdpa.py:122-153); here the MLX affine
    tuple goes to the staged-attention kernel (bits 2/4/8, any head dims,
    mask arrays), and the symmetric s8 pair, which has no staged form, to
    int8_quantized_sdpa. Like every sparkq operator it runs only on the
    device."""
    if len(keys) == 3:
        return ext.staged_quantized_sdpa(queries, keys, values, scale=scale,
                                         group_size=getattr(cache, "group_size", 32),
                                         bits=getattr(cache, "bits", 8), mask=mask)
    return ext.int8_quantized_sdpa(queries, keys, values, scale=scale,
                                   group_size=getattr(cache, "group_size", 32),
                                   bits=getattr(cache, "bits", 8), mask=mask)


def _int8_attention(queries, keys, values, *, cache, scale, mask):
    return ext.int8_quantized_sdpa(queries, keys, values, scale=scale,
                                   group_size=getattr(cache, "group_size", 32),
                                   bits=cache.bits, mask=mask)


def causal_mask(length: int, n: int, device=None) -> torch.Tensor:
    """Boolean [length, n] mask of MLX's "causal": aligned bottom-right, so
    query i of the last ``length`` positions sees tokens 0 .. n-length+i
    (mlx-lm's create_causal_mask; X/spark_mlx_ext/int8_quantized_sdpa.py:
    141-142 builds the same mask as arange(n-L, n)[:, None] >= arange(n))."""
    return torch.ones((length, n), dtype=torch.bool, device=device).tril(n - length)


def _native_attention(queries, keys, values, *, scale, mask):
    heads, kv_heads = queries.shape[1], keys.shape[1]
    if heads != kv_heads:
        keys = keys.repeat_interleave(heads // kv_heads, dim=1)
        values = values.repeat_interleave(heads // kv_heads, dim=1)
    length, n = queries.shape[2], keys.shape[2]
    if isinstance(mask, str):
        if mask != "causal":
            raise ValueError("mask string must be 'causal'")
        # torch's is_causal aligns the mask top-left; MLX aligns it bottom-right,
        # which differs whenever the cache already holds tokens (length < n)
        mask = causal_mask(length, n, queries.device) if length > 1 else None
    return torch.nn.functional.scaled_dot_product_attention(
        queries, keys, values, attn_mask=mask, scale=scale)
