"""QKV/RoPE dispatch on torch, mirroring spark_mlx_llm/ops/qkv.py.

dispatch_qkv (:18-88) keeps the reference's routes: one token (B = L = 1)
of an affine W4 projection with a standard non-traditional RoPE goes through
the fused projection + rotation (spark_qkv_rope, :110-137); other shapes
project with the resolved W4 route, split the heads (:140-160) and apply the
rope module (:176-177).
"""

from __future__ import annotations


from .. import ext
from .linear import AffineParameters, LinearConfig, _on_gfx950

__all__ = ["RoPE", "dispatch_qkv"]


class RoPE:
    """torch counterpart of mlx.nn.RoPE: mx.fast.rope(x, dims, traditional,
    base, scale, offset) on the gfx950 kernel."""

    def __init__(self, dims: int, traditional: bool = False, base: float = 10000.0,
                 scale: float = 1.0):
        self.dims = dims
        self.traditional = traditional
        self.base = base
        self.scale = scale

    def __call__(self, x, offset: int = 0):
        return ext.rope(x, self.dims, traditional=self.traditional, base=self.base,
                        scale=self.scale, offset=offset)


def dispatch_qkv(x, projection, rope, *, q_size, kv_size, n_heads, n_kv_heads, head_dim,
                 offset, config: LinearConfig | None = None):
    config = config if config is not None else LinearConfig()
    batch_size, sequence_length, _ = x.shape
    quantized_qkv = _on_gfx950(x) and AffineParameters.accepts(projection)
    splitk_qkv = (
        quantized_qkv
        and config.w4_qmv_backend == "splitk"
        and AffineParameters.supports_splitk(x.shape, x.dtype,
                                             *AffineParameters.from_module(projection))
    )
    use_native_qkv = (
        quantized_qkv
        and not splitk_qkv
        and batch_size == 1
        and sequence_length == 1
        and projection.bits == 4
        and projection.group_size in (32, 64, 128)
        and type(rope) is RoPE
        and not rope.traditional
        and rope.scale == 1.0
        and isinstance(offset, int)
    )
    if use_native_qkv:
        return ext.spark_qkv_rope(x, projection.weight, projection.scales, projection.biases,
                                  q_size, kv_size, n_heads, n_kv_heads, head_dim, rope.dims,
                                  rope.base, offset, projection.group_size, projection.bits)
    if quantized_qkv:
        project, params = AffineParameters.resolve(projection, x.shape, x.dtype, config)
        queries, keys, values = _split_heads(project(x, *params), q_size=q_size, kv_size=kv_size,
                                             n_heads=n_heads, n_kv_heads=n_kv_heads,
                                             head_dim=head_dim)
    else:
        queries, keys, values = _split_heads(projection(x), q_size=q_size, kv_size=kv_size,
                                             n_heads=n_heads, n_kv_heads=n_kv_heads,
                                             head_dim=head_dim)
    return rope(queries, offset=offset), rope(keys, offset=offset), values


def _split_heads(qkv, *, q_size, kv_size, n_heads, n_kv_heads, head_dim):
    """[B, L, q+2kv] -> contiguous [B, H, L, D] queries, keys and values
    (spark_mlx_llm/ops/qkv.py:140-160)."""
    batch_size, sequence_length, _ = qkv.shape
    queries, keys, values = qkv.split([q_size, kv_size, kv_size], dim=-1)

    def heads(t, n):
        return t.reshape(batch_size, sequence_length, n, head_dim).transpose(1, 2).contiguous()

    return heads(queries, n_heads), heads(keys, n_kv_heads), heads(values, n_kv_heads)
