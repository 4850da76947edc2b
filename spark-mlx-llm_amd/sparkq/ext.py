"""Operator API of the MI355X kernels, mirroring spark_mlx_ext on torch tensors.

Every op validates like its reference wrapper (TypeError/ValueError), then
calls libsparkq on the current HIP stream of the input's device. Ops return
without synchronising; inputs are never modified; non-contiguous inputs are
copied (the reference's ensure_row_contiguous behaviour). There is no CPU or
eager fallback: tensors must live on a gfx950 device.

Reference: extensions/spark-mlx-ext/spark_mlx_ext/__init__.py:12-44.
"""

from __future__ import annotations

import ctypes
import math
from math import prod

import torch
from torch import nn

from . import _lib
from ._lib import BF16, F16, F32, KV_AFFINE_U2, KV_AFFINE_U4, KV_AFFINE_U8, KV_S8_F16SCALE

__all__ = [
    "W8A8Linear",
    "attention_gate",
    "affine_dequantize",
    "affine_quantize",
    "affine_quantized_matmul",
    "fused_ffn",
    "int8_matmul_int32",
    "int8_quantized_sdpa",
    "is_w8a8_available",
    "kv_quantize_s8",
    "QuantizedKVCache",
    "kv_append",
    "prepare_w4a16",
    "prepare_w4a16_nax4",
    "quantize_per_token",
    "rms_norm",
    "rope",
    "spark_qkv_rope",
    "staged_quantized_sdpa",
    "w4a16_multirow",
    "w4a16_qmv",
    "w8a16_per_channel",
    "w8a8_linear",
]

_PACKED = (torch.uint32, torch.int32)
_HALF = (torch.bfloat16, torch.float16)
_REAL = (torch.float16, torch.bfloat16, torch.float32)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _out_buffer(out, shape, dtype, device):
    if out is None:
        return torch.empty(shape, dtype=dtype, device=device)
    if (out.dtype != dtype or out.device != device or not out.is_contiguous()
            or out.numel() != prod(shape)):
        raise ValueError(f"out must be a contiguous {dtype} tensor with {prod(shape)} elements")
    return out.view(shape)


def _require_device(op: str, *tensors):
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError(f"{op} requires GPU execution")


def is_w8a8_available() -> bool:
    """True on a gfx950 device (X/src/spark_w8a8.cpp:204-216 answers the same
    question for Apple M5+)."""
    if not torch.cuda.is_available():
        return False
    try:
        return bool(_lib.lib().sparkq_is_available())
    except (RuntimeError, OSError):
        return False


# ---------------------------------------------------------------------------
# W4A16
# ---------------------------------------------------------------------------

def _w4_check(op, x, weight, scales, biases, group_size, bits):
    if any(not isinstance(v, torch.Tensor) for v in (x, weight, scales, biases)):
        raise TypeError("x, weight, scales and biases must be tensors")
    if bits != 4:
        raise ValueError(f"{op}: only 4-bit affine weights are supported (bits={bits})")
    if weight.dtype not in _PACKED or weight.ndim != 2:
        raise ValueError(f"{op} requires UINT32-packed W4 weights of shape [N,K/8]")
    if x.dtype not in _HALF or scales.dtype != x.dtype or biases.dtype != x.dtype:
        raise ValueError(f"{op} requires BF16 or F16 x with scales and biases of the same dtype")
    if x.ndim < 1 or x.shape[-1] <= 0:
        raise ValueError(f"{op} requires x[..., K] with positive K")
    k = x.shape[-1]
    n = weight.shape[0]
    if n <= 0 or weight.shape[1] * 8 != k:
        raise ValueError(f"{op}: weight must have shape [N,K/8] with K={k}")
    if group_size not in (32, 64, 128) or k % group_size:
        raise ValueError(f"{op}: group_size must be 32, 64 or 128 and divide K")
    if scales.shape != (n, k // group_size) or biases.shape != scales.shape:
        raise ValueError(f"{op} requires scales and biases with shape [N,K/{group_size}]")
    if k % 64:
        raise ValueError(f"{op} requires K divisible by 64")
    _require_device(op, x, weight, scales, biases)


def affine_quantized_matmul(x, weight, scales, biases, *, group_size: int = 64,
                            bits: int = 4, transpose: bool = True, out_dtype=None, out=None,
                            prepared=None):
    """y = x @ dequantize(weight)^T for MLX affine packed weights.

    The equivalent of mx.quantized_matmul(x, weight, scales, biases,
    transpose=True, group_size, bits, mode="affine") as called by
    AffineParameters.native (spark_mlx_llm/ops/linear.py:181-191). Any number
    of rows: up to 32 rows stream the weights (decode, speculative verify),
    more rows use the tiled MFMA GEMM (prefill). bits=8 (weight [N,K/4]) runs
    the groupwise W8 affine MFMA kernel that the reference's W8 layers fall
    back to. out_dtype may be
    torch.float32 to read the unrounded fp32 epilogue; out, when given, is a
    contiguous [..., N] tensor written in place. prepared, when given, is
    the derived buffer of prepare_w4a16 for these very scales and biases
    (bf16 only): the prefill GEMM then skips the weight half of its
    prologue; results are bit-identical either way.
    """
    if not transpose:
        raise ValueError("only transpose=True (x @ W^T) is supported")
    op = "affine_quantized_matmul"
    if bits == 8:
        return _w8_affine_matmul(op, x, weight, scales, biases, group_size, out_dtype, out)
    _w4_check(op, x, weight, scales, biases, group_size, bits)
    k = x.shape[-1]
    n = weight.shape[0]
    lead = x.shape[:-1]
    m = prod(lead)
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if out_dtype not in (x.dtype, torch.float32):
        raise ValueError("out_dtype must be x.dtype or torch.float32")
    y = _out_buffer(out, (m, n), out_dtype, x.device)
    if m == 0:
        return y.reshape(*lead, n)
    x2 = x.reshape(m, k).contiguous()
    weight, scales, biases = weight.contiguous(), scales.contiguous(), biases.contiguous()
    ws, wsb = _lib.workspace(x.device, _lib.lib().sparkq_w4a16_workspace_bytes(m, n, k, group_size),
                             "w4a16")
    if prepared is None:
        _lib.call("sparkq_w4a16_linear", _ptr(x2), _ptr(weight), _ptr(scales), _ptr(biases),
                  _ptr(y), m, n, k, group_size, bits, _lib.dtype_code(x.dtype),
                  _lib.dtype_code(out_dtype), ws, wsb, _lib.stream_handle(x.device),
                  device=x.device)
    else:
        _check_prepared(op, prepared, n, k, group_size, x)
        _lib.call("sparkq_w4a16_linear_prepared", _ptr(x2), _ptr(weight), _ptr(scales),
                  _ptr(biases), _ptr(prepared), _ptr(y), m, n, k, group_size, bits,
                  _lib.dtype_code(x.dtype), _lib.dtype_code(out_dtype), ws, wsb,
                  _lib.stream_handle(x.device), device=x.device)
    return y.reshape(*lead, n)


def _check_prepared(op, prepared, n, k, group_size, x):
    need = _lib.lib().sparkq_w4a16_prepared_bytes(n, k, group_size)
    if (not isinstance(prepared, torch.Tensor) or prepared.dtype != torch.uint8
            or prepared.ndim != 1 or prepared.numel() < need or not prepared.is_contiguous()):
        raise ValueError(f"{op}: prepared must be the uint8 buffer of prepare_w4a16 "
                         f"({need} bytes for N={n}, K={k}, group_size={group_size})")
    if x.dtype != torch.bfloat16:
        raise ValueError(f"{op}: a prepared buffer serves bfloat16 activations only")
    if prepared.device != x.device:
        raise ValueError(f"{op}: prepared must live on the activations' device")


def prepare_w4a16(weight, scales, biases, *, group_size: int | None = None):
    """Derived buffer of one W4 projection for the prefill GEMM: the weight
    half of its prologue (scaled fp16 scales, row shifts, bias slots),
    computed once per weight set instead of on every call. The reference
    derives its prepared W4 buffers the same way, once per source arrays
    and outside the checkpoint tree (spark_mlx_llm/ops/linear.py:260-268).
    Returns a uint8 device tensor, or None where no prepared form exists
    (fp16 scales). Costs about (3*K/G + 16) * 2 + 2*K/G + 4 bytes per row
    (6.6 MB for a 19456 x 2560 G64 projection, 24% of its packed bytes)."""
    if any(not isinstance(v, torch.Tensor) for v in (weight, scales, biases)):
        raise TypeError("weight, scales and biases must be tensors")
    if weight.dtype not in _PACKED or weight.ndim != 2 or scales.ndim != 2:
        raise ValueError("prepare_w4a16 requires UINT32-packed W4 weights [N,K/8] and "
                         "scales [N,K/G]")
    n, k = weight.shape[0], weight.shape[1] * 8
    if scales.shape[0] != n or scales.shape[1] <= 0 or k % scales.shape[1]:
        raise ValueError("prepare_w4a16: scales must have shape [N,K/G]")
    g = k // scales.shape[1] if group_size is None else group_size
    if g not in (32, 64, 128) or scales.shape != (n, k // g) or biases.shape != scales.shape:
        raise ValueError("prepare_w4a16: group_size must be 32, 64 or 128 with scales and "
                         "biases [N,K/G]")
    if scales.dtype != torch.bfloat16 or biases.dtype != torch.bfloat16:
        return None
    _require_device("prepare_w4a16", weight, scales, biases)
    need = _lib.lib().sparkq_w4a16_prepared_bytes(n, k, g)
    prepared = torch.empty(need, dtype=torch.uint8, device=scales.device)
    scales, biases = scales.contiguous(), biases.contiguous()
    _lib.call("sparkq_w4a16_prepare", _ptr(scales), _ptr(biases), _ptr(prepared), need, n, k,
              g, BF16, _lib.stream_handle(scales.device), device=scales.device)
    return prepared


def _w8_affine_matmul(op, x, weight, scales, biases, group_size, out_dtype, out):
    """bits=8 branch of affine_quantized_matmul: packed uint32 [N,K/4] codes
    (byte k%4 of word k/4, unsigned), groupwise scales and biases [N,K/G].
    The result dtype follows MLX's promotion of x with the scales (fp32
    scales, as the converter writes for the lm_head, give an fp32 result)."""
    if any(not isinstance(v, torch.Tensor) for v in (x, weight, scales, biases)):
        raise TypeError("x, weight, scales and biases must be tensors")
    if weight.dtype not in _PACKED or weight.ndim != 2:
        raise ValueError(f"{op} requires UINT32-packed W8 weights of shape [N,K/4]")
    if x.dtype not in _HALF:
        raise ValueError(f"{op} requires BF16 or F16 x for 8-bit affine weights")
    if scales.dtype not in _REAL or biases.dtype != scales.dtype:
        raise ValueError(f"{op} requires floating scales and biases of one dtype")
    if x.ndim < 1 or x.shape[-1] <= 0:
        raise ValueError(f"{op} requires x[..., K] with positive K")
    k, n = x.shape[-1], weight.shape[0]
    if n <= 0 or weight.shape[1] * 4 != k:
        raise ValueError(f"{op}: weight must have shape [N,K/4] with K={k}")
    if group_size not in (32, 64, 128) or k % group_size:
        raise ValueError(f"{op}: group_size must be 32, 64 or 128 and divide K")
    if scales.shape != (n, k // group_size) or biases.shape != scales.shape:
        raise ValueError(f"{op} requires scales and biases with shape [N,K/{group_size}]")
    _require_device(op, x, weight, scales, biases)
    result = torch.promote_types(x.dtype, scales.dtype)
    out_dtype = result if out_dtype is None else out_dtype
    if out_dtype not in (result, torch.float32):
        raise ValueError(f"out_dtype must be {result} or torch.float32")
    lead = x.shape[:-1]
    m = prod(lead)
    y = _out_buffer(out, (m, n), out_dtype, x.device)
    if m == 0:
        return y.reshape(*lead, n)
    x2 = x.reshape(m, k).contiguous()
    weight, scales, biases = weight.contiguous(), scales.contiguous(), biases.contiguous()
    _lib.call("sparkq_w8_affine_linear", _ptr(x2), _ptr(weight), _ptr(scales), _ptr(biases),
              _ptr(y), m, n, k, group_size, _lib.dtype_code(x.dtype),
              _lib.dtype_code(scales.dtype), _lib.dtype_code(out_dtype),
              _lib.stream_handle(x.device), device=x.device)
    return y.reshape(*lead, n)


def w4a16_qmv(x, weight, scales, biases, *, stream=None):
    """One-row affine W4 GEMV (X/spark_mlx_ext/w4a16_qmv.py:37-98).

    Widened from the reference's BF16/G32/K%512 specialisation: group size is
    read from the scales shape (32, 64 or 128), K % 64 == 0, BF16 or F16.
    """
    if any(not isinstance(v, torch.Tensor) for v in (x, weight, scales, biases)):
        raise TypeError("x, weight, scales and biases must be tensors")
    if x.ndim < 1 or prod(x.shape[:-1]) != 1:
        raise ValueError("W4A16 QMV requires exactly one activation row")
    if weight.ndim != 2:
        raise ValueError("W4A16 packed weight must have shape [N,K/8]")
    if scales.ndim != 2 or scales.shape[1] <= 0:
        raise ValueError("W4A16 QMV requires scales and biases with shape [N,K/G]")
    group_size = x.shape[-1] // scales.shape[1]
    return affine_quantized_matmul(x, weight, scales, biases, group_size=group_size, bits=4)


_MULTIROW_ALGORITHMS = ("wide", "p2", "mma", "mma2", "nax", "nax2", "nax4", "split_p2")


def w4a16_multirow(x, weight, scales, biases, *, algorithm: str = "wide", **tuning):
    """Multi-row (speculative verify) affine W4 projection
    (X/spark_mlx_ext/w4a16_multirow.py:238-437).

    The reference selects among eight Apple-specific algorithms; on gfx950 a
    single MFMA weight-streaming kernel serves every row count up to 32, so the
    algorithm name is validated and the tuning keywords are accepted unused.
    """
    if algorithm not in _MULTIROW_ALGORITHMS:
        raise ValueError(f"Unknown multirow algorithm {algorithm!r}")
    if x.ndim < 1 or not 1 <= prod(x.shape[:-1]) <= 32:
        raise ValueError("W4A16 multirow requires between 1 and 32 activation rows")
    group_size = x.shape[-1] // scales.shape[1]
    return affine_quantized_matmul(x, weight, scales, biases, group_size=group_size, bits=4)


def prepare_w4a16_nax4(weight, scales, biases):
    """The reference repacks nibbles into [N/256][K/32][32k][256n] tiles for its
    tensor-op kernel (X/spark_mlx_ext/w4a16_multirow.py:181-222). The gfx950
    kernels read the converter's native [N,K/8] layout with 16-byte loads, so
    the prepared form is the input itself."""
    return weight, scales, biases


def affine_quantize(w, *, group_size: int = 64, bits: int = 4):
    """Quantize BF16/F16 weights [N,K] into the MLX affine 4-bit layout on the
    GPU with the benchmark's formula: per group, scale = (max-min)/15 and
    bias = min, both rounded to w.dtype, codes rint((w-bias)/scale) clamped
    to 0..15. The layout is the one mx.quantize(bits=4) fills for the
    reference (spark_mlx_llm/dspark/draft_quantization.py:119), but the
    tuple is not MLX's: mx.quantize makes the group's larger-magnitude edge
    exactly representable (a negative scale when that edge is the minimum,
    bias equal to the edge), so its codes, scales and biases differ from
    these. Any tuple in this layout runs through the same kernels; bit
    identity with mx.quantize is unpinned (MLX is not available here)."""
    if bits != 4:
        raise ValueError("only 4-bit affine quantization is supported")
    if w.ndim != 2 or w.dtype not in _HALF:
        raise ValueError("w must be a BF16 or F16 matrix [N,K]")
    n, k = w.shape
    if group_size not in (32, 64, 128) or k % group_size:
        raise ValueError("group_size must be 32, 64 or 128 and divide K")
    _require_device("affine_quantize", w)
    w = w.contiguous()
    wq = torch.empty((n, k // 8), dtype=torch.uint32, device=w.device)
    s = torch.empty((n, k // group_size), dtype=w.dtype, device=w.device)
    b = torch.empty_like(s)
    _lib.call("sparkq_w4_quantize", _ptr(w), _ptr(wq), _ptr(s), _ptr(b), n, k, group_size,
              _lib.dtype_code(w.dtype), _lib.stream_handle(w.device), device=w.device)
    return wq, s, b


def affine_dequantize(weight, scales, biases, *, group_size: int = 64, bits: int = 4):
    """Exact fp32 dequantization q*s+b of MLX affine 4-bit weights."""
    if bits != 4 or weight.dtype not in _PACKED or weight.ndim != 2:
        raise ValueError("expected UINT32-packed 4-bit weights [N,K/8]")
    n, k = weight.shape[0], weight.shape[1] * 8
    if scales.dtype not in _HALF or biases.dtype != scales.dtype:
        raise ValueError("scales and biases must be BF16 or F16")
    if scales.shape != (n, k // group_size) or biases.shape != scales.shape:
        raise ValueError("scales and biases must have shape [N,K/group_size]")
    _require_device("affine_dequantize", weight, scales, biases)
    out = torch.empty((n, k), dtype=torch.float32, device=weight.device)
    weight, scales, biases = weight.contiguous(), scales.contiguous(), biases.contiguous()
    _lib.call("sparkq_w4a16_dequantize", _ptr(weight), _ptr(scales),
              _ptr(biases), _ptr(out), n, k, group_size,
              _lib.dtype_code(scales.dtype), _lib.stream_handle(weight.device), device=weight.device)
    return out


# ---------------------------------------------------------------------------
# W8A8
# ---------------------------------------------------------------------------

def _validate_dimensions(x, weight):
    """X/src/spark_w8a8.cpp:51-65"""
    if (x.ndim < 1 or weight.ndim != 2 or x.shape[-1] <= 0 or weight.shape[0] <= 0
            or x.numel() == 0 or x.shape[-1] != weight.shape[1]):
        raise ValueError("Expected nonempty x[..., K] and weight[N, K] with matching K.")
    if x.shape[-1] % 32 or x.shape[-1] > 131040:
        raise ValueError("K must be a multiple of 32 in [32, 131040].")
    if weight.dtype != torch.int8:
        raise ValueError("weight must contain signed INT8 values.")


def quantize_per_token(x):
    """Per-token symmetric int8 activations (X/src/kernels/w8a8_quantize.metal):
    returns (q int8 [M,K], scales fp32 [M]) for x [..., K]."""
    if x.dtype not in _REAL:
        raise ValueError("x must have dtype float16, bfloat16, or float32.")
    _require_device("quantize_per_token", x)
    k = x.shape[-1]
    m = x.numel() // k
    x2 = x.reshape(m, k).contiguous()
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    sc = torch.empty((m,), dtype=torch.float32, device=x.device)
    _lib.call("sparkq_a8_quantize_per_token", _ptr(x2), _ptr(q), _ptr(sc), m, k,
              _lib.dtype_code(x.dtype), _lib.stream_handle(x.device), device=x.device)
    return q, sc


def int8_matmul_int32(x, weight, *, stream=None):
    """Raw int32 x[M,K] @ weight[N,K]^T (X/src/spark_w8a8.cpp:218-228)."""
    _validate_dimensions(x, weight)
    if x.ndim != 2 or x.dtype != torch.int8:
        raise ValueError("int8_matmul_int32 requires x[M, K] with dtype int8.")
    _require_device("int8_matmul_int32", x, weight)
    m, k = x.shape
    n = weight.shape[0]
    c = torch.empty((m, n), dtype=torch.int32, device=x.device)
    ws, wsb = _lib.workspace(x.device, _lib.lib().sparkq_int8_matmul_workspace_bytes(m, n, k),
                             "i8mm")
    x, weight = x.contiguous(), weight.contiguous()
    _lib.call("sparkq_int8_matmul_i32", _ptr(x), _ptr(weight),
              _ptr(c), m, n, k, ws, wsb, _lib.stream_handle(x.device), device=x.device)
    return c


def w8a8_linear(x, weight, scales, bias=None, *, stream=None, out_dtype=None, out=None):
    """Per-token int8 activations x per-channel int8 weights, int32 MACs, then
    T(float(acc)*sa[m]*sw[n] + bias[n]) (X/src/spark_w8a8.cpp:230-257)."""
    _validate_dimensions(x, weight)
    n, k = weight.shape
    if x.dtype not in _REAL:
        raise ValueError("x must have dtype float16, bfloat16, or float32.")
    if scales.dtype != torch.float32 or tuple(scales.shape) not in ((n,), (n, 1)):
        raise ValueError("scales must have shape [N] or [N, 1] and dtype float32.")
    if bias is not None and (tuple(bias.shape) != (n,) or bias.dtype not in _REAL):
        raise ValueError("bias must have shape [N] and a real floating dtype.")
    _require_device("w8a8_linear", x, weight, scales, bias)
    out_dtype = x.dtype if out_dtype is None else out_dtype
    lead = x.shape[:-1]
    m = prod(lead)
    x2 = x.reshape(m, k).contiguous()
    y = _out_buffer(out, (m, n), out_dtype, x.device)
    ws, wsb = _lib.workspace(x.device, _lib.lib().sparkq_w8a8_workspace_bytes(m, n, k), "w8a8")
    bias_c = bias.contiguous() if bias is not None else None
    weight, scales = weight.contiguous(), scales.reshape(n).contiguous()
    _lib.call("sparkq_w8a8_linear", _ptr(x2), _ptr(weight),
              _ptr(scales), _ptr(bias_c),
              _lib.dtype_code(bias.dtype) if bias is not None else F32, _ptr(y), m, n, k,
              _lib.dtype_code(x.dtype), _lib.dtype_code(out_dtype), ws, wsb,
              _lib.stream_handle(x.device), device=x.device)
    return y.reshape(*lead, n)


class W8A8Linear(nn.Module):
    """Linear layer over existing symmetric per-channel INT8 weights
    (X/spark_mlx_ext/linear.py:9-55): weight int8 [N,K], scales fp32 [N] or
    [N,1], optional floating bias [N]. Inference only."""

    def __init__(self, weight, scales, bias=None):
        super().__init__()
        if weight.ndim != 2 or weight.dtype != torch.int8:
            raise ValueError("weight must be an INT8 matrix [N, K]")
        n, k = weight.shape
        if n <= 0 or k <= 0 or k % 32 or k > 131040:
            raise ValueError("N must be positive; K must be a multiple of 32 in [32, 131040]")
        if scales.dtype != torch.float32 or tuple(scales.shape) not in ((n,), (n, 1)):
            raise ValueError("scales must be FP32 with shape [N] or [N, 1]")
        if bias is not None and (tuple(bias.shape) != (n,) or bias.dtype not in _REAL):
            raise ValueError("bias must be a floating array of shape [N]")
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("bias", bias)
        self.requires_grad_(False)

    @property
    def input_dims(self) -> int:
        return self.weight.shape[1]

    @property
    def output_dims(self) -> int:
        return self.weight.shape[0]

    def forward(self, x):
        return w8a8_linear(x, self.weight, self.scales, self.bias)

    def extra_repr(self) -> str:
        return (f"input_dims={self.input_dims}, output_dims={self.output_dims}, "
                f"bias={self.bias is not None}")


# ---------------------------------------------------------------------------
# W8A16
# ---------------------------------------------------------------------------

def w8a16_per_channel(x, weight, scales, *, stream=None, out_dtype=None, out=None):
    """Signed int8 weights [N,K] with an fp32 scale per output channel times
    16-bit activations: y = T(scale[n] * sum_k x[k] * w[n,k])
    (X/src/spark_w8a16.cpp:80-110; checks as there). The reference takes one
    activation row; up to 4 rows are accepted here (short verify batches)."""
    if (x.ndim < 1 or weight.ndim != 2 or x.shape[-1] <= 0 or weight.shape[0] <= 0
            or weight.shape[1] != x.shape[-1] or not 1 <= x.numel() // x.shape[-1] <= 4):
        raise ValueError(
            "w8a16_per_channel requires one activation row x[..., K] with singleton leading "
            "dimensions and nonempty weight[N, K].")
    if x.dtype not in _HALF:
        raise ValueError("w8a16_per_channel x must have dtype bfloat16 or float16.")
    if weight.dtype != torch.int8:
        raise ValueError("w8a16_per_channel weight must have dtype int8.")
    n, k = weight.shape
    if scales.dtype != torch.float32 or tuple(scales.shape) not in ((n,), (n, 1)):
        raise ValueError(
            "w8a16_per_channel scales must have dtype float32 and shape [N] or [N, 1].")
    _require_device("w8a16_per_channel", x, weight, scales)
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if out_dtype not in (x.dtype, torch.float32):
        raise ValueError("out_dtype must be x.dtype or torch.float32")
    lead = x.shape[:-1]
    m = prod(lead)
    x2 = x.reshape(m, k).contiguous()
    y = _out_buffer(out, (m, n), out_dtype, x.device)
    weight, scales = weight.contiguous(), scales.reshape(n).contiguous()
    _lib.call("sparkq_w8a16_linear", _ptr(x2), _ptr(weight), _ptr(scales), _ptr(y), m, n, k,
              _lib.dtype_code(x.dtype), _lib.dtype_code(out_dtype), _lib.stream_handle(x.device), device=x.device)
    return y.reshape(*lead, n)


# ---------------------------------------------------------------------------
# INT8-KV decode attention
# ---------------------------------------------------------------------------

def kv_quantize_s8(x):
    """Symmetric int8 KV rows: codes int8 [..., D] and fp16 scales [...] with
    scale = fp16(amax/127) (1 when zero) and codes from the rounded scale."""
    if x.dtype not in _REAL:
        raise ValueError("x must be float16, bfloat16 or float32")
    _require_device("kv_quantize_s8", x)
    d = x.shape[-1]
    r = x.numel() // d
    x2 = x.reshape(r, d).contiguous()
    codes = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    sc = torch.empty(x.shape[:-1], dtype=torch.float16, device=x.device)
    _lib.call("sparkq_kv_quantize_s8", _ptr(x2), _ptr(codes), _ptr(sc), r, d,
              _lib.dtype_code(x.dtype), _lib.stream_handle(x.device), device=x.device)
    return codes, sc


def _int8_prefill_affine(queries, keys, values, *, scale, causal, group_size, bits, out_dtype,
                         out):
    """L > 1 queries over the MLX affine 8-bit cache: the prefill branch of
    X/spark_mlx_ext/int8_quantized_sdpa.py:236-245 and its kernel
    spark_affine_u8_sdpa_prefill (int8_quantized_sdpa_prefill.py:44-57). K/V
    dequantize to the query dtype, weights are rounded to it for PV; scores,
    normalizer and output accumulate in fp32."""
    batch, heads, length, dim = queries.shape
    kv_heads, n = keys[0].shape[1:3]
    if bits != 8 or group_size not in (32, 64, 128):
        raise ValueError("Supported affine formats: bits 8, group size 32/64/128")
    if queries.dtype not in _HALF:
        raise ValueError("multi-token INT8-KV attention needs float16 or bfloat16 queries")
    if dim not in (64, 128, 256):
        raise ValueError("multi-token INT8-KV attention needs a head dim of 64, 128 or 256")
    if causal and length > n:
        raise ValueError("a causal mask needs L <= N")
    for name, (packed, s, b) in (("key", keys), ("value", values)):
        if (dim % group_size or packed.shape != (batch, kv_heads, n, dim // 4)
                or s.shape != (batch, kv_heads, n, dim // group_size)
                or b.shape != s.shape or packed.dtype not in _PACKED
                or s.dtype != queries.dtype or b.dtype != queries.dtype
                or s.stride() != b.stride()):
            raise ValueError(f"Incompatible {name} packed shape, affine metadata or dtype")
        if packed.stride(3) != 1 or s.stride(3) != 1:
            raise ValueError(f"{name} innermost axis must be contiguous")
    (kc, ks, kb), (vc, vs, vb) = keys, values
    _require_device("int8_quantized_sdpa", queries, kc, ks, kb, vc, vs, vb)
    out_dtype = queries.dtype if out_dtype is None else out_dtype
    q = queries.contiguous()
    y = _out_buffer(out, (batch, heads, length, dim), out_dtype, queries.device)
    st = (ctypes.c_int64 * 12)(*(_kv_strides(kc, ks, 4) + _kv_strides(vc, vs, 4)))
    c = 1 if causal else 0
    ws, wsb = _lib.workspace(queries.device,
                             _lib.lib().sparkq_int8kv_sdpa_prefill_affine_workspace_bytes(
                                 batch, heads, kv_heads, length, n, dim, c),
                             "sdpa_prefill")
    _lib.call("sparkq_int8kv_sdpa_prefill_affine", _ptr(q), _ptr(kc), _ptr(ks), _ptr(kb),
              _ptr(vc), _ptr(vs), _ptr(vb), _ptr(y), batch, heads, kv_heads, length, n, dim,
              group_size, c, _lib.dtype_code(queries.dtype), _lib.dtype_code(out_dtype),
              float(scale), st, ws, wsb, _lib.stream_handle(queries.device), device=queries.device)
    return y


def _int8_prefill(queries, keys, values, *, scale, causal, fmt, out_dtype, out,
                  group_size=32, bits=8):
    """L > 1 queries (the prefill branch of
    X/spark_mlx_ext/int8_quantized_sdpa.py:236-245): tiled QK, online softmax
    and PV in one launch, bottom-right causal or unmasked. The MLX affine
    tuple goes to _int8_prefill_affine; this body serves the symmetric s8
    cache."""
    if fmt == KV_AFFINE_U8:
        return _int8_prefill_affine(queries, keys, values, scale=scale, causal=causal,
                                    group_size=group_size, bits=bits, out_dtype=out_dtype,
                                    out=out)
    batch, heads, length, dim = queries.shape
    kv_heads, n = keys[0].shape[1:3]
    if queries.dtype not in _HALF:
        raise ValueError("multi-token INT8-KV attention needs float16 or bfloat16 queries")
    if causal and length > n:
        raise ValueError("a causal mask needs L <= N")
    for name, (codes, s) in (("key", keys), ("value", values)):
        if (codes.shape != (batch, kv_heads, n, dim) or codes.dtype != torch.int8
                or s.shape != (batch, kv_heads, n) or s.dtype != torch.float16):
            raise ValueError(f"Incompatible {name} int8 codes or fp16 scales")
        if codes.stride(3) != 1:
            raise ValueError(f"{name} innermost axis must be contiguous")
    (kc, ks), (vc, vs) = keys, values
    _require_device("int8_quantized_sdpa", queries, kc, ks, vc, vs)
    out_dtype = queries.dtype if out_dtype is None else out_dtype
    q = queries.contiguous()
    y = _out_buffer(out, (batch, heads, length, dim), out_dtype, queries.device)
    st = (ctypes.c_int64 * 12)(*(_kv_strides(kc, ks, 1) + _kv_strides(vc, vs, 1)))
    _lib.call("sparkq_int8kv_sdpa_prefill", _ptr(q), _ptr(kc), _ptr(ks), _ptr(vc), _ptr(vs),
              _ptr(y), batch, heads, kv_heads, length, n, dim, 1 if causal else 0,
              _lib.dtype_code(queries.dtype), _lib.dtype_code(out_dtype), float(scale), st,
              _lib.stream_handle(queries.device), device=queries.device)
    return y


def kv_append(x, cache, offset: int, *, group_size: int = 32, bits: int = 8):
    """Quantize x [B,H,L,D] into tokens [offset, offset+L) of a preallocated
    cache, in place: cache is (codes int8 [B,H,Ncap,D], scales fp16
    [B,H,Ncap]) for the symmetric format, or the MLX affine tuple of `bits`
    (8, 4 or 2) bits (packed uint32 [B,H,Ncap,D*bits/32], scales, biases
    [B,H,Ncap,D/G] in x.dtype). The quantize-on-append step of mlx-lm's
    QuantizedKVCache."""
    if x.ndim != 4 or x.numel() == 0:
        raise ValueError("x must be a nonempty [B,H,L,D] tensor")
    b, h, length, d = x.shape
    fmt = KV_AFFINE_U8 if len(cache) == 3 else KV_S8_F16SCALE
    if fmt == KV_AFFINE_U8 and bits not in (2, 4, 8):
        raise ValueError("Supported affine formats: bits 2/4/8, group size 32/64/128")
    wpr = d * bits // 32  # packed words per token row
    codes, scales = cache[0], cache[1]
    biases = cache[2] if fmt == KV_AFFINE_U8 else None
    ncap = codes.shape[2]
    if offset < 0 or offset + length > ncap:
        raise ValueError(f"tokens [{offset}, {offset + length}) exceed the cache capacity {ncap}")
    if fmt == KV_AFFINE_U8:
        if x.dtype not in _HALF or scales.dtype != x.dtype or biases.dtype != x.dtype:
            raise ValueError("affine KV needs float16 or bfloat16 x, scales and biases")
        if (codes.shape != (b, h, ncap, wpr) or codes.dtype not in _PACKED
                or scales.shape != (b, h, ncap, d // group_size) or biases.shape != scales.shape
                or scales.stride() != biases.stride() or d % group_size):
            raise ValueError("Incompatible affine KV cache for this input")
        strides = _kv_strides(codes, scales, 4)
        fmt = {8: KV_AFFINE_U8, 4: KV_AFFINE_U4, 2: KV_AFFINE_U2}[bits]
    else:
        if x.dtype not in _REAL:
            raise ValueError("x must be float16, bfloat16 or float32")
        if (codes.shape != (b, h, ncap, d) or codes.dtype != torch.int8
                or scales.shape != (b, h, ncap) or scales.dtype != torch.float16):
            raise ValueError("Incompatible int8 KV cache for this input")
        strides = _kv_strides(codes, scales, 1)
    if codes.stride(3) != 1 or (fmt != KV_S8_F16SCALE and scales.stride(-1) != 1):
        raise ValueError("the cache's innermost axes must be contiguous")
    _require_device("kv_append", x, codes, scales, biases)
    st = (ctypes.c_int64 * 6)(*strides)
    _lib.call("sparkq_kv_append", _ptr(x.contiguous()), _ptr(codes), _ptr(scales), _ptr(biases),
              b, h, length, d, offset, group_size, fmt, _lib.dtype_code(x.dtype), st,
              _lib.stream_handle(x.device), device=x.device)


class QuantizedKVCache:
    """Quantize-on-append INT8 KV cache with the interface of mlx-lm 0.31.3's
    QuantizedKVCache (used by spark_mlx_llm/generation.py:13,377):
    update_and_fetch(keys, values) quantizes [B,Hkv,L,D] keys and values on the
    device into storage that grows in steps of 256 tokens and returns views of
    tokens [0, offset), ready for int8_quantized_sdpa. kv_format "affine_u8"
    keeps MLX's (packed, scales, biases) tuples with group_size and bits
    (8, 4 or 2; mlx-lm's kv_bits); "s8" the symmetric (codes, fp16 scale)
    pairs of the decode benchmark."""

    step = 256

    def __init__(self, group_size: int = 32, bits: int = 8, kv_format: str = "affine_u8"):
        if kv_format not in ("affine_u8", "s8"):
            raise ValueError("kv_format must be 'affine_u8' or 's8'")
        if bits not in ((2, 4, 8) if kv_format == "affine_u8" else (8,)):
            raise ValueError("affine KV caches take bits 2, 4 or 8; the s8 format 8")
        if kv_format == "affine_u8" and group_size not in (32, 64, 128):
            raise ValueError("group_size must be 32, 64 or 128")
        self.group_size, self.bits, self.kv_format = group_size, bits, kv_format
        self.keys = self.values = None
        self.offset = 0

    def _alloc(self, x, capacity):
        b, h, _, d = x.shape
        dev = x.device
        if self.kv_format == "s8":
            return (torch.zeros((b, h, capacity, d), dtype=torch.int8, device=dev),
                    torch.zeros((b, h, capacity), dtype=torch.float16, device=dev))
        g = self.group_size
        return (torch.zeros((b, h, capacity, d * self.bits // 32), dtype=torch.int32, device=dev),
                torch.zeros((b, h, capacity, d // g), dtype=x.dtype, device=dev),
                torch.zeros((b, h, capacity, d // g), dtype=x.dtype, device=dev))

    def _grow(self, old, x, capacity):
        new = self._alloc(x, capacity)
        if old is not None:
            for dst, src in zip(new, old):
                dst[:, :, : self.offset] = src[:, :, : self.offset]
        return new

    def update_and_fetch(self, keys, values):
        if keys.ndim != 4 or values.ndim != 4 or keys.shape[:3] != values.shape[:3]:
            raise ValueError("keys and values must be [B,Hkv,L,D] with matching B, Hkv and L")
        length = keys.shape[2]
        if self.kv_format == "affine_u8" and (keys.shape[-1] % self.group_size
                                              or values.shape[-1] % self.group_size):
            raise ValueError("head dims must be multiples of group_size")
        cap = self.keys[0].shape[2] if self.keys is not None else 0
        if self.keys is None or self.offset + length > cap:
            capacity = -(-(self.offset + length) // self.step) * self.step
            self.keys = self._grow(self.keys, keys, capacity)
            self.values = self._grow(self.values, values, capacity)
        kv_append(keys, self.keys, self.offset, group_size=self.group_size, bits=self.bits)
        kv_append(values, self.values, self.offset, group_size=self.group_size, bits=self.bits)
        self.offset += length
        n = self.offset
        return (tuple(t[:, :, :n] for t in self.keys), tuple(t[:, :, :n] for t in self.values))

    @property
    def state(self):
        return self.keys, self.values


def _kv_strides(codes, scales, elem_bytes_codes):
    st = codes.stride()
    ss = scales.stride()
    return [st[0] * elem_bytes_codes, st[1] * elem_bytes_codes, st[2] * elem_bytes_codes,
            ss[0], ss[1], ss[2]]


def staged_quantized_sdpa(queries, keys, values, *, scale, group_size: int = 32, bits: int = 8,
                          mask=None, out_dtype=None, out=None):
    """Attention over an MLX affine quantized cache in the staged form
    (dequantized keys, scores, softmax, weights times values), whatever the
    fused 8-bit predicate would choose: what mlx-lm's quantized attention
    computes for the reference when its fused kernel is switched off
    (spark_mlx_llm/ops/sdpa.py:39-78 with fused_quantized_sdpa=False), and
    the reference's own _fallback (X/spark_mlx_ext/int8_quantized_sdpa.py:
    122-153). 4- and 2-bit caches at one query token still take the decode
    kernel on their codes, which computes the same arithmetic in one pass.
    Validates as int8_quantized_sdpa does for the affine tuple."""
    if len(keys) != 3:
        raise ValueError("the staged form takes the affine (packed, scales, biases) tuple")
    return int8_quantized_sdpa(queries, keys, values, scale=scale, group_size=group_size,
                               bits=bits, mask=mask, out_dtype=out_dtype, out=out,
                               _allow_fused=False)


def int8_quantized_sdpa(queries, keys, values, *, scale, group_size: int = 32, bits: int = 8,
                        mask=None, single_pass_max_length: int = 1023, out_dtype=None,
                        out=None, _allow_fused: bool = True):
    """Attention over a quantized KV cache
    (X/spark_mlx_ext/int8_quantized_sdpa.py:156-287).

    queries [B,Hq,L,D]. keys/values are either the MLX affine tuple
    (packed uint32 [B,Hkv,N,D*bits/32], scales [B,Hkv,N,D/G], biases) with
    scales in the query dtype, or the symmetric pair (codes int8 [B,Hkv,N,D],
    scales fp16 [B,Hkv,N]). Views with a sliced token capacity are read in
    place (strides are passed through); the innermost axis must be
    contiguous. As in the reference, the affine tuple takes the fused kernels
    when bits == 8, the head dims are equal and 64/128/256 (the reference:
    256 only), the query-to-KV head ratio is 1/2/4/8 and the mask is None or
    "causal" (multi-token queries: 16-bit, and L <= N when causal); every
    other supported combination (bits 2/4, any head dims that are multiples
    of the group size, boolean or additive mask arrays, any head ratio) takes
    the staged attention kernel, the reference's _fallback (:122-153).
    single_pass_max_length is validated for signature compatibility; the
    split policy is the kernels' own.
    """
    if type(single_pass_max_length) is not int or single_pass_max_length < 0:
        raise ValueError("single_pass_max_length must be a nonnegative Python int")
    if queries.ndim != 4 or len(keys) not in (2, 3) or len(values) != len(keys):
        raise ValueError("Expected Q[B,H,L,D] and affine (packed, scales, biases) KV tuples")
    batch, heads, length, dim = queries.shape
    if any(t.ndim != 4 for t in (*keys, *values)) and len(keys) == 3:
        raise ValueError("Every packed KV and metadata array must have four dimensions")
    if any(t.ndim != 4 for t in (keys[0], values[0])):
        raise ValueError("Every packed KV and metadata array must have four dimensions")
    kv_heads, n = keys[0].shape[1:3]
    if min(batch, heads, length, dim, kv_heads, n) <= 0 or heads % kv_heads:
        raise ValueError("Nonempty inputs and query heads divisible by KV heads required")
    if not isinstance(scale, (float, int)) or not math.isfinite(scale):
        raise ValueError("scale must be a finite Python number")
    simple_mask = mask is None or (isinstance(mask, str) and mask == "causal")
    if isinstance(mask, str) and mask != "causal":
        raise ValueError("mask string must be 'causal'")
    if queries.dtype not in _REAL:
        raise ValueError("Q and metadata must be float16, bfloat16 or float32")
    if len(keys) == 2:
        if not simple_mask:
            raise ValueError("the symmetric int8 cache takes mask=None or mask='causal'")
        return _s8_attention(queries, keys, values, scale=scale, causal=mask is not None,
                             out_dtype=out_dtype, out=out)
    # the MLX affine tuple: the reference's validation (:188-224)
    if bits not in (2, 4, 8) or group_size not in (32, 64, 128):
        raise ValueError("Supported affine formats: bits 2/4/8, group size 32/64/128")
    pack = 32 // bits
    dv = values[0].shape[-1] * pack
    for name, (packed, s, b) in (("key", keys), ("value", values)):
        width = dim if name == "key" else dv
        if (width <= 0 or width % group_size
                or packed.shape != (batch, kv_heads, n, width // pack)
                or s.shape != (batch, kv_heads, n, width // group_size)
                or b.shape != s.shape or packed.dtype not in _PACKED
                or s.dtype != queries.dtype or b.dtype != queries.dtype
                or s.stride() != b.stride()):
            raise ValueError(f"Incompatible {name} packed shape, affine metadata or dtype")
        if packed.stride(3) != 1 or s.stride(3) != 1:
            raise ValueError(f"{name} innermost axis must be contiguous")
    gqa = heads // kv_heads
    fused = (_allow_fused and bits == 8 and dim == dv and dim in (64, 128, 256)
             and gqa in (1, 2, 4, 8)
             and simple_mask
             and (length == 1 or (queries.dtype in _HALF and (mask is None or length <= n))))
    # 4- and 2-bit caches at one query token: the decode kernel on their
    # codes (the staged form's arithmetic in one pass; the reference sends
    # them to its _fallback, whose M=1 quantized matmuls stream the cache)
    low_bit_decode = (bits in (2, 4) and length == 1 and dim == dv and dim in (64, 128, 256)
                      and gqa in (1, 2, 4, 8) and simple_mask)
    if low_bit_decode:
        strides = (_kv_strides(keys[0], keys[1], 4) + _kv_strides(values[0], values[1], 4))
        (kc, ks, kb), (vc, vs, vb) = keys, values
        return _decode(queries, kc, ks, kb, vc, vs, vb, strides, group_size,
                       KV_AFFINE_U4 if bits == 4 else KV_AFFINE_U2, scale, out_dtype, out)
    if not fused:
        return _staged_attention(queries, keys, values, scale=scale, group_size=group_size,
                                 bits=bits, mask=mask, out_dtype=out_dtype, out=out)
    if length > 1:
        return _int8_prefill_affine(queries, keys, values, scale=scale, causal=mask is not None,
                                    group_size=group_size, bits=bits, out_dtype=out_dtype,
                                    out=out)
    strides = (_kv_strides(keys[0], keys[1], 4) + _kv_strides(values[0], values[1], 4))
    (kc, ks, kb), (vc, vs, vb) = keys, values
    return _decode(queries, kc, ks, kb, vc, vs, vb, strides, group_size, KV_AFFINE_U8, scale,
                   out_dtype, out)


def _decode(queries, kc, ks, kb, vc, vs, vb, strides, group_size, fmt, scale, out_dtype, out):
    batch, heads, _, dim = queries.shape
    kv_heads, n = kc.shape[1:3]
    _require_device("int8_quantized_sdpa", queries, kc, ks, kb, vc, vs, vb)
    out_dtype = queries.dtype if out_dtype is None else out_dtype
    q = queries.reshape(batch, heads, dim).contiguous()
    out = _out_buffer(out, (batch, heads, 1, dim), out_dtype, queries.device)
    st = (ctypes.c_int64 * 12)(*strides)
    ws, wsb = _lib.workspace(queries.device,
                             _lib.lib().sparkq_int8kv_sdpa_workspace_bytes(batch, heads, n, dim),
                             "sdpa")
    _lib.call("sparkq_int8kv_sdpa_decode", _ptr(q), _ptr(kc), _ptr(ks), _ptr(kb), _ptr(vc),
              _ptr(vs), _ptr(vb), _ptr(out), batch, heads, kv_heads, n, dim, group_size, fmt,
              _lib.dtype_code(queries.dtype), _lib.dtype_code(out_dtype), float(scale), st,
              ws, wsb, _lib.stream_handle(queries.device), device=queries.device)
    return out


def _s8_attention(queries, keys, values, *, scale, causal, out_dtype, out):
    """The symmetric int8 + fp16-scale cache (the decode benchmark's format):
    one query token on the decode kernels, several on the s8 prefill kernel."""
    batch, heads, length, dim = queries.shape
    kv_heads, n = keys[0].shape[1:3]
    if length > 1:
        return _int8_prefill(queries, keys, values, scale=scale, causal=causal,
                             fmt=KV_S8_F16SCALE, out_dtype=out_dtype, out=out)
    for name, (codes, s) in (("key", keys), ("value", values)):
        if (codes.shape != (batch, kv_heads, n, dim) or codes.dtype != torch.int8
                or s.shape != (batch, kv_heads, n) or s.dtype != torch.float16):
            raise ValueError(f"Incompatible {name} int8 codes or fp16 scales")
        if codes.stride(3) != 1:
            raise ValueError(f"{name} innermost axis must be contiguous")
    strides = (_kv_strides(keys[0], keys[1], 1) + _kv_strides(values[0], values[1], 1))
    (kc, ks), (vc, vs) = keys, values
    return _decode(queries, kc, ks, None, vc, vs, None, strides, 32, KV_S8_F16SCALE, scale,
                   out_dtype, out)


_MASK_NONE, _MASK_CAUSAL, _MASK_BOOL, _MASK_ADD = 0, 1, 2, 3


def _staged_attention(queries, keys, values, *, scale, group_size, bits, mask, out_dtype, out):
    """The reference's staged _fallback (X/spark_mlx_ext/int8_quantized_sdpa.py:
    122-153) on the gfx950 staged-attention kernel: any bits in 2/4/8, head
    dims that are multiples of the group size (keys and values may differ),
    any head ratio, and masks None, "causal" (bottom-right), boolean arrays
    (False hides a token: its score becomes the dtype's lowest value, as
    mx.where does) or additive arrays broadcastable to [B,Hq,L,N]."""
    batch, heads, length, dim = queries.shape
    kv_heads, n = keys[0].shape[1:3]
    dv = values[0].shape[-1] * (32 // bits)
    (kc, ks, kb), (vc, vs, vb) = keys, values
    mask_t, mstrides, kind, mdt = None, None, _MASK_NONE, F32
    if isinstance(mask, str):
        kind = _MASK_CAUSAL
    elif mask is not None:
        if not isinstance(mask, torch.Tensor) or mask.ndim > 4:
            raise ValueError("mask must be None, 'causal' or an array of at most 4 dimensions")
        if mask.dtype == torch.bool:
            kind = _MASK_BOOL
        elif mask.dtype in _REAL:
            kind, mdt = _MASK_ADD, _lib.dtype_code(mask.dtype)
        else:
            raise ValueError("mask arrays must be boolean or floating")
        try:
            mask_t = torch.broadcast_to(mask.to(queries.device), (batch, heads, length, n))
        except RuntimeError as err:
            raise ValueError(f"mask of shape {tuple(mask.shape)} does not broadcast to "
                             f"{(batch, heads, length, n)}") from err
        if kind == _MASK_BOOL:
            mask_t = mask_t.view(torch.uint8)
        mstrides = (ctypes.c_int64 * 4)(*mask_t.stride())
    _require_device("int8_quantized_sdpa", queries, kc, ks, kb, vc, vs, vb, mask_t)
    out_dtype = queries.dtype if out_dtype is None else out_dtype
    if out_dtype not in (queries.dtype, torch.float32):
        raise ValueError("out_dtype must be the query dtype or torch.float32")
    q = queries.contiguous()
    y = _out_buffer(out, (batch, heads, length, dv), out_dtype, queries.device)
    st = (ctypes.c_int64 * 12)(*(_kv_strides(kc, ks, 4) + _kv_strides(vc, vs, 4)))
    ws, wsb = _lib.workspace(queries.device,
                             _lib.lib().sparkq_quantized_sdpa_workspace_bytes(
                                 batch, heads, kv_heads, length, n, dv), "sdpa_staged")
    _lib.call("sparkq_quantized_sdpa", _ptr(q), _ptr(kc), _ptr(ks), _ptr(kb), _ptr(vc),
              _ptr(vs), _ptr(vb), _ptr(mask_t), kind, mdt, mstrides, _ptr(y), batch, heads,
              kv_heads, length, n, dim, dv, group_size, bits, _lib.dtype_code(queries.dtype),
              _lib.dtype_code(out_dtype), float(scale), st, ws, wsb,
              _lib.stream_handle(queries.device), device=queries.device)
    return y


# ---------------------------------------------------------------------------
# Decoder-layer steps around the projections
# ---------------------------------------------------------------------------

def _round_up(v: int, a: int) -> int:
    return (v + a - 1) // a * a


def rms_norm(x, weight, eps: float, *, residual=None, return_hidden: bool = False):
    """mx.fast.rms_norm(x (+ residual), weight, eps) over the last axis:
    weight * T(h * rsqrt(mean(h^2) + eps)) with h = x (+ residual) rounded to
    x's dtype (spark_mlx_llm/ops/ffn.py:98-99). With return_hidden, returns
    (normed, h)."""
    if not isinstance(x, torch.Tensor) or not isinstance(weight, torch.Tensor):
        raise TypeError("x and weight must be tensors")
    if x.dtype not in _HALF or weight.dtype != x.dtype:
        raise ValueError("rms_norm requires BF16 or F16 x and a weight of the same dtype")
    k = x.shape[-1]
    if weight.shape != (k,):
        raise ValueError(f"rms_norm weight must have shape [{k}]")
    if residual is not None and (residual.shape != x.shape or residual.dtype != x.dtype):
        raise ValueError("rms_norm residual must match x in shape and dtype")
    _require_device("rms_norm", x, weight, residual)
    m = prod(x.shape[:-1])
    x2 = x.reshape(m, k).contiguous()
    r2 = residual.reshape(m, k).contiguous() if residual is not None else None
    out = torch.empty_like(x2)
    hid = torch.empty_like(x2) if return_hidden else None
    _lib.call("sparkq_rms_norm", _ptr(x2), _ptr(r2), _ptr(weight.contiguous()), float(eps),
              _ptr(hid), _ptr(out), m, k, _lib.dtype_code(x.dtype), _lib.stream_handle(x.device), device=x.device)
    if return_hidden:
        return out.view(x.shape), (hid.view(x.shape) if residual is not None else x)
    return out.view(x.shape)


def rope(x, dims: int, *, traditional: bool = False, base: float = 10000.0,
         scale: float = 1.0, offset: int = 0):
    """mx.fast.rope on x [..., L, D]: position of token l is offset + l; the
    first `dims` features rotate in pairs (i, i + dims/2) (or (2i, 2i+1) when
    traditional) by (scale * position) * base^(-2i/dims); the rest pass
    through (spark_mlx_llm/ops/qkv.py:176-177; X/src/spark_qkv_rope.cpp:
    99-100)."""
    if not isinstance(x, torch.Tensor):
        raise TypeError("x must be a tensor")
    if x.dtype not in _HALF:
        raise ValueError("rope requires a BF16 or F16 input")
    if x.ndim < 2:
        raise ValueError("rope requires x[..., L, D]")
    if not isinstance(offset, int) or isinstance(offset, bool):
        raise ValueError("rope offset must be an int")
    _require_device("rope", x)
    length, d = x.shape[-2], x.shape[-1]
    rows = prod(x.shape[:-1])
    xc = x.contiguous()
    out = torch.empty_like(xc)
    if rows == 0:
        return out
    _lib.call("sparkq_rope", _ptr(xc), _ptr(out), rows, length, d, int(dims), int(bool(traditional)),
              float(base), float(scale), int(offset), _lib.dtype_code(x.dtype),
              _lib.stream_handle(x.device), device=x.device)
    return out


def spark_qkv_rope(x, weight, scales, biases, q_size: int, kv_size: int, num_heads: int,
                   num_key_value_heads: int, head_dim: int, rope_dims: int, rope_base: float,
                   offset: int, group_size: int, bits: int):
    """Fused QKV projection + RoPE of one token, spark_qkv_rope
    (X/src/spark_qkv_rope.cpp:14-102) with its argument checks: x [1,1,hidden]
    -> (queries [1,H,1,D], keys [1,Hkv,1,D], values [1,Hkv,1,D]); queries and
    keys rotated by mx.fast.rope(rope_dims, traditional=False, rope_base,
    scale=1, offset)."""
    if not isinstance(x, torch.Tensor) or x.ndim != 3 or x.shape[0] != 1 or x.shape[1] != 1 \
            or x.shape[2] <= 0:
        raise ValueError("[spark_qkv_rope] x must have shape [1, 1, hidden] with hidden > 0.")
    if not x.dtype.is_floating_point:
        raise ValueError("[spark_qkv_rope] x must have a real floating dtype.")
    if (num_heads <= 0 or num_key_value_heads <= 0 or head_dim <= 0
            or num_heads % num_key_value_heads != 0 or q_size != num_heads * head_dim
            or kv_size != num_key_value_heads * head_dim):
        raise ValueError("[spark_qkv_rope] Invalid head counts, head_dim, q_size, or kv_size.")
    if (rope_dims <= 0 or rope_dims % 2 != 0 or rope_dims > head_dim
            or not math.isfinite(rope_base) or rope_base <= 0):
        raise ValueError("[spark_qkv_rope] rope_dims must be positive, even, and no larger than "
                         "head_dim; rope_base must be positive and finite.")
    if group_size not in (32, 64, 128):
        raise ValueError("[spark_qkv_rope] group_size must be 32, 64, or 128.")
    if bits not in (1, 2, 3, 4, 5, 6, 8):
        raise ValueError("[spark_qkv_rope] bits must be 1, 2, 3, 4, 5, 6, or 8.")
    for t in (weight, scales, biases):
        if not isinstance(t, torch.Tensor) or t.ndim != 2:
            raise ValueError("[spark_qkv_rope] weight, scales, and biases must be matrices.")
    if (weight.dtype not in _PACKED or not scales.dtype.is_floating_point
            or not biases.dtype.is_floating_point):
        raise ValueError("[spark_qkv_rope] weight must be uint32; scales and biases must have "
                         "real floating dtypes.")
    hidden = x.shape[2]
    if (hidden % group_size or weight.shape[0] != q_size + 2 * kv_size
            or weight.shape[1] * 32 != hidden * bits or scales.shape != biases.shape
            or scales.shape[0] != weight.shape[0] or scales.shape[1] != hidden // group_size):
        raise ValueError("[spark_qkv_rope] Packed weight and quantization metadata shapes do "
                         "not match x, q_size, kv_size, group_size, and bits.")
    if x.dtype not in _HALF or scales.dtype != x.dtype or biases.dtype != x.dtype:
        raise ValueError("[spark_qkv_rope] x, scales and biases must share a BF16 or F16 dtype")
    if not isinstance(offset, int) or isinstance(offset, bool):
        raise ValueError("[spark_qkv_rope] offset must be an int")
    _require_device("spark_qkv_rope", x, weight, scales, biases)
    dev = x.device
    q = torch.empty((1, num_heads, 1, head_dim), dtype=x.dtype, device=dev)
    k = torch.empty((1, num_key_value_heads, 1, head_dim), dtype=x.dtype, device=dev)
    v = torch.empty_like(k)
    need = _lib.lib().sparkq_qkv_rope_workspace_bytes(hidden, num_heads, num_key_value_heads,
                                                       head_dim, group_size)
    ws, wsb = _lib.workspace(dev, need, "qkv_rope")
    _lib.call("sparkq_qkv_rope", _ptr(x.contiguous()), _ptr(weight.contiguous()),
              _ptr(scales.contiguous()), _ptr(biases.contiguous()), _ptr(q), _ptr(k), _ptr(v),
              hidden, q_size, kv_size, num_heads, num_key_value_heads, head_dim, rope_dims,
              float(rope_base), int(offset), group_size, bits, _lib.dtype_code(x.dtype), ws, wsb,
              _lib.stream_handle(dev), device=dev)
    return q, k, v


def fused_ffn(x, attention_output, norm_weight, eps: float, gate, up, down, *,
              group_size: int = 64, bits: int = 4, return_intermediates: bool = False):
    """The decoder's FFN block, compiled_ffn (spark_mlx_llm/ops/ffn.py:83-105):
    hidden = x + attention_output; normed = rms_norm(hidden, norm_weight, eps);
    out = hidden + down(gelu(gate(normed)) * up(normed)), in the 16-bit
    graph's rounding. gate, up and down are (weight, scales, biases) of W4
    affine projections. With return_intermediates, returns (out, hidden,
    normed, act)."""
    tensors = (x, attention_output, norm_weight)
    if any(not isinstance(t, torch.Tensor) for t in tensors):
        raise TypeError("x, attention_output and norm_weight must be tensors")
    if bits != 4:
        raise ValueError("fused_ffn: only 4-bit affine projections are supported")
    if x.dtype not in _HALF or attention_output.dtype != x.dtype or norm_weight.dtype != x.dtype:
        raise ValueError("fused_ffn requires BF16 or F16 x, attention_output and norm weight")
    if attention_output.shape != x.shape:
        raise ValueError("fused_ffn: attention_output must have the shape of x")
    k = x.shape[-1]
    if norm_weight.shape != (k,):
        raise ValueError(f"fused_ffn: norm weight must have shape [{k}]")
    (gw, gs, gb), (uw, us, ub), (dw, ds, db) = gate, up, down
    inter = gw.shape[0]
    for name, (w, s, b), n, kk in (("gate", gate, inter, k), ("up", up, inter, k),
                                   ("down", down, k, inter)):
        if (w.dtype not in _PACKED or w.shape != (n, kk // 8) or s.dtype != x.dtype
                or b.dtype != x.dtype or kk % group_size
                or s.shape != (n, kk // group_size) or b.shape != s.shape):
            raise ValueError(f"fused_ffn: {name} projection has the wrong packed shape or dtype")
    if group_size not in (32, 64, 128) or k % 64 or inter % 64:
        raise ValueError("fused_ffn: group_size 32/64/128 and sizes divisible by 64 required")
    _require_device("fused_ffn", x, attention_output, norm_weight, gw, gs, gb, uw, us, ub, dw,
                    ds, db)
    m = prod(x.shape[:-1])
    x2 = x.reshape(m, k).contiguous()
    a2 = attention_output.reshape(m, k).contiguous()
    out = torch.empty_like(x2)
    if m == 0:
        return out.view(x.shape)
    dev = x.device
    need = _lib.lib().sparkq_ffn_workspace_bytes(m, k, inter, group_size)
    buf = _lib.workspace_buffer(dev, need, "ffn")
    c = [t.contiguous() for t in (gw, gs, gb, uw, us, ub, dw, ds, db)]
    _lib.call("sparkq_ffn", _ptr(x2), _ptr(a2), _ptr(norm_weight.contiguous()), float(eps),
              *[_ptr(t) for t in c], _ptr(out), m, k, inter, group_size,
              _lib.dtype_code(x.dtype), ctypes.c_void_p(buf.data_ptr()), buf.numel(),
              _lib.stream_handle(dev), device=dev)
    if not return_intermediates:
        return out.view(x.shape)
    lin = _round_up(max(_lib.lib().sparkq_w4a16_workspace_bytes(m, inter, k, group_size),
                        _lib.lib().sparkq_w4a16_workspace_bytes(m, k, inter, group_size)), 256)
    hk = _round_up(m * k * 2, 256)

    def view(off, n, cols):
        return buf[off:off + 2 * n].view(x.dtype).view(m, cols).clone()

    hidden = view(lin, m * k, k)
    normed = view(lin + hk, m * k, k)
    act = view(lin + 2 * hk, m * inter, inter)
    return out.view(x.shape), hidden, normed, act


def attention_gate(x, output, gate_weight, *, return_gate: bool = False):
    """Head-wise sigmoid gate of the attention output, transposed for the
    output projection (spark_mlx_llm/ops/attention_output.py:69-95):
    x [B,L,hidden], output [B,H,L,D], gate_weight [H,hidden] (a bias-free
    g_proj) -> [B,L,H*D] = (output^T[b,l,h,:] * sigmoid(x[b,l] . g[h])),
    with the 16-bit graph's roundings (the dot and the sigmoid each rounded
    to the dtype, the product rounded once). With return_gate the [B,L,H]
    gate is returned too."""
    if any(not isinstance(t, torch.Tensor) for t in (x, output, gate_weight)):
        raise TypeError("x, output and gate_weight must be tensors")
    if output.ndim != 4 or x.ndim != 3 or gate_weight.ndim != 2:
        raise ValueError("expected x [B,L,hidden], output [B,H,L,D] and gate_weight [H,hidden]")
    b, h, length, d = output.shape
    if x.shape[:2] != (b, length) or gate_weight.shape != (h, x.shape[2]):
        raise ValueError("x, output and gate_weight shapes disagree")
    if x.dtype not in _HALF or output.dtype != x.dtype or gate_weight.dtype != x.dtype:
        raise ValueError("attention_gate requires bfloat16 or float16 tensors of one dtype")
    _require_device("attention_gate", x, output, gate_weight)
    hidden = x.shape[2]
    x, output, gate_weight = x.contiguous(), output.contiguous(), gate_weight.contiguous()
    out = torch.empty((b, length, h * d), dtype=x.dtype, device=x.device)
    gate = torch.empty((b, length, h), dtype=x.dtype, device=x.device) if return_gate else None
    _lib.call("sparkq_attention_gate", _ptr(x), _ptr(output), _ptr(gate_weight), _ptr(out),
              _ptr(gate), b, length, h, d, hidden, _lib.dtype_code(x.dtype),
              _lib.stream_handle(x.device), device=x.device)
    return (out, gate) if return_gate else out
