"""Reader for the converter's on-disk checkpoint format.

spark_mlx_llm/conversion.py writes (convert_to_mlx, :611-656 and :755-843):

- ``model.safetensors`` (and ``model-draft.safetensors`` for draft tensors): an
  8-byte little-endian header length, a JSON header {name: {"dtype", "shape",
  "data_offsets"}, "__metadata__": {"format": "mlx"}} padded with spaces to a
  multiple of 8, then the tensor bytes in header order;
- ``model.safetensors.index.json``: {"metadata": {"total_size"}, "weight_map":
  {name: file}};
- ``config.json`` with ``quantization`` (storage: default {"bits": 4,
  "group_size": 32, "mode": "affine"} plus one entry per quantized module, e.g.
  {"bits": 8, ...} for out_proj/lm_head), ``quantization_config`` (the same
  with "input_activations" on W8A8 modules) and ``w8_qmv_backend``.

A quantized module has ``<module>.weight`` (U32 packed codes, [N, K*bits/32]),
``<module>.scales`` and ``<module>.biases`` ([N, K/G], BF16; F32 for the LM
head). This reader memory-maps the shards, builds the tensors on a device and
wraps each quantized module in the projection its backend selects, the load-time
policy of QuantizedProjections (spark_mlx_llm/ops/linear.py:565-731): W4
modules become QuantizedLinear (sparkq's affine GEMV/GEMM). W8 modules keep
the affine QuantizedLinear (sparkq's groupwise W8 MFMA kernel) and, by
backend, are wrapped after the W8 unpack (ops/linear.py:299-324):
"w8a16" in W8A16PerChannelLinear when the scales are per channel (groupwise
W8 stays affine), "w8a8" in W8A8Projection; "auto" builds
W8A8QuantizedLinear for a module whose quantization_config entry carries
input_activations (ops/linear.py:569-583) and keeps the affine module
otherwise; "native" and "multirow" keep the affine module.
"""

from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass
from math import prod

import numpy as np
import torch

from .ops.linear import (LinearConfig, QuantizedLinear, W8A16PerChannelLinear, W8A8Projection,
                         W8A8QuantizedLinear, unpack_affine_w8, validate_w8a8_activations)

__all__ = ["TensorInfo", "Checkpoint", "quantization_scheme", "load_projection"]

# safetensors dtype names -> (numpy dtype, torch dtype), conversion.py:31
_DTYPES = {
    "BF16": (np.uint16, torch.bfloat16),
    "F16": (np.float16, torch.float16),
    "F32": (np.float32, torch.float32),
    "I8": (np.int8, torch.int8),
    "I32": (np.int32, torch.int32),
    "U32": (np.uint32, torch.int32),    # packed codes: same bits, int32 storage
    "I64": (np.int64, torch.int64),
}


@dataclass(frozen=True)
class TensorInfo:
    file: str
    dtype: str
    shape: tuple
    begin: int   # absolute byte offset in the file
    end: int


def read_header(path: str) -> dict:
    """Parse one safetensors file's header; offsets are made absolute."""
    with open(path, "rb") as f:
        head = f.read(8)
        if len(head) != 8:
            raise ValueError(f"{path}: truncated safetensors header")
        (n,) = struct.unpack("<Q", head)
        if n <= 0 or n > 100 * 1024 * 1024:
            raise ValueError(f"{path}: implausible safetensors header length {n}")
        raw = f.read(n)
    if len(raw) != n:
        raise ValueError(f"{path}: truncated safetensors header")
    header = json.loads(raw.decode("utf-8"))
    size = os.path.getsize(path)
    base = 8 + n
    out = {}
    for name, desc in header.items():
        if name == "__metadata__":
            continue
        dtype, shape, (b, e) = desc["dtype"], tuple(desc["shape"]), desc["data_offsets"]
        if dtype not in _DTYPES:
            raise ValueError(f"{path}: tensor {name} has unsupported dtype {dtype}")
        nbytes = prod(shape) * np.dtype(_DTYPES[dtype][0]).itemsize
        if e - b != nbytes or base + e > size or b < 0:
            raise ValueError(f"{path}: tensor {name} offsets do not match its shape")
        out[name] = TensorInfo(os.path.basename(path), dtype, shape, base + b, base + e)
    return out


class Checkpoint:
    """A converted model directory: config, tensor inventory and lazy reads."""

    def __init__(self, directory: str):
        self.directory = os.path.abspath(directory)
        with open(os.path.join(self.directory, "config.json")) as f:
            self.config = json.load(f)
        index = os.path.join(self.directory, "model.safetensors.index.json")
        if os.path.exists(index):
            with open(index) as f:
                files = sorted(set(json.load(f)["weight_map"].values()))
        else:
            files = ["model.safetensors"]
        self.tensors: dict[str, TensorInfo] = {}
        for name in files:
            for key, info in read_header(os.path.join(self.directory, name)).items():
                if key in self.tensors:
                    raise ValueError(f"tensor {key} appears in more than one shard")
                self.tensors[key] = info
        self._maps: dict[str, np.memmap] = {}

    def numpy(self, name: str) -> np.ndarray:
        """The tensor's bytes as a numpy view of the memory-mapped shard."""
        info = self.tensors[name]
        mm = self._maps.get(info.file)
        if mm is None:
            mm = np.memmap(os.path.join(self.directory, info.file), dtype=np.uint8, mode="r")
            self._maps[info.file] = mm
        npdt = _DTYPES[info.dtype][0]
        return mm[info.begin:info.end].view(npdt).reshape(info.shape)

    def tensor(self, name: str, device="cpu") -> torch.Tensor:
        info = self.tensors[name]
        arr = np.array(self.numpy(name))   # one copy out of the map
        tdt = _DTYPES[info.dtype][1]
        if info.dtype == "BF16":
            t = torch.from_numpy(arr.view(np.int16)).view(torch.bfloat16)
        elif info.dtype == "U32":
            t = torch.from_numpy(arr.view(np.int32))
        else:
            t = torch.from_numpy(arr).to(tdt)
        return t.to(device)

    def quantized_modules(self) -> list[str]:
        """Modules stored as packed affine weights (weight + scales + biases)."""
        return sorted(k[: -len(".scales")] for k in self.tensors
                      if k.endswith(".scales") and k[: -len(".scales")] + ".biases" in self.tensors
                      and k[: -len(".scales")] + ".weight" in self.tensors)


def quantization_scheme(config: dict, module: str) -> dict:
    """Storage scheme of one module: the per-module entry of config
    ["quantization"] over its defaults (conversion.py:755-761)."""
    q = config.get("quantization")
    if not isinstance(q, dict):
        raise ValueError("checkpoint config has no quantization section")
    base = {k: q[k] for k in ("bits", "group_size", "mode") if k in q}
    own = q.get(module)
    if isinstance(own, dict):
        base.update({k: own[k] for k in ("bits", "group_size", "mode") if k in own})
    if base.get("mode", "affine") != "affine":
        raise ValueError(f"{module}: only affine quantization is supported")
    return {"bits": int(base.get("bits", 4)), "group_size": int(base.get("group_size", 32)),
            "mode": "affine"}


def load_projection(ckpt: Checkpoint, module: str, device, *, w8_backend: str | None = None):
    """Build the projection for one quantized module on ``device``.

    W4 -> QuantizedLinear. W8 -> by backend (the checkpoint's w8_qmv_backend
    unless overridden; ops/linear.py:569-583, 651-711): "w8a16"
    W8A16PerChannelLinear over the affine module when the W8 is per channel
    and bias-free, "w8a8" W8A8Projection over it, "auto" W8A8QuantizedLinear
    when the module's quantization_config entry carries input_activations,
    otherwise (and for "native"/"multirow") the affine QuantizedLinear."""
    scheme = quantization_scheme(ckpt.config, module)
    bits, g = scheme["bits"], scheme["group_size"]
    w = ckpt.tensor(module + ".weight", device)
    s = ckpt.tensor(module + ".scales", device)
    b = ckpt.tensor(module + ".biases", device)
    if w.shape[1] * (32 // bits) != s.shape[1] * g:
        raise ValueError(f"{module}: packed weight and scales disagree with group_size={g}")
    bias = ckpt.tensor(module + ".bias", device) if module + ".bias" in ckpt.tensors else None
    affine = QuantizedLinear(w, s, b, group_size=g, bits=bits, bias=bias)
    if bits == 4:
        return affine
    if bits != 8:
        raise ValueError(f"{module}: unsupported bits={bits}")
    backend = w8_backend or ckpt.config.get("w8_qmv_backend", "native")
    LinearConfig(w8_qmv_backend=backend)
    if backend == "auto":
        scheme = (ckpt.config.get("quantization_config") or {}).get(module, {})
        if isinstance(scheme, dict) and scheme.get("input_activations") is not None:
            validate_w8a8_activations(scheme["input_activations"])
            return W8A8QuantizedLinear(w, s, b, group_size=g, bits=8, bias=bias)
        return affine
    if backend == "w8a8":
        w8, sc = unpack_affine_w8(w, s, b, g, module)
        return W8A8Projection(affine, w8, sc)
    if backend == "w8a16" and bias is None:
        unpacked = unpack_affine_w8(w, s, b, g, module, allow_fallback=True)
        if unpacked is None:
            return affine
        return W8A16PerChannelLinear(affine, *unpacked)
    return affine
