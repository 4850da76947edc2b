"""The converter's on-disk format (spark_mlx_llm/conversion.py:611-656,
755-843) through sparkq.checkpoint: a model directory holding the reference
converter's own W4 (G32) and W8 (per-row) tensors from tests/golden, written
as the converter lays them out (safetensors with {"format": "mlx"} metadata,
an index, a config with per-module quantization), read back bit for bit, and
(on the GPU) run through the projections the W8 backend selects."""

import json
import os

import numpy as np
import pytest
import torch
from safetensors.torch import load_file, save_file

import oracle as o
from helpers import down16, up16

GOLD = os.path.join(os.path.dirname(__file__), "golden", "converter_vectors.npz")
W4 = "model.layers.0.mlp.gate_proj"
W8 = "model.layers.0.self_attn.out_proj"


def _write_model(directory, w8_backend="w8a16"):
    g = np.load(GOLD)
    tensors = {
        W4 + ".weight": g["w4_words"], W4 + ".scales": g["w4_scales"],
        W4 + ".biases": g["w4_biases"],
        W8 + ".weight": g["w8_words"], W8 + ".scales": g["w8_scales"],
        W8 + ".biases": g["w8_biases"],
        "model.norm.weight": np.arange(256, dtype=np.uint16),
    }
    shards = {"model.safetensors": [k for k in tensors if k != "model.norm.weight"],
              "model-00002.safetensors": ["model.norm.weight"]}
    def as_torch(a):
        # the converter's dtypes: U32 packed codes, BF16 coefficients and norms
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint32:
            return torch.from_numpy(a.view(np.int32)).view(torch.uint32)
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)

    for name, keys in shards.items():
        save_file({k: as_torch(tensors[k]) for k in keys},
                  os.path.join(directory, name), metadata={"format": "mlx"})
    index = {"metadata": {"total_size": sum(v.nbytes for v in tensors.values())},
             "weight_map": {k: f for f, ks in shards.items() for k in ks}}
    with open(os.path.join(directory, "model.safetensors.index.json"), "w") as f:
        json.dump(index, f)
    storage = {"bits": 4, "group_size": 32, "mode": "affine",
               W4: {"bits": 4, "group_size": 32, "mode": "affine"},
               W8: {"bits": 8, "group_size": 32, "mode": "affine"}}
    config = {"quantization": storage, "quantization_config": storage,
              "w8_qmv_backend": w8_backend, "dtype": "bfloat16"}
    with open(os.path.join(directory, "config.json"), "w") as f:
        json.dump(config, f)
    return tensors


def test_reader_matches_safetensors(tmp_path):
    from sparkq.checkpoint import Checkpoint, quantization_scheme

    tensors = _write_model(tmp_path)
    ck = Checkpoint(str(tmp_path))
    assert set(ck.tensors) == set(tensors)
    ref = load_file(str(tmp_path / "model.safetensors"))
    for k, v in ref.items():
        assert ck.tensors[k].shape == tuple(v.shape)
        raw = v.view(torch.int32) if v.dtype == torch.uint32 else v.view(torch.int16)
        assert np.array_equal(ck.numpy(k).view(raw.numpy().dtype), raw.numpy())
        assert np.array_equal(ck.numpy(k), tensors[k])
    assert ck.tensors[W4 + ".weight"].dtype == "U32"
    assert ck.tensors[W8 + ".scales"].dtype == "BF16"
    assert np.array_equal(ck.numpy("model.norm.weight"), tensors["model.norm.weight"])
    assert ck.quantized_modules() == sorted([W4, W8])
    # bf16 tensors come back as torch.bfloat16 with the same bits
    s = ck.tensor(W4 + ".scales")
    assert s.dtype == torch.bfloat16
    assert np.array_equal(s.view(torch.int16).numpy().view(np.uint16), tensors[W4 + ".scales"])
    assert quantization_scheme(ck.config, W8) == {"bits": 8, "group_size": 32, "mode": "affine"}
    assert quantization_scheme(ck.config, "model.layers.1.mlp.up_proj")["bits"] == 4


def test_reader_rejects_bad_files(tmp_path):
    from sparkq.checkpoint import read_header

    p = tmp_path / "bad.safetensors"
    p.write_bytes(b"\x10\x00\x00\x00\x00\x00\x00\x00{}")
    with pytest.raises(ValueError, match="truncated"):
        read_header(str(p))
    hdr = json.dumps({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 8]}}).encode()
    p.write_bytes(len(hdr).to_bytes(8, "little") + hdr + b"\0" * 8)
    with pytest.raises(ValueError, match="offsets"):
        read_header(str(p))


@pytest.mark.gpu
@pytest.mark.parametrize("backend", ["w8a16", "w8a8"])
def test_loaded_projections_match_oracle(gpu, tmp_path, backend):
    """The golden rows span a wide dynamic range (outputs from 0.05 to 4600),
    so the fp32 epilogue is checked per element relative to its magnitude, and
    each layer's 16-bit output must be the rounding of that fp32 value."""
    import sparkq
    from sparkq.checkpoint import Checkpoint, load_projection
    from sparkq.ops import W8A16PerChannelLinear, W8A8Projection

    tensors = _write_model(tmp_path, w8_backend=backend)
    ck = Checkpoint(str(tmp_path))
    x = o.randn16(3, 1, 256).reshape(1, 256)
    xt = up16(x, o.BF16, gpu)

    def close(y, ref):
        assert np.all(np.abs(y - ref) <= 1e-4 * (np.abs(ref) + 1.0)), float(np.abs(y - ref).max())

    # W4 G32 module written by the reference converter
    p4 = load_projection(ck, W4, gpu)
    y32 = sparkq.affine_quantized_matmul(xt, p4.weight, p4.scales, p4.biases, group_size=32,
                                         out_dtype=torch.float32).cpu().numpy()
    close(y32, o.w4a16_matmul(x, tensors[W4 + ".weight"], tensors[W4 + ".scales"],
                              tensors[W4 + ".biases"], 32))
    assert np.array_equal(down16(p4(xt)), o.round16(y32, o.BF16))
    # W8 per-row module through the configured adapter
    p8 = load_projection(ck, W8, gpu)
    w8 = o.w8_unpack_affine(tensors[W8 + ".weight"])
    sc = o.bits_to_f32(tensors[W8 + ".scales"], o.BF16)[:, 0].copy()
    if backend == "w8a16":
        assert isinstance(p8, W8A16PerChannelLinear)
        y32 = sparkq.w8a16_per_channel(xt, p8.weight, p8.scales,
                                       out_dtype=torch.float32).cpu().numpy()
        close(y32, o.w8a16_matmul(x, w8, sc))
    else:
        assert isinstance(p8, W8A8Projection)
        w8t, sct = p8.projection.weight, p8.projection.scales
        assert np.array_equal(w8t.cpu().numpy(), w8)
        y32 = sparkq.w8a8_linear(xt, w8t, sct, out_dtype=torch.float32).cpu().numpy()
        q, sa = o.a8_quantize(o.bits_to_f32(x, o.BF16))
        assert np.array_equal(y32, o.w8a8_epilogue(o.int8_matmul(q, w8), sa, sc))
    assert np.array_equal(down16(p8(xt)), o.round16(y32, o.BF16))
