"""Write golden vectors of the reference converter's weight quantizers.

The reference converter (spark_mlx_llm/conversion.py) defines the packed
checkpoint format the kernels read. Its quantizers are `_rows`
(conversion.py:551-608) for the schemes `bf16-int4` (G32 affine: min/max
clamped to include 0, scale/15 rounded to bf16, rint zero point and codes,
bias -zero*scale in bf16) and `bf16-int8` (per-row symmetric: max|w|/127 in
bf16, codes rint(w/scale)+128, bias -128*scale, both repeated per 32), with
`_packed` (:429-433) and `bf16` (:154-159).

This script imports that module from a reference checkout in the build
container only (it needs NumPy and the standard library), feeds it seeded
bf16 weight rows through a raw file descriptor of the form `_rows` reads
(`read`/`floats`, :134-152), and stores the inputs and the outputs as
`converter_vectors.npz` next to this file. Only that fixture is committed;
the tests compare the oracle's restatement with it.

Usage: python tests/golden/make_converter_vectors.py [/path/to/reference]
"""

from __future__ import annotations

import os
import pathlib
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "converter_vectors.npz")
K = 256  # 8 groups of 32 per row


def bf16_bits(x):
    """float32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    w = np.asarray(x, np.float32).view(np.uint32)
    return ((w + 0x7FFF + ((w >> 16) & 1)) >> 16).astype(np.uint16)


def weight_rows(rng):
    """bf16 weight rows covering the quantizers' edge cases, one row each:
    random N(0, 0.02); a zero group; all-positive and all-negative groups
    (the clamp of min/max to include 0); a single nonzero value; a wide
    dynamic range; values placed on half-step ties of the rounded scale;
    large magnitudes; tiny magnitudes."""
    rows = []
    for _ in range(24):
        rows.append(rng.standard_normal(K) * 0.02)
    r = rng.standard_normal(K) * 0.05
    r[32:64] = 0.0
    rows.append(r)
    rows.append(np.abs(rng.standard_normal(K)) * 0.03 + 0.01)
    rows.append(-np.abs(rng.standard_normal(K)) * 0.03 - 0.01)
    r = np.zeros(K)
    r[::37] = 0.25
    rows.append(r)
    rows.append(rng.standard_normal(K) * 10.0 ** rng.uniform(-6, 2, K))
    # near-ties: two anchors fix a group's range, the other values sit at
    # lo + (j + 0.5) * s for the bf16-rounded scale s, so w/s lands near .5
    for lo, hi in ((-0.75, 0.75), (0.0, 1.5), (-1.5, 0.0)):
        r = np.zeros(K, np.float64)
        for g in range(K // 32):
            s = float(np.float32((hi - lo) / 15.0))
            s_b = float((bf16_bits(np.float32(s)).astype(np.uint32) << 16).view(np.float32))
            vals = lo + (np.arange(32) % 15 + 0.5) * s_b
            vals[0], vals[1] = lo, hi
            r[32 * g:32 * g + 32] = vals
        rows.append(r)
    rows.append(rng.standard_normal(K) * 300.0)
    rows.append(rng.standard_normal(K) * 1e-4)
    w = np.stack(rows).astype(np.float32)
    return bf16_bits(w)


def run_rows(cv, kind, bits, w16):
    n, k = w16.shape
    module = "model.layers.0.mlp.up_proj"
    with tempfile.TemporaryDirectory() as d:
        path = pathlib.Path(d) / "weight.bin"
        path.write_bytes(w16.astype("<u2").tobytes())
        desc = {"path": path, "offset": 0, "bytes": w16.nbytes, "shape": [n, k], "dtype": "BF16"}
        out, _ = cv._rows(module, {"kind": kind, "bits": bits, "shape": [n, k]},
                          {module + ".weight": desc}, 0, n)
    words = np.frombuffer(out["weight"], "<u4").reshape(n, -1)
    scales = np.frombuffer(out["scales"], "<u2").reshape(n, -1)
    biases = np.frombuffer(out["biases"], "<u2").reshape(n, -1)
    return words.copy(), scales.copy(), biases.copy()


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, ref)
    from spark_mlx_llm import conversion as cv  # noqa: E402  (NumPy-only module)

    rng = np.random.default_rng(20260101)
    w16 = weight_rows(rng)
    w4 = run_rows(cv, "bf16-int4", 4, w16)
    w8 = run_rows(cv, "bf16-int8", 8, w16)
    # bf16(): special values (finite only; the converter rejects overflow)
    probe = np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.0e38, -1.5e-39, 1e-45,
                      65504.0, 0.1, 1.0 / 3.0, -2.5e-8], np.float32)
    enc, _ = cv.bf16(probe)
    np.savez_compressed(OUT, w16=w16, w4_words=w4[0], w4_scales=w4[1], w4_biases=w4[2],
                        w8_words=w8[0], w8_scales=w8[1], w8_biases=w8[2],
                        bf16_in=probe, bf16_out=np.asarray(enc, np.uint16))
    print(f"wrote {OUT}: {w16.shape[0]} rows x {K}")


if __name__ == "__main__":
    main()
