"""GPU parity of the W8A16 per-channel GEMV (libsparkq via sparkq.ext) against
the oracle: the fp32 output within max-abs 2e-2 and rel-L2 1e-3 of the fp64
scale * (x . w), the 16-bit output within one unit of its correctly rounded
value, and one-hot activations picking w[:, k] * scale exactly."""

import numpy as np
import pytest
import torch

import oracle as o
from helpers import check_fp32, check_rounded16, down16, up16

pytestmark = pytest.mark.gpu


def _problem(m, n, k, dtype, seed):
    """Per-channel symmetric codes of N(0, 0.02) weights (the converter's
    channel formula), one row starting with the extreme code -128, and N(0,1)
    activations."""
    w = o.randn(seed, 900 + n, n * k, 0.02).reshape(n, k)
    w8, sc = o.w8_quantize_channel(w)
    w8[0, : min(k, 16)] = -128
    x = o.randn16(seed, 500 + m, m * k, 1.0, dtype).reshape(m, k)
    return x, w8, sc


def _run(dev, x, w8, sc, dtype, out_dtype=None):
    import sparkq

    return sparkq.w8a16_per_channel(up16(x, dtype, dev), torch.from_numpy(w8).to(dev),
                                    torch.from_numpy(sc).to(dev), out_dtype=out_dtype)


@pytest.mark.parametrize("dtype", [o.BF16, o.F16])
@pytest.mark.parametrize("m,n,k", [(1, 2560, 4096), (1, 37, 528), (1, 5, 16), (2, 130, 1040),
                                   (3, 64, 256), (4, 1030, 2560), (1, 600, 9728)])
def test_w8a16_matches_oracle(gpu, m, n, k, dtype):
    """Reference production shape (N=2560, K=4096), a partial last span
    (K % 256 != 0), a partial row quad (N % 4 != 0), K = 16, more row quads
    than CUs, and 2..4 activation rows."""
    x, w8, sc = _problem(m, n, k, dtype, seed=n + k)
    ref = o.w8a16_matmul(x, w8, sc, dtype)
    y32 = _run(gpu, x, w8, sc, dtype, out_dtype=torch.float32).cpu().numpy()
    check_fp32(y32, ref)
    check_rounded16(down16(_run(gpu, x, w8, sc, dtype)), ref, dtype)


@pytest.mark.parametrize("n,k", [(3584, 2560), (19456, 2560), (37, 512), (1030, 2560), (5, 256),
                                 (300, 1024), (600, 2304)])
def test_w8a16_one_round(gpu, n, k, monkeypatch):
    """M = 1 over whole 256-k spans up to K = 2560 on the one-round kernel (one
    row quad per wave, spans in order with one, two or every load in flight):
    the three issue depths give identical bits, each within the oracle's
    tolerance, as is the streaming kernel on the same problem; a partial row
    quad, fewer quads than CUs and more than eight per CU."""
    for dtype in (o.BF16, o.F16):
        x, w8, sc = _problem(1, n, k, dtype, seed=n + 3 * k)
        ref = o.w8a16_matmul(x, w8, sc, dtype)
        outs = []
        for depth in ("8", "1", "2"):
            monkeypatch.setenv("SPARKQ_W8A16_Q_DEPTH", depth)
            outs.append(_run(gpu, x, w8, sc, dtype, out_dtype=torch.float32))
        check_fp32(outs[0].cpu().numpy(), ref)
        assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
        check_rounded16(down16(_run(gpu, x, w8, sc, dtype)), ref, dtype)
        monkeypatch.setenv("SPARKQ_W8A16_NO_Q", "1")
        check_fp32(_run(gpu, x, w8, sc, dtype, out_dtype=torch.float32).cpu().numpy(), ref)
        monkeypatch.delenv("SPARKQ_W8A16_NO_Q")


def test_one_hot_picks_scaled_column(gpu):
    n, k = 300, 1024
    _, w8, sc = _problem(1, n, k, o.BF16, seed=3)
    for kk in (0, 77, 1023):
        x = np.zeros((1, k), np.float32)
        x[0, kk] = 1.0
        y = _run(gpu, o.bf16_bits(x), w8, sc, o.BF16, out_dtype=torch.float32).cpu().numpy()[0]
        want = (w8[:, kk].astype(np.float64) * sc.astype(np.float64)).astype(np.float32)
        assert np.array_equal(y, want), kk


def test_converter_w8_rows(gpu):
    """The reference converter's per-row W8 vectors (tests/golden), unpacked
    by the operator layer, through the GEMV: matches the oracle on the same
    int8 codes and channel scales."""
    import sparkq
    from sparkq.ops.linear import unpack_affine_w8

    g = np.load(__file__.rsplit("/", 1)[0] + "/golden/converter_vectors.npz")
    w8, ch = unpack_affine_w8(torch.from_numpy(g["w8_words"].view(np.int32)),
                              torch.from_numpy(g["w8_scales"].view(np.int16)).view(torch.bfloat16),
                              torch.from_numpy(g["w8_biases"].view(np.int16)).view(torch.bfloat16),
                              group_size=32)
    n, k = w8.shape
    x = o.randn16(4, 1, k).reshape(1, k)
    ref = o.w8a16_matmul(x, w8.numpy(), ch.numpy())
    y = sparkq.w8a16_per_channel(up16(x, o.BF16, gpu), w8.to(gpu), ch.to(gpu),
                                 out_dtype=torch.float32).cpu().numpy()
    check_fp32(y, ref)


def test_lm_head_sampled(gpu):
    """The W8 lm_head shape (131072 x 2560, 335 MB): sampled rows against the
    oracle, and two calls bit-identical."""
    import sparkq

    n, k = 131072, 2560
    gen = torch.Generator(device=gpu).manual_seed(5)
    w8 = torch.randint(-128, 128, (n, k), dtype=torch.int8, device=gpu, generator=gen)
    sc = torch.rand(n, device=gpu, generator=gen) * 0.01 + 1e-4
    x16 = o.randn16(6, 1, k).reshape(1, k)
    xt = up16(x16, o.BF16, gpu)
    y = sparkq.w8a16_per_channel(xt, w8, sc, out_dtype=torch.float32)
    assert torch.equal(y, sparkq.w8a16_per_channel(xt, w8, sc, out_dtype=torch.float32))
    rows = np.sort(np.random.default_rng(1).choice(n, 512, replace=False))
    ref = o.w8a16_matmul(x16, w8[rows].cpu().numpy(), sc[rows].cpu().numpy())
    check_fp32(y.cpu().numpy()[:, rows], ref)


def test_rejects_bad_inputs(gpu):
    import sparkq

    x = torch.zeros((1, 64), dtype=torch.bfloat16, device=gpu)
    w = torch.zeros((8, 64), dtype=torch.int8, device=gpu)
    sc = torch.ones(8, dtype=torch.float32, device=gpu)
    with pytest.raises(ValueError, match="dtype int8"):
        sparkq.w8a16_per_channel(x, w.to(torch.int16), sc)
    with pytest.raises(ValueError, match="float32"):
        sparkq.w8a16_per_channel(x, w, sc.to(torch.float16))
    with pytest.raises(ValueError, match="bfloat16 or float16"):
        sparkq.w8a16_per_channel(x.float(), w, sc)
    with pytest.raises(ValueError, match="one activation row"):
        sparkq.w8a16_per_channel(torch.zeros((5, 64), dtype=torch.bfloat16, device=gpu), w, sc)
