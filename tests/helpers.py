"""Shared helpers for the parity tests: seeded inputs from the oracle's
generator, uploads to the device, and the comparison metrics."""

import numpy as np
import torch

import oracle as o

TORCH16 = {o.BF16: torch.bfloat16, o.F16: torch.float16}


def up16(bits, dtype, device):
    """uint16 bit patterns -> device tensor of the 16-bit float dtype."""
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16))
    return t.view(TORCH16[dtype]).to(device)


def up32(words, device):
    return torch.from_numpy(np.ascontiguousarray(words).view(np.int32)).to(device)


def down16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def w4_problem(m, n, k, g, dtype=o.BF16, seed=0, wstd=0.02):
    """Weights N(0, wstd) rounded to dtype and quantized with the benchmark's
    affine formula; activations N(0,1) rounded to dtype."""
    w = o.bits_to_f32(o.randn16(seed, 1000 + n, n * k, wstd, dtype), dtype).reshape(n, k)
    wq, s, b = o.w4_quantize(w, g, dtype)
    x = o.randn16(seed, 2000 + m, m * k, 1.0, dtype).reshape(m, k)
    return x, wq, s, b


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def ulp_distance16(a_bits, b_bits, dtype):
    """Distance in units of the 16-bit format between two bit arrays."""
    def ordered(x):
        x = x.astype(np.int64)
        return np.where(x & 0x8000, -(x & 0x7FFF), x)

    return np.abs(ordered(a_bits) - ordered(b_bits))


def check_fp32(out, ref, atol=2e-2, rtol_l2=1e-3):
    """The north-star tolerance (max-abs 2e-2, relative L2 1e-3 against the
    fp64 dequantize-then-matmul) applied to the unrounded fp32 epilogue."""
    ma, rl = max_abs(out, ref), rel_l2(out, ref)
    print(f"[fp32] max_abs={ma:.3e} rel_l2={rl:.3e}")
    assert ma <= atol and rl <= rtol_l2, f"max_abs={ma:.3e} rel_l2={rl:.3e}"
    return ma, rl


def check_rounded16(out_bits, ref64, dtype, atol=2e-2, near_zero=2.0 ** -7,
                    max_flip_frac=0.05):
    """A 16-bit output against the correctly rounded oracle: every element
    within atol of it or a 1-unit boundary flip (one unit of bf16 is 2^-5 at
    |y| >= 4, above atol, so flips are allowed and counted rather than held
    to atol); every element whose magnitude is at least near_zero * rms(ref)
    within one unit of the format (an fp32 accumulation error of ~1e-6*rms is
    many units of a near-zero result, so those are held to atol only); and
    the fraction of 1-unit flips bounded and reported."""
    ref = np.asarray(ref64, np.float64)
    ref_bits = o.round16(ref.astype(np.float32), dtype)
    diff = np.abs(o.bits_to_f32(out_bits, dtype).astype(np.float64)
                  - o.bits_to_f32(ref_bits, dtype).astype(np.float64))
    d = ulp_distance16(out_bits, ref_bits, dtype)
    ma = float(diff.max())
    ma_noflip = float(diff[d > 1].max()) if (d > 1).any() else 0.0
    rms = float(np.sqrt(np.mean(ref ** 2)))
    big = np.abs(ref) >= near_zero * rms
    frac = float((d > 0).mean())
    print(f"[16-bit] max_abs_vs_rounded={ma:.3e} (beyond 1-unit flips {ma_noflip:.3e}) "
          f"max_ulp(|y|>={near_zero:g}rms)={int(d[big].max()) if big.any() else 0} "
          f"flips={frac:.4f} max_ulp_all={int(d.max())}")
    assert ma_noflip <= atol, f"max_abs vs rounded oracle beyond 1-unit flips {ma_noflip:.3e}"
    assert not big.any() or d[big].max() <= 1, f"max ulp distance {d[big].max()}"
    assert frac <= max_flip_frac, f"1-ulp flips {frac:.4f}"
    return frac
