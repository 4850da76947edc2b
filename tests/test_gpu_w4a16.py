"""GPU parity of the W4A16 path (libsparkq via sparkq.ext) against the oracle.

Bars: dequantized weights and the quantizer bit-exact; the fp32 epilogue
within max-abs 2e-2 and rel-L2 1e-3 of the fp64 dequantize-then-matmul; the
16-bit output within one unit of the correctly rounded oracle.
"""

import numpy as np
import pytest
import torch

import oracle as o
from helpers import (check_fp32, check_rounded16, down16, up16, up32, w4_problem)

pytestmark = pytest.mark.gpu


def _run(dev, x, wq, s, b, g, dtype, out_dtype=None):
    import sparkq

    return sparkq.affine_quantized_matmul(
        up16(x, dtype, dev), up32(wq, dev), up16(s, dtype, dev), up16(b, dtype, dev),
        group_size=g, out_dtype=out_dtype)


@pytest.mark.parametrize("dtype", [o.BF16, o.F16])
@pytest.mark.parametrize("g", [32, 64, 128])
def test_dequantize_bit_exact(gpu, g, dtype):
    import sparkq

    n, k = 64, 512
    rng = np.random.default_rng(g)
    codes = rng.integers(0, 16, (n, k), dtype=np.uint8)
    wq = o.pack4(codes)
    sv = (rng.standard_normal((n, k // g)) * 10 ** rng.uniform(-5, 2, (n, k // g))).astype(np.float32)
    bv = (rng.standard_normal((n, k // g)) * 10 ** rng.uniform(-5, 2, (n, k // g))).astype(np.float32)
    s16, b16 = o.round16(sv, dtype), o.round16(bv, dtype)
    s16[0, 0], b16[0, 0] = 0x0000, 0x8000
    if dtype == o.BF16:
        s16[1, 0], b16[1, 0] = 0x0003, 0x8005   # subnormals
        s16[2, 0], b16[2, 0] = 0x7F00, 0xFE00   # large exponents
    ref = o.w4_dequantize(wq, s16, b16, g, dtype)
    out = sparkq.affine_dequantize(up32(wq, gpu), up16(s16, dtype, gpu), up16(b16, dtype, gpu),
                                   group_size=g).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dtype", [o.BF16, o.F16])
@pytest.mark.parametrize("g", [32, 64, 128])
def test_quantizer_bit_exact(gpu, g, dtype):
    import sparkq

    n, k = 96, 512
    w16 = o.randn16(7, g, n * k, 0.02, dtype).reshape(n, k)
    w16[0, :g] = o.round16(np.full(g, 0.5, np.float32), dtype)   # constant group
    wq, s, b = sparkq.affine_quantize(up16(w16, dtype, gpu), group_size=g)
    rwq, rs, rb = o.w4_quantize(o.bits_to_f32(w16, dtype), g, dtype)
    assert np.array_equal(wq.cpu().view(torch.int32).numpy().view(np.uint32), rwq)
    assert np.array_equal(down16(s), rs)
    assert np.array_equal(down16(b), rb)


SKINNY = [1, 2, 3, 8, 13, 16, 17, 32]


@pytest.mark.parametrize("m", SKINNY)
@pytest.mark.parametrize("g", [32, 64, 128])
def test_linear_skinny(gpu, m, g):
    n, k = 96, 1024
    x, wq, s, b = w4_problem(m, n, k, g, seed=m)
    ref = o.w4a16_matmul(x, wq, s, b, g)
    y32 = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32).cpu().numpy()
    check_fp32(y32, ref)
    y16 = down16(_run(gpu, x, wq, s, b, g, o.BF16))
    check_rounded16(y16, ref, o.BF16)


@pytest.mark.parametrize("m", [1, 8, 40])
def test_linear_f16(gpu, m):
    n, k, g = 160, 512, 64
    x, wq, s, b = w4_problem(m, n, k, g, dtype=o.F16, seed=3)
    ref = o.w4a16_matmul(x, wq, s, b, g, o.F16)
    y32 = _run(gpu, x, wq, s, b, g, o.F16, out_dtype=torch.float32).cpu().numpy()
    check_fp32(y32, ref)
    check_rounded16(down16(_run(gpu, x, wq, s, b, g, o.F16)), ref, o.F16)


@pytest.mark.parametrize("m", [33, 130, 256])
@pytest.mark.parametrize("g", [32, 64, 128])
def test_linear_gemm(gpu, m, g):
    n, k = 200, 512   # N tail inside a 128-wide tile
    x, wq, s, b = w4_problem(m, n, k, g, seed=m + g)
    ref = o.w4a16_matmul(x, wq, s, b, g)
    y32 = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32).cpu().numpy()
    check_fp32(y32, ref)
    check_rounded16(down16(_run(gpu, x, wq, s, b, g, o.BF16)), ref, o.BF16)


@pytest.mark.parametrize("m,n,k", [(1, 64, 4096), (4, 8192, 256), (16, 40, 2048)])
def test_split_plans(gpu, m, n, k):
    """Cross-workgroup split-K (few row tiles, long K) and a single split."""
    g = 64
    x, wq, s, b = w4_problem(m, n, k, g, seed=5)
    ref = o.w4a16_matmul(x, wq, s, b, g)
    y32 = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32).cpu().numpy()
    check_fp32(y32, ref)


@pytest.mark.parametrize("m,n,k,g", [(33, 200, 4096, 32), (300, 520, 4096, 64), (130, 90, 9728, 128),
                                     (2048, 256, 4096, 64)])
def test_gemm_split_k(gpu, m, n, k, g):
    """Few output tiles and long K: the bf16 GEMM splits K across workgroups
    and the last one of each tile sums the partials (ragged M and N tiles)."""
    x, wq, s, b = w4_problem(m, n, k, g, seed=m + n)
    ref = o.w4a16_matmul(x, wq, s, b, g)
    y32 = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32)
    check_fp32(y32.cpu().numpy(), ref)
    check_rounded16(down16(_run(gpu, x, wq, s, b, g, o.BF16)), ref, o.BF16)
    # repeated calls on the same workspace are bit-identical (counters reset)
    assert torch.equal(y32, _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32))


def test_gemm_one_tile_per_cu_split(gpu, monkeypatch):
    """A grid of more 128-row tiles than CUs but fewer than two per CU keeps
    one whole tile per CU and splits the tiles past the CUs into k pieces
    (270 tiles on 256 CUs: 14 tiles in three pieces); it matches the oracle
    on the columns either side of the first split tile (the last row tile's
    columns 19456..) and at the end, and, to fp32 rounding, the unsplit grid."""
    m, n, k, g = 384, 23040, 1536, 64
    x, wq, s, b = w4_problem(m, n, k, g, seed=7)
    cols = np.r_[18944:19968, 22528:23040]
    ref = o.w4a16_matmul(x, wq[cols], s[cols], b[cols], g)
    y = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32)
    check_fp32(y.cpu().numpy()[:, cols], ref)
    check_rounded16(down16(_run(gpu, x, wq, s, b, g, o.BF16))[:, cols], ref, o.BF16)
    monkeypatch.setenv("SPARKQ_W4_GEMM_NO_CU1", "1")
    y1 = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32)
    assert torch.allclose(y, y1, rtol=1e-5, atol=1e-6 * float(y1.abs().max()))


@pytest.mark.parametrize("m,n,k,gm,same_split", [(2048, 2560, 9728, "4", True), (1024, 3584, 2560, "8", True),
                                                 (300, 1000, 1024, "4", True), (640, 4096, 2048, "2", True),
                                                 (512, 19456, 2560, "4", False)])
def test_gemm_tile_order(gpu, m, n, k, gm, same_split, monkeypatch):
    """The XCD-grouped tile order of the prefill GEMM (each XCD's work items
    take a contiguous chunk of the order, walked in groups of gm tile rows)
    against row-major order. Where every tile or none is split along k, each
    output's products are summed in the same order either way: identical
    bits (whole grids in k pieces, tile counts that are and are not
    multiples of eight, 64- and 128-row tiles). Where only the tiles past one
    per CU are split (304 tiles on 256 CUs), the order picks which tiles
    those are, and a split tile adds its fp32 partials in a different order:
    within the oracle's tolerance and fp32 rounding of each other."""
    g = 64
    x, wq, s, b = w4_problem(m, n, k, g, seed=m + 5 * n)
    monkeypatch.setenv("SPARKQ_W4_GEMM_GM", gm)
    y = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32)
    monkeypatch.setenv("SPARKQ_W4_GEMM_ROWMAJOR", "1")
    y0 = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32)
    if same_split:
        assert torch.equal(y, y0)
    else:
        assert torch.allclose(y, y0, rtol=1e-5, atol=1e-6 * float(y0.abs().max()))
    cols = np.sort(np.random.default_rng(n).choice(n, 64, replace=False))
    check_fp32(y.cpu().numpy()[:, cols], o.w4a16_matmul(x, wq[cols], s[cols], b[cols], g))


@pytest.mark.parametrize("m,n,k,g", [(40, 96, 2048, 64), (33, 64, 2560, 32), (48, 40, 9728, 64),
                                     (36, 32, 16384, 128), (34, 16, 16896, 64)])
def test_gemm_prologue_row_paths(gpu, m, n, k, g, monkeypatch):
    """The prologue keeps an activation row in registers up to K = 16384 (one,
    two, four or eight 16-byte chunks per thread, the last ones past the row
    end) and loops over longer rows; both paths give the same bits, and match
    the oracle."""
    x, wq, s, b = w4_problem(m, n, k, g, seed=m + n + k)
    ref = o.w4a16_matmul(x, wq, s, b, g)
    outs = {}
    for no_reg in ("0", "1"):
        monkeypatch.setenv("SPARKQ_PREP_NO_REG", no_reg)
        outs[no_reg] = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32)
        check_fp32(outs[no_reg].cpu().numpy(), ref)
    assert torch.equal(outs["0"], outs["1"])


@pytest.mark.parametrize("m,n,k,g", [(100, 520, 1024, 64), (200, 200, 4096, 32), (130, 90, 9728, 128),
                                     (512, 2560, 9728, 64)])
def test_gemm_tile_rows(gpu, m, n, k, g, monkeypatch):
    """Small grids take 64-row tiles (two 32-row fragments per wave) instead
    of 128-row ones. Without a K split both tilings add every output's
    products in the same order, so they agree bit for bit; with the planned
    split both match the oracle."""
    x, wq, s, b = w4_problem(m, n, k, g, seed=m + k)
    ref = o.w4a16_matmul(x, wq, s, b, g)
    outs = {}
    for mx4 in ("0", "1"):
        monkeypatch.setenv("SPARKQ_W4_GEMM_MX4", mx4)
        monkeypatch.delenv("SPARKQ_W4_SPLITS", raising=False)
        y32 = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32)
        check_fp32(y32.cpu().numpy(), ref)
        check_rounded16(down16(_run(gpu, x, wq, s, b, g, o.BF16)), ref, o.BF16)
        monkeypatch.setenv("SPARKQ_W4_SPLITS", "1")
        outs[mx4] = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32)
    assert torch.equal(outs["0"], outs["1"])


@pytest.mark.parametrize("m,n,k", [(1024, 4096, 2560), (1024, 4096, 2624), (1024, 4096, 2688),
                                   (1024, 4096, 2752), (384, 23040, 1536)])
def test_gemm_schedule_variants_bit_identical(gpu, m, n, k, monkeypatch):
    """The 128-row-tile GEMM's schedule variants (wave priority over the MFMA
    phase; four A slots with a barrier every second step) change neither
    the operands nor the summation order: every variant gives the default's
    bits, over step counts of every remainder mod 4 and a grid whose tiles
    past the CUs split along k; the default matches the oracle."""
    g = 64
    x, wq, s, b = w4_problem(m, n, k, g, seed=k + n)
    outs = {}
    for sch in ("8", "1", "2", "3"):   # 8: the plain schedule; 3: the default
        monkeypatch.setenv("SPARKQ_W4_GEMM_SCH", sch)
        outs[sch] = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32)
    for sch in ("1", "2", "3"):
        assert torch.equal(outs[sch], outs["8"]), sch
    cols = np.sort(np.random.default_rng(k).choice(n, size=96, replace=False))
    check_fp32(outs["3"].cpu().numpy()[:, cols], o.w4a16_matmul(x, wq[cols], s[cols], b[cols], g))


@pytest.mark.parametrize("m,n,k,g", [(1, 37, 576, 32), (3, 41, 576, 64), (2, 4, 64, 32),
                                     (4, 130, 9728, 32), (1, 5, 10240, 128), (3, 9, 4608, 64)])
def test_decode_ragged_shapes(gpu, m, n, k, g):
    """Row counts that leave a partial row quad, rows whose last 512-k span is
    partial, the longest rows the decode kernel takes, and K = 64."""
    x, wq, s, b = w4_problem(m, n, k, g, seed=n + k)
    ref = o.w4a16_matmul(x, wq, s, b, g)
    y32 = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32).cpu().numpy()
    check_fp32(y32, ref)
    check_rounded16(down16(_run(gpu, x, wq, s, b, g, o.BF16)), ref, o.BF16)


@pytest.mark.parametrize("n,k,g", [(37, 5632, 64), (36, 3712, 64), (1030, 6144, 128),
                                   (2600, 3072, 32), (4, 9728, 64), (100, 6144, 128), (2048, 8192, 64),
                                   (1024, 10240, 32)])
def test_decode_long_rows(gpu, n, k, g):
    """M = 1 with rows longer than 2560 k: rows of up to 8 whole 512-k spans
    and whole row quads take the one-round kernel, the rest the streaming
    kernel (one workgroup per CU, row quads split evenly, items dealt
    round-robin): a partial last row quad, a partial last span, more row
    quads than CUs (uneven split) and fewer row quads than CUs."""
    for dtype in (o.BF16, o.F16):
        x, wq, s, b = w4_problem(1, n, k, g, dtype=dtype, seed=n + g)
        ref = o.w4a16_matmul(x, wq, s, b, g, dtype)
        y32 = _run(gpu, x, wq, s, b, g, dtype, out_dtype=torch.float32).cpu().numpy()
        check_fp32(y32, ref)
        check_rounded16(down16(_run(gpu, x, wq, s, b, g, dtype)), ref, dtype)


@pytest.mark.parametrize("quads", ["0", "1"])
@pytest.mark.parametrize("m,n,k,g", [(3, 1100, 4096, 64), (5, 1100, 3072, 32), (12, 260, 1536, 128),
                                     (16, 1028, 2048, 64), (2, 8, 9728, 64), (4, 2600, 9728, 64)])
def test_decode_multirow_stream(gpu, m, n, k, g, quads, monkeypatch):
    """2 <= M <= 16 on the multi-row streaming kernel (the 16x16x32 kernel
    switched off): more row quads than CUs (uneven split), fewer, a row-quad
    count below the wave count, M not a multiple of 4 (the last row quartet
    repeats row M-1) and long rows; each with equal row ranges per workgroup
    (groups per row a multiple of 8; the ranges need not be whole quads) and
    with whole row quads."""
    monkeypatch.setenv("SPARKQ_W4_NO_MR", "1")
    monkeypatch.setenv("SPARKQ_W4_NO_GEMVQ", "1")
    monkeypatch.setenv("SPARKQ_W4_DEC_QUADS", quads)
    x, wq, s, b = w4_problem(m, n, k, g, seed=m * n)
    ref = o.w4a16_matmul(x, wq, s, b, g)
    y32 = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32).cpu().numpy()
    check_fp32(y32, ref)
    check_rounded16(down16(_run(gpu, x, wq, s, b, g, o.BF16)), ref, o.BF16)


@pytest.mark.parametrize("m,n,k,g", [(5, 1100, 3072, 32), (8, 3584, 2560, 64), (16, 19456, 2560, 64),
                                     (16, 1000, 1152, 128), (5, 40, 9728, 64), (16, 16, 128, 32),
                                     (11, 2560, 4096, 64), (16, 2560, 9728, 64), (9, 3584, 2560, 32)])
@pytest.mark.parametrize("tiled", ["0", "1"])
def test_decode_mfma_rows(gpu, m, n, k, g, tiled, monkeypatch):
    """5 <= M <= 16 on the 16x16x32 kernels (taken from 9 rows by default),
    the segment-major one (activations loaded once per workgroup into
    registers, group sums from an all-ones MFMA) and the tile-major one
    (activations staged in LDS): a partial last row tile, the benchmark's
    QKV, gate+up and down shapes, one-segment rows (K = 128), long rows with
    one tile per workgroup, both dtypes."""
    monkeypatch.setenv("SPARKQ_W4_MR_MIN", "5")
    monkeypatch.setenv("SPARKQ_W4_NO_GEMVQ", "1")
    monkeypatch.setenv("SPARKQ_W4_MR_TILED", tiled)
    monkeypatch.setenv("SPARKQ_W4_MR_SEG", "1" if tiled == "0" else "0")
    for dtype in (o.BF16, o.F16):
        x, wq, s, b = w4_problem(m, n, k, g, dtype=dtype, seed=m + n + k)
        ref = o.w4a16_matmul(x, wq, s, b, g, dtype)
        y32 = _run(gpu, x, wq, s, b, g, dtype, out_dtype=torch.float32).cpu().numpy()
        check_fp32(y32, ref)
        check_rounded16(down16(_run(gpu, x, wq, s, b, g, dtype)), ref, dtype)


@pytest.mark.parametrize("m,n,k,g", [(16, 2560, 9728, 64), (9, 100, 9728, 32), (8, 2560, 9728, 64),
                                     (6, 300, 8192, 128), (12, 1000, 16384, 64), (5, 48, 9728, 64)])
def test_decode_mfma_rows_split_k(gpu, m, n, k, g, monkeypatch):
    """Rows whose activations exceed the tile-major 16x16x32 kernel's staging
    split K into ranges (the down projection at 9..16 rows; 5..8 rows when
    the kernel is asked to take them); the last workgroup of a tile range
    adds the ranges' partials. Ragged N, G32..128, both dtypes, repeated
    calls bit-identical (the counters are left zero)."""
    monkeypatch.setenv("SPARKQ_W4_MR_MIN", "5")
    monkeypatch.setenv("SPARKQ_W4_MR_TILED", "1")
    for dtype in (o.BF16, o.F16):
        x, wq, s, b = w4_problem(m, n, k, g, dtype=dtype, seed=m + n + k)
        ref = o.w4a16_matmul(x, wq, s, b, g, dtype)
        y32 = _run(gpu, x, wq, s, b, g, dtype, out_dtype=torch.float32)
        check_fp32(y32.cpu().numpy(), ref)
        check_rounded16(down16(_run(gpu, x, wq, s, b, g, dtype)), ref, dtype)
        assert torch.equal(y32, _run(gpu, x, wq, s, b, g, dtype, out_dtype=torch.float32))


@pytest.mark.parametrize("m,n,k,g", [(2, 3584, 2560, 64), (3, 100, 1024, 32), (4, 19456, 2560, 64),
                                     (4, 1024, 4096, 128), (2, 44, 2048, 128), (3, 1028, 2560, 32),
                                     (4, 8, 512, 64)])
def test_decode_one_round_rows(gpu, m, n, k, g):
    """2 <= M <= 4 on the one-round kernel (rows of whole 512-k spans, whole
    row quads): each output row matches the oracle and equals, bit for bit,
    the M = 1 result for that activation row alone (the summation order of a
    row does not depend on how many rows share the launch), both dtypes;
    rows of one and two spans (two MFMA chains), rows of eight spans, more
    row quads than waves per workgroup, fewer row quads than CUs."""
    for dtype in (o.BF16, o.F16):
        x, wq, s, b = w4_problem(m, n, k, g, dtype=dtype, seed=m * n + k)
        ref = o.w4a16_matmul(x, wq, s, b, g, dtype)
        y32 = _run(gpu, x, wq, s, b, g, dtype, out_dtype=torch.float32)
        check_fp32(y32.cpu().numpy(), ref)
        check_rounded16(down16(_run(gpu, x, wq, s, b, g, dtype)), ref, dtype)
        for r in sorted({0, m // 2, m - 1}):
            y1 = _run(gpu, x[r:r + 1], wq, s, b, g, dtype, out_dtype=torch.float32)
            assert torch.equal(y32[r:r + 1], y1), r


@pytest.mark.parametrize("depth", ["1", "2"])
@pytest.mark.parametrize("m,n,k,g", [(1, 19456, 2560, 64), (1, 1100, 3072, 32), (3, 1028, 4096, 128),
                                     (4, 3584, 2560, 64), (1, 8, 512, 64)])
def test_decode_one_round_load_depth(gpu, m, n, k, g, depth, monkeypatch):
    """The one-round kernel with one or two weight loads per wave in flight
    (each next span's load issued as a span is taken up; rows of 1..8 spans,
    spans past the row's end, fewer row quads than waves): the output is bit
    for bit that of all spans in flight, and within the oracle's tolerance."""
    x, wq, s, b = w4_problem(m, n, k, g, seed=n + k + m)
    ref = o.w4a16_matmul(x, wq, s, b, g)
    monkeypatch.setenv("SPARKQ_W4_GEMVQ_DEPTH", "8")
    y_all = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32)
    monkeypatch.setenv("SPARKQ_W4_GEMVQ_DEPTH", depth)
    y = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32)
    check_fp32(y.cpu().numpy(), ref)
    assert torch.equal(y, y_all)


@pytest.mark.parametrize("m,n,k,g", [(8, 19456, 2560, 64), (4, 2560, 9728, 64), (6, 1100, 3072, 32),
                                     (5, 40, 9728, 64)])
def test_decode_multirow_stream_load_depth(gpu, m, n, k, g, monkeypatch):
    """The multi-row streaming kernel with one weight item of a wave in flight
    (each next item's load issued as an item is taken up) and with every item
    in flight: bit-identical outputs, within the oracle's tolerance."""
    monkeypatch.setenv("SPARKQ_W4_NO_MR", "1")
    monkeypatch.setenv("SPARKQ_W4_NO_GEMVQ", "1")
    x, wq, s, b = w4_problem(m, n, k, g, seed=m * 7 + n)
    ref = o.w4a16_matmul(x, wq, s, b, g)
    outs = []
    for depth in ("8", "1"):
        monkeypatch.setenv("SPARKQ_W4_DEC_DEPTH", depth)
        outs.append(_run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32))
    check_fp32(outs[1].cpu().numpy(), ref)
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("m,n,k,g,phases", [(7, 2560, 9728, 64, "1"), (8, 2560, 9728, 32, "1"),
                                            (8, 8, 9728, 64, "1"), (6, 1000, 12288, 128, "1"),
                                            (7, 1028, 9728, 32, "1"), (5, 300, 16384, 64, "1"),
                                            (5, 1100, 3072, 32, "2"), (5, 1100, 3072, 32, "4"),
                                            (8, 3584, 2560, 64, "3"), (6, 44, 4096, 32, "2")])
def test_decode_multirow_stream_phased(gpu, m, n, k, g, phases, monkeypatch):
    """The multi-row streaming kernel with its activations staged in K phases
    (5..8 rows, opt-in): the down projection at 7 and 8 rows (two phases of 10
    and 9 spans), slabs past LDS at 6 rows (K = 12288) and past the staging
    registers at 5 rows (K = 16384), a partial last row quad, fewer row quads
    than CUs, and more phases asked for on short rows (spans per phase 3 / 2 /
    2 / 4, a shorter last phase); both dtypes within the oracle's tolerance,
    repeated calls bit-identical."""
    monkeypatch.setenv("SPARKQ_W4_NO_MR", "1")
    monkeypatch.setenv("SPARKQ_W4_NO_GEMVQ", "1")
    monkeypatch.setenv("SPARKQ_W4_DEC_PHASES", phases)
    for dtype in (o.BF16, o.F16):
        x, wq, s, b = w4_problem(m, n, k, g, dtype=dtype, seed=m * 13 + n + k)
        ref = o.w4a16_matmul(x, wq, s, b, g, dtype)
        y32 = _run(gpu, x, wq, s, b, g, dtype, out_dtype=torch.float32)
        check_fp32(y32.cpu().numpy(), ref)
        check_rounded16(down16(_run(gpu, x, wq, s, b, g, dtype)), ref, dtype)
        assert torch.equal(y32, _run(gpu, x, wq, s, b, g, dtype, out_dtype=torch.float32))


@pytest.mark.parametrize("m,n,k,g", [(16, 19456, 2560, 64), (12, 2560, 9728, 64), (9, 1000, 1152, 128)])
def test_decode_mfma_rows_load_depth(gpu, m, n, k, g, monkeypatch):
    """The tile-major 16x16x32 kernel with one, two or all weight items of a
    wave in flight (each next item's load issued as an item is taken up;
    whole K and K ranges): bit-identical outputs, within the oracle's
    tolerance."""
    monkeypatch.setenv("SPARKQ_W4_MR_TILED", "1")
    x, wq, s, b = w4_problem(m, n, k, g, seed=m + n)
    ref = o.w4a16_matmul(x, wq, s, b, g)
    outs = []
    for depth in ("0", "1", "2"):
        monkeypatch.setenv("SPARKQ_W4_MR_DEPTH", depth)
        outs.append(_run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32))
    check_fp32(outs[1].cpu().numpy(), ref)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


@pytest.mark.parametrize("m", [2, 3, 4])
def test_decode_mfma_rows_few(gpu, m, monkeypatch):
    """The 16x16x32 kernel below 5 rows stays correct."""
    monkeypatch.setenv("SPARKQ_W4_MR_MIN", "2")
    monkeypatch.setenv("SPARKQ_W4_NO_GEMVQ", "1")
    n, k, g = 700, 2560, 64
    x, wq, s, b = w4_problem(m, n, k, g, seed=m)
    ref = o.w4a16_matmul(x, wq, s, b, g)
    y32 = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32).cpu().numpy()
    check_fp32(y32, ref)


@pytest.mark.parametrize("g", [32, 64, 128])
def test_gemm_row_shifts(gpu, g):
    """The bf16 GEMM runs on fp16 operands after per-row power-of-two shifts
    of the activations and of the scales. Rows far outside the fp16 range in
    either direction, an all-zero row, a row of zero scales and a row whose
    scales span 2^20 must keep the fp32 dot-product error bound: |err| <=
    2^-14 * sum_k |x_k| * (|w_k| + 8|s_g(k)|) per element."""
    m, n, k = 40, 72, 512
    x, wq, s, b = w4_problem(m, n, k, g, seed=g)
    xf = o.bits_to_f32(x, o.BF16).copy()
    xf[0] *= 2.0 ** 40
    xf[1] *= 2.0 ** -60
    xf[2] = 0.0
    xf[3, ::7] *= 2.0 ** 30
    sf, bf = o.bits_to_f32(s, o.BF16).copy(), o.bits_to_f32(b, o.BF16).copy()
    sf[0] *= 2.0 ** -40
    bf[0] *= 2.0 ** -40
    sf[1] *= 2.0 ** 40
    bf[1] *= 2.0 ** 40
    sf[2] = 0.0
    sf[3, 1] *= 2.0 ** 20
    x, s, b = o.round16(xf, o.BF16), o.round16(sf, o.BF16), o.round16(bf, o.BF16)
    ref = o.w4a16_matmul(x, wq, s, b, g)
    y = _run(gpu, x, wq, s, b, g, o.BF16, out_dtype=torch.float32).cpu().numpy().astype(np.float64)
    xa = np.abs(o.bits_to_f32(x, o.BF16).astype(np.float64))
    deq = np.abs(o.w4_dequantize(wq, s, b, g).astype(np.float64))
    s8 = np.repeat(8.0 * np.abs(o.bits_to_f32(s, o.BF16).astype(np.float64)), g, axis=1)
    bound = 2.0 ** -14 * (xa @ (deq + s8).T)
    err = np.abs(y - ref)
    assert np.isfinite(y).all()
    worst = float(np.max(err / np.maximum(bound, 1e-300)))
    print(f"worst err/bound = {worst:.3e}")
    assert (err <= bound).all(), worst
    assert np.all(y[2] == 0.0)


def test_one_hot_rows_pick_weight_columns(gpu):
    import sparkq

    n, k, g = 64, 256, 64
    _, wq, s, b = w4_problem(1, n, k, g, seed=9)
    x = np.zeros((3, k), np.float32)
    x[0, 0], x[1, 77], x[2, 255] = 1.0, 1.0, 1.0
    y = _run(gpu, o.bf16_bits(x), wq, s, b, g, o.BF16, out_dtype=torch.float32).cpu().numpy()
    deq = o.w4_dequantize(wq, s, b, g)
    assert np.array_equal(y[0], deq[:, 0]) and np.array_equal(y[1], deq[:, 77])
    assert np.array_equal(y[2], deq[:, 255])
    # the qmv / multirow entry points reach the same kernel
    xt = up16(o.bf16_bits(x[:1]), o.BF16, gpu)
    args = (up32(wq, gpu), up16(s, o.BF16, gpu), up16(b, o.BF16, gpu))
    assert torch.equal(sparkq.w4a16_qmv(xt, *args), _run(gpu, o.bf16_bits(x[:1]), wq, s, b, g, o.BF16))


@pytest.mark.parametrize("g", [32, 64, 128])
def test_gemm_one_hot_rows_pick_weight_columns(gpu, g):
    """M > 32 takes the bf16 GEMM. A one-hot activation row picks one column
    of the dequantized weights: the s*(q-8) part is exact, so the only error
    left is the bf16-pair split of the bias b + 8s, under 2^-15 |b + 8s|."""
    n, k, m = 300, 1024, 64
    _, wq, s, b = w4_problem(1, n, k, g, seed=21 + g)
    ks = np.random.default_rng(g).choice(k, m, replace=False)
    x = np.zeros((m, k), np.float32)
    x[np.arange(m), ks] = 1.0
    y = _run(gpu, o.bf16_bits(x), wq, s, b, g, o.BF16, out_dtype=torch.float32).cpu().numpy()
    deq = o.w4_dequantize(wq, s, b, g).astype(np.float64)
    ref = deq[:, ks].T
    sf = o.bits_to_f32(s, o.BF16).astype(np.float64)[:, ks // g].T
    bf = o.bits_to_f32(b, o.BF16).astype(np.float64)[:, ks // g].T
    err = np.abs(y - ref)
    bound = 2.0 ** -15 * np.abs(bf + 8.0 * sf)
    assert (err <= bound).all(), float(np.max(err - bound))


def test_deterministic(gpu):
    x, wq, s, b = w4_problem(4, 512, 2560, 64, seed=11)
    a = _run(gpu, x, wq, s, b, 64, o.BF16, out_dtype=torch.float32)
    c = _run(gpu, x, wq, s, b, 64, o.BF16, out_dtype=torch.float32)
    assert torch.equal(a, c)


# ---------------------------------------------------------------------------
# benchmark shapes: full kernels, oracle on sampled rows/columns
# ---------------------------------------------------------------------------

# the single 2560x2560 projection and the three projections of one layer
PROJ = {"square": (2560, 2560), "qkv": (3584, 2560), "gate_up": (19456, 2560),
        "down": (2560, 9728)}


def _gpu_weights(dev, n, k, g, seed):
    """Benchmark-style weights: N(0,0.02) bf16 quantized on the device."""
    import sparkq

    w16 = o.randn16(seed, n, n * k, 0.02, o.BF16).reshape(n, k)
    wq, s, b = sparkq.affine_quantize(up16(w16, o.BF16, dev), group_size=g)
    return wq, s, b


@pytest.mark.parametrize("proj", list(PROJ))
@pytest.mark.parametrize("m", [1, 4, 8, 16, 512, 2048])
def test_benchmark_shapes_sampled(gpu, proj, m):
    import sparkq

    n, k = PROJ[proj]
    g = 64
    wq, s, b = _gpu_weights(gpu, n, k, g, seed=1)
    x16 = o.randn16(0, 77 + m, m * k).reshape(m, k)
    y = sparkq.affine_quantized_matmul(up16(x16, o.BF16, gpu), wq, s, b, group_size=g,
                                       out_dtype=torch.float32).cpu().numpy()
    assert np.isfinite(y).all()
    rng = np.random.default_rng(m)
    rows = np.sort(rng.choice(m, size=min(m, 24), replace=False))
    cols = np.sort(rng.choice(n, size=256, replace=False))
    wq_h = wq.cpu().numpy().view(np.uint32)[cols]
    s_h, b_h = down16(s)[cols], down16(b)[cols]
    ref = o.w4a16_matmul(x16[rows], wq_h, s_h, b_h, g)
    check_fp32(y[np.ix_(rows, cols)], ref)


def test_linearity_full_size(gpu):
    """y(x1 + x2) = y(x1) + y(x2) at the largest prefill shape (fp32 epilogue);
    x1, x2 are chosen so that x1 + x2 is exact in bf16."""
    import sparkq

    n, k, g, m = 19456, 2560, 64, 2048
    wq, s, b = _gpu_weights(gpu, n, k, g, seed=2)
    x1 = torch.randint(-8, 8, (m, k), device=gpu).to(torch.bfloat16) / 8
    x2 = torch.randint(-8, 8, (m, k), device=gpu).to(torch.bfloat16) / 8
    f = lambda x: sparkq.affine_quantized_matmul(x, wq, s, b, group_size=g, out_dtype=torch.float32)
    lhs, rhs = f(x1 + x2), f(x1) + f(x2)
    rel = (torch.linalg.norm(lhs - rhs) / torch.linalg.norm(rhs)).item()
    assert rel < 1e-5, rel
