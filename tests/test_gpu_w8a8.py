"""GPU parity of the W8A8 path against the oracle: the per-token quantizer and
the int32 accumulators bit-exact, and (because the epilogue is the same
fmaf in both) the fp32 output bit-exact too; 16-bit outputs are its
correctly rounded value."""

import numpy as np
import pytest
import torch

import oracle as o
from helpers import TORCH16, down16, up16

pytestmark = pytest.mark.gpu


def _x(m, k, dtype, seed=0):
    return o.randn16(seed, 300 + m, m * k, 1.0, dtype).reshape(m, k)


@pytest.mark.parametrize("dtype", [o.BF16, o.F16, o.F32])
@pytest.mark.parametrize("m,k", [(1, 2560), (8, 9728), (16, 2560), (5, 32), (3, 131040)])
def test_quantize_per_token_bit_exact(gpu, m, k, dtype):
    import sparkq

    if dtype == o.F32:
        xf = o.randn(1, m, m * k).reshape(m, k)
        xt = torch.from_numpy(xf).to(gpu)
    else:
        x16 = _x(m, k, dtype)
        xf = o.bits_to_f32(x16, dtype)
        xt = up16(x16, dtype, gpu)
    if m >= 3:
        xf[2] = 0.0
        xt[2] = 0.0
    q, sc = sparkq.quantize_per_token(xt)
    rq, rsc = o.a8_quantize(xf)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(sc.cpu().numpy().view(np.uint32), rsc.view(np.uint32))


def test_quantize_ties_round_to_even(gpu):
    import sparkq

    x = np.zeros((1, 64), np.float32)
    x[0, :5] = [127.0, 2.5, 1.5, -0.5, -2.5]   # scale 1: ties at .5
    q, sc = sparkq.quantize_per_token(torch.from_numpy(x).to(gpu))
    assert sc.item() == 1.0
    assert q[0, :5].tolist() == [127, 2, 2, 0, -2]


@pytest.mark.parametrize("m,n,k", [(1, 3584, 2560), (8, 2560, 9728), (16, 19456, 2560),
                                   (33, 96, 256), (70, 130, 512), (2, 40, 32),
                                   (3, 37, 32), (4, 130, 9728), (2, 5, 10240), (1, 9, 4864),
                                   (4, 2560, 2560), (5, 37, 64), (13, 100, 192), (16, 17, 2560),
                                   (7, 101, 4096), (11, 203, 2560), (9, 3, 9728)])
def test_int8_matmul_int32_bit_exact(gpu, m, n, k):
    import sparkq

    rng = np.random.default_rng(m * 7 + n)
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    b = rng.integers(-128, 128, (n, k), dtype=np.int8)
    c = sparkq.int8_matmul_int32(torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu))
    if m * n * k > 2e8:
        cols = np.sort(rng.choice(n, 256, replace=False))
        assert np.array_equal(c.cpu().numpy()[:, cols], o.int8_matmul(a, b[cols]))
    else:
        assert np.array_equal(c.cpu().numpy(), o.int8_matmul(a, b))


@pytest.mark.parametrize("m,n,k", [(3, 16390, 2560), (16, 16384, 1024), (8, 19456, 3072),
                                   (5, 17000, 1536), (12, 20000, 2048), (16, 19456, 2560)])
def test_int8_rows_one_round(gpu, m, n, k, monkeypatch):
    """3..16 rows over at least two 16-row tiles per workgroup slot (the
    one-round kernel: activations staged once per workgroup, K in quarters):
    a partial last tile, K = 1024..3072, bit-exact against the oracle on the
    first and last tiles and sampled columns, and equal in full to the
    per-tile kernel."""
    import sparkq

    rng = np.random.default_rng(m * 11 + n + k)
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    b = rng.integers(-128, 128, (n, k), dtype=np.int8)
    at, bt = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    c = sparkq.int8_matmul_int32(at, bt)
    cols = np.unique(np.concatenate([np.arange(16), np.arange(n - 16, n),
                                     rng.choice(n, 256, replace=False)]))
    assert np.array_equal(c.cpu().numpy()[:, cols], o.int8_matmul(a, b[cols]))
    monkeypatch.setenv("SPARKQ_I8_NO_ROWSQ", "1")
    assert torch.equal(c, sparkq.int8_matmul_int32(at, bt))


@pytest.mark.parametrize("m,n,k,dtype,with_bias", [(3, 16390, 2560, o.BF16, True), (8, 19456, 2560, o.F16, False),
                                                   (5, 17000, 1536, o.BF16, False), (9, 16384, 2560, o.BF16, True),
                                                   (6, 20000, 3072, o.F16, True), (8, 19456, 2560, o.BF16, False)])
def test_w8a8_linear_rows_one_round(gpu, m, n, k, dtype, with_bias, monkeypatch):
    """W8A8 projections over the one-round rows kernel (epilogue with and
    without bias): the fp32 output bit for bit against the oracle on the
    first and last row tiles and sampled columns, and equal in full, in fp32
    and in the 16-bit dtype, to the per-tile rows kernel."""
    import sparkq

    x16 = _x(m, k, dtype, seed=n)
    xf = o.bits_to_f32(x16, dtype)
    wq, wsc = _w8(n, k, seed=m)
    rng = np.random.default_rng(n + k)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float32) if with_bias else None
    xt = up16(x16, dtype, gpu)
    wt, st = torch.from_numpy(wq).to(gpu), torch.from_numpy(wsc).to(gpu)
    bt = torch.from_numpy(bias).to(gpu) if with_bias else None
    y32 = sparkq.w8a8_linear(xt, wt, st, bias=bt, out_dtype=torch.float32)
    y16 = sparkq.w8a8_linear(xt, wt, st, bias=bt)
    cols = np.unique(np.concatenate([np.arange(16), np.arange(n - 16, n), rng.choice(n, 256, replace=False)]))
    qa, sa = o.a8_quantize(xf)
    ref = o.w8a8_epilogue(o.int8_matmul(qa, wq[cols]), sa, wsc[cols], None if bias is None else bias[cols])
    assert np.array_equal(y32.cpu().numpy()[:, cols].view(np.uint32), ref.view(np.uint32))
    monkeypatch.setenv("SPARKQ_I8_NO_ROWSQ", "1")
    assert torch.equal(y32, sparkq.w8a8_linear(xt, wt, st, bias=bt, out_dtype=torch.float32))
    assert torch.equal(y16, sparkq.w8a8_linear(xt, wt, st, bias=bt))


@pytest.mark.parametrize("m,n,k,dtype", [(8, 3584, 2560, o.BF16), (16, 19456, 2560, o.BF16), (5, 2560, 9728, o.F16),
                                         (3, 100, 512, o.BF16), (16, 17, 2560, o.F16), (12, 1000, 16384, o.BF16)])
def test_w8a8_one_launch_quantizer(gpu, m, n, k, dtype, monkeypatch):
    """3..16 rows in one launch (producer workgroups quantize the rows while
    the others stream their weights): equal to the quantizer launch followed
    by the int8 kernel, on consecutive calls with different activations (the
    ready counter is left zero between calls), with the workgroups'
    self-quantizing fallback forced, and bit for bit against the oracle on
    sampled columns."""
    import sparkq

    monkeypatch.setenv("SPARKQ_I8_SYNCQ_ALL", "1")  # every row length, not only K > 4096
    wq, wsc = _w8(n, k, seed=m + 1)
    wt, st = torch.from_numpy(wq).to(gpu), torch.from_numpy(wsc).to(gpu)
    xs = [_x(m, k, dtype, seed=s) for s in (n, n + 1)]
    xts = [up16(x, dtype, gpu) for x in xs]
    one = [sparkq.w8a8_linear(xt, wt, st, out_dtype=torch.float32) for xt in (xts[0], xts[1], xts[0])]
    monkeypatch.setenv("SPARKQ_I8_SELF_QUANTIZE", "1")
    own = [sparkq.w8a8_linear(xt, wt, st, out_dtype=torch.float32) for xt in xts]
    monkeypatch.setenv("SPARKQ_I8_NO_SYNCQ", "1")
    two = [sparkq.w8a8_linear(xt, wt, st, out_dtype=torch.float32) for xt in xts]
    assert torch.equal(one[0], two[0]) and torch.equal(one[1], two[1]) and torch.equal(one[2], two[0])
    assert torch.equal(own[0], two[0]) and torch.equal(own[1], two[1])
    cols = np.sort(np.random.default_rng(n).choice(n, min(n, 256), replace=False))
    qa, sa = o.a8_quantize(o.bits_to_f32(xs[1], dtype))
    ref = o.w8a8_epilogue(o.int8_matmul(qa, wq[cols]), sa, wsc[cols])
    assert np.array_equal(one[1].cpu().numpy()[:, cols].view(np.uint32), ref.view(np.uint32))


def test_int8_matmul_extreme_range(gpu):
    import sparkq

    k = 131040
    a = np.full((2, k), -128, np.int8)
    b = np.full((33, k), -128, np.int8)
    b[1] = 127
    c = sparkq.int8_matmul_int32(torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu))
    assert c[0, 0].item() == 16384 * k and c[0, 1].item() == -128 * 127 * k


def _w8(n, k, seed=0):
    w = o.randn(seed, 500 + n, n * k, 0.02).reshape(n, k)
    return o.w8_quantize_channel(w)


@pytest.mark.parametrize("dtype", [o.BF16, o.F16, o.F32])
@pytest.mark.parametrize("m,n,k", [(1, 3584, 2560), (8, 2560, 9728), (16, 19456, 2560),
                                   (40, 100, 256), (1, 2560, 9728), (3, 37, 32), (4, 130, 4096),
                                   (2, 21, 10240), (5, 37, 64), (12, 100, 9728), (6, 101, 512),
                                   (16, 4, 256), (9, 203, 2560), (7, 45, 9728)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_w8a8_linear_bit_exact(gpu, m, n, k, dtype, with_bias):
    import sparkq

    wq, wsc = _w8(n, k)
    if dtype == o.F32:
        xf = o.randn(2, m, m * k).reshape(m, k)
        xt = torch.from_numpy(xf).to(gpu)
    else:
        x16 = _x(m, k, dtype, seed=1)
        xf = o.bits_to_f32(x16, dtype)
        xt = up16(x16, dtype, gpu)
    bias = o.randn(3, n, n) if with_bias else None
    bias_t = torch.from_numpy(bias).to(gpu) if with_bias else None
    wt, st = torch.from_numpy(wq).to(gpu), torch.from_numpy(wsc).to(gpu)
    y32 = sparkq.w8a8_linear(xt, wt, st, bias_t, out_dtype=torch.float32).cpu().numpy()
    qa, sa = o.a8_quantize(xf)
    rng = np.random.default_rng(0)
    cols = np.sort(rng.choice(n, min(n, 512), replace=False))
    acc = o.int8_matmul(qa, wq[cols])
    ref = o.w8a8_epilogue(acc, sa, wsc[cols], bias[cols] if with_bias else None)
    assert np.array_equal(y32[:, cols].view(np.uint32), ref.view(np.uint32))
    y = sparkq.w8a8_linear(xt, wt, st, bias_t)
    assert y.dtype == (torch.float32 if dtype == o.F32 else TORCH16[dtype])
    if dtype != o.F32:
        assert np.array_equal(down16(y)[:, cols], o.round16(ref, dtype))


@pytest.mark.parametrize("dtype", [o.BF16, o.F16, o.F32])
@pytest.mark.parametrize("m,n,k", [(1, 2560, 9728), (2, 2560, 9728), (1, 3584, 2560), (2, 19456, 2560),
                                   (1, 37, 1056), (2, 300, 4096), (1, 257, 1024), (2, 100, 8192),
                                   (1, 9, 2048)])
def test_w8a8_linear_stream(gpu, m, n, k, dtype, monkeypatch):
    """1..2 rows on the streaming int8 GEMV (one workgroup per CU over a
    contiguous run of weight rows, 1 KB items that may cross a row end, the
    quantizer fused): the fp32 epilogue bit for bit against the oracle on
    sampled columns and the first and last rows of every run, and equal in
    full to the kernels that serve these shapes without it."""
    import sparkq

    print(f"[case] w8a8 stream m={m} n={n} k={k} dtype={dtype}", flush=True)
    wq, wsc = _w8(n, k, seed=4)
    if dtype == o.F32:
        xf = o.randn(5, m, m * k).reshape(m, k)
        xt = torch.from_numpy(xf).to(gpu)
    else:
        x16 = _x(m, k, dtype, seed=5)
        xf = o.bits_to_f32(x16, dtype)
        xt = up16(x16, dtype, gpu)
    bias = o.randn(6, n, n)
    bias_t = torch.from_numpy(bias).to(gpu)
    wt, st = torch.from_numpy(wq).to(gpu), torch.from_numpy(wsc).to(gpu)
    monkeypatch.setenv("SPARKQ_I8_STREAM", "1")
    y32 = sparkq.w8a8_linear(xt, wt, st, bias_t, out_dtype=torch.float32)
    y16 = sparkq.w8a8_linear(xt, wt, st, bias_t)
    monkeypatch.setenv("SPARKQ_I8_NO_STREAM", "1")
    assert torch.equal(y32, sparkq.w8a8_linear(xt, wt, st, bias_t, out_dtype=torch.float32))
    assert torch.equal(y16, sparkq.w8a8_linear(xt, wt, st, bias_t))
    p = min(n, 256)
    edges = {r for i in range(p) for r in (i * n // p, (i + 1) * n // p - 1)}
    rng = np.random.default_rng(n + k)
    cols = np.array(sorted(edges | set(rng.choice(n, min(n, 256), replace=False).tolist())))
    cols = cols[:768]
    qa, sa = o.a8_quantize(xf)
    ref = o.w8a8_epilogue(o.int8_matmul(qa, wq[cols]), sa, wsc[cols], bias[cols])
    assert np.array_equal(y32.cpu().numpy()[:, cols].view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dtype", [o.BF16, o.F16, o.F32])
@pytest.mark.parametrize("m,n,k", [(1, 3584, 2560), (2, 3584, 2560), (1, 19456, 2560), (2, 19456, 2560),
                                   (1, 37, 512), (2, 1030, 2560), (1, 5, 256), (2, 300, 1024)])
def test_w8a8_linear_one_round(gpu, m, n, k, dtype, monkeypatch):
    """1..2 rows over whole 256-k spans up to K = 2560 on the one-round int8
    GEMV (one row quad per wave over its whole row, the quantizer fused, one,
    two or every span in flight): the fp32 epilogue bit for bit against the
    oracle on the first and last rows and sampled columns, and equal in full
    to the kernels that serve these shapes without it; a partial row quad,
    fewer quads than CUs and more than eight per CU."""
    import sparkq

    print(f"[case] w8a8 one-round m={m} n={n} k={k} dtype={dtype}", flush=True)
    wq, wsc = _w8(n, k, seed=8)
    if dtype == o.F32:
        xf = o.randn(9, m, m * k).reshape(m, k)
        xt = torch.from_numpy(xf).to(gpu)
    else:
        x16 = _x(m, k, dtype, seed=9)
        xf = o.bits_to_f32(x16, dtype)
        xt = up16(x16, dtype, gpu)
    bias = o.randn(10, n, n)
    bias_t = torch.from_numpy(bias).to(gpu)
    wt, st = torch.from_numpy(wq).to(gpu), torch.from_numpy(wsc).to(gpu)
    monkeypatch.setenv("SPARKQ_I8_Q", "1")
    outs = []
    for depth in ("8", "1", "2"):
        monkeypatch.setenv("SPARKQ_I8_Q_DEPTH", depth)
        outs.append(sparkq.w8a8_linear(xt, wt, st, bias_t, out_dtype=torch.float32))
    y16 = sparkq.w8a8_linear(xt, wt, st, bias_t)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    monkeypatch.setenv("SPARKQ_I8_NO_Q", "1")
    monkeypatch.delenv("SPARKQ_I8_Q")
    assert torch.equal(outs[0], sparkq.w8a8_linear(xt, wt, st, bias_t, out_dtype=torch.float32))
    assert torch.equal(y16, sparkq.w8a8_linear(xt, wt, st, bias_t))
    rng = np.random.default_rng(n + k + m)
    cols = np.unique(np.concatenate([np.arange(min(n, 8)), np.arange(max(0, n - 8), n),
                                     rng.choice(n, min(n, 256), replace=False)]))
    qa, sa = o.a8_quantize(xf)
    ref = o.w8a8_epilogue(o.int8_matmul(qa, wq[cols]), sa, wsc[cols], bias[cols])
    assert np.array_equal(outs[0].cpu().numpy()[:, cols].view(np.uint32), ref.view(np.uint32))


BENCH_PROJ = {"qkv": (3584, 2560), "gate_up": (19456, 2560), "down": (2560, 9728)}


@pytest.mark.parametrize("proj", list(BENCH_PROJ))
@pytest.mark.parametrize("m", [1, 8, 16])
def test_w8a8_benchmark_pairs_bit_exact(gpu, m, proj):
    """Every (rows, projection) pair of the W8A8 decode benchmark: int32
    accumulators (through the raw entry point) and the fp32 epilogue bit for
    bit on sampled columns."""
    import sparkq

    n, k = BENCH_PROJ[proj]
    print(f"[case] w8a8 m={m} proj={proj}", flush=True)
    wq, wsc = _w8(n, k, seed=9)
    x16 = _x(m, k, o.BF16, seed=m)
    xf = o.bits_to_f32(x16, o.BF16)
    xt = up16(x16, o.BF16, gpu)
    wt, st = torch.from_numpy(wq).to(gpu), torch.from_numpy(wsc).to(gpu)
    y32 = sparkq.w8a8_linear(xt, wt, st, out_dtype=torch.float32).cpu().numpy()
    qa, sa = o.a8_quantize(xf)
    qt, sat = sparkq.quantize_per_token(xt)
    assert np.array_equal(qt.cpu().numpy(), qa) and np.array_equal(sat.cpu().numpy(), sa)
    acc_t = sparkq.int8_matmul_int32(qt, wt).cpu().numpy()
    cols = np.sort(np.random.default_rng(m + n).choice(n, 512, replace=False))
    acc = o.int8_matmul(qa, wq[cols])
    assert np.array_equal(acc_t[:, cols], acc)
    ref = o.w8a8_epilogue(acc, sa, wsc[cols])
    assert np.array_equal(y32[:, cols].view(np.uint32), ref.view(np.uint32))


def test_w8a8_decode_zero_row_and_repeat(gpu):
    """Decode GEMV with an all-zero activation row (scale 1, zero codes) and a
    second call on the same buffers giving identical bits."""
    import sparkq

    m, n, k = 3, 260, 2560
    wq, wsc = _w8(n, k, seed=4)
    x16 = _x(m, k, o.BF16, seed=5)
    x16[1] = 0
    xt = up16(x16, o.BF16, gpu)
    wt, st = torch.from_numpy(wq).to(gpu), torch.from_numpy(wsc).to(gpu)
    y1 = sparkq.w8a8_linear(xt, wt, st, out_dtype=torch.float32)
    y2 = sparkq.w8a8_linear(xt, wt, st, out_dtype=torch.float32)
    assert torch.equal(y1, y2)
    qa, sa = o.a8_quantize(o.bits_to_f32(x16, o.BF16))
    ref = o.w8a8_epilogue(o.int8_matmul(qa, wq), sa, wsc)
    assert np.array_equal(y1.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert np.all(y1[1].cpu().numpy() == 0)


def test_readme_known_answer(gpu):
    """ones(32) activations x ones(4,32) int8 weights, scale 1 -> 32
    (X/README.md:41-46, adapted from W8A16 to W8A8)."""
    import sparkq

    lin = sparkq.W8A8Linear(torch.ones((4, 32), dtype=torch.int8, device=gpu),
                            torch.ones(4, dtype=torch.float32, device=gpu))
    y = lin(torch.ones((1, 32), dtype=torch.bfloat16, device=gpu))
    assert y.float().cpu().tolist() == [[32.0] * 4]


@pytest.mark.parametrize("m", [512, 2048])
def test_w8a8_prefill_out_proj_bit_exact(gpu, m):
    """W8A8 at prefill sizes, the reference's out_proj at any M
    (X/src/spark_w8a8.cpp:71-151): N=2560, K=4096. int32 accumulators
    (raw entry point) and the fp32 epilogue bit for bit on sampled rows and
    columns, the bf16 output its correctly rounded value."""
    import sparkq

    n, k = 2560, 4096
    print(f"[case] w8a8 prefill m={m}", flush=True)
    wq, wsc = _w8(n, k, seed=m)
    x16 = _x(m, k, o.BF16, seed=m + 1)
    xt = up16(x16, o.BF16, gpu)
    wt, st = torch.from_numpy(wq).to(gpu), torch.from_numpy(wsc).to(gpu)
    y32 = sparkq.w8a8_linear(xt, wt, st, out_dtype=torch.float32).cpu().numpy()
    y16 = down16(sparkq.w8a8_linear(xt, wt, st))
    qa, sa = o.a8_quantize(o.bits_to_f32(x16, o.BF16))
    qt, _ = sparkq.quantize_per_token(xt)
    acc_t = sparkq.int8_matmul_int32(qt, wt).cpu().numpy()
    rng = np.random.default_rng(m)
    rows = np.sort(rng.choice(m, 96, replace=False))
    cols = np.sort(rng.choice(n, 160, replace=False))
    acc = o.int8_matmul(qa[rows], wq[cols])
    assert np.array_equal(acc_t[np.ix_(rows, cols)], acc)
    ref = o.w8a8_epilogue(acc, sa[rows], wsc[cols])
    assert np.array_equal(y32[np.ix_(rows, cols)].view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(y16[np.ix_(rows, cols)], o.round16(ref, o.BF16))


@pytest.mark.parametrize("m,n,k", [(2048, 2176, 2048), (2048, 2560, 4096)])
def test_int8_gemm_whole_and_split_tiles(gpu, m, n, k, monkeypatch):
    """Between one and two 128 x 128 tiles per CU, the tiled int8 GEMM runs one
    whole tile per CU and splits only the tiles past them (the last row tile's
    columns here): the int32 accumulators of rows in both regions equal the
    int64 oracle, and equal the unsplit grid's bit for bit."""
    import sparkq

    print(f"[case] int8 gemm whole+split m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m + n + k)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    at, bt = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    c = sparkq.int8_matmul_int32(at, bt).cpu().numpy()
    rows = np.sort(np.concatenate([rng.choice(m - 128, 48, replace=False),
                                   m - 128 + rng.choice(128, 48, replace=False)]))
    cols = np.sort(rng.choice(n, 128, replace=False))
    assert np.array_equal(c[np.ix_(rows, cols)], o.int8_matmul(a[rows], b[cols]))
    monkeypatch.setenv("SPARKQ_I8_GEMM_NO_CU1", "1")
    assert np.array_equal(sparkq.int8_matmul_int32(at, bt).cpu().numpy(), c)


@pytest.mark.parametrize("m,n,k,gm", [(2048, 2560, 1024, "4"), (4096, 2560, 512, "2"), (640, 1000, 256, "4"),
                                      (300, 300, 384, "8"), (2048, 2176, 2048, "4")])
def test_int8_gemm_tile_order(gpu, m, n, k, gm, monkeypatch):
    """The XCD-grouped tile order (each XCD's work items take a contiguous
    chunk of the order, walked in groups of gm tile rows) against row-major
    order: identical int32 accumulators over whole grids, tile counts that
    are and are not multiples of eight, with and without k pieces; sampled
    elements equal the int64 oracle."""
    import sparkq

    print(f"[case] int8 gemm tile order m={m} n={n} k={k} gm={gm}", flush=True)
    rng = np.random.default_rng(m * 3 + n + k)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    at, bt = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    monkeypatch.setenv("SPARKQ_I8_GEMM_GM", gm)
    c = sparkq.int8_matmul_int32(at, bt)
    monkeypatch.setenv("SPARKQ_I8_GEMM_ROWMAJOR", "1")
    assert torch.equal(c, sparkq.int8_matmul_int32(at, bt))
    rows = np.sort(rng.choice(m, 64, replace=False))
    cols = np.sort(rng.choice(n, 96, replace=False))
    assert np.array_equal(c.cpu().numpy()[np.ix_(rows, cols)], o.int8_matmul(a[rows], b[cols]))


@pytest.mark.parametrize("m,n,k", [(64, 96, 256), (130, 300, 512), (200, 2560, 1024),
                                   (1000, 130, 384), (257, 64, 8192), (96, 4100, 128)])
@pytest.mark.parametrize("splits", ["0", "1", "3"])
def test_int8_gemm_tiled_bit_exact(gpu, m, n, k, splits, monkeypatch):
    """The tiled int8 GEMM (64 rows and more, K % 128 == 0): rows and columns
    that leave partial 128 x 128 tiles, one k step, long rows, and K split
    into pieces (the planned count, forced to 1, forced to 3): the raw int32
    accumulators equal the int64 oracle in every element, and so do the
    fp32 epilogue values of w8a8_linear."""
    import sparkq

    monkeypatch.setenv("SPARKQ_I8_GEMM_SPLITS", splits)
    print(f"[case] int8 gemm m={m} n={n} k={k} splits={splits}", flush=True)
    rng = np.random.default_rng(m + n + k)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    a[3] = 127
    b[5] = -127
    c = sparkq.int8_matmul_int32(torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu))
    assert np.array_equal(c.cpu().numpy(), o.int8_matmul(a, b))
    wq, wsc = _w8(n, k, seed=n)
    x16 = _x(m, k, o.BF16, seed=k)
    xt = up16(x16, o.BF16, gpu)
    y32 = sparkq.w8a8_linear(xt, torch.from_numpy(wq).to(gpu), torch.from_numpy(wsc).to(gpu),
                             out_dtype=torch.float32).cpu().numpy()
    qa, sa = o.a8_quantize(o.bits_to_f32(x16, o.BF16))
    ref = o.w8a8_epilogue(o.int8_matmul(qa, wq), sa, wsc)
    assert np.array_equal(y32.view(np.uint32), ref.view(np.uint32))
