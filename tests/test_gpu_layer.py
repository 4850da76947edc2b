"""GPU parity of the decoder-layer steps around the W4 projections: the FFN
block (compiled_ffn, spark_mlx_llm/ops/ffn.py:83-105) fused into two launches
for up to 4 rows and composed beyond, the fused QKV projection + RoPE of one
token (spark_qkv_rope, X/src/spark_qkv_rope.cpp:14-102) and its composed
fallback, and the standalone RoPE and RMSNorm kernels.

Each stage is held to the oracle where the arithmetic is fixed: the residual
adds and the GELU*up epilogue bit for bit (given the same 16-bit inputs), the
projections bit for bit against the plain W4 kernels on the same inputs, and
the reductions (RMSNorm's mean square, the projections' dots) within one
16-bit unit of the float64 oracle."""

import math

import numpy as np
import pytest
import torch

import oracle as o
from helpers import down16, ulp_distance16, up16, up32

pytestmark = pytest.mark.gpu


def _mat(seed, stream, n, k, g, dtype):
    w = o.bits_to_f32(o.randn16(seed, stream, n * k, 0.02, dtype), dtype).reshape(n, k)
    return o.w4_quantize(w, g, dtype)


def _dev(m, dev, dtype):
    wq, s, b = m
    return up32(wq, dev), up16(s, dtype, dev), up16(b, dtype, dev)


def _ulps(a, b, dtype, floor):
    """Unit distance where |b| >= floor, 0 elsewhere (a near-zero result is
    many units of itself for an fp32 rounding difference)."""
    d = ulp_distance16(a, b, dtype)
    return np.where(np.abs(o.bits_to_f32(b, dtype)) >= floor, d, 0)


def _ulp(v, dtype):
    """One unit of the 16-bit format at |v| (normal range)."""
    mant = 7 if dtype == o.BF16 else 10
    e = np.floor(np.log2(np.maximum(np.abs(np.asarray(v, np.float64)), 2.0 ** -60)))
    return 2.0 ** (e - mant)


def _plain(x16, mats, g, dtype, dev):
    """The plain W4 projection of 16-bit rows on the device, rounded."""
    import sparkq

    y = sparkq.affine_quantized_matmul(up16(x16, dtype, dev), *_dev(mats, dev, dtype), group_size=g)
    return down16(y)


FFN_CASES = [
    # m, k, inter, g, dtype
    (1, 2560, 9728, 64, o.BF16),     # the benchmark layer: fused gate/up, streamed down
    (1, 2560, 9728, 32, o.BF16),
    (1, 2048, 1536, 128, o.F16),
    (2, 2560, 2048, 64, o.BF16),
    (4, 2048, 4096, 32, o.BF16),
    (3, 1024, 1024, 64, o.BF16),     # rows of 2 spans: composed
    (5, 2560, 2048, 64, o.BF16),     # 5 rows: composed
    (16, 512, 1024, 32, o.F16),
]


@pytest.mark.parametrize("m,k,inter,g,dtype", FFN_CASES)
def test_ffn_stages(gpu, m, k, inter, g, dtype):
    import sparkq

    seed = m + k + inter + g
    x = o.randn16(seed, 1, m * k, 1.0, dtype).reshape(m, k)
    a = o.randn16(seed, 2, m * k, 1.0, dtype).reshape(m, k)
    nw = o.round16(1.0 + 0.2 * o.randn(seed, 3, k), dtype)
    gate = _mat(seed, 4, inter, k, g, dtype)
    up = _mat(seed, 5, inter, k, g, dtype)
    down = _mat(seed, 6, k, inter, g, dtype)
    print(f"ffn m={m} k={k} I={inter} g={g} dtype={dtype}", flush=True)
    out, hid, nrm, act = sparkq.fused_ffn(
        up16(x, dtype, gpu), up16(a, dtype, gpu), up16(nw, dtype, gpu), 1e-6,
        _dev(gate, gpu, dtype), _dev(up, gpu, dtype), _dev(down, gpu, dtype), group_size=g,
        return_intermediates=True)
    out, hid, nrm, act = (down16(t) for t in (out, hid, nrm, act))
    # residual add: exact
    assert np.array_equal(hid, o.add16(x, a, dtype))
    # RMSNorm: the mean square is a reduction, so within one unit
    ref_n = o.rms_norm16(hid, nw, 1e-6, dtype)
    dn = ulp_distance16(nrm, ref_n, dtype)
    print(f"normed: max_ulp={int(dn.max())} exact={float((dn == 0).mean()):.5f}")
    assert dn.max() <= 1 and (dn == 0).mean() > 0.99
    # gate/up on the device's own normed rows through the plain kernels, then
    # the GELU*up epilogue: bit for bit
    g16 = _plain(nrm, gate, g, dtype, gpu)
    u16 = _plain(nrm, up, g, dtype, gpu)
    assert np.array_equal(act, o.gelu_mul16(g16, u16, dtype))
    # down projection of act + the residual epilogue: bit for bit
    assert np.array_equal(out, o.add16(hid, _plain(act, down, g, dtype, gpu), dtype))
    # end to end against the float64 oracle staged in the 16-bit graph
    # (a one-unit flip of a rounded gate value can move gelu's 16-bit
    # 1 + erf(.) by a whole unit of 1, so act may differ widely in a few
    # elements; the down projection dilutes that to a fraction of the MLP
    # output's scale)
    ref = o.ffn_block(x, a, nw, 1e-6, gate, up, down, g, dtype)
    got, want = o.bits_to_f32(out, dtype), o.bits_to_f32(ref["out"], dtype)
    mlp_rms = float(np.sqrt(np.mean(ref["mlp"] ** 2)))
    err = np.abs(got.astype(np.float64) - want)
    print(f"out: exact={float((out == ref['out']).mean()):.4f} max_err={err.max():.3e} "
          f"mlp_rms={mlp_rms:.3e}")
    assert np.all(err <= 2 * _ulp(want, dtype) + 0.02 * mlp_rms)


def test_ffn_fused_equals_composed(gpu, monkeypatch):
    """The fused launch and the composed steps agree (same rounding points;
    the two RMSNorm reductions may differ in a last unit)."""
    import sparkq

    m, k, inter, g, dtype = 1, 2560, 9728, 64, o.BF16
    x = o.randn16(9, 1, m * k).reshape(m, k)
    a = o.randn16(9, 2, m * k).reshape(m, k)
    nw = o.round16(1.0 + 0.2 * o.randn(9, 3, k), dtype)
    mats = [_dev(_mat(9, s, n, kk, g, dtype), gpu, dtype)
            for s, n, kk in ((4, inter, k), (5, inter, k), (6, k, inter))]
    args = (up16(x, dtype, gpu), up16(a, dtype, gpu), up16(nw, dtype, gpu), 1e-6, *mats)
    fused = [down16(t) for t in sparkq.fused_ffn(*args, group_size=g, return_intermediates=True)]
    monkeypatch.setenv("SPARKQ_NO_FUSED_FFN", "1")
    comp = [down16(t) for t in sparkq.fused_ffn(*args, group_size=g, return_intermediates=True)]
    assert np.array_equal(fused[1], comp[1])
    assert ulp_distance16(fused[2], comp[2], dtype).max() <= 1
    if np.array_equal(fused[2], comp[2]):
        assert np.array_equal(fused[3], comp[3]) and np.array_equal(fused[0], comp[0])


QKV_CASES = [
    # k, heads, kv heads, head_dim, rope_dims, g, offset, dtype
    (2560, 32, 8, 128, 128, 64, 0, o.BF16),      # the benchmark's attention shape
    (2560, 32, 8, 128, 128, 64, 4095, o.BF16),
    (2560, 16, 4, 256, 64, 32, 30000, o.BF16),   # head_dim 256, partial rotation, G32
    (2048, 16, 16, 64, 64, 128, 17, o.F16),
    (2560, 8, 2, 128, 6, 64, 100, o.BF16),       # rope_dims % 8 != 0: composed
    (1024, 8, 8, 64, 64, 64, 3, o.BF16),         # rows of 2 spans: composed
]


@pytest.mark.parametrize("k,nh,nkv,hd,rd,g,off,dtype", QKV_CASES)
def test_qkv_rope(gpu, k, nh, nkv, hd, rd, g, off, dtype):
    import sparkq

    n = (nh + 2 * nkv) * hd
    mats = _mat(k + n, 7, n, k, g, dtype)
    x = o.randn16(k + n, 8, k, 1.0, dtype)
    base = 10000.0 if off < 10000 else 1000000.0
    print(f"qkv k={k} heads={nh}/{nkv} hd={hd} rd={rd} g={g} offset={off}", flush=True)
    q, kk, v = sparkq.spark_qkv_rope(up16(x, dtype, gpu).view(1, 1, k), *_dev(mats, gpu, dtype),
                                     nh * hd, nkv * hd, nh, nkv, hd, rd, base, off, g, 4)
    assert q.shape == (1, nh, 1, hd) and kk.shape == (1, nkv, 1, hd) and v.shape == kk.shape
    q, kk, v = down16(q).reshape(nh, hd), down16(kk).reshape(nkv, hd), down16(v).reshape(nkv, hd)
    # the projection through the plain kernel: values and unrotated dims are
    # bit for bit, the rotated dims within one unit of the oracle's rope of it
    y = _plain(x.reshape(1, k), mats, g, dtype, gpu)[0]
    qs, ks = nh * hd, nkv * hd
    yq, yk, yv = y[:qs].reshape(nh, 1, hd), y[qs:qs + ks].reshape(nkv, 1, hd), y[qs + ks:]
    assert np.array_equal(v.reshape(-1), yv)
    assert np.array_equal(q[:, rd:], yq[:, 0, rd:]) and np.array_equal(kk[:, rd:], yk[:, 0, rd:])
    for got, src in ((q, yq), (kk, yk)):
        ref = o.rope16(src, rd, base, off, dtype)[:, 0]
        rms = float(np.sqrt(np.mean(o.bits_to_f32(ref, dtype) ** 2)))
        d = _ulps(got, ref, dtype, rms / 64)
        assert d.max() <= 1, int(d.max())
    # end to end against the float64 projection
    rq, rk, rv, _ = o.qkv_rope(x, *mats, g, nh, nkv, hd, rd, base, off, dtype)
    assert ulp_distance16(v, rv, dtype).max() <= 1
    for got, ref in ((q, rq), (kk, rk)):
        # one-unit flips of the rounded projection enter both rotated terms
        gf, rf = o.bits_to_f32(got, dtype), o.bits_to_f32(ref, dtype)
        rms = float(np.sqrt(np.mean(rf.astype(np.float64) ** 2)))
        err = np.abs(gf.astype(np.float64) - rf)
        print(f"rotated: exact={float((got == ref).mean()):.4f} max_err/rms={err.max() / rms:.3e}")
        assert np.all(err <= 2 * _ulp(rf, dtype) + 2.0 ** -7 * rms)


@pytest.mark.parametrize("shape,dims,trad,base,scale,off", [
    ((1, 32, 7, 128), 128, False, 10000.0, 1.0, 0),
    ((2, 8, 33, 128), 128, False, 500000.0, 1.0, 1000),
    ((1, 4, 5, 256), 64, False, 10000.0, 1.0, 12),
    ((1, 4, 9, 64), 64, True, 10000.0, 0.5, 3),
    ((3, 2, 1, 80), 40, True, 10000.0, 1.0, 70000)])
def test_rope_op(gpu, shape, dims, trad, base, scale, off):
    import sparkq

    for dtype in (o.BF16, o.F16):
        x = o.randn16(len(shape) + dims, 9, int(np.prod(shape)), 1.0, dtype).reshape(shape)
        y = down16(sparkq.rope(up16(x, dtype, gpu), dims, traditional=trad, base=base,
                               scale=scale, offset=off))
        ref = o.rope16(x, dims, base, off, dtype, traditional=trad, scale=scale)
        assert np.array_equal(y[..., dims:], x[..., dims:])
        assert _ulps(y, ref, dtype, 2.0 ** -6).max() <= 1


@pytest.mark.parametrize("m,k", [(1, 2560), (7, 4096), (64, 1000)])
def test_rms_norm_op(gpu, m, k):
    import sparkq

    for dtype in (o.BF16, o.F16):
        x = o.randn16(m, 10, m * k, 1.0, dtype).reshape(m, k)
        r = o.randn16(m, 11, m * k, 1.0, dtype).reshape(m, k)
        w = o.round16(1.0 + 0.2 * o.randn(m, 12, k), dtype)
        n, h = sparkq.rms_norm(up16(x, dtype, gpu), up16(w, dtype, gpu), 1e-5,
                               residual=up16(r, dtype, gpu), return_hidden=True)
        assert np.array_equal(down16(h), o.add16(x, r, dtype))
        d = ulp_distance16(down16(n), o.rms_norm16(o.add16(x, r, dtype), w, 1e-5, dtype), dtype)
        assert d.max() <= 1 and (d == 0).mean() > 0.99


def test_dispatch_routes(gpu):
    """sparkq.ops.dispatch_ffn / dispatch_qkv take the fused kernels for the
    standard modules and one token, and the composed route otherwise, with
    the results of the direct ops."""
    import sparkq
    from sparkq.ops import QuantizedLinear, RMSNorm, RoPE, dispatch_ffn, dispatch_qkv

    dtype, g, k, inter = o.BF16, 64, 2560, 2048
    t16 = torch.bfloat16

    def layer(seed, n, kk):
        wq, s, b = _dev(_mat(seed, 1, n, kk, g, dtype), gpu, dtype)
        return QuantizedLinear(wq, s, b, group_size=g, bits=4)

    class MLP(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_proj, self.up_proj, self.down_proj = (
                layer(1, inter, k), layer(2, inter, k), layer(3, k, inter))

        def forward(self, x):
            raise AssertionError("the standard MLP must take the fused route")

    mlp = MLP()
    norm = RMSNorm(k, 1e-6, weight=up16(o.round16(1.0 + 0.1 * o.randn(1, 4, k), dtype), dtype, gpu))
    x = up16(o.randn16(1, 5, k), dtype, gpu).view(1, 1, k)
    a = up16(o.randn16(1, 6, k), dtype, gpu).view(1, 1, k)
    y = dispatch_ffn(x, a, norm, mlp, mlp_type=MLP)
    p = lambda m: (m.weight, m.scales, m.biases)  # noqa: E731
    ref = sparkq.fused_ffn(x, a, norm.weight, 1e-6, p(mlp.gate_proj), p(mlp.up_proj),
                           p(mlp.down_proj), group_size=g)
    assert torch.equal(y, ref)

    nh, nkv, hd = 8, 2, 128
    proj = layer(7, (nh + 2 * nkv) * hd, k)
    rope = RoPE(hd, base=10000.0)
    kw = dict(q_size=nh * hd, kv_size=nkv * hd, n_heads=nh, n_kv_heads=nkv, head_dim=hd)
    q1, k1, v1 = dispatch_qkv(x, proj, rope, offset=5, **kw)
    fq, fk, fv = sparkq.spark_qkv_rope(x, proj.weight, proj.scales, proj.biases, nh * hd,
                                       nkv * hd, nh, nkv, hd, hd, 10000.0, 5, g, 4)
    assert torch.equal(q1, fq) and torch.equal(k1, fk) and torch.equal(v1, fv)
    # four tokens: projection, head split, rope at positions 5..8
    x4 = up16(o.randn16(1, 8, 4 * k), dtype, gpu).view(1, 4, k)
    q4, k4, v4 = dispatch_qkv(x4, proj, rope, offset=5, **kw)
    y4 = sparkq.affine_quantized_matmul(x4, proj.weight, proj.scales, proj.biases, group_size=g)
    yq = y4[..., :nh * hd].reshape(1, 4, nh, hd).transpose(1, 2)
    assert q4.shape == (1, nh, 4, hd) and v4.shape == (1, nkv, 4, hd)
    assert torch.equal(q4, sparkq.rope(yq.contiguous(), hd, base=10000.0, offset=5))
    assert torch.equal(v4, y4[..., (nh + nkv) * hd:].reshape(1, 4, nkv, hd).transpose(1, 2))
    # token 3 of the four equals the single-token fused route at offset 8
    # up to the projection's row count (same per-row arithmetic)
    s1 = dispatch_qkv(x4[:, 3:4].contiguous(), proj, rope, offset=8, **kw)
    assert torch.equal(s1[2][:, :, 0], v4[:, :, 3])
    assert t16 == q4.dtype


def test_layer_graph_replay_matches_eager(gpu):
    """The fused FFN block (one token and 16 rows), QKV + RoPE and the KV
    append captured in one HIP graph: every replay, with eager work and
    synchronisation between them, equals the eager results bit for bit."""
    import sparkq

    dtype, g, k, inter = o.BF16, 64, 2560, 9728
    mats = [_dev(_mat(3, s, n, kk, g, dtype), gpu, dtype)
            for s, n, kk in ((4, inter, k), (5, inter, k), (6, k, inter))]
    qkv = _dev(_mat(3, 7, 3584, k, g, dtype), gpu, dtype)
    nw = up16(o.round16(1.0 + 0.1 * o.randn(3, 3, k), dtype), dtype, gpu)
    x1 = up16(o.randn16(3, 1, k), dtype, gpu).view(1, k)
    a1 = up16(o.randn16(3, 2, k), dtype, gpu).view(1, k)
    x16 = up16(o.randn16(3, 8, 16 * k), dtype, gpu).view(16, k)
    a16 = up16(o.randn16(3, 9, 16 * k), dtype, gpu).view(16, k)
    cache = sparkq.QuantizedKVCache(group_size=32, kv_format="affine_u8")
    kv = up16(o.randn16(3, 10, 4 * 128), dtype, gpu).view(1, 4, 1, 128)
    cache.update_and_fetch(kv, kv)   # allocate the storage before capture

    def step():
        f1 = sparkq.fused_ffn(x1, a1, nw, 1e-6, *mats, group_size=g)
        f16 = sparkq.fused_ffn(x16, a16, nw, 1e-6, *mats, group_size=g)
        q, kk, v = sparkq.spark_qkv_rope(x1.view(1, 1, k), *qkv, 2560, 512, 20, 4, 128, 128,
                                         10000.0, 77, g, 4)
        cache.offset = 1
        keys, _ = cache.update_and_fetch(kk, v)
        return [f1, f16, q, kk, v, keys[0]]

    eager = [t.clone() for t in step()]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    for _ in range(3):
        junk = torch.randn(1 << 20, device=gpu).sum()   # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert float(junk) == float(junk)
        for got, want in zip(outs, eager):
            assert torch.equal(got, want)
