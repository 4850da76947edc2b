"""The allocation-free INT8-KV decode (sparkq_int8kv_sdpa_decode_noalloc)
against the workspace entry point it shares its kernels with, called
through the C-ABI on the same inputs: the outputs must be identical, on two
calls in a row whose second is smaller (the fixed scratch keeps the first
call's partials and counters), for both cache formats and a split and an
unsplit context."""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(dev, b, hq, hkv, n, d, fmt, g, seed):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn((b, hq, d), generator=gen).to(torch.bfloat16).to(dev)
    if fmt == 0:
        kc = torch.randint(-127, 128, (b, hkv, n, d), generator=gen, dtype=torch.int8).to(dev)
        vc = torch.randint(-127, 128, (b, hkv, n, d), generator=gen, dtype=torch.int8).to(dev)
        ks = (torch.rand((b, hkv, n), generator=gen) * 0.02 + 1e-3).to(torch.float16).to(dev)
        vs = (torch.rand((b, hkv, n), generator=gen) * 0.02 + 1e-3).to(torch.float16).to(dev)
        kb = vb = None
        strides = [n * d * hkv, n * d, d, n * hkv, n, 1] * 2
    else:
        def packed():
            return torch.randint(-2 ** 31, 2 ** 31 - 1, (b, hkv, n, d // 4), generator=gen,
                                 dtype=torch.int32).to(dev)
        kc, vc = packed(), packed()
        ks = (torch.rand((b, hkv, n, d // g), generator=gen) * 0.01).to(torch.bfloat16).to(dev)
        vs = (torch.rand((b, hkv, n, d // g), generator=gen) * 0.01).to(torch.bfloat16).to(dev)
        kb = (-torch.rand((b, hkv, n, d // g), generator=gen)).to(torch.bfloat16).to(dev)
        vb = (-torch.rand((b, hkv, n, d // g), generator=gen)).to(torch.bfloat16).to(dev)
        strides = [n * d * hkv, n * d, d, n * hkv * (d // g), n * (d // g), d // g] * 2
    return q, kc, ks, kb, vc, vs, vb, strides


def _call(noalloc, dev, args, b, hq, hkv, n, d, fmt, g):
    from sparkq import _lib

    q, kc, ks, kb, vc, vs, vb, strides = args
    out = torch.full((b, hq, d), float("nan"), dtype=torch.float32, device=dev)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    st = (ctypes.c_int64 * 12)(*strides)
    stream = _lib.stream_handle(dev)
    head = (ptr(q), ptr(kc), ptr(ks), ptr(kb), ptr(vc), ptr(vs), ptr(vb), ptr(out), b, hq, hkv,
            n, d, g, fmt, _lib.BF16, _lib.F32, ctypes.c_float(d ** -0.5), st)
    if noalloc:
        rc = _lib.lib().sparkq_int8kv_sdpa_decode_noalloc(*head, stream)
    else:
        nbytes = _lib.lib().sparkq_int8kv_sdpa_workspace_bytes(b, hq, n, d)
        ws = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=dev)
        rc = _lib.lib().sparkq_int8kv_sdpa_decode(*head, ctypes.c_void_p(ws.data_ptr()),
                                                  nbytes, stream)
    assert rc == 0, _lib.lib().sparkq_last_error().decode()
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("fmt,g", [(0, 128), (1, 32)])
def test_noalloc_decode_matches_workspace_entry(gpu, fmt, g):
    shapes = [(4, 32, 8, 8192, 128), (1, 16, 4, 1000, 64), (2, 8, 8, 20000, 256)]
    for i, (b, hq, hkv, n, d) in enumerate(shapes):
        print(f"[case] noalloc fmt={fmt} g={g} B={b} Hq={hq} Hkv={hkv} N={n} D={d}", flush=True)
        args = _inputs(gpu, b, hq, hkv, n, d, fmt, g if fmt else d, seed=10 * i + fmt)
        ref = _call(False, gpu, args, b, hq, hkv, n, d, fmt, g)
        got = _call(True, gpu, args, b, hq, hkv, n, d, fmt, g)
        assert np.isfinite(ref).all()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (
            f"shape {i}: max diff {np.abs(got - ref).max()}")
        # a second call in a row on the same scratch gives the same bits
        again = _call(True, gpu, args, b, hq, hkv, n, d, fmt, g)
        assert np.array_equal(again.view(np.uint32), ref.view(np.uint32))
