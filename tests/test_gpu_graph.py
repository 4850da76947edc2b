"""Stream-ordered behaviour of the split-K entry points: workspaces shared
across calls of different shapes and paths, repeated calls, and HIP-graph
capture with replays checked bit-for-bit against eager results (with eager
work and synchronisation between the replays)."""

import math

import numpy as np
import pytest
import torch

import oracle as o
from helpers import check_fp32, up16, up32, w4_problem

pytestmark = pytest.mark.gpu


def _w4(dev, m, n, k, g=64, seed=0):
    x, wq, s, b = w4_problem(m, n, k, g, seed=seed)
    ref = o.w4a16_matmul(x, wq, s, b, g)
    return (up16(x, o.BF16, dev), up32(wq, dev), up16(s, o.BF16, dev), up16(b, o.BF16, dev)), ref


def test_split_k_after_gemm_on_shared_workspace(gpu):
    import sparkq

    split_args, split_ref = _w4(gpu, 1, 64, 4096, seed=1)     # splits K across workgroups
    gemm_args, gemm_ref = _w4(gpu, 96, 200, 512, seed=2)      # M > 32: GEMM path
    f = lambda a: sparkq.affine_quantized_matmul(*a, group_size=64, out_dtype=torch.float32)
    for _ in range(3):
        check_fp32(f(split_args).cpu().numpy(), split_ref)
        check_fp32(f(gemm_args).cpu().numpy(), gemm_ref)


def test_repeated_split_k_calls_are_identical(gpu):
    import sparkq

    args, ref = _w4(gpu, 4, 2560, 9728, seed=3)
    outs = [sparkq.affine_quantized_matmul(*args, group_size=64, out_dtype=torch.float32)
            for _ in range(40)]
    for y in outs[1:]:
        assert torch.equal(y, outs[0])
    check_fp32(outs[0].cpu().numpy(), ref)


def test_graph_replay_matches_eager(gpu):
    import sparkq

    w4_args, _ = _w4(gpu, 1, 3584, 2560, seed=4)
    w4b_args, _ = _w4(gpu, 8, 2560, 9728, seed=5)
    n, k = 2560, 9728
    w8, sc8 = o.w8_quantize_channel(o.randn(0, 6, n * k, 0.02).reshape(n, k))
    w8t, sc8t = torch.from_numpy(w8).to(gpu), torch.from_numpy(sc8).to(gpu)
    x8 = torch.randn((8, k), device=gpu).to(torch.bfloat16)
    kc, ks = sparkq.kv_quantize_s8(torch.randn((1, 8, 4096, 128), device=gpu).to(torch.bfloat16))
    vc, vs = sparkq.kv_quantize_s8(torch.randn((1, 8, 4096, 128), device=gpu).to(torch.bfloat16))
    q = torch.randn((1, 32, 1, 128), device=gpu).to(torch.bfloat16)
    # prefill over the MLX affine cache with a context split (tile counters
    # reset by the kernel on every call)
    aff = []
    for _ in range(2):
        cache = (torch.zeros((1, 4, 900, 64), dtype=torch.int32, device=gpu),
                 torch.zeros((1, 4, 900, 8), dtype=torch.bfloat16, device=gpu),
                 torch.zeros((1, 4, 900, 8), dtype=torch.bfloat16, device=gpu))
        sparkq.kv_append(torch.randn((1, 4, 900, 256), device=gpu).to(torch.bfloat16), cache, 0)
        aff.append(cache)
    qp = torch.randn((1, 16, 300, 256), device=gpu).to(torch.bfloat16)
    assert sparkq._lib.lib().sparkq_int8kv_sdpa_prefill_affine_workspace_bytes(
        1, 16, 4, 300, 900, 256, 1) > 0

    outs = {
        "w4": torch.empty((1, 3584), dtype=torch.bfloat16, device=gpu),
        "w4b": torch.empty((8, 2560), dtype=torch.bfloat16, device=gpu),
        "w8": torch.empty((8, 2560), dtype=torch.bfloat16, device=gpu),
        "sdpa": torch.empty((1, 32, 1, 128), dtype=torch.bfloat16, device=gpu),
        "prefill_affine": torch.empty((1, 16, 300, 256), dtype=torch.bfloat16, device=gpu),
    }

    def step():
        sparkq.affine_quantized_matmul(*w4_args, group_size=64, out=outs["w4"])
        sparkq.affine_quantized_matmul(*w4b_args, group_size=64, out=outs["w4b"])
        sparkq.w8a8_linear(x8, w8t, sc8t, out=outs["w8"])
        sparkq.int8_quantized_sdpa(q, (kc, ks), (vc, vs), scale=1 / math.sqrt(128),
                                   out=outs["sdpa"])
        sparkq.int8_quantized_sdpa(qp, aff[0], aff[1], scale=0.0625, mask="causal",
                                   out=outs["prefill_affine"])

    step()
    torch.cuda.synchronize()
    eager = {key: v.clone() for key, v in outs.items()}
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for replay in range(4):
        for v in outs.values():
            v.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for key in outs:
            assert torch.equal(outs[key], eager[key]), (replay, key)
        # eager work between replays on the same workspaces
        step()
        torch.cuda.synchronize()
        for key in outs:
            assert torch.equal(outs[key], eager[key]), ("eager", replay, key)
