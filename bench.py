#!/usr/bin/env python3
"""Benchmark of the quantized-linear hot path on one MI355X.

Headline (value): W4A16 G64 decode GEMV weight GB/s at M=1 over a 36-layer
sweep of {QKV 3584x2560, gate+up 19456x2560, down 2560x9728} with distinct
weight buffers per layer (1.70 GB per sweep, so the weights are cold in the
256 MB MALL). One step = one sweep = 108 projections, captured once in a HIP
graph and replayed; inputs are resident in HBM before the timed region.

Also reported in the same JSON line: the M=4/8/16 sweeps, the prefill GEMM
per shape (M in 16/512/2048 over the same 36 layers of distinct weights;
GB/s at M=16, TFLOPS above) with its own roofline block (gate+up M=2048),
W8A8 GB/s (M in 1/8/16), INT8-KV decode attention GB/s (B in 1/8, N in
4096/32768), the roofline of the dominant kernel, and the CPU legs timed on
this host's cores (the headline GEMV sweep, the GEMM, W8A8 and INT8-KV
attention).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-extras]
       python bench.py --only-dominant | --only-gemm all|NAME:M   (profiler drivers)
       python bench.py --trace-summary RUN_results.db             (per-shape rows)
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "spark-mlx-llm_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
INT8_PEAK_TOPS = 5000.0
LAYERS = 36
G = 64
PROJ = {"qkv": (3584, 2560), "gate_up": (19456, 2560), "down": (2560, 9728)}
METRIC = "W4A16 GEMV weight GB/s (% HBM peak) at M=1; prefill GEMM TFLOPS (% MFMA)"


def w4_bytes(n, k, g=G):
    return n * k // 2 + 2 * 2 * n * (k // g)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Timer:
    """HIP events on the current stream (the stream the kernels run on)."""

    def __init__(self, torch):
        self.torch = torch

    def time(self, fn, iters, warmup=2):
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / iters  # ms


def capture(torch, fn):
    """Capture fn into a HIP graph (after one eager warm-up call)."""
    fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize()
    return graph


def make_w4_layers(torch, sparkq, dev, layers):
    out = []
    gen = torch.Generator(device=dev).manual_seed(0)
    for _ in range(layers):
        layer = {}
        for name, (n, k) in PROJ.items():
            w = (torch.randn((n, k), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
            layer[name] = sparkq.affine_quantize(w, group_size=G)
            del w
        out.append(layer)
    return out


def w4_sweep_fn(torch, sparkq, layers, xs, outs):
    def fn():
        for li, layer in enumerate(layers):
            for name, (wq, s, b) in layer.items():
                sparkq.affine_quantized_matmul(xs[PROJ[name][1]], wq, s, b, group_size=G,
                                               out=outs[li][name])
    return fn


def bench_w4_decode(torch, sparkq, dev, layers, steps, warmup, m):
    xs = {k: torch.randn((m, k), device=dev).to(torch.bfloat16) for k in (2560, 9728)}
    outs = [{n: torch.empty((m, PROJ[n][0]), dtype=torch.bfloat16, device=dev) for n in PROJ}
            for _ in layers]
    graph = capture(torch, w4_sweep_fn(torch, sparkq, layers, xs, outs))
    ms = Timer(torch).time(graph.replay, steps, warmup)
    # replay check against eager: the kernels are deterministic
    graph.replay()
    torch.cuda.synchronize()
    wq, s, b = layers[0]["gate_up"]
    eager = sparkq.affine_quantized_matmul(xs[2560], wq, s, b, group_size=G)
    torch.cuda.synchronize()
    ok = bool(torch.equal(eager, outs[0]["gate_up"]))
    return ms, ok


def bench_w4_projection(torch, sparkq, dev, layers, name, m, iters):
    n, k = PROJ[name]
    x = torch.randn((m, k), device=dev).to(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)

    def fn():
        for layer in layers:
            wq, s, b = layer[name]
            sparkq.affine_quantized_matmul(x, wq, s, b, group_size=G, out=y)

    graph = capture(torch, fn)
    ms = Timer(torch).time(graph.replay, iters, 2)
    return ms / len(layers)  # per projection


def bench_square_cold(torch, sparkq, dev, iters, copies=128):
    """The single-linear workload: W4A16 G64 at M=1, K=N=2560, over `copies`
    distinct weight sets (472 MB, cold in the 256 MB MALL) in one graph
    replay; returns ms per launch."""
    n = k = 2560
    gen = torch.Generator(device=dev).manual_seed(3)
    ws = []
    for _ in range(copies):
        w = (torch.randn((n, k), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
        ws.append(sparkq.affine_quantize(w, group_size=G))
        del w
    x = torch.randn((1, k), device=dev).to(torch.bfloat16)
    y = torch.empty((1, n), dtype=torch.bfloat16, device=dev)

    def fn():
        for wq, s, b in ws:
            sparkq.affine_quantized_matmul(x, wq, s, b, group_size=G, out=y)

    graph = capture(torch, fn)
    ms = Timer(torch).time(graph.replay, iters, 2) / copies
    del graph, ws
    return ms


def prepare_layers(sparkq, layers):
    """Each layer's derived prefill buffers (sparkq.prepare_w4a16), made once
    per weight set at load time, outside any timed region."""
    return [{name: sparkq.prepare_w4a16(*layer[name], group_size=G) for name in layer}
            for layer in layers]


def bench_gemm(torch, sparkq, dev, layers, name, m, iters, prepared=None):
    """One W4A16 projection at M rows over every layer's distinct weights in
    one graph replay (36 launches, weights cold in the MALL); returns ms per
    launch. With prepared (prepare_layers), each call passes its layer's
    derived buffer, so the GEMM prologue converts the activations only."""
    n, k = PROJ[name]
    x = torch.randn((m, k), device=dev).to(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)

    def fn():
        for li, layer in enumerate(layers):
            wq, s, b = layer[name]
            sparkq.affine_quantized_matmul(x, wq, s, b, group_size=G, out=y,
                                           prepared=None if prepared is None else prepared[li][name])

    graph = capture(torch, fn)
    ms = Timer(torch).time(graph.replay, iters, 2) / len(layers)
    del graph
    return ms


def gemm_line(name, m, ms):
    n, k = PROJ[name]
    tf = 2 * m * n * k / (ms / 1e3) / 1e12
    line = {"ms": round(ms, 5), "TFLOP/s": round(tf, 1), "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)}
    if m <= 32:  # weight-streaming regime: the bound is HBM
        gbs = w4_bytes(n, k) / (ms / 1e3) / 1e9
        line.update({"GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)})
    return line


def bench_w8a8(torch, sparkq, dev, m, iters, copies=36):
    res = {}
    gen = torch.Generator(device=dev).manual_seed(1)
    for name, (n, k) in PROJ.items():
        ws = []
        for _ in range(copies):
            w = torch.randn((n, k), generator=gen, device=dev) * 0.02
            sc = (w.abs().amax(1) / 127).clamp_min(1e-12)
            q = torch.round(w / sc[:, None]).clamp(-127, 127).to(torch.int8)
            ws.append((q, sc.float()))
            del w
        x = torch.randn((m, k), device=dev).to(torch.bfloat16)
        y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)

        def fn():
            for q, sc in ws:
                sparkq.w8a8_linear(x, q, sc, out=y)

        graph = capture(torch, fn)
        ms = Timer(torch).time(graph.replay, iters, 2) / copies
        nbytes = n * k + 4 * n
        res[name] = {"ms": round(ms, 5), "GB/s": round(nbytes / ms / 1e6, 1)}
        del ws, graph
    return res


def bench_w8a8_prefill(torch, sparkq, dev, iters, copies=8):
    """W8A8 at prefill sizes on the out_proj shape N=2560, K=4096 (the
    reference serves out_proj at any M): the whole w8a8_linear call (per-token
    quantizer, int8 GEMM, fp32 epilogue, bf16 out) over 8 distinct weight
    sets per graph replay; int8 ops 2*M*N*K against the 5 POP/s dense peak."""
    res = {}
    n, k = 2560, 4096
    gen = torch.Generator(device=dev).manual_seed(3)
    ws = [(torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=gen),
           torch.rand(n, device=dev, generator=gen) * 1e-3) for _ in range(copies)]
    for m in (512, 2048):
        x = torch.randn((m, k), device=dev).to(torch.bfloat16)
        y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)

        def fn():
            for q, sc in ws:
                sparkq.w8a8_linear(x, q, sc, out=y)

        graph = capture(torch, fn)
        ms = Timer(torch).time(graph.replay, iters, 2) / copies
        tops = 2 * m * n * k / (ms / 1e3) / 1e12
        res[f"M={m} N={n} K={k}"] = {"ms": round(ms, 5), "TOP/s": round(tops, 1),
                                     "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        del graph
    del ws
    return res


def bench_w8a16(torch, sparkq, dev, iters):
    """W8A16 per-channel GEMV at M=1: the projections (36 distinct weight
    sets) and the W8 lm_head 131072 x 2560 (335 MB, 3 distinct copies)."""
    res = {}
    gen = torch.Generator(device=dev).manual_seed(2)
    shapes = dict(PROJ)
    shapes["lm_head"] = (131072, 2560)
    for name, (n, k) in shapes.items():
        copies = 3 if name == "lm_head" else 36
        ws = [(torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=gen),
               torch.rand(n, device=dev, generator=gen) * 1e-3) for _ in range(copies)]
        x = torch.randn((1, k), device=dev).to(torch.bfloat16)
        y = torch.empty((1, n), dtype=torch.bfloat16, device=dev)

        def fn():
            for q, sc in ws:
                sparkq.w8a16_per_channel(x, q, sc, out=y)

        graph = capture(torch, fn)
        ms = Timer(torch).time(graph.replay, iters, 2) / copies
        nbytes = n * k + 4 * n
        res[name] = {"ms": round(ms, 5), "GB/s": round(nbytes / ms / 1e6, 1),
                     "frac_hbm": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4)}
        del ws, graph
    return res


def bench_sdpa(torch, sparkq, dev, b, n, iters):
    hq, hkv, d = 32, 8, 128
    kv_bytes = 2 * b * hkv * n * d + 2 * b * hkv * n * 2
    copies = max(1, min(32, (600 << 20) // kv_bytes))
    caches = []
    for c in range(copies):
        kc, ks = sparkq.kv_quantize_s8(torch.randn((b, hkv, n, d), device=dev, dtype=torch.bfloat16))
        vc, vs = sparkq.kv_quantize_s8(torch.randn((b, hkv, n, d), device=dev, dtype=torch.bfloat16))
        caches.append(((kc, ks), (vc, vs)))
    q = torch.randn((b, hq, 1, d), device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(d)

    def fn():
        for keys, vals in caches:
            sparkq.int8_quantized_sdpa(q, keys, vals, scale=scale, out=out)

    graph = capture(torch, fn)
    ms = Timer(torch).time(graph.replay, iters, 2) / copies
    return {"ms": round(ms, 5), "GB/s": round(kv_bytes / ms / 1e6, 1),
            "frac_hbm": round(kv_bytes / ms / 1e6 / HBM_PEAK_GBS, 4), "kv_bytes": kv_bytes}


def bench_low_bit_decode(torch, sparkq, dev, n, iters, bits=4, g=64, staged=False, b=1):
    """Decode attention over an MLX affine cache: by default 4-bit (mlx-lm's
    kv_bits=4, group 64; the reference attends it through its staged
    _fallback), with bits=8, g=32 the reference's fused-kernel format. 32/8
    heads, D=128, one query token, on the one-pass decode kernel over the
    codes, or (staged=True) on the staged-attention kernel, forced with an
    all-visible boolean mask. GB/s of the cache bytes read (codes plus bf16
    scales and biases)."""
    hq, hkv, d = 32, 8, 128
    words = d * bits // 32
    kv_bytes = 2 * b * hkv * n * (words * 4 + 2 * 2 * (d // g))
    copies = max(1, min(32, (600 << 20) // kv_bytes))
    gen = torch.Generator(device=dev).manual_seed(4)

    def part():
        packed = torch.randint(-2 ** 31, 2 ** 31 - 1, (b, hkv, n, words), dtype=torch.int32,
                               device=dev, generator=gen)
        sc = (torch.rand((b, hkv, n, d // g), device=dev, generator=gen) * 0.1 + 0.01)
        bi = -sc * 7.5
        return packed, sc.to(torch.bfloat16), bi.to(torch.bfloat16)

    caches = [(part(), part()) for _ in range(copies)]
    q = torch.randn((b, hq, 1, d), device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(d)

    mask = torch.ones((1, n), dtype=torch.bool, device=dev) if staged else None

    def fn():
        for keys, vals in caches:
            sparkq.int8_quantized_sdpa(q, keys, vals, scale=scale, group_size=g, bits=bits,
                                       mask=mask, out=out)

    graph = capture(torch, fn)
    ms = Timer(torch).time(graph.replay, iters, 2) / copies
    del graph, caches
    return {"ms": round(ms, 5), "GB/s": round(kv_bytes / ms / 1e6, 1),
            "frac_hbm": round(kv_bytes / ms / 1e6 / HBM_PEAK_GBS, 4), "kv_bytes": kv_bytes}


def bench_prefill(torch, sparkq, dev, length, n, iters, fmt="s8", hq=32, hkv=8, d=128, g=32):
    """INT8-KV prefill attention, B=1, bottom-right causal, over the s8 cache
    or the MLX affine u8 cache (group size g, quantized on append). Useful
    flop: 4*Hq*D per visible (query, token) pair."""
    b = 1
    kv = [torch.randn((b, hkv, n, d), device=dev, dtype=torch.bfloat16) for _ in range(2)]
    if fmt == "s8":
        keys, vals = (sparkq.kv_quantize_s8(t) for t in kv)
        group = {}
    else:
        def affine(t):
            cache = (torch.zeros((b, hkv, n, d // 4), device=dev, dtype=torch.int32),
                     torch.zeros((b, hkv, n, d // g), device=dev, dtype=torch.bfloat16),
                     torch.zeros((b, hkv, n, d // g), device=dev, dtype=torch.bfloat16))
            sparkq.kv_append(t, cache, 0, group_size=g)
            return cache
        keys, vals = affine(kv[0]), affine(kv[1])
        group = {"group_size": g}
    q = torch.randn((b, hq, length, d), device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(d)

    def fn():
        sparkq.int8_quantized_sdpa(q, keys, vals, scale=scale, mask="causal", out=out, **group)

    graph = capture(torch, fn)
    ms = Timer(torch).time(graph.replay, iters, 2)
    pairs = sum(n - length + i + 1 for i in range(length))
    flop = 4.0 * b * hq * d * pairs
    return {"ms": round(ms, 4), "TFLOP/s": round(flop / ms / 1e9, 1),
            "frac_f16_peak": round(flop / ms / 1e9 / BF16_PEAK_TFLOPS, 4)}


def bench_kv_append(torch, sparkq, dev, iters):
    """Quantize-on-append of one decode token and of a 2048-token prefill
    chunk into 8 KV heads of D=128 (both formats): bytes read + written."""
    res = {}
    for fmt, g in (("s8", 32), ("affine_u8", 32)):
        for length in (1, 2048):
            cache = sparkq.QuantizedKVCache(group_size=g, kv_format=fmt)
            x = torch.randn((1, 8, length, 128), device=dev).to(torch.bfloat16)
            cache.update_and_fetch(x, x)
            store = cache.keys

            def fn():
                for _ in range(32):
                    sparkq.kv_append(x, store, 0, group_size=g)

            graph = capture(torch, fn)
            ms = Timer(torch).time(graph.replay, iters, 2) / 32
            nbytes = x.numel() * 2 + x.numel() + (8 * length * (2 if fmt == "s8" else 2 * 2 * 128 // g))
            res[f"{fmt} L={length}"] = {"ms": round(ms, 5), "GB/s": round(nbytes / ms / 1e6, 1)}
    return res


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "w4_gemv_gate_up_m1_pmc.md")


def bench_layer(torch, sparkq, dev, layers, iters):
    """The fused decoder-layer steps at one token over the 36 layers: the FFN
    block (residual + RMSNorm + gate/up + gelu*up in one launch, down +
    residual in another; gate and up are the two halves of the fused
    gate_up weights) and the QKV projection with RoPE (3584 = 2560 + 2 * 512
    rows: 20 query and 4 key/value heads of 128, full rotation, position
    4095)."""
    inter = PROJ["gate_up"][0] // 2
    hidden = PROJ["down"][0]
    x = torch.randn((1, hidden), device=dev).to(torch.bfloat16)
    a = torch.randn((1, hidden), device=dev).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(hidden, device=dev)).to(torch.bfloat16)

    def halves(t):
        return t[:inter], t[inter:]

    ffn_args = []
    for layer in layers:
        (gw, uw), (gs, us), (gb, ub) = (halves(t) for t in layer["gate_up"])
        ffn_args.append(((gw, gs, gb), (uw, us, ub), layer["down"]))

    def ffn():
        for gate, up, down in ffn_args:
            sparkq.fused_ffn(x, a, nw, 1e-6, gate, up, down, group_size=G)

    xq = x.view(1, 1, hidden)

    def qkv():
        for layer in layers:
            wq, s, b = layer["qkv"]
            sparkq.spark_qkv_rope(xq, wq, s, b, 2560, 512, 20, 4, 128, 128, 500000.0, 4095, G, 4)

    res = {}
    for name, fn, nbytes in (
            ("ffn_block", ffn, w4_bytes(*PROJ["gate_up"]) + w4_bytes(*PROJ["down"])),
            ("qkv_rope", qkv, w4_bytes(*PROJ["qkv"]))):
        graph = capture(torch, fn)
        ms = Timer(torch).time(graph.replay, iters, 2) / len(layers)
        res[name] = {"ms": round(ms, 5), "GB/s": round(nbytes / ms / 1e6, 1),
                     "frac_hbm": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4)}
        del graph
    return res


def measured_traffic():
    """HBM bytes per launch of the dominant kernel, from the committed PMC
    summary (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the same counters
    on a copy kernel of known size), or None when there is none."""
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1].strip()))
    except (OSError, ValueError):
        pass
    return None


def only_dominant(torch, sparkq, dev, iters):
    """Driver for rocprofv3 --pmc runs: the dominant kernel alone (gate+up
    GEMV at M=1 over 36 distinct weight sets), then a 256 MiB device copy whose
    byte count calibrates the counters."""
    n, k = PROJ["gate_up"]
    layers = []
    gen = torch.Generator(device=dev).manual_seed(0)
    for _ in range(LAYERS):
        w = (torch.randn((n, k), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
        layers.append(sparkq.affine_quantize(w, group_size=G))
        del w
    x = torch.randn((1, k), device=dev).to(torch.bfloat16)
    y = torch.empty((1, n), dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    for _ in range(iters):
        for wq, s, b in layers:
            sparkq.affine_quantized_matmul(x, wq, s, b, group_size=G, out=y)
    torch.cuda.synchronize()
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"dominant kernel x {iters * LAYERS} launches, then 5 copies of {256 << 20} bytes")


GEMM_PMC_FILE = os.path.join(ROOT, "profiles", "w4_gemm_gate_up_m2048_pmc.md")


GEMM_TRACE_FILE = os.path.join(ROOT, "profiles", "w4a16_gemm_per_shape_trace.md")


def gemm_trace():
    """Kernel-only and prologue average durations (us) of the dominant GEMM
    shape (gate+up, M=2048, prepared weights) from the committed per-shape
    kernel trace, or {} when there is none."""
    out = {}
    try:
        for line in open(GEMM_TRACE_FILE):
            key, _, val = line.partition(":")
            if key in ("gate_up_m2048_kernel_us", "gate_up_m2048_prologue_us"):
                out[key] = float(val.strip())
    except (OSError, ValueError):
        pass
    return out


def only_sdpa(torch, sparkq, dev, which, iters):
    """Driver for rocprofv3 runs over the INT8-KV decode (32/8 heads, D=128):
    each "B:N" of which over the symmetric s8 cache, or "FMT:B:N" with FMT
    s8, u8 (the MLX affine u8 G32 tuple, the reference's fused format) or u4
    (4-bit G64), iters graph-free launches over rotated caches."""
    hq, hkv, d = 32, 8, 128
    for spec in which.split(","):
        parts = spec.split(":")
        fmt = parts[0] if len(parts) == 3 else "s8"
        b, n = (int(v) for v in parts[-2:])
        bits, g = {"s8": (8, 0), "u8": (8, 32), "u4": (4, 64)}[fmt]
        if fmt == "s8":
            kv_bytes = 2 * b * hkv * n * d + 2 * b * hkv * n * 2
        else:
            kv_bytes = 2 * b * hkv * n * (d * bits // 8 + 2 * 2 * (d // g))
        copies = max(1, min(32, (600 << 20) // kv_bytes))
        gen = torch.Generator(device=dev).manual_seed(4)

        def part():
            words = d * bits // 32
            packed = torch.randint(-2 ** 31, 2 ** 31 - 1, (b, hkv, n, words), dtype=torch.int32,
                                   device=dev, generator=gen)
            sc = torch.rand((b, hkv, n, d // g), device=dev, generator=gen) * 0.01 + 0.001
            return packed, sc.to(torch.bfloat16), (-sc * (1 << (bits - 1))).to(torch.bfloat16)

        caches = []
        for _ in range(copies):
            if fmt == "s8":
                kc, ks = sparkq.kv_quantize_s8(torch.randn((b, hkv, n, d), device=dev, dtype=torch.bfloat16))
                vc, vs = sparkq.kv_quantize_s8(torch.randn((b, hkv, n, d), device=dev, dtype=torch.bfloat16))
                caches.append(((kc, ks), (vc, vs)))
            else:
                caches.append((part(), part()))
        q = torch.randn((b, hq, 1, d), device=dev).to(torch.bfloat16)
        out = torch.empty_like(q)
        kw = {} if fmt == "s8" else {"group_size": g, "bits": bits}
        torch.cuda.synchronize()
        for _ in range(iters):
            for keys, vals in caches:
                sparkq.int8_quantized_sdpa(q, keys, vals, scale=1.0 / math.sqrt(d), out=out, **kw)
        torch.cuda.synchronize()
        log(f"INT8-KV decode {fmt} B={b} N={n}: {iters * copies} launches ({kv_bytes} KV bytes each)")
        del caches


def gemm_counters():
    """MFMA and VALU busy fractions of the dominant GEMM shape (gate+up,
    M=2048) from the committed PMC summary, or {} when there is none."""
    out = {}
    try:
        for line in open(GEMM_PMC_FILE):
            key, _, val = line.partition(":")
            if key in ("mfma_busy_frac", "valu_busy_frac", "mfma_flop_frac"):
                out[key] = float(val.strip())
    except (OSError, ValueError):
        pass
    return out


def only_gemm(torch, sparkq, dev, which, iters):
    """Driver for rocprofv3 runs over the prefill GEMM: every (projection, M)
    of the GEMM sweep (which == "all"), or one of them ("gate_up:2048"), each
    over 36 layers of distinct weights with their derived prefill buffers
    (as the bench times them), iters graph-free passes."""
    shapes = [(name, m) for name in PROJ for m in (16, 512, 2048)]
    if which != "all":
        name, m = which.split(":")
        shapes = [(name, int(m))]
    gen = torch.Generator(device=dev).manual_seed(0)
    for name, m in shapes:
        n, k = PROJ[name]
        ws = []
        for _ in range(LAYERS):
            w = (torch.randn((n, k), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
            wq, s, b = sparkq.affine_quantize(w, group_size=G)
            ws.append((wq, s, b, sparkq.prepare_w4a16(wq, s, b, group_size=G)))
            del w
        x = torch.randn((m, k), device=dev).to(torch.bfloat16)
        y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        torch.cuda.synchronize()
        for _ in range(iters):
            for wq, s, b, prep in ws:
                sparkq.affine_quantized_matmul(x, wq, s, b, group_size=G, out=y, prepared=prep)
        torch.cuda.synchronize()
        log(f"{name} M={m}: {iters * LAYERS} launches")
        del ws


def trace_summary(path):
    """Per-shape rows of a rocprofv3 kernel trace, from its rocpd database
    (*_results.db, the default output) or a *_kernel_trace.csv: launches,
    average and total duration per (kernel, grid size) in first-launch order;
    the GEMM shapes have distinct grids."""
    rows = {}

    def add(name, grid, dur_ns):
        e = rows.setdefault((name, grid), [0, 0.0])
        e[0] += 1
        e[1] += dur_ns / 1e3

    if path.endswith(".db"):
        import sqlite3

        con = sqlite3.connect(path)
        for name, gx, gy, gz, start, end in con.execute(
                "select name, grid_x, grid_y, grid_z, start, end from kernels order by start"):
            add(name, f"{gx}x{gy}x{gz}", end - start)
    else:
        import csv

        with open(path) as f:
            for r in csv.DictReader(f):
                grid = "x".join(r.get(f"Grid_Size_{a}", "?") for a in "XYZ")
                add(r["Kernel_Name"], grid, int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    print("| kernel | grid (work-items) | launches | avg us | total us |")
    print("|---|---|---|---|---|")
    for (name, grid), (cnt, tot) in rows.items():
        short = name if len(name) < 90 else name[:87] + "..."
        print(f"| `{short}` | {grid} | {cnt} | {tot / cnt:.2f} | {tot:.1f} |")


def cpu_threads():
    """Host threads for the CPU legs: OMP_NUM_THREADS when set (the GPU host
    allots a fixed share of its cores per GPU that way), else every core in
    this process's affinity mask."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else len(os.sched_getaffinity(0))


def host_cpu():
    import subprocess

    import oracle as o

    model = "unknown"
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        model = next(l.split(":", 1)[1].strip() for l in out.splitlines() if l.startswith("Model name"))
    except (OSError, StopIteration, subprocess.SubprocessError):
        try:
            model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo")
                         if l.startswith("model name"))
        except (OSError, StopIteration):
            pass
    return {"model": model, "logical_cpus": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "isa": o.cpu_isa()}


def _run_for(fn, budget_s, min_runs=1):
    """Calls fn until budget_s has passed (at least min_runs times, after one
    untimed call); returns (runs, seconds)."""
    fn()
    runs, t0 = 0, time.perf_counter()
    while True:
        fn()
        runs += 1
        el = time.perf_counter() - t0
        if el >= budget_s and runs >= min_runs:
            return runs, el


def cpu_baseline(layers_host, threads, cpu, budget_s=10.0):
    """Headline CPU leg: the oracle's OpenMP fp32 dequantize-then-dot GEMV on
    this host at M=1 over the same 36 layers of distinct weights as the GPU
    sweep (1.70 GB, cold in the host caches), for about budget_s."""
    import oracle as o

    x = {k: o.randn16(0, k, k).reshape(1, k) for k in (2560, 9728)}
    per_layer = sum(w4_bytes(*PROJ[n]) for n in PROJ)
    done = [0]

    def sweep_part():
        layer = layers_host[done[0] % len(layers_host)]
        for name, (wq, s, b) in layer.items():
            o.cpu_w4a16_gemv(x[PROJ[name][1]], wq, s, b, G, threads)
        done[0] += 1

    runs, el = _run_for(sweep_part, budget_s)
    gbs = per_layer * runs / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": (f"{runs} layers (QKV+gate_up+down, {per_layer} weight bytes each) of the 36-layer "
                       f"W4A16 G64 GEMV sweep at M=1, cycled in order, in {el:.1f} s on {threads} threads "
                       f"({cpu['isa']}) of {cpu['model']} ({cpu['logical_cpus']} logical CPUs); "
                       "MLX CPU backend unavailable (mlx not installed)")}


def cpu_legs(layers_host, threads, budget_s=2.0):
    """The CPU legs of the other workloads, each run for about budget_s:
    the single W4A16 2560x2560 linear at M=1, W4A16 GEMM (gate+up at
    M=16/512/2048), W8A8 (gate+up at M=1/8/16 over 4
    distinct int8 weight sets) and INT8-KV decode attention (32/8 heads,
    D=128; B=8 N=32768 is left out: 545 MB of cache per call)."""
    import numpy as np

    import oracle as o

    res = {}
    # the single 2560 x 2560 linear at M=1: the first 2560 rows of each
    # layer's QKV weights (36 distinct sets)
    xq = o.randn16(0, 2560, 2560).reshape(1, 2560)
    iq = [0]

    def square():
        wq, s, b = layers_host[iq[0] % len(layers_host)]["qkv"]
        o.cpu_w4a16_gemv(xq, wq[:2560], s[:2560], b[:2560], G, threads)
        iq[0] += 1

    runs, el = _run_for(square, budget_s)
    ms = el / runs * 1e3
    res["w4a16 2560x2560 M=1"] = {"ms": round(ms, 4), "GB/s": round(w4_bytes(2560, 2560) / ms / 1e6, 2),
                                  "runs": runs}
    n, k = PROJ["gate_up"]
    for m in (16, 512, 2048):
        x = o.randn16(0, 100 + m, m * k).reshape(m, k)
        i = [0]

        def gemm():
            wq, s, b = layers_host[i[0] % len(layers_host)]["gate_up"]
            o.cpu_w4a16_gemv(x, wq, s, b, G, threads)
            i[0] += 1

        runs, el = _run_for(gemm, budget_s if m < 2048 else 0.0)
        ms = el / runs * 1e3
        line = {"ms": round(ms, 3), "TFLOP/s": round(2 * m * n * k / ms / 1e9, 4), "runs": runs}
        if m <= 32:
            line["GB/s"] = round(w4_bytes(n, k) / ms / 1e6, 2)
        res[f"w4a16 gate_up M={m}"] = line
    rng = np.random.default_rng(0)
    ws = [(rng.integers(-127, 128, (n, k), dtype=np.int8), (rng.random(n) * 1e-3).astype(np.float32))
          for _ in range(4)]
    for m in (1, 8, 16):
        x = o.randn16(0, 200 + m, m * k).reshape(m, k)
        i = [0]

        def w8a8():
            wq, sw = ws[i[0] % len(ws)]
            o.cpu_w8a8_linear(x, wq, sw, threads)
            i[0] += 1

        runs, el = _run_for(w8a8, budget_s)
        ms = el / runs * 1e3
        res[f"w8a8 gate_up M={m}"] = {"ms": round(ms, 3), "GB/s": round((n * k + 4 * n) / ms / 1e6, 2),
                                      "runs": runs}
    del ws
    hq, hkv, d = 32, 8, 128
    for b, nn in ((1, 4096), (1, 32768), (8, 4096)):
        kc = rng.integers(-127, 128, (b, hkv, nn, d), dtype=np.int8)
        vc = rng.integers(-127, 128, (b, hkv, nn, d), dtype=np.int8)
        sc = np.full((b, hkv, nn), 0x2000, np.uint16)  # fp16 2^-7
        q = o.randn16(0, 300 + b, b * hq * d).reshape(b, hq, d)
        runs, el = _run_for(lambda: o.cpu_int8kv_sdpa(q, kc, sc, vc, sc, 1 / math.sqrt(d), threads),
                            budget_s)
        ms = el / runs * 1e3
        kv_bytes = 2 * b * hkv * nn * d + 2 * b * hkv * nn * 2
        res[f"int8kv_sdpa B={b} N={nn}"] = {"ms": round(ms, 3), "GB/s": round(kv_bytes / ms / 1e6, 2),
                                            "runs": runs}
    res["threads"] = threads
    return res


def launch_floor(torch, sparkq, dev, iters):
    """Launch-to-launch floor of graph replay: back-to-back W4A16 G64 launches
    at M=1 and K=512 (one 1 KB span per row quad, next to no work) for N = 4,
    1024 and 8192 (1, 256 and 512 workgroups), 256 launches captured in one
    graph; prints a markdown row per case with the time per launch (HIP
    events over the replays). Under rocprofv3 --kernel-trace the kernel's own
    duration is the rest: the launch-to-launch gap is the difference."""
    k, launches = 512, 256
    print("| N x K | launches per replay | us per launch (graph replay) |")
    print("|---|---|---|")
    for n in (4, 1024, 8192):
        w = (torch.randn((n, k), device=dev) * 0.02).to(torch.bfloat16)
        wq, s, b = sparkq.affine_quantize(w, group_size=G)
        x = torch.randn((1, k), device=dev).to(torch.bfloat16)
        y = torch.empty((1, n), dtype=torch.bfloat16, device=dev)

        def fn():
            for _ in range(launches):
                sparkq.affine_quantized_matmul(x, wq, s, b, group_size=G, out=y)

        graph = capture(torch, fn)
        ms = Timer(torch).time(graph.replay, iters, 2)
        print(f"| {n} x {k} | {launches} | {ms * 1e3 / launches:.3f} |", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--skip-extras", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--only-dominant", action="store_true",
                    help="run only the dominant kernel and a calibration copy (for rocprofv3 --pmc)")
    ap.add_argument("--only-gemm", default=None, metavar="all|NAME:M",
                    help="run only prefill GEMM launches (for rocprofv3 --kernel-trace / --pmc)")
    ap.add_argument("--only-sdpa", default=None, metavar="[FMT:]B:N[,...]",
                    help="run only INT8-KV decode launches (for rocprofv3 --kernel-trace / --pmc); "
                         "FMT s8 (default), u8 (affine G32) or u4 (affine G64)")
    ap.add_argument("--launch-floor", action="store_true",
                    help="time back-to-back near-empty GEMV launches in graph replay and exit")
    ap.add_argument("--trace-summary", default=None, metavar="CSV",
                    help="print per-(kernel, grid) rows of a rocprofv3 kernel trace and exit")
    args = ap.parse_args()
    if args.trace_summary is not None:
        trace_summary(args.trace_summary)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU; multi-GPU runs are not part of "
                                   "it (--gpus must be 1)"}))
        sys.exit(2)

    import numpy as np
    import torch

    import sparkq

    dev = torch.device("cuda:0")
    if not sparkq.is_w8a8_available():
        raise RuntimeError("libsparkq unusable on cuda:0 (needs gfx950)")
    if args.only_dominant:
        only_dominant(torch, sparkq, dev, max(args.steps, 1))
        return
    if args.only_gemm:
        only_gemm(torch, sparkq, dev, args.only_gemm, max(args.steps, 1))
        return
    if args.only_sdpa:
        only_sdpa(torch, sparkq, dev, args.only_sdpa, max(args.steps, 1))
        return
    if args.launch_floor:
        launch_floor(torch, sparkq, dev, max(args.steps, 1))
        return
    log("generating 36 layers of W4A16 G64 weights")
    layers = make_w4_layers(torch, sparkq, dev, LAYERS)
    sweep_bytes = LAYERS * sum(w4_bytes(*PROJ[n]) for n in PROJ)

    log(f"timing M=1 sweep: {args.warmup} warmup + {args.steps} steps")
    ms, graph_ok = bench_w4_decode(torch, sparkq, dev, layers, args.steps, args.warmup, 1)
    value = sweep_bytes / (ms / 1e3) / 1e9

    # dominant kernel: the gate+up projection (59% of the sweep's bytes)
    gu_ms = bench_w4_projection(torch, sparkq, dev, layers, "gate_up", 1, max(args.steps, 10))
    gu_bytes = w4_bytes(*PROJ["gate_up"])
    achieved = gu_bytes / (gu_ms / 1e3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic(),
                "kernel": "w4_gemv_q_kernel<BF16,64,5,1,2> (gate+up 19456x2560, M=1)",
                "bytes_per_launch": gu_bytes, "avg_launch_ms": round(gu_ms, 5)}

    extras = {}
    if not args.skip_extras:
        log("per-projection and M=4/8/16 sweeps")
        per = {}
        for name in PROJ:
            pm = bench_w4_projection(torch, sparkq, dev, layers, name, 1, 10)
            per[name] = {"ms": round(pm, 5), "GB/s": round(w4_bytes(*PROJ[name]) / pm / 1e6, 1)}
        extras["w4a16_decode_m1_per_projection"] = per
        sq = bench_square_cold(torch, sparkq, dev, 10)
        sq_gbs = w4_bytes(2560, 2560) / sq / 1e6
        extras["w4a16_m1_2560x2560_cold"] = {"ms": round(sq, 5), "GB/s": round(sq_gbs, 1),
                                              "frac_hbm": round(sq_gbs / HBM_PEAK_GBS, 4),
                                              "weight_bytes": w4_bytes(2560, 2560), "copies": 128}
        sweeps = {}
        for m in (4, 8, 16):
            sm, _ = bench_w4_decode(torch, sparkq, dev, layers, 10, 2, m)
            gbs = sweep_bytes / (sm / 1e3) / 1e9
            sweeps[f"M={m}"] = {"ms_per_sweep": round(sm, 4), "GB/s": round(gbs, 1),
                                "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        extras["w4a16_decode_sweep"] = sweeps
        log("prefill GEMM")
        prepared = prepare_layers(sparkq, layers)
        gemm, unprepared = {}, {}
        for name in PROJ:
            for m in (16, 512, 2048):
                gm = bench_gemm(torch, sparkq, dev, layers, name, m, 3 if m == 2048 else 5,
                                prepared)
                gemm[f"{name} M={m}"] = gemm_line(name, m, gm)
                if m > 32:  # the same calls computing the weight half of the prologue each time
                    um = bench_gemm(torch, sparkq, dev, layers, name, m, 3 if m == 2048 else 5)
                    unprepared[f"{name} M={m}"] = gemm_line(name, m, um)
        extras["w4a16_prefill_gemm"] = gemm
        extras["w4a16_prefill_gemm_unprepared"] = unprepared
        del prepared
        log("W8A8")
        extras["w8a8"] = {f"M={m}": bench_w8a8(torch, sparkq, dev, m, 5) for m in (1, 8, 16)}
        extras["w8a8_prefill"] = bench_w8a8_prefill(torch, sparkq, dev, 5)
        log("W8A16")
        extras["w8a16_m1"] = bench_w8a16(torch, sparkq, dev, 5)
        log("INT8-KV decode attention")
        extras["int8kv_sdpa_decode"] = {f"B={b} N={n}": bench_sdpa(torch, sparkq, dev, b, n, 5)
                                        for b in (1, 8) for n in (4096, 32768)}
        extras["sdpa_decode_4bit"] = {f"B=1 N={n}": bench_low_bit_decode(torch, sparkq, dev, n, 5)
                                      for n in (4096, 32768)}
        extras["sdpa_decode_affine_u8"] = {
            f"B={b} N={n}": bench_low_bit_decode(torch, sparkq, dev, n, 5, bits=8, g=32, b=b)
            for b in (1, 8) for n in (4096, 32768)}
        extras["staged_sdpa_decode_4bit"] = {
            f"B=1 N={n}": bench_low_bit_decode(torch, sparkq, dev, n, 3, staged=True)
            for n in (4096, 32768)}
        log("INT8-KV prefill attention and KV append")
        extras["int8kv_sdpa_prefill_causal"] = {
            f"L={l} N={n}": bench_prefill(torch, sparkq, dev, l, n, 5)
            for l, n in ((2048, 2048), (512, 4096))}
        extras["int8kv_sdpa_prefill_affine_causal"] = {
            f"L={l} N={n} Hq/Hkv={hq}/{hkv} D={d}": bench_prefill(
                torch, sparkq, dev, l, n, 5, fmt="affine_u8", hq=hq, hkv=hkv, d=d)
            for l, n in ((2048, 2048), (512, 4096)) for hq, hkv, d in ((32, 8, 128), (16, 4, 256))}
        extras["kv_append"] = bench_kv_append(torch, sparkq, dev, 10)
        log("fused FFN block and QKV+RoPE")
        extras["layer_m1"] = bench_layer(torch, sparkq, dev, layers, 10)

    cpu = None
    if not args.skip_cpu:
        log("CPU baseline")
        host = []
        for layer in layers:
            host.append({name: (wq.cpu().view(torch.int32).numpy().view(np.uint32),
                                s.cpu().view(torch.int16).numpy().view(np.uint16),
                                b.cpu().view(torch.int16).numpy().view(np.uint16))
                         for name, (wq, s, b) in layer.items()})
        threads, cpu_info = cpu_threads(), host_cpu()
        cpu = cpu_baseline(host, threads, cpu_info)
        cpu["host"] = cpu_info
        if not args.skip_extras:
            log("CPU legs of the other workloads")
            extras["cpu_legs"] = cpu_legs(host, threads)
        del host

    prefill = extras.get("w4a16_prefill_gemm", {}).get("gate_up M=2048")
    roofline_gemm = None
    if prefill:
        n, k = PROJ["gate_up"]
        flop = 2 * 2048 * n * k
        roofline_gemm = {"bound": "mfma", "achieved": prefill["TFLOP/s"], "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": prefill["frac_bf16_peak"],
                         "kernel": "gemm_prep_kernel (activation rows) + w4_gemm_x16w_kernel "
                                   "(gate+up 19456x2560, M=2048, weights prepared once per set)",
                         "flop_per_launch": flop, "avg_launch_ms": prefill["ms"],
                         "prologue_included": True}
        unprep = extras.get("w4a16_prefill_gemm_unprepared", {}).get("gate_up M=2048")
        if unprep:
            roofline_gemm["unprepared_TFLOP/s"] = unprep["TFLOP/s"]
        tr = gemm_trace()
        if "gate_up_m2048_kernel_us" in tr:
            ku = tr["gate_up_m2048_kernel_us"]
            roofline_gemm["kernel_only_avg_us_rocprof"] = ku
            roofline_gemm["kernel_only_TFLOP/s_rocprof"] = round(flop / ku / 1e6, 1)
            roofline_gemm["kernel_only_frac_rocprof"] = round(flop / ku / 1e6 / BF16_PEAK_TFLOPS, 4)
        if "gate_up_m2048_prologue_us" in tr:
            roofline_gemm["prologue_avg_us_rocprof"] = tr["gate_up_m2048_prologue_us"]
        roofline_gemm.update(gemm_counters())
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,0.02) weights quantized on device, N(0,1) activations)",
        "config": {"workload": "W4A16 G64 decode GEMV sweep, M=1, 36 layers x {QKV 3584x2560, "
                               "gate+up 19456x2560, down 2560x9728}, distinct weights per layer",
                   "bytes_per_step": sweep_bytes, "frac_hbm": round(value / HBM_PEAK_GBS, 4),
                   "graph_replay_matches_eager": graph_ok},
        "prefill_gemm_tflops": prefill["TFLOP/s"] if prefill else None,
        "prefill_gemm_frac_bf16_peak": prefill["frac_bf16_peak"] if prefill else None,
        "roofline": roofline,
        "roofline_gemm": roofline_gemm,
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
