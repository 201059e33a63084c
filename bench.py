#!/usr/bin/env python3
"""Benchmark of the int8 / int8-dyn quantized-linear path on one MI355X.

Headline (``value``): int8 weight-only decode at M=1 - one step is one pass
over the fused-QKV [6144x4096], gate+up [24576x4096] and down [4096x12288]
projections (int8 per-channel weights, fp16 activations, fp16 outputs), with
inputs resident in HBM.  ``value`` = algorithmic bytes per step (N*K weights +
4N scales + M*K*2 activations + M*N*2 outputs) x steps / time, in GB/s.
Weights rotate over enough distinct copies (>= 512 MB) that the 256 MB
Infinity Cache cannot serve them.  The steps run as HIP graph replays, one
graph holding one step per weight copy.

Also reported (``extra``): M=4/16 decode, the 4096x4096 single GEMV (fp32 and
fp16 activations), the prefill GEMM at M=512/2048/8192 (N=12288, K=4096,
TFLOP/s vs the 2.5 PFLOP/s dense fp16 peak), int8-dyn at M=1/128/512/2048
(and the opt-in per-token symmetric scheme at M=1/128/2048), and
one decode step through all 539 linears of a random-init 36-layer hybrid
model (hidden 4096, FFN 12288, vocab 151936) at M=1 and M=8, unfused and with
the layers that read the same input fused (223 launches, same weight bytes),
and fused and grouped (171 launches) at this model's and at the real
checkpoint's sizes (hidden 2560, FFN 9728), the latter also with fp32
activations and in int8-dyn mode.

``roofline`` covers the dominant kernel (the gate+up GEMV launch): its average
duration is measured with HIP events around a graph of back-to-back launches
on the stream the kernel runs on.  ``cpu_baseline`` times the reference's CPU
path (the int8 block loop of quant.py:46-53, restated with torch CPU ops) on
the host cores for the same decode step.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "spikingbrain-cpu_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "int8 W-only GEMV GB/s (%HBM peak) at M=1; prefill GEMM TFLOPS (%MFMA) M=2048"
HBM_PEAK_GBS = 8000.0
F16_PEAK_TFLOPS = 2500.0
I8_PEAK_TOPS = 5000.0
DECODE_SHAPES = [(6144, 4096), (24576, 4096), (4096, 12288)]  # fused QKV, gate+up, down
DOMINANT = (24576, 4096)
ROTATE_BYTES = 512 << 20
WARM_MS = 100.0  # untimed sustained load before each timed region
SOFTMAX_LAYERS = (0, 1, 2, 3, 6, 12, 17, 21, 24, 35)


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def gemv_bytes(M, N, K, xbytes=2, ybytes=2):
    return N * K + 4 * N + M * K * xbytes + M * N * ybytes


class Ctx:
    def __init__(self):
        import torch

        from sbq import quant

        self.torch = torch
        self.quant = quant
        self.dev = torch.device("cuda", 0)
        torch.cuda.set_device(self.dev)

    def weights(self, N, K, seed, colsum=False):
        """Random N(0, 0.02) weights quantized and packed on the GPU."""
        torch = self.torch
        g = torch.Generator(device=self.dev).manual_seed(seed)
        w = torch.randn(N, K, generator=g, device=self.dev) * 0.02
        q, s = self.quant.quantize_per_channel_gpu(w)
        del w
        packed, cs = self.quant.repack(q, with_colsum=colsum)
        del q
        return packed, s, cs

    def act(self, M, K, seed, dtype=None, outliers=False):
        torch = self.torch
        g = torch.Generator(device=self.dev).manual_seed(seed)
        x = torch.randn(M, K, generator=g, device=self.dev)
        if outliers:
            idx = torch.randperm(K, generator=g, device=self.dev)[: max(1, K // 100)]
            x[:, idx] *= 20
        return x.to(dtype or torch.float16)

    def graph(self, fn):
        torch = self.torch
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()  # warm the launch path outside capture
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        return g

    def time_graphs(self, graphs, steps, warmup, warm_ms=WARM_MS):
        """Replay graphs round-robin; return ms per replay (events on the
        stream the graphs are launched on, synchronize on both sides).  Untimed
        warmup: `warmup` replays, then more until `warm_ms` of wall time."""
        torch = self.torch
        for i in range(warmup):
            graphs[i % len(graphs)].replay()
        torch.cuda.synchronize()
        t0, i = time.perf_counter(), 0
        while (time.perf_counter() - t0) * 1e3 < warm_ms:
            graphs[i % len(graphs)].replay()
            torch.cuda.synchronize()
            i += 1
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            graphs[i % len(graphs)].replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    def time_steps(self, step, copies, steps, warmup, warm_ms=WARM_MS):
        """ms per step for exactly `steps` steps; step(c) runs one step on weight
        copy c.  One graph holds `copies` consecutive steps (so the host replays
        once per `copies` steps); a second graph holds the remainder.  Untimed
        warmup: `warmup` steps, then replays of the same graph until `warm_ms`
        of wall time has passed (the shader clock settles under sustained load)."""
        torch = self.torch
        full = self.graph(lambda: [step(c) for c in range(copies)])
        rem_n = steps % copies
        rem = self.graph(lambda: [step(c) for c in range(rem_n)]) if rem_n else None
        for _ in range(max(1, -(-warmup // copies))):
            full.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        while (time.perf_counter() - t0) * 1e3 < warm_ms:
            full.replay()
            torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps // copies):
            full.replay()
        if rem is not None:
            rem.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps


# ---------------------------------------------------------------------------
# decode (weight-only GEMV)
# ---------------------------------------------------------------------------
def decode_setup(ctx, M, shapes, xdtype=None, seed=0):
    torch = ctx.torch
    step_bytes = sum(gemv_bytes(M, N, K, 4 if xdtype == torch.float32 else 2) for N, K in shapes)
    weight_bytes = sum(N * K for N, K in shapes)
    copies = max(1, math.ceil(ROTATE_BYTES / weight_bytes)) + (1 if weight_bytes < ROTATE_BYTES else 0)
    layers = [[ctx.weights(N, K, seed + 17 * c + i) for i, (N, K) in enumerate(shapes)] for c in range(copies)]
    xs = [ctx.act(M, K, 100 + i, xdtype) for i, (N, K) in enumerate(shapes)]
    ys = [torch.empty((M, N), dtype=torch.float16, device=ctx.dev) for N, K in shapes]
    return layers, xs, ys, step_bytes, copies


def decode_bench(ctx, M, steps, warmup, shapes=DECODE_SHAPES, xdtype=None):
    quant = ctx.quant
    layers, xs, ys, step_bytes, copies = decode_setup(ctx, M, shapes, xdtype)

    def step(c):
        for (packed, s, _), x, y, (N, K) in zip(layers[c], xs, ys, shapes):
            quant.linear_w8(x, packed, s, None, N, out=y)

    ms = ctx.time_steps(step, copies, steps, warmup)
    gbs = step_bytes / (ms * 1e-3) / 1e9
    out = {"ms_per_step": ms, "GBps": gbs, "hbm_frac": gbs / HBM_PEAK_GBS, "bytes_per_step": step_bytes,
           "weight_copies": copies}
    del layers
    return out


def gemv_grouped4_bench(ctx, N=4096, K=4096, steps=40, warmup=5, xdtype=None):
    """Four independent N x K projections at M=1 (distinct weights, inputs
    and outputs) as one grouped launch (sbq_linear_w8_grouped: the launch gap
    and ramp paid once for the four), weights rotating beyond the Infinity
    Cache: per-projection time and the group's GB/s."""
    torch, quant = ctx.torch, ctx.quant
    shapes = [(N, K)] * 4
    layers, xs, ys, step_bytes, copies = decode_setup(ctx, 1, shapes, xdtype, seed=900)

    def step(c):
        L = layers[c]
        quant.linear_w8_grouped(xs, [l[0] for l in L], [l[1] for l in L], [None] * 4, [N] * 4,
                                out_dtype=torch.float16, outs=ys)

    ms = ctx.time_steps(step, copies, steps, warmup)
    gbs = step_bytes / (ms * 1e-3) / 1e9
    del layers
    return {"us_per_launch": ms * 1e3, "us_per_projection": ms * 1e3 / 4, "GBps": gbs, "hbm_frac": gbs / HBM_PEAK_GBS}


def stream_floor_bench(ctx, steps=40, warmup=5):
    """What one dependent launch of other kernels takes to read the same bytes
    as a 4096x4096 (16.8 MB) and a 24576x4096 (100.7 MB) int8 GEMV at M=1,
    rotating beyond the Infinity Cache as the GEMV benches' weights do:
    torch's copy_ moving as many HBM bytes (half read, half written; a plain
    elementwise kernel, safe to capture in a graph), and the vendor library's
    GEMV on fp16 weights of the same shape (torch.matmul, hipBLASLt: twice
    the weight bytes).  Reference points for the per-launch floor of the
    GEMV; not part of this library."""
    torch = ctx.torch
    out = {}
    for N, K in ((4096, 4096), (24576, 4096)):
        nbytes = N * K
        copies = math.ceil(ROTATE_BYTES / nbytes) + 1
        src = [torch.empty(nbytes // 2, dtype=torch.uint8, device=ctx.dev).fill_(c) for c in range(copies)]
        dst = [torch.empty(nbytes // 2, dtype=torch.uint8, device=ctx.dev) for _ in range(copies)]
        ms = ctx.time_steps(lambda c: dst[c].copy_(src[c]), copies, steps, warmup)
        r = {"copy_us": ms * 1e3, "copy_GBps": nbytes / (ms * 1e-3) / 1e9}
        del src, dst
        copies16 = math.ceil(ROTATE_BYTES / (2 * nbytes)) + 1
        ws = [(torch.randn(K, N, device=ctx.dev) * 0.02).half() for _ in range(copies16)]
        x = torch.randn(1, K, device=ctx.dev).half()
        y = torch.empty((1, N), dtype=torch.float16, device=ctx.dev)
        ms = ctx.time_steps(lambda c: torch.matmul(x, ws[c], out=y), copies16, steps, warmup)
        r["fp16_matmul_us"] = ms * 1e3
        r["fp16_matmul_GBps"] = 2 * nbytes / (ms * 1e-3) / 1e9
        del ws
        out[f"{N}x{K}"] = r
    return out


def dominant_kernel(ctx, M=1, launches_per_copy=8, reps=5):
    """Average duration of the gate+up GEMV launch: a graph of back-to-back
    launches (rotating weight copies), HIP events around the replays."""
    quant = ctx.quant
    N, K = DOMINANT
    wbytes = N * K
    copies = math.ceil(ROTATE_BYTES / wbytes) + 1
    layers = [ctx.weights(N, K, 500 + c) for c in range(copies)]
    x = ctx.act(M, K, 7)
    y = ctx.torch.empty((M, N), dtype=ctx.torch.float16, device=ctx.dev)

    def run():
        for _ in range(launches_per_copy):
            for packed, s, _ in layers:
                quant.linear_w8(x, packed, s, None, N, out=y)

    g = ctx.graph(run)
    n = launches_per_copy * copies
    ms = ctx.time_graphs([g], reps, 1)
    us = ms * 1e3 / n
    bytes_per_launch = gemv_bytes(M, N, K)
    return {"kernel": "sbq::gemv_fast_kernel (gate+up 24576x4096, M=1, fp16 x, fp16 y)", "avg_us": us,
            "bytes_per_launch": bytes_per_launch, "GBps": bytes_per_launch / (us * 1e-6) / 1e9,
            "launches": n * reps}


def lm_head_greedy_bench(ctx, V=151936, K=4096, M=1, steps=40, warmup=5):
    """lm_head (model.py:445-447) at M=1 with fp32 activations and logits (the
    reference model's dtypes), three ways: the logits alone; the logits and
    the greedy token in one pass (sbq_linear_w8_argmax); the logits then the
    separate row argmax (sbq_argmax_rows).  Weights rotate over 2 copies
    (1.24 GB, beyond the Infinity Cache)."""
    torch, quant = ctx.torch, ctx.quant
    layers = [ctx.weights(V, K, 800 + c) for c in range(2)]
    x = ctx.act(M, K, 801, torch.float32)
    y = torch.empty((M, V), dtype=torch.float32, device=ctx.dev)
    idx = torch.empty((M,), dtype=torch.int64, device=ctx.dev)
    state = quant.argmax_state(ctx.dev)
    nbytes = gemv_bytes(M, V, K, 4, 4)

    def plain(c):
        packed, s, _ = layers[c % 2]
        quant.linear_w8(x, packed, s, None, V, out=y)

    def fused(c):
        packed, s, _ = layers[c % 2]
        quant.linear_w8_argmax(x, packed, s, None, V, state, out=y, idx=idx)

    def separate(c):
        plain(c)
        quant.greedy_tokens(y)

    res = {"V": V, "K": K, "M": M, "bytes": nbytes}
    for name, fn in (("logits_us", plain), ("logits_and_token_one_pass_us", fused),
                     ("logits_then_argmax_us", separate)):
        res[name] = ctx.time_steps(fn, 4, steps, warmup) * 1e3
    res["one_pass_extra_us"] = res["logits_and_token_one_pass_us"] - res["logits_us"]
    res["GBps_one_pass"] = nbytes / (res["logits_and_token_one_pass_us"] * 1e-6) / 1e9
    return res


def sample_bench(ctx, V=151936, M=1, steps=40, warmup=5):
    """The engine's non-greedy sampling step (engine.py:29-42) over one row of
    lm_head logits (fp32, N(0, 2.5)), with the logits left on the GPU:
    sbq_sample_rows (radix selection, no sort) for the engine's default
    parameters (temperature 0.7, top_p 0.9), with top-k 50 as well, and with
    neither; beside it the reference's expression run by torch's own GPU ops
    (division, topk, softmax, sort, cumsum, scatter, multinomial with a GPU
    generator), timed over the same number of eager calls."""
    torch, quant = ctx.torch, ctx.quant
    logits = torch.randn(M, V, generator=torch.Generator().manual_seed(5)).mul_(2.5).to(ctx.dev)
    u = torch.rand(M, generator=torch.Generator().manual_seed(6)).to(ctx.dev)
    ws = quant.sample_workspace(M, V, ctx.dev)
    res = {"V": V, "M": M}
    for name, (T, k, p) in (("default_T0.7_p0.9", (0.7, 0, 0.9)), ("T0.7_k50_p0.9", (0.7, 50, 0.9)),
                            ("T1_no_cut", (1.0, 0, 1.0))):
        res[f"sbq_{name}_us"] = ctx.time_steps(lambda c, T=T, k=k, p=p: quant.sample_tokens(logits, T, p, k, u=u,
                                                                                              workspace=ws),
                                               4, steps, warmup) * 1e3
    gen = torch.Generator(device=ctx.dev).manual_seed(7)

    def torch_sample(T, k, p):
        z = logits[0] / T
        if k > 0:
            z = z.masked_fill(z < torch.topk(z, min(k, z.numel())).values[-1], float("-inf"))
        pr = torch.softmax(z, -1)
        if 0 < p < 1:
            sp, order = pr.sort(descending=True)
            sp = sp * (sp.cumsum(0) - sp < p)
            pr = torch.zeros_like(pr).scatter_(0, order, sp)
        return torch.multinomial(pr / pr.sum(), 1, generator=gen)

    for name, (T, k, p) in (("default_T0.7_p0.9", (0.7, 0, 0.9)), ("T0.7_k50_p0.9", (0.7, 50, 0.9))):
        for _ in range(warmup):
            torch_sample(T, k, p)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            torch_sample(T, k, p)
        e1.record()
        torch.cuda.synchronize()
        res[f"torch_ops_{name}_us"] = e0.elapsed_time(e1) / steps * 1e3
    return res


def device_state_bench(ctx, fmt="int8", H=2048, F=5632, blocks=4, V=32000, heads=16, max_len=512, steps=48):
    """Greedy decoding with a toy decoder (tests/toy_decoder.py: our own
    small model of the reference's projection pattern, random weights) in
    three placements: state on the CPU as the reference model keeps it (every
    projection copies x up and y back, argmax on the CPU); state on the GPU
    with eager launches; state on the GPU with one HIP graph replay per token.
    Reports per-token time and tokens/s (the linears' share is what this path
    owns; attention and norms are plain torch)."""
    torch = ctx.torch
    sys.path.insert(0, str(ROOT / "tests"))
    from toy_decoder import ToyDecoder, toy_weights

    w, emb = toy_weights(H, F, blocks, V)
    res = {"fmt": fmt, "H": H, "F": F, "blocks": blocks, "vocab": V, "heads": heads, "max_len": max_len,
           "steps": steps, "linears_per_token": 7 * blocks + 1}

    def per_token(run, n, sync):
        run(2)  # warm
        sync()
        t0 = time.perf_counter()
        run(n)
        sync()
        return (time.perf_counter() - t0) / n

    cpu = ToyDecoder(fmt, w, emb, heads, max_len, "cpu")
    cpu.reset(1)
    t = per_token(lambda n: [cpu.step_cpu_state() for _ in range(n)], min(steps, 16), torch.cuda.synchronize)
    res["cpu_state_ms_per_token"] = t * 1e3
    del cpu
    gpu = ToyDecoder(fmt, w, emb, heads, max_len, ctx.dev)
    gpu.reset(1)
    t = per_token(lambda n: [gpu.step_device() for _ in range(n)], steps, torch.cuda.synchronize)
    res["device_eager_ms_per_token"] = t * 1e3
    gpu.reset(1)
    g = ctx.graph(gpu.step_device)
    gpu.reset(1)
    t = per_token(lambda n: [g.replay() for _ in range(n)], steps, torch.cuda.synchronize)
    res["device_graph_ms_per_token"] = t * 1e3
    for k in ("cpu_state", "device_eager", "device_graph"):
        res[k + "_tokens_per_s"] = 1e3 / res[k + "_ms_per_token"]
    return res


def device_state_hybrid_bench(ctx, fmt="int8", steps=32, weights=None):
    """Greedy decoding with the hybrid decoder of tests/hybrid_decoder.py
    (our own model of the hybrid layer's launch pattern at the real
    checkpoint's sizes: hidden 2560, FFN 9728, 32 heads of 128, 8 kv heads,
    vocab 151936; layers hybrid, softmax, hybrid; random weights) over the
    device-resident state of sbq.state, in three placements: the state on the
    CPU (every projection copies x up and y back, the token by argmax on the
    CPU), the state on the GPU with eager launches, and one HIP graph replay
    per token.  Reports per-token time and tokens/s; the non-projection math
    (recurrences, attention, norms) is plain torch."""
    torch = ctx.torch
    sys.path.insert(0, str(ROOT / "tests"))
    from hybrid_decoder import Dims, HybridDecoder, SbqLinears, layer_shapes, make_weights

    dm = Dims()
    w, emb = weights if weights is not None else make_weights(dm)
    lin = SbqLinears(fmt, w, emb, dm, ctx.dev)
    wbytes = sum(N * K for i in range(len(dm.hybrid)) for N, K in layer_shapes(dm, i).values()) + dm.V * dm.H
    res = {"fmt": fmt, "H": dm.H, "F": dm.F, "layers": "hybrid, softmax, hybrid", "vocab": dm.V, "steps": steps,
           "linears_per_token": len(w) + 1, "weight_bytes_per_token": wbytes}

    def per_token(run, n):
        run(2)  # warm
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        run(n)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n

    with torch.no_grad():
        cpu = HybridDecoder(lin, emb, dm, "cpu")
        cpu.reset(1)
        res["cpu_state_ms_per_token"] = per_token(lambda n: [cpu.step() for _ in range(n)], min(steps, 8)) * 1e3
        del cpu
        gpu = HybridDecoder(lin, emb, dm, ctx.dev)
        gpu.reset(1)
        res["device_eager_ms_per_token"] = per_token(lambda n: [gpu.step() for _ in range(n)], steps) * 1e3
        gpu.reset(1)
        g = ctx.graph(gpu.step)
        gpu.reset(1)
        res["device_graph_ms_per_token"] = per_token(lambda n: [g.replay() for _ in range(n)], steps) * 1e3
    for k in ("cpu_state", "device_eager", "device_graph"):
        res[k + "_tokens_per_s"] = 1e3 / res[k + "_ms_per_token"]
    res["device_graph_weight_GBps"] = wbytes / (res["device_graph_ms_per_token"] * 1e-3) / 1e9
    del g, gpu, lin
    return res


def device_state_hybrid_both(ctx):
    """device_state_hybrid_bench for int8 and int8-dyn on one set of weights."""
    sys.path.insert(0, str(ROOT / "tests"))
    from hybrid_decoder import Dims, make_weights

    wts = make_weights(Dims())
    return {f: device_state_hybrid_bench(ctx, f, weights=wts) for f in ("int8", "int8-dyn")}


# ---------------------------------------------------------------------------
# prefill GEMM and int8-dyn
# ---------------------------------------------------------------------------
def prefill_bench(ctx, M, N=12288, K=4096, steps=20, warmup=5, xdtype=None, per_graph=5, ydtype=None):
    quant = ctx.quant
    packed, s, _ = ctx.weights(N, K, 900)
    x = ctx.act(M, K, 901)
    if xdtype is not None:
        x = x.to(xdtype)
    y = ctx.torch.empty((M, N), dtype=ydtype or ctx.torch.float16, device=ctx.dev)
    ws = quant.w8_workspace(M, K, ctx.dev, x.dtype, N)  # the pre-passes are part of each timed step
    # per_graph steps per graph replay: the launch gap between replays is not the kernel's
    ms = ctx.time_steps(lambda c: quant.linear_w8(x, packed, s, None, N, out=y, workspace=ws), per_graph, steps,
                        warmup)
    tflops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    return {"M": M, "N": N, "K": K, "x": str(x.dtype).replace("torch.", ""), "y": str(y.dtype).replace("torch.", ""),
            "ms": ms, "TFLOPs": tflops, "mfma_frac": tflops / F16_PEAK_TFLOPS}


def midm_bench(ctx, M, N, fmt, K=4096, steps=20, warmup=5):
    """One mid-sized linear (fp16 x and y): the whole call (pre-passes, GEMM,
    split-K fixup) with weights rotating over copies beyond the 256 MB
    Infinity Cache, as a layer-by-layer forward reads them."""
    torch, quant = ctx.torch, ctx.quant
    copies = math.ceil(ROTATE_BYTES / (N * K)) + 1
    layers = [ctx.weights(N, K, 960 + c, colsum=fmt == "int8-dyn") for c in range(copies)]
    x = ctx.act(M, K, 961, outliers=fmt == "int8-dyn")
    y = torch.empty((M, N), dtype=torch.float16, device=ctx.dev)
    if fmt == "int8-dyn":
        ws = quant.w8a8_workspace(M, K, ctx.dev, N)

        def step(c):
            L = layers[c]
            quant.linear_w8a8(x, L[0], L[1], L[2], None, N, torch.float16, workspace=ws, out=y)
    else:
        ws = quant.w8_workspace(M, K, ctx.dev, x.dtype, N)

        def step(c):
            L = layers[c]
            quant.linear_w8(x, L[0], L[1], None, N, out=y, workspace=ws)

    ms = ctx.time_steps(step, copies, max(steps, copies), warmup)
    ops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    peak = I8_PEAK_TOPS if fmt == "int8-dyn" else F16_PEAK_TFLOPS
    del layers
    return {"format": fmt, "M": M, "N": N, "K": K, "us": ms * 1e3, "TOPs_or_TFLOPs": ops, "peak_frac": ops / peak,
            "GBps": gemv_bytes(M, N, K) / (ms * 1e-3) / 1e9}


def w8a8_bench(ctx, M, N, K=4096, steps=20, warmup=5, token=False):
    """int8-dyn linear, whole call (activation quantization included): fbgemm's
    per-tensor asymmetric scheme, or with token=True the opt-in per-token
    symmetric one (row quantizer, then the s8 GEMV / GEMM)."""
    torch, quant = ctx.torch, ctx.quant
    wbytes = N * K
    # decode sizes rotate weight copies (HBM-bound); prefill sizes reuse one copy, 5 steps per graph replay
    ncopy = 1 if M >= 128 else math.ceil(ROTATE_BYTES / wbytes) + 1
    copies = 5 if M >= 128 else ncopy
    layers = [ctx.weights(N, K, 950 + c, colsum=True) for c in range(ncopy)]
    x = ctx.act(M, K, 951, outliers=True)
    y = torch.empty((M, N), dtype=torch.float16, device=ctx.dev)
    ws = quant.w8a8_workspace(M, K, ctx.dev, N)
    def step(c):
        L = layers[c % ncopy]
        if token:
            quant.linear_w8a8_token(x, L[0], L[1], None, N, torch.float16, workspace=ws, out=y)
        else:
            quant.linear_w8a8(x, L[0], L[1], L[2], None, N, torch.float16, workspace=ws, out=y)

    ms = ctx.time_steps(step, copies, max(steps, copies), warmup)
    res = {"M": M, "N": N, "K": K, "ms": ms}
    tops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    res["TOPs"] = tops
    res["i8_frac"] = tops / I8_PEAK_TOPS
    res["GBps"] = gemv_bytes(M, N, K) / (ms * 1e-3) / 1e9
    return res


def vendor_gemm_bench(ctx, K=4096, steps=20, warmup=5):
    """The vendor library's own GEMMs at the prefill and mid-sized shapes, as
    reference points for the kernels above (not part of this library):
    torch.matmul on fp16 weights [K, N] (hipBLASLt; an fp16 model with no
    int8 weights at all, twice the weight bytes), and torch._int_mm on s8
    operands (hipBLASLt's int8 GEMM: the int32 product alone, without the
    activation quantization, the zero-point correction or the scaled fp16
    output of an int8-dyn call).  Five steps per graph replay on one weight
    copy, as prefill_bench and w8a8_bench time theirs."""
    torch = ctx.torch
    gen = torch.Generator(device=ctx.dev).manual_seed(970)
    out = {"fp16_matmul": [], "int8_int_mm": []}
    for M, N in ((128, 4096), (128, 12288), (512, 12288), (2048, 12288), (8192, 12288)):
        w = (torch.randn(K, N, generator=gen, device=ctx.dev) * 0.02).half()
        x = torch.randn(M, K, generator=gen, device=ctx.dev).half()
        y = torch.empty(M, N, dtype=torch.float16, device=ctx.dev)
        ms = ctx.time_steps(lambda c: torch.matmul(x, w, out=y), 5, steps, warmup)
        tf = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        out["fp16_matmul"].append({"M": M, "N": N, "K": K, "us": ms * 1e3, "TFLOPs": tf,
                                   "mfma_frac": tf / F16_PEAK_TFLOPS})
        del w, x, y
    for M, N in ((128, 4096), (128, 12288), (512, 12288), (2048, 4096), (2048, 12288)):
        a = torch.randint(-127, 128, (M, K), generator=gen, device=ctx.dev, dtype=torch.int8)
        b = torch.randint(-127, 128, (K, N), generator=gen, device=ctx.dev, dtype=torch.int8)
        try:  # eager first: a shape the library refuses is reported, not captured
            torch._int_mm(a, b)
            torch.cuda.synchronize()
        except RuntimeError as e:
            out["int8_int_mm"].append({"M": M, "N": N, "K": K, "error": str(e).splitlines()[0][:160]})
            continue
        ms = ctx.time_steps(lambda c: torch._int_mm(a, b), 5, steps, warmup)
        tops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        out["int8_int_mm"].append({"M": M, "N": N, "K": K, "us": ms * 1e3, "TOPs": tops, "i8_frac": tops / I8_PEAK_TOPS})
        del a, b
    return out


# ---------------------------------------------------------------------------
# one decode step through every quantized linear of the 36-layer hybrid model
# ---------------------------------------------------------------------------
def hybrid_stack_shapes(H=4096, F=12288, heads=32, kv_heads=8, d=128, routers=4, vocab=151936, layers=36,
                        fused=False):
    """(N, K) of every quantized linear of one decode step.  fused=True
    concatenates the layers that read the same input (FusedLinear): per hybrid
    block sse_q/k/v + lora_q[0]/lora_k[0] + sse_a/b/e + swa_q/k/v (N=18820),
    and gate+up; per softmax block q/k/v and gate+up.  Same weight bytes."""
    shapes = []
    for i in range(layers):
        if i in SOFTMAX_LAYERS:
            qkv = [(heads * d, H), (kv_heads * d, H), (kv_heads * d, H)]
            shapes += [(sum(n for n, _ in qkv), H)] if fused else qkv
            shapes += [(H, heads * d)]
        else:
            reads_x = [(heads * d, H)] * 3                      # sse_q, sse_k, sse_v
            reads_x += [(d, H), (d, H)]                         # lora_q[0], lora_k[0]
            reads_x += [(2 * heads, H), (2 * heads, H), (routers, H)]  # sse_a, sse_b, sse_e
            reads_x += [(heads * d, H), (kv_heads * d, H), (kv_heads * d, H)]  # swa q, k, v
            shapes += [(sum(n for n, _ in reads_x), H)] if fused else reads_x
            shapes += [(heads * d, d), (heads * d, d)]          # lora_q[1], lora_k[1]
            shapes += [(H, heads * d), (H, heads * d)]          # sse_o, swa_o
        shapes += [(2 * F, H)] if fused else [(F, H), (F, H)]   # gate, up
        shapes += [(H, F)]                                      # down
    shapes.append((vocab, H))                                   # lm_head
    return shapes


def grouped_stack_launches(H=4096, F=12288, heads=32, d=128):
    """The fused stack's launches with the independent pairs of each hybrid
    layer grouped (sbq_linear_w8_grouped / sbq_linear_w8a8_grouped): lora_q[1] + lora_k[1] (two inputs
    of K = 128) and sse_o + swa_o (two attention outputs of K = 4096).  Each
    launch is a list of (N, K); the weight bytes are the fused stack's."""
    pair_lora = [(heads * d, d), (heads * d, d)]
    pair_o = [(H, heads * d), (H, heads * d)]
    shapes = hybrid_stack_shapes(H=H, F=F, fused=True)
    out, i = [], 0
    while i < len(shapes):
        if shapes[i:i + 2] == pair_lora or shapes[i:i + 2] == pair_o:
            out.append(shapes[i:i + 2])
            i += 2
        else:
            out.append([shapes[i]])
            i += 1
    return out


def stack_step(quant, launches, layers, xs, ys, wss, w8a8):
    """The decode step of a stack as one function of launches: `launches` as
    grouped_stack_launches / hybrid_stack_shapes give them, `layers` the
    (packed, scale, colsum) of every linear in launch order, xs[K] two
    [M, K] inputs per K (a grouped pair reads both; single launches read the
    first), ys the output of every linear, wss[K] the int8-dyn workspaces.
    The bench times it and the GPU tests check every output it writes
    against the oracle."""
    plan, j = [], 0
    for grp in launches:
        plan.append((grp, layers[j:j + len(grp)], ys[j:j + len(grp)]))
        j += len(grp)

    def step():
        for grp, lays, outs in plan:
            if w8a8 and len(grp) == 1:
                (N, K), (packed, s, cs) = grp[0], lays[0]
                quant.linear_w8a8(xs[K][0], packed, s, cs, None, N, workspace=wss[K], out=outs[0])
            elif w8a8:
                K = grp[0][1]
                quant.linear_w8a8_grouped([xs[K][i] for i in range(len(grp))], [p for p, _, _ in lays],
                                          [s for _, s, _ in lays], [c for _, _, c in lays], [None] * len(grp),
                                          [N for N, _ in grp], outs=outs, workspace=wss[K])
            elif len(grp) == 1:
                (N, K), (packed, s, _) = grp[0], lays[0]
                quant.linear_w8(xs[K][0], packed, s, None, N, out=outs[0])
            else:
                K = grp[0][1]
                quant.linear_w8_grouped([xs[K][i] for i in range(len(grp))], [p for p, _, _ in lays],
                                        [s for _, s, _ in lays], [None] * len(grp), [N for N, _ in grp],
                                        outs=outs)

    return step


def stack_bench(ctx, Ms=(1, 8), steps=10, warmup=3, fused=False, grouped=False, H=4096, F=12288, xdtype=None,
                w8a8=False):
    """One decode step through every quantized linear of the 36-layer hybrid
    model (hidden H, FFN F; H=2560, F=9728 is the reference's real checkpoint),
    one launch per linear, or fused / fused and grouped; w8a8: int8-dyn
    linears (DynamicInt8Linear), fused, one launch each or grouped."""
    torch, quant = ctx.torch, ctx.quant
    launches = (grouped_stack_launches(H=H, F=F) if grouped
                else [[sh] for sh in hybrid_stack_shapes(H=H, F=F, fused=fused)])
    shapes = [sh for grp in launches for sh in grp]
    layers = [ctx.weights(N, K, 2000 + i, colsum=w8a8) for i, (N, K) in enumerate(shapes)]
    wbytes = sum(N * K for N, K in shapes)
    res = {"linears": len(shapes), "launches": len(launches), "weight_bytes": wbytes}
    for M in Ms:
        xs = {}
        for N, K in shapes:
            if K not in xs:
                xs[K] = [ctx.act(M, K, 3000 + K, xdtype), ctx.act(M, K, 3500 + K, xdtype)]  # a grouped pair reads two inputs
        ys = [torch.empty((M, N), dtype=torch.float16, device=ctx.dev) for N, K in shapes]
        wss = {K: quant.w8a8_workspace(M, K, ctx.dev, None, xs[K][0].dtype) for K in xs} if w8a8 else {}
        step = stack_step(quant, launches, layers, xs, ys, wss, w8a8)
        g = ctx.graph(step)
        ms = ctx.time_graphs([g], steps, warmup)
        nbytes = sum(gemv_bytes(M, N, K) for N, K in shapes)
        res[f"M{M}"] = {"ms_per_step": ms, "tokens_per_s": M / (ms * 1e-3), "GBps": nbytes / (ms * 1e-3) / 1e9}
        del g, ys, wss
    del layers
    return res


# ---------------------------------------------------------------------------
# profile helpers: the workload of the two rocprofv3 --pmc passes, and the
# summaries of rocprofv3 output that are committed under profiles/
# ---------------------------------------------------------------------------
CAL_BYTES = 1 << 30  # calibration copy: 1 GiB read + 1 GiB written, beyond the 256 MB Infinity Cache
# the gate+up launch at M=1 (fp16 x): sbq::gemv_fast_kernel, two 16-row tiles per
# 256-lane workgroup (4 waves splitting K)
DOMINANT_KERNEL = "gemv_fast_kernel"
DOMINANT_BLOCK = 256
DOMINANT_GRID = ((DOMINANT[0] + 31) // 32) * DOMINANT_BLOCK


def traffic_probe(ctx, launches=24, cal_reps=4):
    """Eager launches of the dominant kernel (weights rotating beyond the
    Infinity Cache) followed by a plain copy kernel of known size (torch.neg
    on 1 GiB of fp16), for FETCH_SIZE / WRITE_SIZE counter passes."""
    torch, quant = ctx.torch, ctx.quant
    N, K = DOMINANT
    copies = math.ceil(ROTATE_BYTES / (N * K)) + 1
    layers = [ctx.weights(N, K, 500 + c) for c in range(copies)]
    x = ctx.act(1, K, 7)
    y = torch.empty((1, N), dtype=torch.float16, device=ctx.dev)
    a = torch.ones(CAL_BYTES // 2, dtype=torch.float16, device=ctx.dev)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for i in range(launches):
        packed, s, _ = layers[i % copies]
        quant.linear_w8(x, packed, s, None, N, out=y)
    torch.cuda.synchronize()
    for _ in range(cal_reps):
        torch.neg(a, out=b)
    torch.cuda.synchronize()
    log(f"traffic probe: {launches} gate+up launches, {cal_reps} copies of {CAL_BYTES >> 20} MiB")


def gemv_probe(ctx, N=4096, K=4096, M=1, launches_per_copy=8, reps=20):
    """Back-to-back decode GEMV launches (fp16 x and y, weights rotating over
    >= 512 MB of copies) captured in one HIP graph and replayed `reps` times:
    the workload of the kernel-trace pass that splits each launch's duration
    from the gap to the next launch."""
    torch, quant = ctx.torch, ctx.quant
    copies = math.ceil(ROTATE_BYTES / (N * K)) + 1
    layers = [ctx.weights(N, K, 700 + c) for c in range(copies)]
    x = ctx.act(M, K, 7)
    y = torch.empty((M, N), dtype=torch.float16, device=ctx.dev)

    def run():
        for _ in range(launches_per_copy):
            for packed, s, _ in layers:
                quant.linear_w8(x, packed, s, None, N, out=y)

    g = ctx.graph(run)
    ms = ctx.time_graphs([g], reps, 1)
    n = launches_per_copy * copies
    log(f"gemv probe: M={M} N={N} K={K}, {reps} replays of {n} launches, {ms * 1e3 / n:.3f} us per launch (events)")


def summarize_gaps(d, match, command):
    """Markdown: per-dispatch duration and the gap from each dispatch's end to
    the next dispatch's start, over runs of consecutive dispatches of the
    kernels whose name contains `match` (the back-to-back launches of a graph)."""
    import statistics

    rows = sorted(_csv_rows(d, "kernel_trace.csv"), key=lambda r: int(r["Start_Timestamp"]))
    dur, gap, period = [], [], []
    for a, b in zip(rows, rows[1:]):
        if match in a["Kernel_Name"] and match in b["Kernel_Name"]:
            s0, e0, s1 = int(a["Start_Timestamp"]), int(a["End_Timestamp"]), int(b["Start_Timestamp"])
            dur.append((e0 - s0) / 1e3)
            gap.append((s1 - e0) / 1e3)
            period.append((s1 - s0) / 1e3)
    if not dur:
        raise SystemExit(f"no consecutive dispatches of {match} in {d}")
    name = _short(next(r["Kernel_Name"] for r in rows if match in r["Kernel_Name"]))

    def line(label, v):
        q = statistics.quantiles(v, n=20)
        return (f"| {label} | {statistics.mean(v):.3f} | {statistics.median(v):.3f} | {q[0]:.3f} | {q[-1]:.3f} |")

    out = [f"# Launch duration vs launch-to-launch gap: `{name}`", "", "Command:", "", "```", command, "```", "",
           f"Pairs of consecutive dispatches: {len(dur)}.", "",
           "| us | mean | median | p5 | p95 |", "|---|---|---|---|---|",
           line("duration (start to end)", dur), line("gap (end to next start)", gap),
           line("period (start to next start)", period)]
    return "\n".join(out) + "\n"


def prefill_probe(ctx, M=2048, N=12288, K=4096, launches=100, xdtype=None):
    """The prefill operation alone (row-sum or staging pre-pass + GEMM; int8
    weights, fp16 x unless xdtype says otherwise, fp16 y), for counter passes;
    enough back-to-back launches (~17 ms) for the shader clock to settle under
    the load."""
    torch, quant = ctx.torch, ctx.quant
    packed, s, _ = ctx.weights(N, K, 900)
    x = ctx.act(M, K, 901)
    if xdtype is not None:
        x = x.to(xdtype)
    y = torch.empty((M, N), dtype=torch.float16, device=ctx.dev)
    ws = quant.w8_workspace(M, K, ctx.dev, x.dtype, N)
    torch.cuda.synchronize()
    for _ in range(launches):
        quant.linear_w8(x, packed, s, None, N, out=y, workspace=ws)
    torch.cuda.synchronize()
    log(f"prefill probe: {launches} launches of M={M} N={N} K={K}")


def w8a8_probe(ctx, M=2048, N=12288, K=4096, launches=100):
    """The int8-dyn prefill operation alone (activation min/max and quantize
    pre-passes + the i8 GEMM; fp16 x with 1% outlier channels, fp16 y), for
    counter passes; enough back-to-back launches for the clock to settle."""
    torch, quant = ctx.torch, ctx.quant
    packed, s, cs = ctx.weights(N, K, 950, colsum=True)
    x = ctx.act(M, K, 951, outliers=True)
    y = torch.empty((M, N), dtype=torch.float16, device=ctx.dev)
    ws = quant.w8a8_workspace(M, K, ctx.dev, N)
    torch.cuda.synchronize()
    for _ in range(launches):
        quant.linear_w8a8(x, packed, s, cs, None, N, torch.float16, workspace=ws, out=y)
    torch.cuda.synchronize()
    log(f"w8a8 probe: {launches} launches of M={M} N={N} K={K}")


def summarize_counters(dirs, match, command):
    """Markdown table: per-dispatch averages of every counter collected in the
    rocprofv3 --pmc output directories, for kernels whose name contains match."""
    rows = []
    for d in dirs:
        acc = {}
        for r in _csv_rows(d, "counter_collection.csv"):
            if match not in r["Kernel_Name"]:
                continue
            k = (r["Dispatch_Id"], r["Counter_Name"])
            acc[k] = acc.get(k, 0.0) + float(r["Counter_Value"])
        per = {}
        for (_, c), v in acc.items():
            per.setdefault(c, []).append(v)
        rows += [(c, sum(v) / len(v), len(v)) for c, v in sorted(per.items())]
    out = [f"# rocprofv3 counters of `{match}`", "", "Command:", "", "```", command, "```", "",
           "| counter | average per dispatch | dispatches |", "|---|---|---|"]
    out += [f"| {c} | {v:.6g} | {n} |" for c, v, n in rows]
    return "\n".join(out) + "\n"


def _csv_rows(d, suffix):
    import csv

    files = sorted(Path(d).rglob(f"*{suffix}"))
    if not files:
        raise SystemExit(f"no *{suffix} under {d}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows += list(csv.DictReader(fh))
    return rows


def _short(name):
    name = name.replace("void ", "")
    return name.split("(")[0] if name.startswith("sbq::") else name[:60]


def summarize_trace(d, command, title="the default bench run"):
    """Markdown summary of a rocprofv3 --kernel-trace --stats run: kernels by
    total time, split by launch grid, and the dominant kernel's average."""
    import statistics

    rows = _csv_rows(d, "kernel_trace.csv")
    agg = {}
    for r in rows:
        grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        key = (_short(r["Kernel_Name"]), grid, int(r["Workgroup_Size_X"]))
        agg.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    total = sum(sum(v) for v in agg.values())
    out = [f"# rocprofv3 kernel trace of {title}", "", "Command:", "", "```", command, "```", "",
           f"Dispatches: {sum(len(v) for v in agg.values())}, kernel time {total / 1e3:.1f} ms.", "",
           "| kernel | grid (work-items) | block | calls | avg us | median us | min us | % time |",
           "|---|---|---|---|---|---|---|---|"]
    for (name, grid, wg), v in sorted(agg.items(), key=lambda kv: -sum(kv[1]))[:25]:
        out.append(f"| `{name}` | {grid} | {wg} | {len(v)} | {statistics.mean(v):.2f} | {statistics.median(v):.2f} | "
                   f"{min(v):.2f} | {100 * sum(v) / total:.1f} |")
    # the dominant launch signature; the M=1 back-to-back run that bench.py's
    # roofline times is the part of it whose neighbours are the same launch
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    is_dom = [DOMINANT_KERNEL in r["Kernel_Name"] and int(r["Workgroup_Size_X"]) == DOMINANT_BLOCK and
              int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"]) == DOMINANT_GRID for r in rows]
    dur = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0 for r in rows]
    allv = [d for d, f in zip(dur, is_dom) if f]
    run = [dur[i] for i in range(1, len(rows) - 1) if is_dom[i - 1] and is_dom[i] and is_dom[i + 1]]
    if run:
        nbytes = gemv_bytes(1, *DOMINANT)
        name = _short(next(r["Kernel_Name"] for r, f in zip(rows, is_dom) if f))
        out += ["", f"Dominant kernel (gate+up {DOMINANT[0]}x{DOMINANT[1]}, M=1): `{name}`, grid {DOMINANT_GRID}, "
                f"block {DOMINANT_BLOCK}.",
                f"Back-to-back launches (the run bench.py's roofline times): {len(run)}, average "
                f"{statistics.mean(run):.3f} us, median {statistics.median(run):.3f} us -> "
                f"{nbytes / (statistics.mean(run) * 1e3):.0f} GB/s of algorithmic bytes ({nbytes} per launch).",
                f"All launches with this signature (also the M=1 and M=4 decode steps): {len(allv)}, average "
                f"{statistics.mean(allv):.3f} us."]
    stats = sorted(Path(d).rglob("*kernel_stats.csv"))
    if stats:
        out += ["", "rocprofv3 --stats (by kernel name, top 12):", "", "```"]
        for line in stats[0].read_text().splitlines()[:13]:
            name, _, rest = line.partition('",')
            out.append((name[:110] + ('..."' if len(name) > 110 else '"')) + "," + rest)
        out += ["```"]
    return "\n".join(out) + "\n"


def summarize_pmc(fetch_dir, write_dir, commands):
    """HBM traffic per launch of the dominant kernel from FETCH_SIZE and
    WRITE_SIZE (KiB per dispatch), each scaled by what the same counter reads
    for the calibration copy of CAL_BYTES."""
    import statistics

    def per_dispatch(d, counter):
        acc = {}
        for r in _csv_rows(d, "counter_collection.csv"):
            if r["Counter_Name"] != counter:
                continue
            k = (r["Dispatch_Id"], r["Kernel_Name"], int(r["Grid_Size"]), int(r["Workgroup_Size"]))
            acc[k] = acc.get(k, 0.0) + float(r["Counter_Value"])
        return acc

    res = {"commands": commands, "calibration": f"torch.neg on {CAL_BYTES} bytes of fp16 (reads and writes "
                                                 f"{CAL_BYTES} bytes)"}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        acc = per_dispatch(d, counter)
        dom = [v for (i, n, g, b), v in acc.items()
               if DOMINANT_KERNEL in n and g == DOMINANT_GRID and b == DOMINANT_BLOCK]
        cal = [v for (i, n, g, b), v in acc.items() if "neg" in n.lower() and v > CAL_BYTES / 1024 / 4]
        if not dom or not cal:
            raise SystemExit(f"{counter}: dominant ({len(dom)}) or calibration ({len(cal)}) dispatches not found")
        factor = (CAL_BYTES / 1024) / statistics.median(cal)
        res[counter] = {"dominant_KiB_per_dispatch": statistics.median(dom), "dispatches": len(dom),
                        "calibration_KiB": statistics.median(cal), "scale": factor,
                        "bytes_per_launch": statistics.median(dom) * 1024 * factor}
    res["algorithmic_bytes_per_launch"] = gemv_bytes(1, *DOMINANT)
    res["traffic_bytes_per_launch"] = res["FETCH_SIZE"]["bytes_per_launch"] + res["WRITE_SIZE"]["bytes_per_launch"]
    res["traffic_over_algorithmic"] = res["traffic_bytes_per_launch"] / res["algorithmic_bytes_per_launch"]
    return json.dumps(res, indent=1) + "\n"


def traffic_from_profiles():
    """HBM bytes per launch of the dominant kernel from the committed PMC
    summary (FETCH_SIZE + WRITE_SIZE, scaled by a copy-kernel calibration)."""
    p = ROOT / "profiles" / "gemv_w8_gateup_m1_traffic.json"
    try:
        return float(json.loads(p.read_text())["traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def cpu_baseline(budget_s):
    """The reference's CPU path (oracle/cpu_baseline.py restates quant.py's
    two int8 forwards with torch CPU operators) on this host's cores: the M=1
    decode step of the headline over a thread sweep (the best count is the
    reported value; the reference's default is 4 threads, bench.py:231), the
    fbgemm int8-dyn decode step, and the prefill legs at M=512 and 2048."""
    import torch

    import oracle.cpu_baseline as cb

    info = cb.cpu_info()
    host = info["host_threads"]
    counts = sorted({t for t in (1, 2, 4, 8, 16, 32, host) if t <= host})
    per = budget_s / (len(counts) + 6)
    sweep = {}
    for t in counts:
        r = cb.decode_step_baseline(DECODE_SHAPES, 1, t, per)
        sweep[t] = r["bytes_per_step"] / r["seconds_per_step"] / 1e9
        log(f"cpu baseline: int8 decode step, {t} threads: {sweep[t]:.2f} GB/s")
    best = max(sweep, key=sweep.get)
    r = cb.decode_step_baseline(DECODE_SHAPES, 1, best, per, fmt="int8-dyn")
    dyn_gbs = r["bytes_per_step"] / r["seconds_per_step"] / 1e9
    # prefill GEMMs are large enough to use every core: all host threads there
    prefill = [cb.prefill_baseline(M, 12288, 4096, host, per, fmt) for fmt in ("int8", "int8-dyn") for M in (512, 2048)]
    torch.set_num_threads(host)
    return {"value": sweep[best], "unit": "GB/s", "cores": best, "kind": "port",
            "sample": (f"int8 block loop of quant.py:46-53 (torch CPU restatement) over the same M=1 decode step "
                       f"(QKV, gate+up, down), median of repetitions over ~{per:.1f} s per thread count; the best "
                       f"of {counts} threads"),
            "GBps_by_threads": {str(t): round(v, 3) for t, v in sweep.items()},
            "GBps_4_threads": sweep.get(4),
            "int8_dyn_decode_GBps": dyn_gbs,
            "prefill": [{k: (round(v, 6) if isinstance(v, float) else v) for k, v in p.items()} for p in prefill],
            **info}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-budget", type=float, default=24.0, help="seconds of CPU baseline sampling")
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary measurements")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only run the dominant kernel and a calibration copy (workload of the --pmc passes)")
    ap.add_argument("--summarize-trace", metavar="DIR", help="print a markdown summary of a rocprofv3 kernel trace")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="print the traffic JSON from FETCH_SIZE and WRITE_SIZE passes over --traffic-probe")
    ap.add_argument("--prefill-probe", nargs="*", type=int, metavar="M N K",
                    help="only run the weight-only GEMM, M=2048 N=12288 K=4096 unless given (counter passes)")
    ap.add_argument("--probe-x", default="float16", choices=("float16", "bfloat16", "float32"),
                    help="activation dtype of --prefill-probe")
    ap.add_argument("--w8a8-probe", nargs="*", type=int, metavar="M N K",
                    help="only run the int8-dyn linear, M=2048 N=12288 K=4096 unless given (counter passes)")
    ap.add_argument("--only", metavar="NAME", help="run one extra measurement and print it (e.g. lm_head_greedy)")
    ap.add_argument("--gemv-probe", nargs=3, type=int, metavar=("M", "N", "K"),
                    help="only run back-to-back decode GEMV launches in a graph (workload of the gap trace)")
    ap.add_argument("--summarize-gaps", metavar="DIR",
                    help="print launch duration vs launch-to-launch gap from a rocprofv3 kernel trace")
    ap.add_argument("--summarize-counters", nargs="+", metavar="DIR",
                    help="print per-dispatch counter averages from rocprofv3 --pmc directories")
    ap.add_argument("--match", default="gemm_dl_kernel", help="kernel-name filter for --summarize-counters")
    ap.add_argument("--command", default="", help="the profiling command(s), recorded in the summary")
    ap.add_argument("--title", default="the default bench run", help="what --summarize-trace's run measured")
    ap.add_argument("--stack-m", type=int, nargs="+", default=[1, 8], metavar="M",
                    help="decode batch sizes of the --only stack_* measurements")
    args = ap.parse_args()
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace, args.command, args.title), end="")
        return
    if args.summarize_pmc:
        print(summarize_pmc(*args.summarize_pmc, args.command), end="")
        return
    if args.summarize_counters:
        print(summarize_counters(args.summarize_counters, args.match, args.command), end="")
        return
    if args.summarize_gaps:
        print(summarize_gaps(args.summarize_gaps, args.match, args.command), end="")
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(multi-GPU sharding of this path is a design note, not built)", file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py runs one process on one GPU; WORLD_SIZE > 1 is not supported", file=sys.stderr)
        sys.exit(2)

    ctx = Ctx()
    torch = ctx.torch
    if args.traffic_probe:
        traffic_probe(ctx)
        return
    if args.prefill_probe is not None:
        prefill_probe(ctx, *(args.prefill_probe or (2048, 12288, 4096)), xdtype=getattr(ctx.torch, args.probe_x))
        return
    if args.w8a8_probe is not None:
        w8a8_probe(ctx, *(args.w8a8_probe or (2048, 12288, 4096)))
        return
    if args.gemv_probe:
        M, N, K = args.gemv_probe
        gemv_probe(ctx, N, K, M)
        return
    if args.only:
        sm = tuple(args.stack_m)
        fn = {"lm_head_greedy": lm_head_greedy_bench, "device_state": device_state_bench,
              "device_state_hybrid": device_state_hybrid_both,
              "sample": sample_bench,
              "vendor_gemm": vendor_gemm_bench,
              "stream_floor": stream_floor_bench,
              "gemv_4096_grouped4": gemv_grouped4_bench,
              "stack_fused": lambda ctx: stack_bench(ctx, Ms=sm, fused=True),
              "w8a8": lambda ctx: [w8a8_bench(ctx, M, N) for M in (1, 128, 512, 2048) for N in (4096, 12288)],
              "prefill": lambda ctx: [prefill_bench(ctx, M) for M in (512, 2048, 8192)],
              "prefill_other_x": lambda ctx: [prefill_bench(ctx, 2048, xdtype=dt)
                                              for dt in (ctx.torch.bfloat16, ctx.torch.float32)],
              "w8a8_token": lambda ctx: [w8a8_bench(ctx, M, N, token=True) for M in (1, 128, 2048)
                                         for N in (4096, 12288)],
              "mid_m": lambda ctx: [midm_bench(ctx, M, N, fmt) for fmt in ("int8", "int8-dyn") for M in (64, 128, 256)
                                    for N in (4096, 12288)],
              "prefill_fp32_y": lambda ctx: [prefill_bench(ctx, M, xdtype=xd, ydtype=ctx.torch.float32)
                                             for M in (512, 2048) for xd in (ctx.torch.float16, ctx.torch.float32)],
              "stack_grouped": lambda ctx: stack_bench(ctx, Ms=sm, grouped=True),
              "stack_checkpoint_grouped": lambda ctx: stack_bench(ctx, Ms=sm, grouped=True, H=2560, F=9728),
              "stack_checkpoint_grouped_f32x": lambda ctx: stack_bench(ctx, Ms=sm, grouped=True, H=2560, F=9728,
                                                                       xdtype=ctx.torch.float32),
              "stack_checkpoint_w8a8": lambda ctx: {xd: stack_bench(ctx, Ms=sm, grouped=True, H=2560, F=9728, w8a8=True,
                                                                    xdtype=getattr(ctx.torch, xd))
                                                    for xd in ("float16", "float32")},
              "stack_checkpoint_w8a8_ungrouped": lambda ctx: {
                  xd: stack_bench(ctx, Ms=sm, fused=True, H=2560, F=9728, w8a8=True, xdtype=getattr(ctx.torch, xd))
                  for xd in ("float16", "float32")},
              "cpu_baseline": lambda ctx: cpu_baseline(args.cpu_budget)}[args.only]
        print(json.dumps({args.only: fn(ctx)}), flush=True)
        return
    log("decode M=1 (headline)")
    head = decode_bench(ctx, 1, args.steps, args.warmup)
    log(f"  {head['GBps']:.0f} GB/s, {head['ms_per_step'] * 1e3:.1f} us/step")
    dom = dominant_kernel(ctx)
    log(f"  dominant kernel {dom['avg_us']:.2f} us, {dom['GBps']:.0f} GB/s")
    extra = {}
    if not args.no_extra:
        for M in (4, 16):
            log(f"decode M={M}")
            extra[f"decode_M{M}"] = decode_bench(ctx, M, args.steps, args.warmup)
        # the same step with fp32 activations, the reference model's own dtype
        log("decode M=1, fp32 activations")
        extra["decode_M1_f32x"] = decode_bench(ctx, 1, args.steps, args.warmup, xdtype=torch.float32)
        log("single 4096x4096 GEMV")
        extra["gemv_4096_f16x"] = decode_bench(ctx, 1, args.steps, args.warmup, shapes=[(4096, 4096)])
        extra["gemv_4096_f32x"] = decode_bench(ctx, 1, args.steps, args.warmup, shapes=[(4096, 4096)],
                                               xdtype=torch.float32)
        extra["gemv_4096_grouped4"] = gemv_grouped4_bench(ctx)
        log("other kernels reading the GEMV's bytes (reference points)")
        extra["stream_floor"] = stream_floor_bench(ctx)
        log("prefill GEMM")
        extra["prefill"] = [prefill_bench(ctx, M) for M in (512, 2048, 8192)]
        # the reference model's own activations are fp32: staged as a scaled fp16 plane
        extra["prefill_other_x"] = [prefill_bench(ctx, 2048, xdtype=dt)
                                    for dt in (ctx.torch.bfloat16, ctx.torch.float32)]
        # fp32 outputs (the reference returns fp32), with fp16 and fp32 activations
        f32 = ctx.torch.float32
        extra["prefill_fp32_y"] = [prefill_bench(ctx, M, xdtype=xd, ydtype=f32)
                                   for M in (512, 2048) for xd in (ctx.torch.float16, f32)]
        log("mid-sized M (whole calls, weights rotating)")
        extra["mid_m"] = [midm_bench(ctx, M, N, fmt) for fmt in ("int8", "int8-dyn") for M in (64, 128, 256)
                          for N in (4096, 12288)]
        log("lm_head and its greedy token")
        extra["lm_head_greedy"] = lm_head_greedy_bench(ctx)
        log("sampling step over the lm_head logits (temperature, top-k, top-p)")
        extra["sample"] = sample_bench(ctx)
        log("device-resident decode (toy decoder)")
        extra["device_state"] = device_state_bench(ctx)
        log("device-resident decode, hybrid layer pattern at the checkpoint's sizes")
        extra["device_state_hybrid"] = device_state_hybrid_both(ctx)
        log("int8-dyn")
        extra["w8a8"] = [w8a8_bench(ctx, M, N) for M in (1, 128, 512, 2048) for N in (4096, 12288)]
        log("int8-dyn, per-token symmetric activations (opt-in)")
        extra["w8a8_token"] = [w8a8_bench(ctx, M, N, token=True) for M in (1, 128, 2048) for N in (4096, 12288)]
        log("vendor GEMMs at the same shapes (reference points)")
        extra["vendor_gemm"] = vendor_gemm_bench(ctx)
        torch.cuda.empty_cache()
        log("36-layer linear stack")
        extra["stack"] = stack_bench(ctx)
        log("36-layer linear stack, layers reading the same input fused")
        extra["stack_fused"] = stack_bench(ctx, fused=True)
        log("36-layer linear stack, fused, independent pairs grouped")
        extra["stack_grouped"] = stack_bench(ctx, grouped=True)
        log("decode step of the real checkpoint's shapes (hidden 2560, FFN 9728), fused and grouped")
        extra["stack_checkpoint_grouped"] = stack_bench(ctx, grouped=True, H=2560, F=9728)
        log("the same step with fp32 activations, the reference model's own dtype")
        extra["stack_checkpoint_grouped_f32x"] = stack_bench(ctx, grouped=True, H=2560, F=9728, xdtype=torch.float32)
        log("the same step in int8-dyn mode (DynamicInt8Linear), fused and grouped, fp16 and fp32 activations")
        extra["stack_checkpoint_w8a8"] = {xd: stack_bench(ctx, grouped=True, H=2560, F=9728, w8a8=True,
                                                          xdtype=getattr(torch, xd)) for xd in ("float16", "float32")}
        torch.cuda.empty_cache()

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_budget)

    pre2048 = next((p for p in extra.get("prefill", []) if p["M"] == 2048), None)

    def gemv_4096(key):  # the single 4096x4096 GEMV at M=1 (the metric's quoted shape)
        r = extra.get(key)
        return None if r is None else {"us": round(r["ms_per_step"] * 1e3, 3), "GBps": round(r["GBps"], 1),
                                       "hbm_frac": round(r["hbm_frac"], 4)}

    line = {
        "metric": METRIC,
        "value": round(head["GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (random N(0,0.02) weights quantized per channel, N(0,1) activations)",
        "config": {
            "workload": "int8 weight-only decode step at M=1: fused QKV 6144x4096 + gate+up 24576x4096 + "
                        "down 4096x12288, fp16 activations and outputs, weights rotating over "
                        f"{head['weight_copies']} copies",
            "hbm_frac": round(head["hbm_frac"], 4),
            "prefill_M2048_TFLOPs": None if pre2048 is None else round(pre2048["TFLOPs"], 1),
            "prefill_M2048_mfma_frac": None if pre2048 is None else round(pre2048["mfma_frac"], 4),
            "gemv_4096x4096_M1_f16x": gemv_4096("gemv_4096_f16x"),
            "gemv_4096x4096_M1_f32x": gemv_4096("gemv_4096_f32x"),
            # four independent 4096x4096 projections in one grouped launch (fp16 x)
            "gemv_4096x4096_M1_grouped4": None if "gemv_4096_grouped4" not in extra else {
                "us_per_projection": round(extra["gemv_4096_grouped4"]["us_per_projection"], 3),
                "GBps": round(extra["gemv_4096_grouped4"]["GBps"], 1),
                "hbm_frac": round(extra["gemv_4096_grouped4"]["hbm_frac"], 4)},
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(dom["GBps"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles(),
            "kernel": dom["kernel"],
            "avg_us": round(dom["avg_us"], 3),
            "bytes_per_launch": dom["bytes_per_launch"],
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
