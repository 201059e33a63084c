"""CPU baseline timing of the reference path (TEST/BENCH INFRASTRUCTURE ONLY).

Used only by bench.py's cpu_baseline leg.  The reference's own files are not
shipped with this package, so this restates, with torch CPU operators, what
the reference executes (paths relative to the reference repository):

* int8:     Int8Linear.forward, quant.py:46-53 - 128-row blocks dequantized to
            fp32, fp32 sgemm per block, torch.cat, then * scale.
* int8-dyn: DynamicInt8Linear.forward, quant.py:57-66 - fbgemm prepack of the
            per-channel qint8 weight, then torch.ops.quantized.linear_dynamic.
"""
from __future__ import annotations

import os
import platform
import time

import numpy as np
import torch


def int8_forward(x2: torch.Tensor, qweight: torch.Tensor, scale: torch.Tensor, block: int = 128) -> torch.Tensor:
    parts = [x2 @ qweight[lo:lo + block].float().t() for lo in range(0, qweight.shape[0], block)]
    return torch.cat(parts, -1) * scale


def dyn_prepack(q: torch.Tensor, scale: torch.Tensor):
    qw = torch._make_per_channel_quantized_tensor(q, scale.double(), torch.zeros_like(scale, dtype=torch.long), 0)
    return torch.ops.quantized.linear_prepack(qw, None)


def dyn_forward(x2: torch.Tensor, packed) -> torch.Tensor:
    return torch.ops.quantized.linear_dynamic(x2.contiguous(), packed)


def cpu_info() -> dict:
    """Host CPU model, torch's CPU capability, and the CPU share this process
    may use: the affinity mask and the cgroup quota (cpu.max), which can be
    smaller than the mask (then more threads than the quota only queue)."""
    model = platform.processor()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()
        quota = None if q == "max" else round(int(q) / int(period), 2)
    except (OSError, ValueError):
        pass
    smt = None
    try:
        smt = open("/sys/devices/system/cpu/smt/active").read().strip() == "1"
    except OSError:
        pass
    return {"cpu": model, "capability": torch.backends.cpu.get_cpu_capability(), "torch": torch.__version__,
            "host_threads": len(os.sched_getaffinity(0)), "cgroup_cpu_quota": quota, "smt_active": smt,
            "os_cpu_count": os.cpu_count()}


def time_calls(fn, budget_s: float, min_reps: int = 2) -> float:
    """Median seconds per call over repetitions filling about budget_s."""
    fn()  # warm-up
    times = []
    start = time.perf_counter()
    while len(times) < min_reps or (time.perf_counter() - start) < budget_s:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= 1000:
            break
    return float(np.median(times))


def _with_threads(threads: int, fn):
    old = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        return fn()
    finally:
        torch.set_num_threads(old)


def _quantized(N: int, K: int, g: torch.Generator):
    """N(0, 0.02) weights quantized as quant.py:25-29 does."""
    w = torch.randn(N, K, generator=g) * 0.02
    s = w.abs().amax(dim=1).clamp(min=1e-8) / 127.0
    q = torch.round(w / s[:, None]).clamp(-127, 127).to(torch.int8)
    return q, s


def decode_step_baseline(shapes, M: int, threads: int, budget_s: float, seed: int = 0, fmt: str = "int8") -> dict:
    """Time one pass of the int8 weight-only forward (fmt "int8", quant.py:46-53)
    or of fbgemm's dynamic linear (fmt "int8-dyn", quant.py:60-65) over
    `shapes` [(N, K)] at batch M on `threads` host threads; returns seconds
    per step and the algorithmic bytes (N*K + 4N + M*K*2 + M*N*2, the GPU
    bench's accounting)."""
    def run():
        g = torch.Generator().manual_seed(seed)
        layers = []
        nbytes = 0
        for N, K in shapes:
            q, s = _quantized(N, K, g)
            x = torch.randn(M, K, generator=g).half().float()
            layers.append((x, dyn_prepack(q, s) if fmt == "int8-dyn" else (q, s)))
            nbytes += N * K + 4 * N + M * K * 2 + M * N * 2

        def step():
            for x, w in layers:
                if fmt == "int8-dyn":
                    dyn_forward(x, w)
                else:
                    int8_forward(x, *w)

        return {"seconds_per_step": time_calls(step, budget_s), "bytes_per_step": nbytes, "threads": threads,
                "fmt": fmt}

    return _with_threads(threads, run)


def prefill_baseline(M: int, N: int, K: int, threads: int, budget_s: float, fmt: str = "int8", seed: int = 0) -> dict:
    """Time the int8 weight-only forward (quant.py:46-53) or fbgemm's dynamic
    linear (quant.py:60-65) at M x N x K on `threads` host threads; returns
    seconds per call and TFLOP/s (2*M*N*K)."""
    def run():
        g = torch.Generator().manual_seed(seed)
        q, s = _quantized(N, K, g)
        x = torch.randn(M, K, generator=g).half().float()
        w = dyn_prepack(q, s) if fmt == "int8-dyn" else None
        fn = (lambda: dyn_forward(x, w)) if fmt == "int8-dyn" else (lambda: int8_forward(x, q, s))
        sec = time_calls(fn, budget_s, min_reps=2)
        return {"M": M, "N": N, "K": K, "fmt": fmt, "threads": threads, "seconds": sec,
                "TFLOPs": 2.0 * M * N * K / sec / 1e12}

    return _with_threads(threads, run)
