"""Time every prefill GEMM configuration of the fitted picker on one GPU.

For each shape (M, N, K) it prepares operands with the library (random
N(0, 0.02) weights quantized and packed on the GPU, N(0, 1) fp16
activations), runs each configuration of the picker's table through the
tuning harness (libsbq_tune.so, `make -C spikingbrain-cpu_amd tune`) in a
HIP graph of 4 back-to-back launches, interleaving the configurations over 4
rounds, and writes one JSON line per shape:

    {"f": "w8" | "w8a8", "M": .., "N": .., "K": .., "t": {"<id>": us, ...}}

(the GEMM alone, best of the rounds).  Every configuration's output is
checked against the library's own call first: bit-identical for int8-dyn,
within fp32 summation order for weight-only.

    python sweep.py --format w8a8 --out sweep_w8a8.jsonl            # the default 255 shapes
    python sweep.py --format w8 --shapes 2048x12288x4096,512x4096x4096
"""
from __future__ import annotations

import argparse
import ctypes
import json
import sys
import time
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

import torch  # noqa: E402

from sbq import quant  # noqa: E402

from fit import CONFIGS  # noqa: E402

P, I, L = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64


def default_shapes():
    """M = 192 .. 4096 by N = 2048 .. 24576 (18820: the fused hybrid group) at
    K = 4096, and by N = 2048 .. 8192 at K = 12288."""
    ms = [192, 256, 320, 384, 448, 512, 576, 640, 768, 896, 1024, 1280, 1536, 1792, 2048, 3072, 4096]
    shapes = [(m, n, 4096) for n in (2048, 3072, 4096, 5120, 6144, 8192, 10240, 12288, 16384, 18820, 24576) for m in ms]
    shapes += [(m, n, 12288) for n in (2048, 4096, 6144, 8192) for m in ms]
    return shapes


def load_harness():
    lib = ctypes.CDLL(str(HERE / "libsbq_tune.so"))
    lib.sbq_tune_gemm_w8.argtypes = [I, P, L, I, I, P, P, I, P, P, P]
    lib.sbq_tune_gemm_w8a8.argtypes = [I, P, I, I, P, P, P, I, P, P, P]
    lib.sbq_tune_rowsum_f16.argtypes = [P, L, I, I, P, P]
    lib.sbq_tune_pick.argtypes = [I, I, I, I]
    return lib


def graph(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def time_graph(g, launches, reps=5):
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * launches)


def sweep_shape(lib, fmt, M, N, K, dev):
    w8a8 = fmt == "w8a8"
    st = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    gen = torch.Generator(device=dev).manual_seed(1)
    q, s = quant.quantize_per_channel_gpu(torch.randn(N, K, generator=gen, device=dev) * 0.02)
    packed, colsum = quant.repack(q, with_colsum=True)
    del q
    x = torch.randn(M, K, generator=gen, device=dev).half()
    y = torch.empty(M, N, device=dev, dtype=torch.float16)
    if w8a8:
        ws = quant.w8a8_workspace(M, K, dev)
        ref = quant.linear_w8a8(x, packed, s, colsum, None, N, torch.float16, workspace=ws)
        # the W8A8 workspace from its first 256-byte boundary: 2048 bytes of
        # min/max partials, (s_x, zp) in 256 bytes, then the s8 rows (sbq_abi.hip)
        base = (ws.data_ptr() + 255) & ~255
        qp, xq = base + 2048, base + 2304

        def run(cfg):
            return lib.sbq_tune_gemm_w8a8(cfg, P(xq), M, K, packed.data_ptr(), s.data_ptr(), colsum.data_ptr(), N,
                                          y.data_ptr(), P(qp), st())
    else:
        ref = quant.linear_w8(x, packed, s, None, N, torch.float16)
        rsum = torch.empty(M, device=dev, dtype=torch.float32)
        assert lib.sbq_tune_rowsum_f16(x.data_ptr(), K, M, K, rsum.data_ptr(), st()) == 0

        def run(cfg):
            return lib.sbq_tune_gemm_w8(cfg, x.data_ptr(), K, M, K, packed.data_ptr(), s.data_ptr(), N, y.data_ptr(),
                                        rsum.data_ptr(), st())
    graphs = []
    for cfg in CONFIGS[fmt]:
        if run(cfg) != 0:
            torch.cuda.synchronize()
            continue
        torch.cuda.synchronize()
        ok = torch.equal(y, ref) if w8a8 else torch.allclose(y.float(), ref.float(), rtol=2e-3, atol=2e-3)
        if not ok:
            raise RuntimeError(f"configuration {cfg} differs from the library's output at M={M} N={N} K={K}")

        def body(cfg=cfg):
            for _ in range(4):
                run(cfg)
        graphs.append((cfg, graph(body)))
    times = {cfg: [] for cfg, _ in graphs}
    for _ in range(4):
        for cfg, g in graphs:
            times[cfg].append(time_graph(g, 4))
    return {"f": fmt, "M": M, "N": N, "K": K, "t": {str(c): min(v) for c, v in times.items()}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--format", choices=["w8", "w8a8"], required=True)
    ap.add_argument("--shapes", help="comma-separated MxNxK (default: the 255-shape grid)")
    ap.add_argument("--out", help="JSON lines file (default: stdout)")
    args = ap.parse_args()
    shapes = ([tuple(int(v) for v in t.split("x")) for t in args.shapes.split(",")] if args.shapes
              else default_shapes())
    dev = torch.device("cuda", 0)
    lib = load_harness()
    warm = torch.randn(4096, 4096, device=dev)  # bring the clocks up before the first shape
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.5:
        warm.mul_(1.0)
    out = open(args.out, "w") if args.out else sys.stdout
    for M, N, K in shapes:
        out.write(json.dumps(sweep_shape(lib, args.format, M, N, K, dev)) + "\n")
        out.flush()


if __name__ == "__main__":
    main()
