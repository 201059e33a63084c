"""Generate the golden fixtures in this directory (run once, commit the .npz).

The expected values come from torch's own CPU operators, not from the build's
oracle and not from importing the reference package:

* quantize_per_channel.npz - the expression of spikingbrain_cpu/quant.py:25-29
  evaluated by torch CPU ops (abs/amax/clamp/div/round), including an all-zero
  row, a row of exact .5 ties and bf16 inputs (loader.py passes bf16 weights).
* int8_linear.npz - Int8Linear.forward's block loop (quant.py:47-52:
  128-row blocks, fp32 sgemm, cat, then * scale) evaluated by torch CPU.
* int8_dyn.npz - torch.ops.quantized.linear_dynamic (fbgemm), the operator
  DynamicInt8Linear.forward calls (quant.py:60-65), on seeded inputs with 1 %
  outlier channels x20, an all-zero input, a tiny-range input, one-signed
  inputs and a bias.

* int8_dyn_token.npz - the opt-in per-token symmetric W8A8 (see
  gen_int8_dyn_token), torch CPU ops only.

Usage: python tests/golden/make_golden.py [fixture names]
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def torch_quantize(w: torch.Tensor):
    w = w.float()
    scale = w.abs().amax(dim=1).clamp(min=1e-8) / 127.0
    q = torch.round(w / scale[:, None]).clamp(-127, 127).to(torch.int8)
    return q, scale


def torch_int8_forward(x: torch.Tensor, q: torch.Tensor, scale: torch.Tensor, block: int = 128):
    x2 = x.reshape(-1, x.shape[-1]).float()
    parts = [x2 @ q[lo:lo + block].float().t() for lo in range(0, q.shape[0], block)]
    return torch.cat(parts, -1) * scale


def gen_quantize(out: dict):
    g = torch.Generator().manual_seed(100)
    w = torch.randn(64, 256, generator=g) * 0.02
    w[3] = 0.0
    # row 5: scale is exactly 2**-7, every other entry sits on an exact .5 tie
    s = 2.0 ** -7
    j = torch.arange(-127, 127, dtype=torch.float32)  # j + 0.5 in [-126.5, 126.5]
    row = torch.empty(256)
    row[0] = 127 * s
    row[1:255] = (j + 0.5) * s
    row[255] = 2.5 * s
    w[5] = row
    w[7] = -w[7].abs()  # one-signed row
    q, sc = torch_quantize(w)
    out["f32_w"], out["f32_q"], out["f32_scale"] = w.numpy(), q.numpy(), sc.numpy()
    wb = (torch.randn(32, 128, generator=g) * 0.02).to(torch.bfloat16)
    q, sc = torch_quantize(wb)
    # bf16 stored as its raw bits (numpy has no bf16)
    out["bf16_w_bits"] = wb.view(torch.int16).numpy()
    out["bf16_q"], out["bf16_scale"] = q.numpy(), sc.numpy()


def gen_int8_linear(out: dict):
    cases = [(1, 4, 4096), (3, 64, 1024), (17, 128, 512), (1, 1024, 128), (3, 96, 256), (17, 200, 96)]
    for i, (M, N, K) in enumerate(cases):
        g = torch.Generator().manual_seed(200 + i)
        w = torch.randn(N, K, generator=g) * 0.02
        x = torch.randn(M, K, generator=g)
        q, sc = torch_quantize(w)
        y = torch_int8_forward(x, q, sc)
        out[f"c{i}_x"], out[f"c{i}_q"], out[f"c{i}_scale"], out[f"c{i}_y"] = x.numpy(), q.numpy(), sc.numpy(), y.numpy()
    out["cases"] = np.array(cases, dtype=np.int64)


def _dyn(x, q, sc, bias=None):
    qw = torch._make_per_channel_quantized_tensor(q, sc.double(), torch.zeros_like(sc, dtype=torch.long), 0)
    packed = torch.ops.quantized.linear_prepack(qw, bias)
    return torch.ops.quantized.linear_dynamic(x.contiguous(), packed)


def gen_int8_dyn(out: dict):
    cases = []
    for i, M in enumerate((1, 5, 33)):
        cases.append(("outliers", M, 64, 4096, 300 + i))
    cases += [("zeros", 3, 16, 256, 310), ("tiny", 4, 16, 256, 311), ("positive", 4, 16, 256, 312),
              ("negative", 4, 16, 256, 313), ("bias", 6, 40, 512, 314), ("tail", 7, 13, 200, 315)]
    names = []
    for i, (kind, M, N, K, seed) in enumerate(cases):
        g = torch.Generator().manual_seed(seed)
        w = torch.randn(N, K, generator=g) * 0.02
        x = torch.randn(M, K, generator=g)
        bias = None
        if kind == "outliers":
            idx = torch.randperm(K, generator=g)[: K // 100]
            x[:, idx] *= 20
        elif kind == "zeros":
            x.zero_()
        elif kind == "tiny":
            x *= 1e-6
        elif kind == "positive":
            x = x.abs() + 1.0
        elif kind == "negative":
            x = -x.abs() - 1.0
        elif kind == "bias":
            bias = torch.randn(N, generator=g)
        q, sc = torch_quantize(w)
        y = _dyn(x, q, sc, bias)
        out[f"c{i}_x"], out[f"c{i}_q"], out[f"c{i}_scale"], out[f"c{i}_y"] = x.numpy(), q.numpy(), sc.numpy(), y.numpy()
        if bias is not None:
            out[f"c{i}_bias"] = bias.numpy()
        names.append(kind)
    out["kinds"] = np.array(names)


def gen_int8_dyn_token(out: dict):
    """Per-token symmetric W8A8 (the opt-in granularity; no reference operator
    exists): rows quantized by the quant.py:25-29 expression in torch ops, the
    int32 product by torch._int_mm, y = fp32(acc) * fp32(s_t * s_w) in torch
    fp32.  No bias here: its fused multiply-add has no exact torch CPU op."""
    cases = [(1, 64, 4096), (5, 64, 4096), (33, 64, 1024)]
    for i, (M, N, K) in enumerate(cases):
        g = torch.Generator().manual_seed(400 + i)
        w = torch.randn(N, K, generator=g) * 0.02
        x = torch.randn(M, K, generator=g)
        idx = torch.randperm(K, generator=g)[: K // 100]
        x[:, idx] *= 20
        q, sc = torch_quantize(w)
        xq, st = torch_quantize(x)
        xp = torch.zeros(max(M, 17), K, dtype=torch.int8)  # _int_mm wants at least 17 rows
        xp[:M] = xq
        acc = torch._int_mm(xp, q.t().contiguous())[:M]
        y = acc.float() * (st[:, None] * sc[None, :])
        out[f"c{i}_x"], out[f"c{i}_q"], out[f"c{i}_scale"] = x.numpy(), q.numpy(), sc.numpy()
        out[f"c{i}_st"], out[f"c{i}_xq"], out[f"c{i}_acc"], out[f"c{i}_y"] = st.numpy(), xq.numpy(), acc.numpy(), y.numpy()
    out["cases"] = np.array(cases, dtype=np.int64)


GENERATORS = (("quantize_per_channel", gen_quantize), ("int8_linear", gen_int8_linear), ("int8_dyn", gen_int8_dyn),
              ("int8_dyn_token", gen_int8_dyn_token))


def main(names=None):
    for name, fn in GENERATORS:
        if names and name not in names:
            continue
        out: dict = {}
        fn(out)
        np.savez_compressed(HERE / f"{name}.npz", **out)
        print(name, sum(v.nbytes for v in out.values()), "bytes raw")


if __name__ == "__main__":
    import sys

    main(sys.argv[1:])
