"""sbq_linear_w8a8_noalloc - the int8-dyn linear with no workspace, for callers
that cannot allocate - against sbq_linear_w8a8 (the entry point with a
workspace) on the same inputs: int32 accumulators and outputs bit-exact.

The no-allocation calls run back to back on one stream, sharing the
library's static per-GPU scratch, each followed by a smaller or different
input (the second call's quantized activations are shorter than the first's,
so stale bytes of the first would show); the largest input the scratch holds
is accepted, one row more is rejected before any launch."""
import numpy as np
import pytest
import torch

from conftest import announce
from sbq import _lib, quant

pytestmark = pytest.mark.gpu

# (M, N, K, x dtype): the tiled GEMM (min/max and quantize passes into the
# scratch), then smaller inputs through each path that uses the scratch
CASES = [
    (700, 1024, 4096, torch.float16),
    (40, 1024, 4096, torch.float16),    # smaller GEMM input
    (8, 1024, 4096, torch.float32),     # decode GEMV with the min/max pre-pass
    (1, 1024, 4096, torch.float32),     # decode GEMV reducing min/max itself (no scratch)
    (2048, 512, 4096, torch.bfloat16),  # the largest xq the scratch holds: 2048 * 4096 bytes
    (33, 130, 200, torch.float16),      # ragged K (Kp = 256) through the GEMM
    (3, 300, 200, torch.float16),       # ragged K, general GEMV
]


def _layer(N, K, seed, dev):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02
    b = torch.randn(N, generator=g) if seed % 2 else None
    return quant.DynamicInt8Linear(w.to(dev), None if b is None else b.to(dev))


def _x(M, K, dtype, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[: max(1, K // 100)]] *= 20
    return x.to(dtype).to(dev)


def test_noalloc_matches_workspace_entry_point(dev):
    layers, xs, refs = [], [], []
    for i, (M, N, K, dt) in enumerate(CASES):
        announce(f"noalloc reference M={M} N={N} K={K} x={dt}")
        lin = _layer(N, K, 10 + i, dev)
        x = _x(M, K, dt, 50 + i, dev)
        acc = torch.empty((M, N), dtype=torch.int32, device=dev)
        y = quant.linear_w8a8(x, lin.packed, lin.scale, lin.colsum, lin.bias, N, acc_out=acc)
        layers.append(lin)
        xs.append(x)
        refs.append((y, acc))
    torch.cuda.synchronize()
    outs = []
    announce("noalloc calls back to back")
    for (M, N, K, dt), lin, x in zip(CASES, layers, xs):
        y = torch.full((M, N), float("nan"), device=dev)
        acc = torch.full((M, N), -1, dtype=torch.int32, device=dev)
        quant.linear_w8a8_noalloc(x, lin.packed, lin.scale, lin.colsum, lin.bias, N, out=y, acc_out=acc)
        outs.append((y, acc))
    torch.cuda.synchronize()
    for (M, N, K, dt), (y, acc), (yr, accr) in zip(CASES, outs, refs):
        np.testing.assert_array_equal(acc.cpu().numpy(), accr.cpu().numpy(), err_msg=f"acc M={M} N={N} K={K}")
        np.testing.assert_array_equal(y.cpu().numpy(), yr.cpu().numpy(), err_msg=f"y M={M} N={N} K={K}")


def test_noalloc_second_call_smaller_fp16_out(dev):
    """Two calls in a row with fp16 outputs, the second smaller."""
    for M, N in ((512, 768), (64, 768)):
        announce(f"noalloc fp16 out M={M}")
        K = 4096
        lin = _layer(N, K, 3, dev)
        x = _x(M, K, torch.float16, 4 + M, dev)
        ref = quant.linear_w8a8(x, lin.packed, lin.scale, lin.colsum, lin.bias, N, torch.float16)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        quant.linear_w8a8_noalloc(x, lin.packed, lin.scale, lin.colsum, lin.bias, N, out=y)
        np.testing.assert_array_equal(y.cpu().numpy(), ref.cpu().numpy())


def test_noalloc_rejects_inputs_beyond_the_scratch(dev):
    announce("noalloc oversize rejection")
    K, N = 4096, 64
    M = _lib.SBQ_NOALLOC_XQ_BYTES // K + 1
    lin = _layer(N, K, 5, dev)
    x = torch.zeros((M, K), dtype=torch.float16, device=dev)
    y = torch.full((M, N), 7.0, device=dev)
    with pytest.raises(ValueError, match="workspace"):
        quant.linear_w8a8_noalloc(x, lin.packed, lin.scale, lin.colsum, None, N, out=y)
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())


def test_noalloc_graph_replays(dev):
    """No-allocation calls captured in a HIP graph: one eager call per case
    first (it looks the scratch up), then the calls captured back to back and
    the graph replayed three times with new activations written between
    replays; every replay's int32 accumulators and outputs equal
    sbq_linear_w8a8 (the workspace entry point) on the same inputs bit for
    bit."""
    cases = [(1, 1024, 4096, torch.float32), (8, 1024, 4096, torch.float16), (200, 768, 4096, torch.float16),
             (40, 512, 4096, torch.bfloat16)]
    layers, xs, ys, accs = [], [], [], []
    for i, (M, N, K, dt) in enumerate(cases):
        announce(f"noalloc graph warm-up M={M} N={N} K={K} x={dt}")
        layers.append(_layer(N, K, 30 + i, dev))
        xs.append(_x(M, K, dt, 60 + i, dev))
        ys.append(torch.empty((M, N), device=dev))
        accs.append(torch.empty((M, N), dtype=torch.int32, device=dev))
        quant.linear_w8a8_noalloc(xs[i], layers[i].packed, layers[i].scale, layers[i].colsum, layers[i].bias, N,
                                  out=ys[i], acc_out=accs[i])
    torch.cuda.synchronize()

    def body():
        for (M, N, K, dt), lin, x, y, acc in zip(cases, layers, xs, ys, accs):
            quant.linear_w8a8_noalloc(x, lin.packed, lin.scale, lin.colsum, lin.bias, N, out=y, acc_out=acc)

    announce("noalloc graph capture")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        body()
    for rep in range(3):
        announce(f"noalloc graph replay {rep}")
        for i, (M, N, K, dt) in enumerate(cases):
            xs[i].copy_(_x(M, K, dt, 100 * rep + i, dev))
            ys[i].fill_(float("nan"))
            accs[i].fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        for (M, N, K, dt), lin, x, y, acc in zip(cases, layers, xs, ys, accs):
            acc_ref = torch.empty((M, N), dtype=torch.int32, device=dev)
            y_ref = quant.linear_w8a8(x, lin.packed, lin.scale, lin.colsum, lin.bias, N, acc_out=acc_ref)
            np.testing.assert_array_equal(acc.cpu().numpy(), acc_ref.cpu().numpy(), err_msg=f"acc rep {rep} M={M}")
            np.testing.assert_array_equal(y.cpu().numpy(), y_ref.cpu().numpy(), err_msg=f"y rep {rep} M={M}")
    del g
