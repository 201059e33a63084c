"""The engine's sampling step on the GPU (sbq_sample_rows, sbq.quant.sample_tokens)
against the oracle's restatement of engine.py:29-42 (paths relative to the
reference repository), with the same uniform for the draw.

The kernel finds the top-k value and the top-p boundary by radix selection
and sums probabilities in 2^-40 fixed point; the oracle sorts and sums in
float64.  So a token may differ only where the oracle itself changes its
answer under a perturbation of 2e-6 of the uniform or of top_p (a draw or a
kept-set boundary that close); every other token must be equal, and the
count of boundary cases is checked to stay small.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import announce
from sbq import quant

pytestmark = pytest.mark.gpu

PARAMS = [  # (temperature, top_k, top_p): the engine's defaults first (engine.py:21-26)
    (0.7, 0, 0.9), (1.0, 50, 1.0), (0.7, 40, 0.8), (1.3, 0, 1.0), (0.9, 1, 1.0), (1.0, 0, 0.02),
    (0.6, 200000, 0.95), (1.0, 7, 0.5),
]
DELTA = 2e-6


def _accept(x, T, k, p, u, tok):
    """The oracle's token, and whether `tok` is acceptable: equal to it, or to
    the oracle's answer under a 2e-6 perturbation of u or top_p."""
    want = oracle.sample_token(x, T, k, p, u)
    if tok == want:
        return want, True, False
    alts = {oracle.sample_token(x, T, k, pp, uu) for uu in (max(u - DELTA, 0.0), u, min(u + DELTA, 1 - 1e-9))
            for pp in ((p - DELTA, p, p + DELTA) if 0 < p < 1 else (p,))}
    return want, tok in alts, True


def _run(logits, T, k, p, u):
    return quant.sample_tokens(logits, T, p, k, u=u).cpu().numpy()


@pytest.mark.parametrize("T,k,p", PARAMS)
def test_sample_vocab_rows_match_oracle(dev, T, k, p):
    """V = 151936 (the lm_head's vocabulary), two rows of different logit
    scales, 24 uniforms per row (the last ones at 0 and just below 1)."""
    announce(f"sample V=151936 T={T} k={k} p={p}")
    V = 151936
    g = torch.Generator().manual_seed(int(T * 100) + k % 1000 + int(p * 1000))
    x = torch.randn(2, V, generator=g) * torch.tensor([[2.5], [0.8]])
    xd = x.to(dev)
    xn = x.numpy()
    us = np.concatenate([np.random.default_rng(11).random(22), [0.0, 1 - 2 ** -24]]).astype(np.float32)
    boundary = 0
    for j, u0 in enumerate(us):
        u = torch.tensor([u0, us[(j + 7) % len(us)]], dtype=torch.float32, device=dev)
        toks = _run(xd, T, k, p, u)
        for r in range(2):
            want, ok, near = _accept(xn[r], T, k, p, float(u[r]), int(toks[r]))
            assert ok, (r, float(u[r]), int(toks[r]), want)
            boundary += near
    assert boundary <= 2, boundary


@pytest.mark.parametrize("V", [1, 2, 37, 1000, 4097, 70000])
def test_sample_small_and_ragged_vocab(dev, V):
    """Vocabularies from one token up, ragged against the 2048-token
    workgroup slices; three rows sampled in one call."""
    announce(f"sample small V={V}")
    g = torch.Generator().manual_seed(V)
    x = torch.randn(3, V, generator=g) * 3
    us = torch.tensor([0.1, 0.5, 0.93], dtype=torch.float32)
    for T, k, p in PARAMS[:4]:
        toks = _run(x.to(dev), T, k, p, us.to(dev))
        for r in range(3):
            want, ok, _ = _accept(x[r].numpy(), T, k, p, float(us[r]), int(toks[r]))
            assert ok, (V, T, k, p, r, int(toks[r]), want)


def test_sample_ties_greedy_and_invalid_rows(dev):
    """Ties at the k-th value are all kept; temperature 0 is the greedy token;
    a NaN or an infinite logit gives -1 (the reference raises); -inf logits
    are never drawn."""
    announce("sample ties / greedy / invalid rows")
    V = 5000
    x = torch.full((4, V), -3.0)
    x[0, [10, 20, 30, 40]] = 4.0             # four-way tie at the top, k = 2 keeps all four
    x[1] = torch.randn(V, generator=torch.Generator().manual_seed(3))
    x[1, 123] = float("nan")
    x[2] = torch.randn(V, generator=torch.Generator().manual_seed(4))
    x[2, 77] = float("inf")
    x[3] = torch.randn(V, generator=torch.Generator().manual_seed(5))
    x[3, ::2] = float("-inf")
    xd = x.to(dev)
    seen = set()
    for u0 in np.linspace(0.0, 0.999, 41):
        u = torch.full((4,), float(u0), device=dev)
        toks = _run(xd, 1.0, 2, 1.0, u)
        seen.add(int(toks[0]))
        assert int(toks[1]) == -1 and int(toks[2]) == -1
        assert int(toks[3]) % 2 == 1
        assert int(toks[0]) == oracle.sample_token(x[0].numpy(), 1.0, 2, 1.0, float(u0))
    assert seen == {10, 20, 30, 40}
    greedy = quant.sample_tokens(xd, 0.0).cpu()
    assert int(greedy[0]) == 10 and int(greedy[1]) == 123 and int(greedy[3]) == int(torch.argmax(x[3]))


def test_sample_strided_rows(dev):
    """Rows of a wider buffer (row stride above V) and one row viewed from a
    column (stride(0) below V): the same tokens as the contiguous copies."""
    announce("sample strided rows")
    V = 5000
    big = torch.randn(3, V + 37, generator=torch.Generator().manual_seed(12)).to(dev) * 2
    rows = big[:, :V]
    u = torch.tensor([0.2, 0.6, 0.9], dtype=torch.float32, device=dev)
    assert torch.equal(quant.sample_tokens(rows, 0.8, 0.9, 30, u=u), quant.sample_tokens(rows.contiguous(), 0.8, 0.9, 30, u=u))
    assert torch.equal(quant.greedy_tokens(rows), quant.greedy_tokens(rows.contiguous()))
    col = torch.randn(V, 1, generator=torch.Generator().manual_seed(13)).to(dev)
    one = col.t()  # [1, V], stride (1, 1)
    assert torch.equal(quant.sample_tokens(one, 1.0, 0.95, 0, u=u[:1]), quant.sample_tokens(one.contiguous(), 1.0, 0.95, 0, u=u[:1]))
    assert torch.equal(quant.greedy_tokens(one), quant.greedy_tokens(one.contiguous()))


def test_sample_drop_in_and_graph_replay(dev):
    """sbq.quant.sample(logits, params, generator) draws its uniform from the
    caller's CPU generator, as the engine passes one; sample_tokens captured
    in a HIP graph (logits and uniforms rewritten between replays) equals the
    eager calls."""
    announce("sample drop-in and graph replay")

    class Params:
        temperature, top_p, top_k = 0.7, 0.9, 0

    V = 151936
    x = (torch.randn(1, V, generator=torch.Generator().manual_seed(8)) * 2).to(dev)
    g1, g2 = torch.Generator().manual_seed(42), torch.Generator().manual_seed(42)
    for _ in range(5):
        tok = quant.sample(x[0], Params, g1)
        u = float(torch.rand((1,), generator=g2)[0])
        want, ok, _ = _accept(x[0].cpu().numpy(), 0.7, 0, 0.9, u, tok)
        assert ok, (tok, want)
    # graph capture with a workspace and device uniforms of its own
    M = 2
    logits = (torch.randn(M, V, generator=torch.Generator().manual_seed(9)) * 2).to(dev)
    u = torch.rand(M, generator=torch.Generator().manual_seed(10)).to(dev)
    ws = quant.sample_workspace(M, V, dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        quant.sample_tokens(logits, 0.8, 0.9, 40, u=u, workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = quant.sample_tokens(logits, 0.8, 0.9, 40, u=u, workspace=ws)
    for rep in range(4):
        logits.copy_((torch.randn(M, V, generator=torch.Generator().manual_seed(20 + rep)) * 2).to(dev))
        u.copy_(torch.rand(M, generator=torch.Generator().manual_seed(30 + rep)).to(dev))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = quant.sample_tokens(logits, 0.8, 0.9, 40, u=u, workspace=quant.sample_workspace(M, V, dev))
        assert torch.equal(out, eager), rep
    del graph
