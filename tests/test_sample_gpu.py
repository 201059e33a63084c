"""The engine's sampling step on the GPU (sbq_sample_rows, sbq.quant.sample_tokens)
against the oracle's restatement of engine.py:29-42 (paths relative to the
reference repository), with the same uniform for the draw.

The kernel finds the top-k value and the top-p boundary by radix selection
and sums probabilities in 2^-40 fixed point; the oracle sorts and sums in
float64.  So a token may differ only where its interval of the kept mass
comes within 2e-6 of the uniform's point, for top_p or 2e-6 beside it (a
draw or a kept-set boundary that close), or where tokens of equal fp32 probability
meet the top-p boundary: engine.py:38 sorts with probs.sort(descending=True),
which leaves the order of equal values open; the oracle takes them in index
order, the kernel in the order of z (larger first), and both are the
reference's rule.  Every other token must be equal, and the count of
boundary cases is checked to stay small.
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


def _probs_ties_by_z(x, T, k, p):
    """The oracle's kept probabilities with tokens of equal fp32 probability
    taken in the order of z (larger first, then index) instead of index order
    when the top-p rule walks the sorted probabilities (engine.py:38-40)."""
    pf = oracle.sample_probs(x, T, k, 1.0)
    if not 0 < p < 1:
        return pf
    z = (np.asarray(x, np.float32) / np.float32(T)).astype(np.float32)
    order = np.lexsort((np.arange(z.size), -z, -pf))
    sp = pf[order]
    keep = (np.cumsum(sp.astype(np.float64)).astype(np.float32) - sp) < np.float32(p)
    kept = np.zeros_like(pf)
    kept[order] = sp * keep
    return kept


def _token_ties_by_z(x, T, k, p, u):
    """The draw from _probs_ties_by_z, as oracle.sample_token draws."""
    c = np.cumsum(_probs_ties_by_z(x, T, k, p).astype(np.float64))
    return int(np.searchsorted(c, u * c[-1], side="right"))


def _near_draw(probs, u, tok):
    """tok is kept and its interval of the cumulative kept mass comes within
    DELTA (of the kept mass) of the uniform's point u."""
    if not 0 <= tok < probs.size or probs[tok] <= 0:
        return False
    c = np.cumsum(probs.astype(np.float64))
    lo = c[tok - 1] if tok else 0.0
    return lo <= (u + DELTA) * c[-1] and c[tok] > (u - DELTA) * c[-1]


def _accept(x, T, k, p, u, tok):
    """The oracle's token, and whether `tok` is acceptable: equal to it, or a
    kept token whose interval comes within 2e-6 of the uniform's point, for
    top_p itself or 2e-6 beside it, with equal probabilities at the top-p
    boundary in index or in z order."""
    want = oracle.sample_token(x, T, k, p, u)
    if tok == want:
        return want, True, False
    if want < 0 or T <= 0:
        return want, False, True
    for pp in ((p - DELTA, p, p + DELTA) if 0 < p < 1 else (p,)):
        for probs in (oracle.sample_probs(x, T, k, pp), _probs_ties_by_z(x, T, k, pp)):
            if _near_draw(probs, u, tok):
                return want, True, True
    return want, False, True


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


def test_sample_top_p_boundary_probability_ties(dev):
    """Two tokens whose z differ by one ulp (0.2 at index 0, 0.20000002 at
    index 2) have the same fp32 probability, and top_p cuts between them.
    The reference's sort leaves their order open (engine.py:38); the kernel
    keeps the larger z (index 2), the oracle's index order keeps index 0, and
    the draws from the two kept sets differ.  A regression case from a
    randomized run (V = 131183, T = 1, top_p 0.3)."""
    announce("sample top-p boundary probability ties")
    x = np.array([0.2, -1.0, 0.20000002, -0.7, -2.0, 1.5], np.float32)
    pf = oracle.sample_probs(x, 1.0, 0, 1.0)
    assert pf[0] == pf[2] and x[0] != x[2]  # equal fp32 probabilities of different z
    top_p = float(pf[5] + pf[0] / 2)  # keeps index 5 and one of the pair
    xd = torch.from_numpy(np.stack([x, x])).to(dev)
    for u0 in (0.01, 0.05, 0.15):
        assert oracle.sample_token(x, 1.0, 0, top_p, u0) == 0
        assert _token_ties_by_z(x, 1.0, 0, top_p, u0) == 2
        toks = _run(xd, 1.0, 0, top_p, torch.full((2,), u0, dtype=torch.float32, device=dev))
        assert toks.tolist() == [2, 2], toks
        assert _accept(x, 1.0, 0, top_p, u0, 2)[1]
    # the randomized run's rows (row 0 met such a pair at the boundary)
    big = torch.randn(5, 131183, generator=torch.Generator().manual_seed(160384264)) * 0.3
    us = torch.tensor([0.4574942, 0.953343, 0.942172, 0.29724792, 0.47127655], dtype=torch.float32)
    toks = _run(big.to(dev), 1.0, 0, 0.3, us.to(dev))
    xn = big.numpy()
    assert oracle.sample_token(xn[0], 1.0, 0, 0.3, float(us[0])) != _token_ties_by_z(xn[0], 1.0, 0, 0.3, float(us[0]))
    assert int(toks[0]) == _token_ties_by_z(xn[0], 1.0, 0, 0.3, float(us[0]))
    for r in range(5):
        assert _accept(xn[r], 1.0, 0, 0.3, float(us[r]), int(toks[r]))[1], r


def _mid_uniforms(x, T, k, p, idx):
    """For each token i in idx, the uniform at the middle of its interval of
    the oracle's kept distribution (None where the token is not kept)."""
    c = np.cumsum(oracle.sample_probs(x, T, k, p).astype(np.float64))
    out = []
    for i in idx:
        lo = c[i - 1] if i > 0 else 0.0
        out.append(None if c[i] == lo else float((lo + c[i]) / 2 / c[-1]))
    return out


@pytest.mark.parametrize("case", ["small", "topk", "slices"])
def test_sample_top_p_boundary_z_ties(dev, case):
    """Tokens of equal z at the top-p boundary: the reference's sort puts them
    together and its rule (cumsum - p < top_p, engine.py:38-40) keeps only
    the first of them that fit, in vocabulary order for a stable sort; the
    kernel keeps the same first n.  Cases: four ties in six tokens with top_p
    keeping two of them; the same with top-k's k-th value at the ties (top-k
    keeps all four, top-p two); twenty ties spread over the workgroup slices
    of a 50000-token row with top_p keeping seven.  Every tie top_p keeps is
    drawn by a uniform at the middle of its interval, the dropped ones never,
    and the tokens after them keep their intervals."""
    announce(f"sample top-p boundary z ties {case}")
    T = 1.0
    if case in ("small", "topk"):
        x = np.array([1.0, 0.3, 0.3, 2.0, 0.3, -1.0, 0.3], np.float32)
        ties, keep_n, k = [1, 2, 4, 6], 2, (3 if case == "topk" else 0)
    else:
        rng = np.random.default_rng(21)
        x = rng.standard_normal(50000).astype(np.float32)
        ties = [i * 2400 + 7 for i in range(20)]
        x[ties] = np.float32(1.25)
        keep_n, k = 7, 0
    full = oracle.sample_probs(x, T, k, 1.0)
    pt = float(full[ties[0]])
    above = float(full[full > pt].astype(np.float64).sum())
    top_p = above + (keep_n - 0.5) * pt
    kept = oracle.sample_probs(x, T, k, top_p)
    assert [i for i in ties if kept[i] > 0] == ties[:keep_n]
    others = [i for i in range(x.size) if kept[i] > 0 and i not in ties][:40]
    probe = ties + others
    us = _mid_uniforms(x, T, k, top_p, probe)
    xd = torch.from_numpy(x).reshape(1, -1).to(dev)
    for i, u0 in zip(probe, us):
        if u0 is None:
            continue
        tok = int(_run(xd, T, k, top_p, torch.tensor([u0], dtype=torch.float32, device=dev))[0])
        assert tok == i == oracle.sample_token(x, T, k, top_p, u0), (i, tok)
    drawn = {int(_run(xd, T, k, top_p, torch.tensor([u0], dtype=torch.float32, device=dev))[0])
             for u0 in np.linspace(0.0, 0.999, 97)}
    assert not drawn & set(ties[keep_n:]), drawn & set(ties[keep_n:])


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
