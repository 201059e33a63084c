"""Pins the CPU oracle (oracle/) before the GPU results are compared with it.

Each oracle function is checked against something it does not share code
with: torch's CPU operators evaluating the reference expressions
(spikingbrain_cpu/quant.py:25-29, :47-52), the live fbgemm operator
torch.ops.quantized.linear_dynamic (quant.py:65), the committed golden
fixtures, and closed forms (integer-valued activations make every dot product
exact).  Planted mistakes - in copies of the oracle's arithmetic, on the CPU -
must be caught by the same checks.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle

GOLD = Path(__file__).resolve().parent / "golden"


def torch_quantize(w):
    w = torch.as_tensor(w).float()
    scale = w.abs().amax(dim=1).clamp(min=1e-8) / 127.0
    q = torch.round(w / scale[:, None]).clamp(-127, 127).to(torch.int8)
    return q.numpy(), scale.numpy()


def torch_dyn(x, q, scale, bias=None):
    qw = torch._make_per_channel_quantized_tensor(torch.as_tensor(q), torch.as_tensor(scale).double(),
                                                  torch.zeros(len(scale), dtype=torch.long), 0)
    packed = torch.ops.quantized.linear_prepack(qw, None if bias is None else torch.as_tensor(bias))
    return torch.ops.quantized.linear_dynamic(torch.as_tensor(x).contiguous(), packed).numpy()


def rand_x(M, K, seed, outliers=True, scale=1.0):
    g = np.random.default_rng(seed)
    x = (g.standard_normal((M, K)) * scale).astype(np.float32)
    if outliers:
        idx = g.permutation(K)[: max(1, K // 100)]
        x[:, idx] *= 20
    return x


def rand_q(N, K, seed):
    g = np.random.default_rng(seed)
    return oracle.quantize_per_channel((g.standard_normal((N, K)) * 0.02).astype(np.float32))


# ---------------------------------------------------------------------------
# quantize_per_channel (quant.py:25-29)
# ---------------------------------------------------------------------------
def test_quantize_matches_golden_fixture():
    d = np.load(GOLD / "quantize_per_channel.npz")
    for impl in (oracle.quantize_per_channel, oracle.quantize_per_channel_c):
        q, s = impl(d["f32_w"])
        np.testing.assert_array_equal(q, d["f32_q"])
        np.testing.assert_array_equal(s.view(np.uint32), d["f32_scale"].view(np.uint32))
        wb = torch.from_numpy(d["bf16_w_bits"]).view(torch.bfloat16).float().numpy()
        q, s = impl(wb)
        np.testing.assert_array_equal(q, d["bf16_q"])
        np.testing.assert_array_equal(s.view(np.uint32), d["bf16_scale"].view(np.uint32))


def test_quantize_fixture_has_ties_and_zero_row():
    d = np.load(GOLD / "quantize_per_channel.npz")
    w, s = d["f32_w"][5], d["f32_scale"][5]
    t = w / s
    ties = np.abs(t - np.trunc(t)) == 0.5
    assert ties.sum() >= 200
    # round-half-even on every tie
    assert np.all(d["f32_q"][5][ties] % 2 == 0)
    assert np.all(d["f32_q"][3] == 0) and d["f32_scale"][3] == np.float32(np.float32(1e-8) / np.float32(127))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_quantize_matches_torch_live(seed):
    g = np.random.default_rng(seed)
    w = (g.standard_normal((257, 300)) * 0.02).astype(np.float32)
    w[0] = 0
    qt, st = torch_quantize(w)
    for impl in (oracle.quantize_per_channel, oracle.quantize_per_channel_c):
        q, s = impl(w)
        np.testing.assert_array_equal(q, qt)
        np.testing.assert_array_equal(s, st)


def test_quantize_mutants_are_caught():
    """Plausible slips: the scale formed by reciprocal multiply instead of IEEE
    division, and round-half-away-from-zero instead of half-even."""
    d = np.load(GOLD / "quantize_per_channel.npz")
    w = d["f32_w"]
    s = d["f32_scale"]
    away = np.clip(np.sign(w / s[:, None]) * np.floor(np.abs(w / s[:, None]) + 0.5), -127, 127).astype(np.int8)
    assert not np.array_equal(away, d["f32_q"])
    big = (np.random.default_rng(9).standard_normal((4096, 512)) * 0.02).astype(np.float32)
    _, st = torch_quantize(big)
    amax = np.abs(big).max(axis=1)
    s_recip = (amax * (np.float32(1) / np.float32(127))).astype(np.float32)
    assert not np.array_equal(s_recip, st)
    _, so = oracle.quantize_per_channel_c(big)
    np.testing.assert_array_equal(so, st)


# ---------------------------------------------------------------------------
# Int8Linear.forward (quant.py:41-53)
# ---------------------------------------------------------------------------
def test_int8_linear_golden_fixture():
    d = np.load(GOLD / "int8_linear.npz")
    for i in range(len(d["cases"])):
        x, q, s, y = d[f"c{i}_x"], d[f"c{i}_q"], d[f"c{i}_scale"], d[f"c{i}_y"]
        assert oracle.rel_l2(oracle.int8_linear(x, q, s), y) < 1e-6
        assert oracle.rel_l2(oracle.int8_linear_c(x, q, s), y) < 1e-6


def test_int8_linear_exact_on_integer_activations():
    """With small-integer x every dot product is an exact integer, so the
    result is fixed bit for bit: fp32(sum) * scale, scale applied last."""
    g = np.random.default_rng(4)
    q, s = rand_q(96, 512, 5)
    x = g.integers(-3, 4, size=(9, 512)).astype(np.float32)
    exact = (x.astype(np.int64) @ q.astype(np.int64).T).astype(np.float32) * s
    np.testing.assert_array_equal(oracle.int8_linear(x, q, s), exact)
    np.testing.assert_array_equal(oracle.int8_linear_c(x, q, s), exact)
    # the torch block loop of the reference agrees exactly too
    yt = (torch.from_numpy(x) @ torch.from_numpy(q).float().t() * torch.from_numpy(s)).numpy()
    np.testing.assert_array_equal(yt, exact)
    # planted mistake: scale folded into the weights before the sum
    folded = (x @ (q.astype(np.float32) * s[:, None]).T).astype(np.float32)
    assert not np.array_equal(folded, exact)


def test_int8_linear_transposed_operand_mutant_caught():
    q, s = rand_q(256, 256, 7)
    x = rand_x(4, 256, 8, outliers=False)
    good = oracle.int8_linear(x, q, s)
    bad = (x.astype(np.float64) @ q.astype(np.float64)).astype(np.float32) * s
    assert oracle.rel_l2(bad, good) > 0.5


def test_int8_linear_bias_and_batch_shape():
    q, s = rand_q(40, 128, 11)
    x = rand_x(6, 128, 12, outliers=False).reshape(2, 3, 128)
    b = np.random.default_rng(13).standard_normal(40).astype(np.float32)
    y = oracle.int8_linear(x, q, s, b)
    assert y.shape == (2, 3, 40)
    ref = torch.from_numpy(x.reshape(6, 128)) @ torch.from_numpy(q).float().t() * torch.from_numpy(s) + torch.from_numpy(b)
    assert oracle.rel_l2(y.reshape(6, 40), ref.numpy()) < 1e-6


# ---------------------------------------------------------------------------
# int8-dyn (fbgemm dynamic linear, quant.py:63-66)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("M,N,K,seed", [(1, 512, 4096, 0), (128, 512, 4096, 1), (2048, 64, 4096, 2), (5, 4, 4096, 3),
                                        (3, 64, 2560, 4), (7, 13, 256, 5), (33, 1024, 256, 6), (17, 128, 96, 7)])
def test_dyn_bit_exact_vs_fbgemm(M, N, K, seed):
    x = rand_x(M, K, seed)
    q, s = rand_q(N, K, seed + 100)
    np.testing.assert_array_equal(oracle.dyn_linear(x, q, s), torch_dyn(x, q, s))


@pytest.mark.parametrize("kind", ["zeros", "tiny", "tinypos", "tinyneg", "positive", "negative", "const", "huge"])
def test_dyn_edge_inputs_bit_exact(kind):
    g = np.random.default_rng(42)
    x = g.standard_normal((4, 512)).astype(np.float32)
    x = {"zeros": x * 0, "tiny": x * 1e-6, "tinypos": np.abs(x) * 1e-6, "tinyneg": -np.abs(x) * 1e-6,
         "positive": np.abs(x) + 1, "negative": -np.abs(x) - 1, "const": np.full_like(x, 0.37),
         "huge": x * 3e4}[kind].astype(np.float32)
    q, s = rand_q(24, 512, 43)
    np.testing.assert_array_equal(oracle.dyn_linear(x, q, s), torch_dyn(x, q, s))


def test_dyn_bias_is_fused_like_fbgemm():
    x = rand_x(64, 512, 50)
    q, s = rand_q(96, 512, 51)
    b = np.random.default_rng(52).standard_normal(96).astype(np.float32)
    ref = torch_dyn(x, q, s, b)
    np.testing.assert_array_equal(oracle.dyn_linear(x, q, s, b), ref)
    # planted mistake: bias added after a separately rounded product
    sep = (oracle.dyn_linear(x, q, s) + b).astype(np.float32)
    assert not np.array_equal(sep, ref)


def test_dyn_golden_fixture():
    d = np.load(GOLD / "int8_dyn.npz")
    for i, kind in enumerate(d["kinds"]):
        bias = d[f"c{i}_bias"] if f"c{i}_bias" in d else None
        y = oracle.dyn_linear(d[f"c{i}_x"], d[f"c{i}_q"], d[f"c{i}_scale"], bias)
        np.testing.assert_array_equal(y, d[f"c{i}_y"], err_msg=str(kind))


def test_dyn_c_and_numpy_layers_agree():
    x = rand_x(9, 700, 60)
    q, s = rand_q(33, 700, 61)
    b = np.random.default_rng(62).standard_normal(33).astype(np.float32)
    yn, info_n = oracle.dyn_linear(x, q, s, b, return_intermediates=True)
    yc, info_c = oracle.dyn_linear_c(x, q, s, b)
    np.testing.assert_array_equal(yn, yc)
    np.testing.assert_array_equal(info_n["xq"], info_c["xq"])
    np.testing.assert_array_equal(info_n["acc"], info_c["acc"])
    assert (info_n["scale"], info_n["zero_point"]) == (info_c["scale"], info_c["zero_point"])


def test_dyn_mutants_are_caught():
    """Quantizing as rint(x*inv)+zp (two roundings) and epilogue (acc*s_x)*s_w
    are the plausible misreadings of fbgemm; both must disagree with it."""
    x = rand_x(2048, 1024, 70)
    q, s = rand_q(64, 1024, 71)
    ref = torch_dyn(x, q, s)
    _, info = oracle.dyn_linear(x, q, s, return_intermediates=True)
    sx, zp = info["scale"], info["zero_point"]
    inv = np.float32(1) / np.float32(sx)
    xq_bad = np.clip(np.rint(x * inv) + zp, 0, 255)
    acc_bad = ((xq_bad.astype(np.float64) - zp) @ q.astype(np.float64).T).astype(np.int32)
    y_bad = acc_bad.astype(np.float32) * (np.float32(sx) * s)
    assert not np.array_equal(y_bad, ref)
    y_bad2 = (info["acc"].astype(np.float32) * np.float32(sx)) * s
    assert not np.array_equal(y_bad2.astype(np.float32), ref)


def test_dyn_acc_is_exact_integer_gemm():
    x = rand_x(16, 4096, 80)
    q, s = rand_q(32, 4096, 81)
    _, info = oracle.dyn_linear(x, q, s, return_intermediates=True)
    exact = (info["xq"].astype(np.int64) - info["zero_point"]) @ q.astype(np.int64).T
    np.testing.assert_array_equal(info["acc"], exact.astype(np.int32))
    # independent route: torch's int8 GEMM on xq - 128, plus the shift times
    # the weight row sums
    xs = torch.from_numpy((info["xq"].astype(np.int16) - 128).astype(np.int8))
    ti = torch._int_mm(xs, torch.from_numpy(q).t().contiguous()).numpy().astype(np.int64)
    colsum = q.astype(np.int64).sum(axis=1)
    np.testing.assert_array_equal(ti + (128 - info["zero_point"]) * colsum, exact)


# ---------------------------------------------------------------------------
# per-token symmetric W8A8 (opt-in granularity)
# ---------------------------------------------------------------------------
def test_dyn_token_quantizer_is_the_weight_quantizer_on_rows():
    """The per-token quantizer restates quant.py:25-29 on activation rows; check
    it against torch CPU ops evaluating that expression (fp32 division, half-even)."""
    g = torch.Generator().manual_seed(31)
    x = torch.randn(37, 1000, generator=g) * torch.linspace(1e-3, 1e3, 37)[:, None]
    x[3] = 0.0                                    # all-zero row: s = 1e-8 / 127
    x[5, :4] = torch.tensor([0.5, 1.5, 2.5, -0.5]) * (x[5].abs().max() / 127)  # ties near the grid
    q = np.random.default_rng(1).integers(-127, 128, (16, 1000)).astype(np.int8)
    s = np.random.default_rng(2).random(16).astype(np.float32)
    _, info = oracle.dyn_linear_token(x.numpy(), q, s, return_intermediates=True)
    st = x.abs().amax(dim=1).clamp_min(1e-8) / 127.0
    xq = torch.clamp(torch.round(x / st[:, None]), -127, 127).to(torch.int8)
    np.testing.assert_array_equal(info["scale"], st.numpy())
    np.testing.assert_array_equal(info["xq"], xq.numpy())


def test_dyn_token_golden_fixture():
    """int8_dyn_token.npz: s_t, xq, int32 acc and y from torch CPU ops alone."""
    d = np.load(GOLD / "int8_dyn_token.npz")
    for i in range(len(d["cases"])):
        y, info = oracle.dyn_linear_token(d[f"c{i}_x"], d[f"c{i}_q"], d[f"c{i}_scale"], return_intermediates=True)
        np.testing.assert_array_equal(info["scale"], d[f"c{i}_st"])
        np.testing.assert_array_equal(info["xq"], d[f"c{i}_xq"])
        np.testing.assert_array_equal(info["acc"], d[f"c{i}_acc"])
        np.testing.assert_array_equal(y, d[f"c{i}_y"])


def test_dyn_token_acc_and_epilogue():
    g = torch.Generator().manual_seed(32)
    M, N, K = 33, 24, 4096
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[:40]] *= 20.0
    q = np.random.default_rng(3).integers(-127, 128, (N, K)).astype(np.int8)
    s = (np.random.default_rng(4).random(N).astype(np.float32) + 0.5) * np.float32(1e-3)
    b = np.random.default_rng(5).standard_normal(N).astype(np.float32)
    y, info = oracle.dyn_linear_token(x.numpy(), q, s, return_intermediates=True)
    # int32 accumulators: an independent route through torch's int8 GEMM
    ti = torch._int_mm(torch.from_numpy(info["xq"]), torch.from_numpy(q).t().contiguous()).numpy()
    np.testing.assert_array_equal(ti, info["acc"])
    # epilogue: fp32(acc) * fp32(s_t * s_w); mutants must fail
    acc = info["acc"].astype(np.float32)
    st = info["scale"]
    np.testing.assert_array_equal(y, acc * (st[:, None] * s[None, :]))
    assert not np.array_equal(y, (acc * st[:, None]) * s[None, :])             # (acc * s_t) * s_w
    assert not np.array_equal(y, acc * (np.float32(st.max()) * s[None, :]))   # one scale for the tensor
    # bias: one fused multiply-add, not a separately rounded add
    yb = oracle.dyn_linear_token(x.numpy(), q, s, bias=b)
    fused = (acc.astype(np.float64) * (st[:, None] * s[None, :]).astype(np.float64) + b).astype(np.float32)
    np.testing.assert_array_equal(yb, fused)
    assert not np.array_equal(yb, (acc * (st[:, None] * s[None, :]) + b).astype(np.float32))


# ---------------------------------------------------------------------------
# packed layout model
# ---------------------------------------------------------------------------
def test_pack_layout_model():
    q = (np.arange(20 * 70) % 251 - 125).astype(np.int8).reshape(20, 70)
    p = oracle.pack_w8(q)
    assert p.size == 32 * 128
    Kc = 2
    for n, k in [(0, 0), (5, 17), (15, 63), (16, 64), (19, 69), (3, 40)]:
        nt, r, kc, g, j = n // 16, n % 16, k // 64, (k % 64) // 16, k % 16
        off = ((nt * Kc + kc) * 64 + g * 16 + r) * 16 + j
        assert p[off] == (int(q[n, k]) & 0xFF) ^ 0x80
    # padding decodes to q = 0
    off = ((1 * Kc + 1) * 64 + 0 * 16 + 10) * 16 + 0  # row 26 (padded)
    assert p[off] == 0x80


# ---------------------------------------------------------------------------
# the engine's sampling step (engine.py:29-42)
# ---------------------------------------------------------------------------
def _torch_kept_probs(x, T, k, p):
    """engine.py:32-41 evaluated by torch CPU ops: torch.topk for the k-th
    value, torch.softmax, a descending torch.sort and torch.cumsum."""
    z = torch.from_numpy(np.asarray(x, np.float32)) / T
    if k > 0:
        z = torch.where(z < torch.topk(z, min(k, z.numel())).values[-1], torch.tensor(float("-inf")), z)
    pr = torch.softmax(z, -1)
    if 0 < p < 1:
        vals, idx = torch.sort(pr, descending=True, stable=True)
        drop = (torch.cumsum(vals, 0) - vals) >= p
        pr = pr.clone()
        pr[idx[drop]] = 0.0
    return pr.numpy()


SAMPLE_PARAMS = [(0.7, 0, 0.9), (1.0, 40, 1.0), (0.7, 40, 0.8), (1.3, 0, 1.0), (0.5, 1, 1.0), (1.0, 0, 0.05),
                 (0.8, 10**6, 0.95)]


@pytest.mark.parametrize("T,k,p", SAMPLE_PARAMS)
def test_sample_probs_match_torch_expression(T, k, p):
    for seed, scale in ((0, 2.0), (1, 0.5), (2, 6.0)):
        x = (np.random.default_rng(seed).standard_normal(5003) * scale).astype(np.float32)
        got = oracle.sample_probs(x, T, k, p)
        ref = _torch_kept_probs(x, T, k, p)
        np.testing.assert_array_equal(got > 0, ref > 0)
        np.testing.assert_allclose(got, ref, rtol=3e-6, atol=1e-30)


def test_sample_probs_defining_properties():
    x = (np.random.default_rng(5).standard_normal(2000) * 3).astype(np.float32)
    # top-k = 1 keeps the argmax alone
    p1 = oracle.sample_probs(x, 0.7, 1, 1.0)
    assert np.flatnonzero(p1).tolist() == [int(np.argmax(x))]
    # top-p: the kept tokens are the most probable ones, their mass reaches
    # top_p, and without the least probable kept token it does not
    full = oracle.sample_probs(x, 0.9, 0, 1.0).astype(np.float64)
    for top_p in (0.3, 0.6, 0.9, 0.99):
        kept = oracle.sample_probs(x, 0.9, 0, top_p) > 0
        assert full[kept].min() >= full[~kept].max()
        assert full[kept].sum() >= top_p - 1e-6
        assert full[kept].sum() - full[kept].min() < top_p + 1e-6
    # ties with the k-th largest value are kept (the mask is z < kth)
    xt = np.array([1.0, 5.0, 3.0, 5.0, 4.0, 5.0, 2.0], np.float32)
    assert np.flatnonzero(oracle.sample_probs(xt, 1.0, 2, 1.0)).tolist() == [1, 3, 5]
    assert np.flatnonzero(oracle.sample_probs(xt, 1.0, 4, 1.0)).tolist() == [1, 3, 4, 5]
    # the temperature divides the logits: p ~ exp(x / T)
    pt = oracle.sample_probs(xt, 2.0, 0, 1.0).astype(np.float64)
    np.testing.assert_allclose(pt, np.exp(xt / 2.0) / np.exp(xt / 2.0).sum(), rtol=1e-6)


def test_sample_probs_mutants_fail():
    # inclusive instead of the reference's exclusive cumsum
    probs = np.array([0.5, 0.3, 0.2], np.float32)
    x = np.log(probs)
    kept = oracle.sample_probs(x, 1.0, 0, 0.5) > 0
    assert kept.tolist() == [True, False, False]
    incl = np.cumsum(probs) < 0.5
    assert incl.tolist() != kept.tolist()
    # dropping the ties at the k-th value
    xt = np.array([1.0, 5.0, 3.0, 5.0, 4.0], np.float32)
    kept = oracle.sample_probs(xt, 1.0, 1, 1.0) > 0
    assert kept.sum() == 2 and kept.sum() != 1
    # multiplying by the temperature instead of dividing
    pt = oracle.sample_probs(xt, 2.0, 0, 1.0).astype(np.float64)
    assert not np.allclose(pt, np.exp(xt * 2.0) / np.exp(xt * 2.0).sum(), rtol=1e-3)


def test_sample_token_draw_and_edge_cases():
    x = (np.random.default_rng(9).standard_normal(300) * 1.5).astype(np.float32)
    T, k, p = 0.8, 25, 0.9
    probs = oracle.sample_probs(x, T, k, p).astype(np.float64)
    probs /= probs.sum()
    n = 20000
    counts = np.bincount([oracle.sample_token(x, T, k, p, (i + 0.5) / n) for i in range(n)], minlength=x.size)
    # inverse CDF over a uniform grid: each token takes its share of the grid to within one point
    assert np.abs(counts - n * probs).max() <= 1.0 + 1e-9
    # greedy branch, NaN and infinite maxima
    assert oracle.sample_token(x, 0.0) == int(np.argmax(x))
    xn = x.copy()
    xn[7] = np.nan
    assert oracle.sample_token(xn, 0.0) == 7 and oracle.sample_token(xn, 0.7, 0, 0.9, 0.5) == -1
    xi = x.copy()
    xi[3] = np.inf
    assert oracle.sample_token(xi, 0.7, 0, 0.9, 0.5) == -1
    xm = x.copy()
    xm[3] = -np.inf
    assert oracle.sample_token(xm, 0.7, 0, 1.0, 0.5) != 3
