"""GPU parity at the full sizes of the benchmark configurations and of the real
checkpoint (run on the MI355X box), against the CPU oracle.

Covered shapes (paths relative to the reference repository):
  * lm_head V=151936 at K=4096 (36-layer benchmark model) and K=2560 (the
    real checkpoint, config.py:16,19), model.py:410,445-447, M=1 and M=8;
  * down projections K=12288 and K=9728 (config.py:18), M=1 and M=8;
  * the 4096x4096 single GEMV and the 24576x4096 gate+up GEMV at M=1;
  * prefill N=12288, K=4096 at M=512, 2048 (fp32 activations, the module
    default) and M=8192 (fp16);
  * int8-dyn at M=1/128/2048 over N=4096/12288;
  * the fused hybrid "reads-x" group (model.py:317-329,363-365: sse_q/k/v,
    lora_q[0]/lora_k[0], sse_a/b/e, swa_q/k/v; N=18820) against the oracle in
    both formats, its parts inside torch.inference_mode();
  * one decode step through all 539 quantized linears of the 36-layer hybrid
    model (26 hybrid + 10 softmax blocks, hidden 4096, FFN 12288, 32/8 heads
    of 128, router 4, vocab 151936) at M=1 and M=8, in both formats, with the
    lora_*[0] -> lora_*[1] chain fed as model.py:318-319 feeds it.

Outputs are checked on samples: one output channel per 16-row weight tile
(every workgroup of the GEMV and every GEMM block is checked) and one token
per 16-token fragment.  Bars, as in the other GPU tests: int8 weight-only
relative L2 <= 1e-3 against the oracle (2e-6 for fp16 activations, which the
kernels use exactly, with fp32 outputs); int8-dyn int32 accumulators and fp32
outputs bit-exact, with the activation quantization parameters of the whole
tensor.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import announce
from sbq import quant

W8_TOL = 1e-3
W8_TOL_EXACT_X = 2e-6
# The fp16 prefill GEMM accumulates (q + 128) * x (weights as exact fp16
# subnormals) and removes 128 * rowsum(x) in the epilogue: at K = 4096 with
# N(0, 1) activations that offset is about 3x the result, so its fp32 rounding
# reaches about 2e-6 relative (a numpy model of the scheme gives 1e-6, plain
# fp32 accumulation 2e-7).  The rounding grows like sqrt(K): at K = 12288 with
# 1% of the channels x20, 3.4-4.05e-6 measured, the same with the row sums
# from the pre-pass or from the K loop (gemm_f16_tol).
W8_TOL_GEMM_F16 = 4e-6


def gemm_f16_tol(K):
    """The fp16 prefill GEMM's bar for fp16 / bf16 inputs at reduction length K."""
    return W8_TOL_GEMM_F16 * max(1.0, (K / 4096) ** 0.5)
DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def gpu_weight(N, K, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(N, K, generator=g, device=dev) * 0.02


def cpu_x(M, K, seed, outliers=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    if outliers:
        idx = torch.randperm(K, generator=g)[: max(1, K // 100)]
        x[:, idx] *= 20
    return x


def tile_sample(n, seed, block=16, cap=None):
    """One index per `block`-sized tile of range(n) (offset varying by tile),
    plus n - 1; `cap` keeps that many tiles (spread over the range)."""
    rng = np.random.default_rng(seed)
    starts = np.arange(0, n, block)
    if cap is not None and len(starts) > cap:
        starts = np.unique(np.linspace(0, len(starts) - 1, cap).astype(int)) * block
    idx = np.minimum(starts + rng.integers(0, block, len(starts)), n - 1)
    return np.unique(np.append(idx, n - 1))


def ref_rows(w_gpu, cols):
    """Oracle quantization of the sampled weight rows (fp32 [len, K] -> q, s)."""
    w = w_gpu[torch.from_numpy(cols).to(w_gpu.device)].float().cpu().numpy()
    return oracle.quantize_per_channel(w)


def ref_w8a8(x_full, rows, q, s, bias=None):
    """int32 accumulators and outputs of the sampled rows x columns, with the
    activation parameters of the WHOLE tensor (fbgemm's per-tensor choice)."""
    sx, zp = oracle.act_qparams(x_full)
    xq = oracle.quantize_act(x_full[rows], sx, zp)
    acc64 = (xq.astype(np.float64) - zp) @ np.asarray(q, np.float64).T  # exact: |acc| < 2^53
    acc = np.ascontiguousarray(acc64.astype(np.int64).astype(np.int32))
    return acc, oracle.dyn_epilogue(acc, sx, s, bias)


def pick(t, rows, cols):
    return t[torch.from_numpy(rows).to(t.device)][:, torch.from_numpy(cols).to(t.device)].float().cpu().numpy()


# ---------------------------------------------------------------------------
# single linears at full size
# ---------------------------------------------------------------------------
W8_FULL = [
    # (M, N, K, x dtype, y dtype)
    (1, 24576, 4096, "f16", "f16"),    # gate+up, the dominant decode launch
    (1, 24576, 4096, "f32", "f32"),
    (16, 24576, 4096, "f16", "f16"),   # six row tiles per workgroup (M > 8, wide, short K)
    (9, 21999, 2560, "bf16", "f32"),   # the same, ragged N and a last workgroup of one row tile
    (1, 4096, 4096, "f16", "f32"),     # single 4096x4096 GEMV
    (1, 4096, 4096, "f32", "f32"),
    (1, 151936, 4096, "f32", "f32"),   # lm_head, 36-layer benchmark model
    (8, 151936, 4096, "f32", "f32"),
    (1, 151936, 2560, "f32", "f32"),   # lm_head, real checkpoint
    (8, 151936, 2560, "f32", "f32"),
    (1, 4096, 12288, "f32", "f32"),    # down
    (8, 4096, 12288, "f16", "f32"),
    (1, 2560, 9728, "f32", "f32"),     # down, real checkpoint
    (8, 2560, 9728, "f32", "f32"),
    (512, 12288, 4096, "f32", "f32"),  # prefill chunk as the model issues it (fp32 in and out)
    (2048, 12288, 4096, "f32", "f32"),
    (8192, 12288, 4096, "f16", "f16"),  # prefill, M=8192
    (8192, 12288, 4096, "f16", "f32"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,xd,yd", W8_FULL)
def test_w8_full_size(dev, M, N, K, xd, yd):
    announce(f"w8 full M={M} N={N} K={K} x={xd} y={yd}")
    w = gpu_weight(N, K, 11, dev)
    lin = quant.Int8Linear(w, None)
    cols = tile_sample(N, 1)
    q, s = ref_rows(w, cols)
    np.testing.assert_array_equal(lin.qweight[torch.from_numpy(cols).to(dev)].cpu().numpy(), q)
    del w
    x = cpu_x(M, K, 2).to(DT[xd])
    out = torch.empty((M, N), dtype=DT[yd], device=dev)
    quant.linear_w8(x.to(dev), lin.packed, lin.scale, None, N, out=out)
    rows = tile_sample(M, 3)
    ref = oracle.int8_linear(x.float().numpy()[rows], q, s)
    tol = (gemm_f16_tol(K) if M > 64 else W8_TOL_EXACT_X) if (xd != "f32" and yd == "f32") else W8_TOL
    assert oracle.rel_l2(pick(out, rows, cols), ref) <= tol


W8A8_FULL = [
    (1, 151936, 4096, "f32"), (8, 151936, 4096, "f32"),   # lm_head
    (1, 151936, 2560, "f32"), (8, 151936, 2560, "f32"),
    (1, 4096, 12288, "f32"), (8, 4096, 12288, "f32"),     # down
    (1, 2560, 9728, "f32"), (8, 2560, 9728, "f32"),
    (1, 12288, 4096, "f16"), (128, 4096, 4096, "f16"),    # int8-dyn benchmark shapes
    (2048, 4096, 4096, "f16"), (512, 12288, 4096, "f32"),
    (8192, 12288, 4096, "f16"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,xd", W8A8_FULL)
def test_w8a8_full_size(dev, M, N, K, xd):
    announce(f"w8a8 full M={M} N={N} K={K} x={xd}")
    w = gpu_weight(N, K, 21, dev)
    lin = quant.DynamicInt8Linear(w, None)
    cols = tile_sample(N, 4)
    q, s = ref_rows(w, cols)
    del w
    x = cpu_x(M, K, 5, outliers=True).to(DT[xd])
    acc = torch.empty((M, N), dtype=torch.int32, device=dev)
    y = quant.linear_w8a8(x.to(dev), lin.packed, lin.scale, lin.colsum, None, N, acc_out=acc)
    rows = tile_sample(M, 6)
    acc_ref, y_ref = ref_w8a8(x.float().numpy(), rows, q, s)
    np.testing.assert_array_equal(acc[torch.from_numpy(rows).to(dev)][:, torch.from_numpy(cols).to(dev)].cpu().numpy(),
                                  acc_ref)
    np.testing.assert_array_equal(pick(y, rows, cols), y_ref)


# ---------------------------------------------------------------------------
# prefill GEMM configurations as the library picks them (M > 128: a fitted
# kernel-time model over the block configurations): one shape per
# configuration in use, with the two-tile W8A8 stages also at an odd number of
# K tiles (their one-tile form of the same block runs); most grids here are not
# a multiple of 8 blocks wide, which takes the XCD block order
# ---------------------------------------------------------------------------
PICK_W8 = [(264, 19648, 4096, 0), (648, 10816, 4096, 2), (136, 16384, 4096, 3), (136, 5504, 4096, 5),
           (136, 256, 4096, 8), (136, 21824, 4096, 16), (136, 10944, 4096, 17), (392, 20992, 4096, 18)]
PICK_W8A8 = [(520, 21824, 4096, 0), (648, 16384, 4096, 2), (328, 16384, 4096, 3), (136, 256, 4096, 8),
             (1536, 8192, 12288, 12), (520, 19648, 4096, 13), (520, 19648, 4032, 13), (264, 19648, 4096, 14),
             (264, 19648, 4032, 14), (136, 5504, 4096, 15), (136, 5504, 4032, 15), (264, 21824, 4096, 16),
             (392, 20992, 4096, 18), (648, 22336, 4096, 19), (136, 21824, 4096, 20), (136, 21824, 4032, 20)]


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,cfg", PICK_W8)
def test_w8_gemm_picked_configs(dev, M, N, K, cfg):
    """fp16 activations with the default workspace (the row-sum pre-pass,
    except on configurations 3, 5 and 16, which sum the rows in their K loop
    either way) and with no workspace (sums accumulated in the K loop), fp32
    outputs."""
    announce(f"w8 picked config {cfg} M={M} N={N} K={K}")
    assert quant.gemm_config(M, N, K, torch.float16) == (cfg, 1)
    w = gpu_weight(N, K, 31, dev)
    lin = quant.Int8Linear(w, None)
    cols = tile_sample(N, 8)
    q, s = ref_rows(w, cols)
    del w
    x = cpu_x(M, K, 9).half()
    rows = tile_sample(M, 10)
    ref = oracle.int8_linear(x.float().numpy()[rows], q, s)
    xd = x.to(dev)
    for ws in (None, torch.empty(0, dtype=torch.uint8, device=dev)):
        y = quant.linear_w8(xd, lin.packed, lin.scale, None, N, workspace=ws)
        assert oracle.rel_l2(pick(y, rows, cols), ref) <= W8_TOL_GEMM_F16, ws is None


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,cfg", PICK_W8A8)
def test_w8a8_gemm_picked_configs(dev, M, N, K, cfg):
    announce(f"w8a8 picked config {cfg} M={M} N={N} K={K}")
    assert quant.gemm_config(M, N, K, torch.float16, w8a8=True) == (cfg, 1)
    w = gpu_weight(N, K, 32, dev)
    lin = quant.DynamicInt8Linear(w, None)
    cols = tile_sample(N, 11)
    q, s = ref_rows(w, cols)
    del w
    x = cpu_x(M, K, 12, outliers=True).half()
    acc = torch.empty((M, N), dtype=torch.int32, device=dev)
    y = quant.linear_w8a8(x.to(dev), lin.packed, lin.scale, lin.colsum, None, N, acc_out=acc)
    rows = tile_sample(M, 13)
    acc_ref, y_ref = ref_w8a8(x.float().numpy(), rows, q, s)
    r_, c_ = torch.from_numpy(rows).to(dev), torch.from_numpy(cols).to(dev)
    np.testing.assert_array_equal(acc[r_][:, c_].cpu().numpy(), acc_ref)
    np.testing.assert_array_equal(pick(y, rows, cols), y_ref)


def _random_prefill_cases(n, seed):
    """Seeded prefill shapes at the model's K (4096, 12288, and 4032 for an odd
    K-tile count): M 129..2048, ragged N (most grids then not a multiple of 8
    blocks wide), every activation dtype, with and without a bias."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        K = int(rng.choice([4032, 4096, 4096, 12288]))
        N = int(rng.integers(2048, 8193 if K == 12288 else 24577))
        out.append((i, int(rng.integers(129, 2049)), N, K, str(rng.choice(["f16", "bf16", "f32"])), bool(rng.integers(0, 2))))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("i,M,N,K,xd,has_bias", _random_prefill_cases(20, 2027))
def test_random_prefill_picks_match_oracle(dev, i, M, N, K, xd, has_bias):
    """Whatever configuration and block order the library picks for the shape:
    W-only within the GEMM's fp16 bar (fp16 / bf16 inputs) or 1e-3 (fp32), W8A8
    acc and y bit-exact, on sampled rows and output channels."""
    cfg8, _ = quant.gemm_config(M, N, K, DT[xd])
    cfg88, _ = quant.gemm_config(M, N, K, DT[xd], w8a8=True)
    announce(f"random prefill pick {i}: M={M} N={N} K={K} x={xd} bias={has_bias} configs {cfg8} / {cfg88}")
    w = gpu_weight(N, K, 1300 + i, dev)
    b = torch.randn(N, generator=torch.Generator().manual_seed(1400 + i)) if has_bias else None
    bd = None if b is None else b.to(dev)
    lin = quant.Int8Linear(w, bd)
    dyn = quant.DynamicInt8Linear(w, bd)
    cols = tile_sample(N, 1500 + i, cap=96)
    q, s = ref_rows(w, cols)
    del w
    x = cpu_x(M, K, 1600 + i, outliers=True).to(DT[xd])
    xv = x.float().numpy()
    xg = x.to(dev)
    rows = tile_sample(M, 1700 + i)
    bc = None if b is None else b.numpy()[cols]
    y = quant.linear_w8(xg, lin.packed, lin.scale, lin.bias, N)
    ref = oracle.int8_linear(xv[rows], q, s, bc)
    assert oracle.rel_l2(pick(y, rows, cols), ref) <= (W8_TOL if xd == "f32" else gemm_f16_tol(K))
    acc = torch.empty((M, N), dtype=torch.int32, device=dev)
    y8 = quant.linear_w8a8(xg, dyn.packed, dyn.scale, dyn.colsum, dyn.bias, N, acc_out=acc)
    acc_ref, y_ref = ref_w8a8(xv, rows, q, s, bc)
    r_, c_ = torch.from_numpy(rows).to(dev), torch.from_numpy(cols).to(dev)
    np.testing.assert_array_equal(acc[r_][:, c_].cpu().numpy(), acc_ref)
    np.testing.assert_array_equal(pick(y8, rows, cols), y_ref)


def _random_decode_cases(n, seed):
    """Seeded decode shapes: M 1..16 (mostly 1 and 4..8), K from the model's
    (128, 2560, 4096, 9728, 12288), other multiples of 64 and a few ragged
    ones, N up to 24576 (often wide enough for five row tiles per workgroup),
    every activation dtype, with and without a bias."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        M = int(rng.choice([1, 1, 1, 2, 3, 4, 5, 6, 7, 8, 8, 12, 16]))
        r = rng.random()
        if r < 0.6:
            K = int(rng.choice([128, 2560, 2560, 4096, 9728, 12288]))
        elif r < 0.9:
            K = 64 * int(rng.integers(1, 161))
        else:
            K = int(rng.integers(65, 4000))
        N = int(rng.integers(16385, 24577)) if rng.random() < 0.4 and K < 8192 else int(rng.integers(1, 12289))
        out.append((i, M, N, K, str(rng.choice(["f16", "bf16", "f32"])), bool(rng.integers(0, 2))))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("i,M,N,K,xd,has_bias", _random_decode_cases(24, 2029))
def test_random_decode_picks_match_oracle(dev, i, M, N, K, xd, has_bias):
    """Whatever decode kernel and configuration the library picks (x in LDS or
    direct fragments, one to five row tiles per workgroup, fused or pre-pass
    min/max, per-token rows quantized in the GEMV or by the row quantizer):
    W-only within 2e-5 (fp32 x: high + remainder keep 16 bits) or 1e-5, per-tensor
    and per-token W8A8 acc and y bit-exact, on sampled output channels."""
    announce(f"random decode {i}: M={M} N={N} K={K} x={xd} bias={has_bias}")
    w = gpu_weight(N, K, 1800 + i, dev)
    b = torch.randn(N, generator=torch.Generator().manual_seed(1900 + i)) if has_bias else None
    bd = None if b is None else b.to(dev)
    lin = quant.Int8Linear(w, bd)
    dyn = quant.DynamicInt8Linear(w, bd)
    tok = quant.DynamicInt8Linear(w, bd, granularity="token")
    cols = tile_sample(N, 2000 + i, cap=96)
    q, s = ref_rows(w, cols)
    del w
    x = cpu_x(M, K, 2100 + i, outliers=True).to(DT[xd])
    xv = x.float().numpy()
    xg = x.to(dev)
    rows = np.arange(M)
    bc = None if b is None else b.numpy()[cols]
    y = quant.linear_w8(xg, lin.packed, lin.scale, lin.bias, N)
    ref = oracle.int8_linear(xv, q, s, bc)
    assert oracle.rel_l2(pick(y, rows, cols), ref) <= (2e-5 if xd == "f32" else 1e-5)
    acc = torch.empty((M, N), dtype=torch.int32, device=dev)
    y8 = quant.linear_w8a8(xg, dyn.packed, dyn.scale, dyn.colsum, dyn.bias, N, acc_out=acc)
    acc_ref, y_ref = ref_w8a8(xv, rows, q, s, bc)
    c_ = torch.from_numpy(cols).to(dev)
    np.testing.assert_array_equal(acc[:, c_].cpu().numpy(), acc_ref)
    np.testing.assert_array_equal(pick(y8, rows, cols), y_ref)
    y_t_ref, info = oracle.dyn_linear_token(xv, q, s, bias=bc, return_intermediates=True)
    y_t = quant.linear_w8a8_token(xg, tok.packed, tok.scale, tok.bias, N, acc_out=acc)
    np.testing.assert_array_equal(acc[:, c_].cpu().numpy(), info["acc"])
    np.testing.assert_array_equal(pick(y_t, rows, cols), y_t_ref)


# ---------------------------------------------------------------------------
# the fused hybrid "reads-x" group (N = 18820)
# ---------------------------------------------------------------------------
HYBRID_READS_X = [("sse_q", 4096), ("sse_k", 4096), ("sse_v", 4096), ("lora_q0", 128), ("lora_k0", 128),
                  ("sse_a", 64), ("sse_b", 64), ("sse_e", 4), ("swa_q", 4096), ("swa_k", 1024), ("swa_v", 1024)]


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int8", "int8-dyn"])
@pytest.mark.parametrize("M", [1, 8])
def test_fused_hybrid_group_vs_oracle(dev, fmt, M):
    announce(f"fused hybrid reads-x group fmt={fmt} M={M}")
    K = 4096
    ws = [gpu_weight(n, K, 40 + i, dev) for i, (_, n) in enumerate(HYBRID_READS_X)]
    mods = [quant.make_linear(fmt, w) for w in ws]
    fused = quant.fuse_linears(mods)
    assert fused.out_features == 18820
    x = cpu_x(M, K, 41)
    outs = fused(x.to(dev))
    parts = [fused.part(i) for i in range(len(mods))]
    with torch.inference_mode():  # as model.py:427 runs the model
        xi = x.to(dev)
        part_outs = [p(xi) for p in parts]
    rows = np.arange(M)
    for (name, n), w, o, po in zip(HYBRID_READS_X, ws, outs, part_outs):
        cols = tile_sample(n, 7)
        q, s = ref_rows(w, cols)
        got = o.cpu().numpy()[:, cols]
        if fmt == "int8":
            assert oracle.rel_l2(got, oracle.int8_linear(x.numpy(), q, s)) <= W8_TOL, name
            np.testing.assert_array_equal(po.cpu().numpy(), o.cpu().numpy())
        else:
            _, y_ref = ref_w8a8(x.numpy(), rows, q, s)
            np.testing.assert_array_equal(got, y_ref, err_msg=name)
            np.testing.assert_array_equal(po.cpu().numpy(), o.cpu().numpy())


@pytest.mark.gpu
def test_fused_parts_share_one_launch_per_call_sequence(dev):
    """FusedLinear.part(i) drop-ins under torch.inference_mode() (inference
    tensors carry no version counter): the parts of one call sequence share
    one launch; once every part has taken its output, the next call launches
    again, so an in-place edit of x between two sequences is seen; a part
    called twice in one sequence launches anew as well."""
    announce("fused parts: one launch per call sequence")
    K = 512
    mods = [quant.make_linear("int8", gpu_weight(n, K, 70 + i, dev)) for i, n in enumerate((64, 32))]
    fused = quant.fuse_linears(mods)
    p0, p1 = fused.part(0), fused.part(1)
    with torch.inference_mode():
        x = cpu_x(1, K, 71).to(dev)
        a0, a1 = p0(x), p1(x)
        for a, m in ((a0, mods[0]), (a1, mods[1])):
            assert oracle.rel_l2(a.cpu().numpy(), m(x).cpu().numpy()) <= 1e-6
        x.mul_(2.0)  # in place: doubles every product and sum exactly
        b0, b1 = p0(x), p1(x)
        assert torch.equal(b0, 2 * a0) and torch.equal(b1, 2 * a1)
        c0 = p0(x)
        x.mul_(0.5)
        c0_again = p0(x)  # part 0 already took its output from the launch before the edit
        assert torch.equal(c0, b0) and torch.equal(c0_again, a0)


# ---------------------------------------------------------------------------
# one decode step through the 539 quantized linears of the 36-layer model
# ---------------------------------------------------------------------------
SOFTMAX_LAYERS = (0, 1, 2, 3, 6, 12, 17, 21, 24, 35)


def stack_layout(H=4096, F=12288, heads=32, kv=8, d=128, routers=4, vocab=151936, layers=36):
    """(name, N, K, input) of every quantized linear of one decode step, in
    model order.  input: "h" (the normed hidden state), "attn" (an attention
    output), "ffn" (the gated MLP activation) or the name of the linear whose
    output it reads (lora_*[1] read lora_*[0], model.py:318-319)."""
    out = []
    for i in range(layers):
        p = f"l{i}."
        if i in SOFTMAX_LAYERS:  # model.py:250-253,262-270
            out += [(p + "q", heads * d, H, "h"), (p + "k", kv * d, H, "h"), (p + "v", kv * d, H, "h"),
                    (p + "o", H, heads * d, "attn")]
        else:  # model.py:284-301,317-329,359-371
            out += [(p + n, heads * d, H, "h") for n in ("sse_q", "sse_k", "sse_v")]
            out += [(p + "lora_q0", d, H, "h"), (p + "lora_k0", d, H, "h")]
            out += [(p + "lora_q1", heads * d, d, p + "lora_q0"), (p + "lora_k1", heads * d, d, p + "lora_k0")]
            out += [(p + "sse_a", 2 * heads, H, "h"), (p + "sse_b", 2 * heads, H, "h"), (p + "sse_e", routers, H, "h")]
            out += [(p + "sse_o", H, heads * d, "attn")]
            out += [(p + "swa_q", heads * d, H, "h"), (p + "swa_k", kv * d, H, "h"), (p + "swa_v", kv * d, H, "h"),
                    (p + "swa_o", H, heads * d, "attn")]
        out += [(p + "gate", F, H, "h"), (p + "up", F, H, "h"), (p + "down", H, F, "ffn")]  # model.py:235-240
    out.append(("lm_head", vocab, H, "h"))  # model.py:410,447
    return out


def test_stack_layout_counts():
    lay = stack_layout()
    assert len(lay) == 539
    assert sum(n * k for _, n, k, _ in lay) == 9381511168


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int8", "int8-dyn"])
def test_decode_step_539_linears(dev, fmt):
    """Every linear's output at M=1 and M=8 checked on up to 48 sampled output
    channels (one per sampled 16-row tile); every distinct (N, K) appears."""
    lay = stack_layout()
    announce(f"539-linear decode step fmt={fmt}: building")
    mods, refs = {}, {}
    for i, (name, n, k, _) in enumerate(lay):
        w = gpu_weight(n, k, 1000 + i, dev)
        mods[name] = quant.make_linear(fmt, w)
        cols = tile_sample(n, i, cap=48)
        refs[name] = (cols, *ref_rows(w, cols))
        del w
    torch.cuda.synchronize()
    for M in (1, 8):
        announce(f"539-linear decode step fmt={fmt} M={M}")
        src = {"h": cpu_x(M, 4096, 51), "attn": cpu_x(M, 4096, 52), "ffn": cpu_x(M, 12288, 53)}
        dsrc = {key: v.to(dev) for key, v in src.items()}
        outs = {}
        with torch.inference_mode():
            for name, n, k, inp in lay:  # eager, in model order
                outs[name] = mods[name](dsrc[inp] if inp in dsrc else outs[inp])
        torch.cuda.synchronize()
        for name, n, k, inp in lay:
            cols, q, s = refs[name]
            x = src[inp].numpy() if inp in src else outs[inp].cpu().numpy()
            got = outs[name].cpu().numpy()[:, cols]
            if fmt == "int8":
                assert oracle.rel_l2(got, oracle.int8_linear(x, q, s)) <= W8_TOL, (name, M)
            else:
                _, y_ref = ref_w8a8(x, np.arange(M), q, s)
                np.testing.assert_array_equal(got, y_ref, err_msg=f"{name} M={M}")
    del mods


def _check_f16_out(got16, ref32, xd, fmt, what):
    """fp16 outputs (what the stack step writes) against the oracle's fp32
    result: int8-dyn bit-exact after the one rounding to fp16; weight-only
    for fp16 inputs (which the kernels use exactly) within one fp16 ulp of the
    rounded oracle plus W8_TOL_EXACT_X of the row's largest output (the fp32
    summation order moves an output by about that much in absolute terms,
    which is several ulps of an output near zero); rel-L2 <= 1e-3 for fp32
    inputs (bf16 high + remainder planes)."""
    ref16 = ref32.astype(np.float16)
    if fmt == "int8-dyn":
        np.testing.assert_array_equal(got16.view(np.uint16), ref16.view(np.uint16), err_msg=what)
    elif xd == torch.float16:
        bar = np.spacing(np.abs(ref16)).astype(np.float32) + W8_TOL_EXACT_X * np.abs(ref32).max(axis=1, keepdims=True)
        assert np.all(np.abs(got16.astype(np.float32) - ref16.astype(np.float32)) <= bar), what
    else:
        assert oracle.rel_l2(got16, ref32) <= W8_TOL, what


@pytest.mark.gpu
@pytest.mark.parametrize("model", ["bench36", "checkpoint"])
def test_grouped_stack_step_vs_oracle(dev, model):
    """The fused and grouped decode step the bench's stack figures come from
    (bench.grouped_stack_launches, run by bench.stack_step exactly as the
    bench runs it: 171 launches for 539 linears) at the 36-layer benchmark
    model's sizes (hidden 4096, FFN 12288) and at the real checkpoint's
    (hidden 2560, FFN 9728), at M = 1 and 8, fp16 and fp32 activations, both
    formats, eager and replayed from a HIP graph: every linear's fp16 output
    against the oracle on up to 48 sampled output channels (one per sampled
    16-row tile, all M rows); int8-dyn bit-exact (the activation parameters
    of each whole input), weight-only within the weight-only bars."""
    import bench

    H, F = (4096, 12288) if model == "bench36" else (2560, 9728)
    launches = bench.grouped_stack_launches(H=H, F=F)
    shapes = [sh for grp in launches for sh in grp]
    assert len(shapes) == 223 and len(launches) == 171
    announce(f"grouped stack step {model}: building {len(shapes)} linears")
    layers, refs = [], []
    for i, (N, K) in enumerate(shapes):
        w = gpu_weight(N, K, 3000 + i, dev)
        q, s = quant.quantize_per_channel_gpu(w)
        packed, cs = quant.repack(q, with_colsum=True)
        cols = tile_sample(N, i, cap=48)
        layers.append((packed, s, cs))
        refs.append((cols, *ref_rows(w, cols)))
        del w, q
    # the input each linear reads: single launches xs[K][0], member j of a
    # grouped launch xs[K][j]
    which = [j if len(grp) > 1 else 0 for grp in launches for j in range(len(grp))]
    torch.cuda.synchronize()
    for fmt in ("int8", "int8-dyn"):
        for M in (1, 8):
            for xd in (torch.float16, torch.float32):
                announce(f"grouped stack step {model} fmt={fmt} M={M} x={xd}")
                xs = {K: [cpu_x(M, K, 60 + K % 97).to(xd).to(dev), cpu_x(M, K, 61 + K % 89).to(xd).to(dev)]
                      for K in {k for _, k in shapes}}
                ys = [torch.empty((M, N), dtype=torch.float16, device=dev) for N, _ in shapes]
                w8a8 = fmt == "int8-dyn"
                wss = {K: quant.w8a8_workspace(M, K, dev, None, xd) for K in xs} if w8a8 else {}
                step = bench.stack_step(quant, launches, layers, xs, ys, wss, w8a8)
                for mode in ("eager", "graph"):
                    for y in ys:
                        y.fill_(float("nan"))
                    if mode == "eager":
                        step()
                    else:
                        s = torch.cuda.Stream()
                        s.wait_stream(torch.cuda.current_stream())
                        with torch.cuda.stream(s):
                            step()
                        torch.cuda.current_stream().wait_stream(s)
                        g = torch.cuda.CUDAGraph()
                        with torch.cuda.graph(g):
                            step()
                        for y in ys:
                            y.fill_(float("nan"))
                        g.replay()
                    torch.cuda.synchronize()
                    xh = {K: [v.float().cpu().numpy() for v in pair] for K, pair in xs.items()}
                    for i, ((N, K), (cols, q, s), y) in enumerate(zip(shapes, refs, ys)):
                        x = xh[K][which[i]]
                        got = y[:, torch.from_numpy(cols).to(dev)].cpu().numpy()
                        if w8a8:
                            _, ref = ref_w8a8(x, np.arange(M), q, s)
                        else:
                            ref = oracle.int8_linear(x, q, s)
                        _check_f16_out(got, ref, xd, fmt, f"{model} {fmt} M={M} {xd} {mode} linear {i} ({N}x{K})")
                    if mode == "graph":
                        del g
                del ys, wss, xs
    del layers


# ---------------------------------------------------------------------------
# the module API under the reference model's calling conventions
# ---------------------------------------------------------------------------
@pytest.mark.gpu
def test_loader_swap_inference_mode_and_dtype_moves(dev):
    """loader.py:43-51 swaps nn.Linear children (including nn.Sequential ones)
    for make_linear modules; model.py:427 then calls them under
    torch.inference_mode().  Fused parts must work there, .half() must leave
    the int8-dyn scales and bias fp32 (they live in fbgemm's packed weight in
    the reference, quant.py:61), and broadcast / transposed-row activations
    must be accepted as the reference's matmul accepts them."""
    announce("loader swap + inference mode + dtype moves")
    K = 256
    model = torch.nn.ModuleDict({"q": torch.nn.Linear(K, 64, bias=False), "k": torch.nn.Linear(K, 32, bias=False),
                                 "lora": torch.nn.Sequential(torch.nn.Linear(K, 16, bias=False),
                                                             torch.nn.Linear(16, 64, bias=False))})
    g = torch.Generator().manual_seed(9)
    for m in model.modules():
        if isinstance(m, torch.nn.Linear):
            m.weight.data = torch.randn(m.weight.shape, generator=g) * 0.02
    for fmt in ("int8", "int8-dyn"):
        swapped = torch.nn.ModuleDict()
        for name, child in model.items():
            if isinstance(child, torch.nn.Sequential):
                swapped[name] = torch.nn.Sequential(*[quant.make_linear(fmt, c.weight.data) for c in child])
            else:
                swapped[name] = quant.make_linear(fmt, child.weight.data)
        fused = quant.fuse_linears([swapped["q"], swapped["k"]])
        x = torch.randn(3, K, generator=g).to(dev)
        with torch.inference_mode():
            xi = x.clone()
            pq, pk = fused.part(0)(xi), fused.part(1)(xi)
            sq, sk = swapped["q"](xi), swapped["k"](xi)
            lo = swapped["lora"](xi)
        if fmt == "int8-dyn":
            np.testing.assert_array_equal(pq.cpu().numpy(), sq.cpu().numpy())
            np.testing.assert_array_equal(pk.cpu().numpy(), sk.cpu().numpy())
        else:
            assert oracle.rel_l2(pq.cpu().numpy(), sq.cpu().numpy()) <= 1e-5
            assert oracle.rel_l2(pk.cpu().numpy(), sk.cpu().numpy()) <= 1e-5
        assert lo.shape == (3, 64)
        # broadcast rows and a transposed [K, 1] row
        xb = x[:1].expand(3, K)
        np.testing.assert_array_equal(swapped["q"](xb).cpu().numpy(), swapped["q"](xb.contiguous()).cpu().numpy())
        xt = x[0].clone().reshape(K, 1).t()  # shape [1, K], strides (1, 1)
        assert xt.stride() == (1, 1)
        np.testing.assert_array_equal(swapped["q"](xt).cpu().numpy(), swapped["q"](x[:1]).cpu().numpy())
    dyn = quant.DynamicInt8Linear(torch.randn(40, K, generator=g) * 0.02, torch.randn(40, generator=g))
    x = torch.randn(2, K, generator=g).to(dev)
    before = dyn(x).cpu().numpy()
    dyn.half()
    assert dyn.scale.dtype == torch.float32 and dyn.bias.dtype == torch.float32
    np.testing.assert_array_equal(dyn(x).cpu().numpy(), before)
    fz = quant.fuse_linears([quant.DynamicInt8Linear(torch.randn(16, K, generator=g) * 0.02, torch.randn(16)),
                             quant.DynamicInt8Linear(torch.randn(16, K, generator=g) * 0.02, None)])
    fb = [o.cpu().numpy() for o in fz(x)]
    fz.to(torch.bfloat16)
    assert fz.scale.dtype == torch.float32 and fz.bias.dtype == torch.float32
    for a, b in zip(fz(x), fb):
        np.testing.assert_array_equal(a.cpu().numpy(), b)


# ---------------------------------------------------------------------------
# lm_head and its greedy token in one pass (model.py:445-447, engine.py:30-31)
# ---------------------------------------------------------------------------
def _check_greedy(y, tok, module=None):
    """tok must be torch.argmax of the logits the same call returned, and
    every argmax state of the module (one per stream it ran on) must be back
    at zero."""
    np.testing.assert_array_equal(tok.cpu().numpy(), torch.argmax(y.cpu(), dim=-1).numpy())
    if module is not None:
        states = module.__dict__.get("_argmax_states", {})
        assert states
        for st in states.values():
            assert int(st.cpu().count_nonzero()) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int8", "int8-dyn"])
@pytest.mark.parametrize("M,K,xd", [(1, 4096, "f32"), (1, 4096, "f16"), (8, 4096, "f32"), (3, 2560, "f32"),
                                    (16, 2560, "f16"), (1, 2560, "bf16")])
def test_lm_head_greedy_one_pass(dev, fmt, M, K, xd):
    announce(f"lm_head greedy fmt={fmt} M={M} K={K} x={xd}")
    V = 151936
    w = gpu_weight(V, K, 61, dev)
    lm = quant.make_linear(fmt, w)
    x = cpu_x(M, K, 62).to(DT[xd]).to(dev)
    y_plain = lm(x)
    for _ in range(3):  # repeated calls reuse the state the last one left at zero
        y, tok = lm.forward_greedy(x)
        np.testing.assert_array_equal(y.cpu().numpy(), y_plain.cpu().numpy())
        _check_greedy(y, tok, lm)
    # against the oracle: its logits over the GPU's 32 best columns and sampled
    # ones must put their maximum at the GPU's token
    cand = np.unique(np.concatenate([torch.topk(y, 32, dim=-1).indices.cpu().numpy().ravel(),
                                     tile_sample(V, 63, cap=64)]))
    q, s = ref_rows(w, cand)
    xf = x.float().cpu().numpy()
    if fmt == "int8":
        ref = oracle.int8_linear(xf, q, s)
    else:
        _, ref = ref_w8a8(xf, np.arange(M), q, s)
    np.testing.assert_array_equal(cand[np.argmax(ref, axis=-1)], tok.cpu().numpy())


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int8", "int8-dyn"])
def test_lm_head_greedy_ties_nan_zeros(dev, fmt):
    """Equal logits far apart (first index wins), NaN logits (the first NaN
    wins), all-zero logits (index 0), through the fused path at V=151936."""
    announce(f"lm_head greedy ties/NaN fmt={fmt}")
    V, K = 151936, 4096
    x = cpu_x(1, K, 64)
    w = gpu_weight(V, K, 65, dev)
    big = 0.1 * torch.sign(x[0]).to(dev)
    for row in (3, 75000, 151000):  # identical rows, far larger than the rest
        w[row] = big
    lm = quant.make_linear(fmt, w)
    y, tok = lm.forward_greedy(x.to(dev))
    assert tok.item() == 3 and y[0, 3].item() == y[0, 151000].item()
    _check_greedy(y, tok, lm)
    b = torch.zeros(V)
    b[90000] = b[140000] = float("nan")
    lmb = quant.make_linear(fmt, w, b.to(dev))
    y, tok = lmb.forward_greedy(x.to(dev))
    assert tok.item() == 90000
    _check_greedy(y, tok, lmb)
    y, tok = lm.forward_greedy(torch.zeros(2, K, device=dev))
    assert tok.tolist() == [0, 0] and float(y.abs().max()) == 0.0
    _check_greedy(y, tok, lm)


@pytest.mark.gpu
@pytest.mark.parametrize("xd", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("M,N,K", [(20, 5000, 1024), (40, 3000, 512), (2, 1000, 200), (20, 845, 2560),
                                   (24, 3520, 2560)])
def test_greedy_one_pass_other_shapes(dev, M, N, K, xd):
    """Shapes the fused GEMV does not take (M > 16, ragged K): the logits
    exactly as forward computes them (for fp16 / bf16 x at 16 < M <= 64 the
    row-tile GEMV or the split GEMM, not the general GEMV), then the row
    argmax; same tokens."""
    announce(f"greedy other shapes M={M} N={N} K={K} x={xd}")
    for fmt in ("int8", "int8-dyn"):
        lm = quant.make_linear(fmt, gpu_weight(N, K, 66, dev))
        x = cpu_x(M, K, 67).to(DT[xd]).to(dev)
        y, tok = lm.forward_greedy(x)
        np.testing.assert_array_equal(y.cpu().numpy(), lm(x).cpu().numpy())
        _check_greedy(y, tok, lm)


@pytest.mark.gpu
def test_greedy_one_pass_graph_replays(dev):
    """The fused call captured in a HIP graph: every replay (new activations,
    eager work in between) gives the argmax of its own logits, and leaves the
    state at zero for the next replay."""
    announce("greedy graph replays")
    V, K = 151936, 4096
    for fmt in ("int8", "int8-dyn"):
        lm = quant.make_linear(fmt, gpu_weight(V, K, 68, dev))
        x = cpu_x(1, K, 69).to(dev)
        lm.forward_greedy(x)  # state and workspace exist before capture
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            lm.forward_greedy(x)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            y, tok = lm.forward_greedy(x)
        for i in range(4):
            x.copy_(cpu_x(1, K, 70 + i).to(dev))
            g.replay()
            torch.cuda.synchronize()
            _check_greedy(y, tok, lm)
            np.testing.assert_array_equal(y.cpu().numpy(), lm(x).cpu().numpy())
            lm(torch.randn(3, K, device=dev))  # eager work between replays


@pytest.mark.gpu
def test_greedy_one_pass_two_streams(dev):
    """One lm_head module used on two streams at once: each stream has its own
    argmax state, so the tokens of both calls are right."""
    announce("greedy two streams")
    V, K = 32000, 4096
    lm = quant.make_linear("int8", gpu_weight(V, K, 71, dev))
    xs = [cpu_x(1, K, 72 + i).to(dev) for i in range(2)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(2)]
    outs = []
    for _ in range(3):
        for st, x in zip(streams, xs):
            st.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(st):
                outs.append(lm.forward_greedy(x))
        torch.cuda.synchronize()
    for y, tok in outs:
        _check_greedy(y, tok, lm)
    assert len(lm.__dict__["_argmax_states"]) >= 2


# ---------------------------------------------------------------------------
# device-resident model state (the callers on either side of the linears)
# ---------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int8", "int8-dyn"])
def test_device_resident_decode(dev, fmt):
    """A toy decoder (tests/toy_decoder.py) generating greedily with its state
    on the GPU: eager steps and one captured HIP graph replayed per token give
    the same tokens and bit-identical logits; the same decoder with its state
    on the CPU (the reference's placement), fed the same tokens, gives the
    same logits to rel-L2 1e-4 (int8) / 5e-3 (int8-dyn: a one-ulp difference
    in a CPU-computed activation can move one quantization step) and the same
    greedy token wherever the top two logits are apart."""
    from toy_decoder import ToyDecoder, toy_weights

    announce(f"device-resident decode fmt={fmt}")
    H, F, B, V, heads, L, steps, first = 256, 768, 2, 1000, 4, 32, 12, 7
    w, emb = toy_weights(H, F, B, V)
    gpu = ToyDecoder(fmt, w, emb, heads, L, dev)
    gpu.reset(first)
    eager_logits, eager_tok = [], []
    for _ in range(steps):
        eager_logits.append(gpu.step_device().clone())
        eager_tok.append(int(gpu.tok.item()))
    # one step captured (the warm-up creates the argmax state and workspaces)
    gpu.reset(first)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        gpu.step_device()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        logits = gpu.step_device()
    gpu.reset(first)
    for i in range(steps):
        g.replay()
        torch.cuda.synchronize()
        assert int(gpu.tok.item()) == eager_tok[i], i
        np.testing.assert_array_equal(logits.cpu().numpy(), eager_logits[i].cpu().numpy())
    assert int(gpu.pos.item()) == steps
    # the reference's placement, teacher-forced with the device's tokens
    cpu = ToyDecoder(fmt, w, emb, heads, L, "cpu")
    cpu.reset(first)
    tol = 1e-4 if fmt == "int8" else 5e-3
    for i in range(steps):
        inp = torch.tensor([first if i == 0 else eager_tok[i - 1]])
        lc = cpu.step_cpu_state(inp)
        ld = eager_logits[i].cpu()
        assert lc.device.type == "cpu"
        assert oracle.rel_l2(lc.numpy(), ld.numpy()) <= tol, i
        top2 = torch.topk(ld, 2).values
        if float(top2[0] - top2[1]) > 1e-2 * float(top2[0].abs()):
            assert int(cpu.tok.item()) == eager_tok[i], i


# ---------------------------------------------------------------------------
# prefill GEMM with K split over workgroups (grids that would leave CUs idle)
# ---------------------------------------------------------------------------
SPLIT_CASES = [  # (M, N, K): 64 x 64 blocks (configuration 22), K split 2 - 4 ways (M <= 128 only); every
    # case reaches the split GEMM in both formats (asserted through sbq_gemm_config): ragged M and N, an odd
    # number of K tiles (4160), short and long K, 16 < M <= 64 on layers the row-tile GEMV leaves to the GEMM
    (64, 4096, 4096), (100, 2048, 4096), (128, 4096, 4096), (120, 1024, 2560), (100, 2000, 4096),
    (128, 4096, 4160), (80, 2560, 9728), (40, 4096, 8192),
]


def _split_bytes(M, N, K, xd, w8a8):
    """(full workspace, workspace without the split area), and asserts that
    the shape runs the tiled GEMM with K split (sbq_gemm_config)."""
    import ctypes

    from sbq import _lib

    L = _lib.load()
    code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[xd]
    splits = ctypes.c_int(-1)
    L.sbq_gemm_config(M, N, K, code, 1 if w8a8 else 0, ctypes.byref(splits))
    assert splits.value >= 2, (M, N, K, xd, w8a8, splits.value)
    base = L.sbq_w8a8_workspace_bytes(M, K) if w8a8 else L.sbq_w8_workspace_bytes(M, K, code)
    return L.sbq_linear_workspace_bytes(M, N, K, code, 1 if w8a8 else 0), base


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", SPLIT_CASES)
def test_w8a8_split_k_bitexact(dev, M, N, K):
    """int8-dyn with K split over workgroups: int32 accumulators and outputs
    bit-exact against the oracle and equal to the unsplit GEMM (the workspace
    without the split area); repeated calls give the same bits."""
    announce(f"w8a8 split-K M={M} N={N} K={K}")
    full, base = _split_bytes(M, N, K, torch.float16, True)
    assert full > base  # the shape splits
    w = gpu_weight(N, K, 81, dev)
    b = torch.randn(N, generator=torch.Generator().manual_seed(82)).to(dev)
    lin = quant.DynamicInt8Linear(w, b)
    cols = tile_sample(N, 83)
    q, s = ref_rows(w, cols)
    for xd in (torch.float16, torch.float32):
        x = cpu_x(M, K, 84, outliers=True).to(xd)
        xg = x.to(dev)
        outs = []
        for ws in (torch.empty(full, dtype=torch.uint8, device=dev), torch.empty(base, dtype=torch.uint8, device=dev)):
            for _ in range(2):
                acc = torch.empty((M, N), dtype=torch.int32, device=dev)
                y = quant.linear_w8a8(xg, lin.packed, lin.scale, lin.colsum, lin.bias, N, acc_out=acc, workspace=ws)
                outs.append((acc.cpu().numpy(), y.cpu().numpy()))
        for o in outs[1:]:
            np.testing.assert_array_equal(o[0], outs[0][0])
            np.testing.assert_array_equal(o[1], outs[0][1])
        acc_ref, y_ref = ref_w8a8(x.float().numpy(), np.arange(M), q, s, b.cpu().numpy()[cols])
        np.testing.assert_array_equal(outs[0][0][:, cols], acc_ref)
        np.testing.assert_array_equal(outs[0][1][:, cols], y_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", SPLIT_CASES)
def test_w8_split_k_matches_oracle(dev, M, N, K):
    """Weight-only with K split over workgroups (fp16 x, and fp32 / bf16 x
    staged as fp16 planes): within the tolerance of the oracle, equal across
    repeated calls (the partials are added in split order), and within fp32
    summation order of the unsplit GEMM."""
    announce(f"w8 split-K M={M} N={N} K={K}")
    w = gpu_weight(N, K, 85, dev)
    lin = quant.Int8Linear(w, None)
    cols = tile_sample(N, 86)
    q, s = ref_rows(w, cols)
    for xd in (torch.float16, torch.bfloat16, torch.float32):
        full, base = _split_bytes(M, N, K, xd, False)
        assert full > base
        x = cpu_x(M, K, 87).to(xd)
        xg = x.to(dev)
        ys = []
        for ws in (torch.empty(full, dtype=torch.uint8, device=dev), torch.empty(full, dtype=torch.uint8, device=dev),
                   torch.empty(base, dtype=torch.uint8, device=dev)):
            ys.append(quant.linear_w8(xg, lin.packed, lin.scale, None, N, workspace=ws).cpu().numpy())
        np.testing.assert_array_equal(ys[0], ys[1])
        assert oracle.rel_l2(ys[0], ys[2]) <= 2e-6
        ref = oracle.int8_linear(x.float().numpy(), q, s)
        tol = W8_TOL if xd == torch.float32 else W8_TOL_EXACT_X
        assert oracle.rel_l2(ys[0][:, cols], ref) <= tol, str(xd)


@pytest.mark.gpu
def test_split_k_graph_replays(dev):
    """Split-K GEMMs captured in a HIP graph: every replay (new activations,
    eager work between) equals the eager call; the counters are zeroed by the
    pre-pass inside each replay."""
    announce("split-K graph replays")
    M, N, K = 128, 4096, 4096
    w = gpu_weight(N, K, 88, dev)
    dyn = quant.DynamicInt8Linear(w, None)
    lin = quant.Int8Linear(w, None)
    x = cpu_x(M, K, 89).half().to(dev)
    ws8a8 = quant.w8a8_workspace(M, K, dev, N)
    ws8 = quant.w8_workspace(M, K, dev, torch.float16, N)
    y1 = torch.empty((M, N), device=dev)
    y2 = torch.empty((M, N), device=dev)

    def run():
        quant.linear_w8a8(x, dyn.packed, dyn.scale, dyn.colsum, None, N, workspace=ws8a8, out=y1)
        quant.linear_w8(x, lin.packed, lin.scale, None, N, workspace=ws8, out=y2)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    for i in range(4):
        x.copy_(cpu_x(M, K, 90 + i).half().to(dev))
        g.replay()
        torch.cuda.synchronize()
        e1 = quant.linear_w8a8(x, dyn.packed, dyn.scale, dyn.colsum, None, N, workspace=quant.w8a8_workspace(M, K, dev, N))
        e2 = quant.linear_w8(x, lin.packed, lin.scale, None, N, workspace=quant.w8_workspace(M, K, dev, torch.float16, N))
        np.testing.assert_array_equal(y1.cpu().numpy(), e1.cpu().numpy())
        np.testing.assert_array_equal(y2.cpu().numpy(), e2.cpu().numpy())


# ---------------------------------------------------------------------------
# grouped launch of independent weight-only linears (sbq_linear_w8_grouped)
# ---------------------------------------------------------------------------
GROUP_CASES = [
    # (M, K, Ns, x dtype): the hybrid layer's pairs (lora up-projections,
    # SSE / SWA output projections), mixed and ragged widths, fp32 / bf16 x,
    # and M > 16 (no grouped kernel: each linear runs as linear_w8 alone, with
    # fp32 x the staged prefill path of its own workspace)
    (1, 128, (4096, 4096), "f16"),
    (1, 4096, (4096, 4096), "f16"),
    (4, 4096, (1000, 64, 4096, 4), "f16"),
    (16, 4096, (2048, 6144), "bf16"),
    (1, 4096, (4096, 4096, 4096), "f32"),
    (1, 12288, (4096, 10), "f16"),
    (24, 4096, (4096, 1000), "f16"), (20, 2560, (4096, 4096), "f32"), (40, 3008, (3888, 7472), "f32"),
    # M = 4 .. 8 over more than 1024 row tiles in all at K = 2560: five row
    # tiles per workgroup with x in LDS (fp32: split from registers), ragged
    # segments
    (8, 2560, (9728, 9728), "f16"), (8, 2560, (9728, 9728), "f32"), (4, 2560, (9000, 8000, 700), "bf16"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,Ns,xd", GROUP_CASES)
def test_grouped_linears(dev, M, K, Ns, xd):
    """Each output of a grouped call equals its linear run alone to fp32
    summation order, and the oracle within the weight-only tolerance; the
    module helper returns what each layer's forward returns."""
    announce(f"grouped linears M={M} K={K} Ns={Ns} x={xd}")
    ws = [gpu_weight(N, K, 900 + i, dev) for i, N in enumerate(Ns)]
    bs = [torch.randn(N, generator=torch.Generator().manual_seed(920 + i)) if i % 2 else None
          for i, N in enumerate(Ns)]
    lins = [quant.Int8Linear(w, None if b is None else b.to(dev)) for w, b in zip(ws, bs)]
    xs = [cpu_x(M, K, 910 + i).to(DT[xd]) for i in range(len(Ns))]
    xg = [x.to(dev) for x in xs]
    biases = [lin.bias for lin in lins]
    for yd in (torch.float32, torch.float16):
        got = quant.linear_w8_grouped(xg, [lin.packed for lin in lins], [lin.scale for lin in lins], biases,
                                      list(Ns), yd)
        for i, (lin, N) in enumerate(zip(lins, Ns)):
            sep = quant.linear_w8(xg[i], lin.packed, lin.scale, biases[i], N, yd)
            g = got[i].float().cpu().numpy()
            assert g.shape == (M, N)
            assert oracle.rel_l2(g, sep.float().cpu().numpy()) <= (1e-5 if yd == torch.float32 else 1e-3), (i, yd)
            cols = tile_sample(N, 930 + i)
            q, s = ref_rows(ws[i], cols)
            b = None if bs[i] is None else bs[i].numpy()[cols]
            ref = oracle.int8_linear(xs[i].float().numpy(), q, s, b)
            tol = W8_TOL_EXACT_X if (xd != "f32" and yd == torch.float32) else W8_TOL
            assert oracle.rel_l2(g[:, cols], ref) <= tol, (i, yd)
    outs = quant.grouped_forward(list(zip(lins, xg)))
    for lin, x, o in zip(lins, xg, outs):
        ref = lin(x)
        assert o.shape == ref.shape and o.dtype == ref.dtype
        assert oracle.rel_l2(o.cpu().numpy(), ref.cpu().numpy()) <= 1e-5


@pytest.mark.gpu
def test_grouped_linears_graph_replays(dev):
    """The grouped launch under HIP graph capture: every replay equals the
    eager result."""
    announce("grouped linears graph replays")
    K, Ns = 4096, (4096, 4096)
    lins = [quant.Int8Linear(gpu_weight(N, K, 940 + i, dev), None) for i, N in enumerate(Ns)]
    dyns = [quant.DynamicInt8Linear(gpu_weight(N, K, 960 + i, dev), None) for i, N in enumerate(Ns)]
    xg = [cpu_x(1, K, 950 + i).half().to(dev) for i in range(len(Ns))]
    outs = [torch.empty((1, N), dtype=torch.float16, device=dev) for N in Ns * 2]
    ws8 = quant.w8a8_workspace(1, K, dev)

    def run():  # weight-only and int8-dyn groups
        quant.linear_w8_grouped(xg, [lin.packed for lin in lins], [lin.scale for lin in lins], [None, None],
                                list(Ns), outs=outs[:2])
        quant.linear_w8a8_grouped(xg, [d.packed for d in dyns], [d.scale for d in dyns], [d.colsum for d in dyns],
                                  [None, None], list(Ns), outs=outs[2:], workspace=ws8)

    run()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    for _ in range(3):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e)


GROUP_W8A8_CASES = [
    # (M, K, Ns, x dtype): int8-dyn pairs of the hybrid layer (one fused
    # launch, each workgroup reducing its own linear's min/max), mixed and
    # ragged widths, and shapes that run one by one.  M = 8 at K = 2560 in
    # fp32 (80 KiB of x) runs as one fused five-row-tile launch (10 chunks per
    # thread) when the pair has enough row tiles, (9728, 9728); with
    # (4096, 4096) it exceeds the fused capacity of the other configurations
    # and runs one by one, as M > 16 does
    (1, 128, (4096, 4096), "f16"),
    (1, 4096, (2560, 2560), "f32"),
    (4, 4096, (1000, 64, 4096, 4), "bf16"),
    (16, 4096, (2048, 6144), "f16"),
    (1, 12288, (4096, 10), "f32"),
    (8, 2560, (9728, 9728), "f16"),
    (8, 2560, (4096, 4096), "f32"),
    (8, 4096, (2560, 2560), "f16"),
    (8, 2560, (9728, 9728), "f32"), (6, 2560, (9000, 9000), "bf16"),
    (24, 4096, (4096, 1000), "f16"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,Ns,xd", GROUP_W8A8_CASES)
def test_grouped_w8a8_linears(dev, M, K, Ns, xd):
    """Each output of a grouped int8-dyn call equals its linear run alone bit
    for bit (every x quantized with its own parameters), and the oracle's
    outputs bit-exactly on sampled channels; grouped_forward on
    DynamicInt8Linear layers returns what each layer's forward returns."""
    announce(f"grouped w8a8 linears M={M} K={K} Ns={Ns} x={xd}")
    ws = [gpu_weight(N, K, 2400 + i, dev) for i, N in enumerate(Ns)]
    bs = [torch.randn(N, generator=torch.Generator().manual_seed(2420 + i)) if i % 2 else None
          for i, N in enumerate(Ns)]
    dyns = [quant.DynamicInt8Linear(w, None if b is None else b.to(dev)) for w, b in zip(ws, bs)]
    xs = [(cpu_x(M, K, 2410 + i, outliers=True) * (1 + i)).to(DT[xd]) for i in range(len(Ns))]
    xg = [x.to(dev) for x in xs]
    for yd in (torch.float32, torch.float16):
        got = quant.linear_w8a8_grouped(xg, [d.packed for d in dyns], [d.scale for d in dyns],
                                        [d.colsum for d in dyns], [d.bias for d in dyns], list(Ns), yd)
        for i, (d, N) in enumerate(zip(dyns, Ns)):
            sep = quant.linear_w8a8(xg[i], d.packed, d.scale, d.colsum, d.bias, N, yd)
            assert got[i].shape == (M, N) and got[i].dtype == yd
            assert torch.equal(got[i], sep), (i, yd)
            if yd == torch.float32:
                cols = tile_sample(N, 2430 + i, cap=96)
                q, s = ref_rows(ws[i], cols)
                b = None if bs[i] is None else bs[i].numpy()[cols]
                _, y_ref = ref_w8a8(xs[i].float().numpy(), np.arange(M), q, s, b)
                np.testing.assert_array_equal(pick(got[i], np.arange(M), cols), y_ref)
    outs = quant.grouped_forward(list(zip(dyns, xg)))
    for d, x, o in zip(dyns, xg, outs):
        assert torch.equal(o, d(x))


# ---------------------------------------------------------------------------
# decode GEMV over several 16-row tiles of x (16 < M <= 64, weight-only)
# ---------------------------------------------------------------------------
MT_CASES = [  # (M, N, K, x dtype): ragged M, narrow / wide (two weight tiles per workgroup) / odd N, short and
    # long K; each within the path's 120 MB of x reads over the grid
    (17, 4096, 4096, "f16"), (24, 1000, 4096, "f16"), (32, 6144, 4096, "bf16"), (26, 18820, 4096, "f16"),
    (18, 4096, 12288, "f16"), (47, 4096, 4096, "bf16"), (64, 6144, 4096, "f16"), (64, 4096, 128, "f16"),
    (64, 10, 4096, "f16"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,xd", MT_CASES)
def test_w8_gemv_row_tiles(dev, M, N, K, xd):
    """fp16 / bf16 x at 16 < M <= 64: within fp32 summation order of the
    oracle for exactly representable inputs (fp32 y), one output rounding for
    2-byte y, with a bias and with strided x rows.  Each case runs twice: with
    the full workspace (the row-tile GEMV only where it beats the tiled GEMM's
    mid-sized-M plan) and with a workspace without the split area (then the
    row-tile GEMV takes every case here)."""
    announce(f"w8 gemv row tiles M={M} N={N} K={K} x={xd}")
    w = gpu_weight(N, K, 960, dev)
    b = torch.randn(N, generator=torch.Generator().manual_seed(961))
    lin = quant.Int8Linear(w, b.to(dev))
    cols = tile_sample(N, 962)
    q, s = ref_rows(w, cols)
    x = cpu_x(M, K, 963).to(DT[xd])
    ref = oracle.int8_linear(x.float().numpy(), q, s, b.numpy()[cols])
    wide = torch.zeros((M, K + 64), dtype=DT[xd], device=dev)
    for ws in (None, quant.w8_workspace(M, K, dev, DT[xd])):
        for xg in (x.to(dev), wide[:, :K].copy_(x.to(dev))):  # dense rows; rows 128 bytes apart beyond K
            y = quant.linear_w8(xg, lin.packed, lin.scale, lin.bias, N, workspace=ws)
            assert oracle.rel_l2(y.cpu().numpy()[:, cols], ref) <= W8_TOL_EXACT_X
            yh = quant.linear_w8(xg, lin.packed, lin.scale, lin.bias, N, torch.float16, workspace=ws)
            np.testing.assert_array_equal(yh.cpu().numpy(), y.half().cpu().numpy())


MT8_CASES = [  # (M, N, K): int8-dyn on the s8 rows of the quantize pre-pass, within the path's x-read cap
    (17, 4096, 4096), (32, 1000, 4096), (33, 6144, 4096), (48, 12288, 4096), (64, 4096, 4096), (40, 4096, 192),
]


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", MT8_CASES)
def test_w8a8_gemv_row_tiles(dev, M, N, K):
    """int8-dyn at 16 < M <= 64: int32 accumulators and outputs bit-exact
    against the oracle, with and without a bias, with the full workspace (the
    row-tile GEMV only where it beats the tiled GEMM's plan) and with one
    without the split area (the row-tile GEMV for every case here)."""
    announce(f"w8a8 gemv row tiles M={M} N={N} K={K}")
    w = gpu_weight(N, K, 970, dev)
    b = torch.randn(N, generator=torch.Generator().manual_seed(971))
    rows = np.arange(M)
    cols = tile_sample(N, 972)
    q, s = ref_rows(w, cols)
    x = cpu_x(M, K, 973, outliers=True)
    for bias, ws in ((None, None), (b, None), (None, quant.w8a8_workspace(M, K, dev)),
                     (b, quant.w8a8_workspace(M, K, dev))):
        lin = quant.DynamicInt8Linear(w, None if bias is None else bias.to(dev))
        acc = torch.empty((M, N), dtype=torch.int32, device=dev)
        y = quant.linear_w8a8(x.to(dev), lin.packed, lin.scale, lin.colsum, lin.bias, N, acc_out=acc, workspace=ws)
        acc_ref, y_ref = ref_w8a8(x.numpy(), rows, q, s, None if bias is None else bias.numpy()[cols])
        r_, c_ = torch.from_numpy(rows).to(dev), torch.from_numpy(cols).to(dev)
        np.testing.assert_array_equal(acc[r_][:, c_].cpu().numpy(), acc_ref)
        np.testing.assert_array_equal(pick(y, rows, cols), y_ref)


# ---------------------------------------------------------------------------
# activation pre-passes over every row layout
# ---------------------------------------------------------------------------
PREPASS_CASES = [  # (M, N, K): the tiled GEMM (M = 300), its split-K plan (M = 100); K = 8192 takes the staging
    # pass's two-read path (rows longer than its registers hold), K = 2576 ragged K tiles
    (300, 1000, 2560), (300, 1000, 8192), (100, 2048, 4096), (300, 520, 2576),
]


def _layout(x, layout, dev):
    """x [M, K] on the GPU as dense rows, 16-byte aligned rows 64 elements
    apart beyond K, or rows starting one element past a 16-byte boundary."""
    M, K = x.shape
    if layout == "dense":
        return x.to(dev)
    wide = torch.zeros((M, K + 64), dtype=x.dtype, device=dev)
    if layout == "strided":
        return wide[:, :K].copy_(x.to(dev))
    return wide[:, 1:1 + K].copy_(x.to(dev))


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", PREPASS_CASES)
@pytest.mark.parametrize("xd", ["f16", "bf16", "f32"])
def test_prepass_row_layouts_match_oracle(dev, M, N, K, xd):
    """The pre-passes in front of the GEMMs read dense rows as one flat array
    (min/max, quantize) and row by row otherwise; the staging pass holds a row
    in registers up to 4096 values and reads it twice beyond.  Every layout
    and activation dtype against the oracle on sampled rows and channels:
    int8-dyn acc and y bit-exact; weight-only within the fp16 GEMM bar for
    fp16 / bf16 x and 1e-3 for fp32 x (one staged fp16 plane)."""
    announce(f"pre-pass layouts M={M} N={N} K={K} x={xd}")
    w = gpu_weight(N, K, 980, dev)
    b = torch.randn(N, generator=torch.Generator().manual_seed(981))
    lin = quant.Int8Linear(w, b.to(dev))
    dyn = quant.DynamicInt8Linear(w, b.to(dev))
    cols = tile_sample(N, 982, cap=64)
    q, s = ref_rows(w, cols)
    del w
    x = cpu_x(M, K, 983, outliers=True).to(DT[xd])
    xv = x.float().numpy()
    rows = tile_sample(M, 984)
    r_, c_ = torch.from_numpy(rows).to(dev), torch.from_numpy(cols).to(dev)
    ref = oracle.int8_linear(xv[rows], q, s, b.numpy()[cols])
    acc_ref, y_ref = ref_w8a8(xv, rows, q, s, b.numpy()[cols])
    for layout in ("dense", "strided", "offset"):
        xg = _layout(x, layout, dev)
        y = quant.linear_w8(xg, lin.packed, lin.scale, lin.bias, N, workspace=quant.w8_workspace(M, K, dev, DT[xd], N))
        assert oracle.rel_l2(pick(y, rows, cols), ref) <= (W8_TOL if xd == "f32" else gemm_f16_tol(K)), layout
        acc = torch.empty((M, N), dtype=torch.int32, device=dev)
        y8 = quant.linear_w8a8(xg, dyn.packed, dyn.scale, dyn.colsum, dyn.bias, N, acc_out=acc,
                               workspace=quant.w8a8_workspace(M, K, dev, N, DT[xd]))
        np.testing.assert_array_equal(acc[r_][:, c_].cpu().numpy(), acc_ref, err_msg=layout)
        np.testing.assert_array_equal(pick(y8, rows, cols), y_ref, err_msg=layout)
