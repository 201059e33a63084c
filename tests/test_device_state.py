"""Device-resident model state (sbq.state) and the hybrid-layer decode step
over it.

CPU tests (no GPU): DeviceKVBuffer against a restatement of the reference's
KVBuffer semantics (model.py:61-85, paths relative to the reference
repository): the keys a query attends to after any sequence of appends,
with and without a window, equal the keys the reference's append returns
under the mask its attention applies (model.py:208-229); truncation;
new_device_state's layout (model.py:412-424).

GPU test: the hybrid decoder (tests/hybrid_decoder.py) at the real
checkpoint's dimensions with its whole state on the GPU, eager and replayed
from one captured HIP graph per token, every projection of every step
checked against the oracle on the device's own inputs, and the whole decode
against a run with the state on the CPU in which every projection is the
oracle's.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import announce
from sbq.state import DeviceKVBuffer, new_device_state


# ---------------------------------------------------------------------------
# state containers (CPU)
# ---------------------------------------------------------------------------
class _RefKV:
    """The reference KVBuffer's contract: append returns the keys / values
    visible to the new tokens (all stored ones, or with a window the last
    `window` stored before the call plus the new ones), positions ending at
    the last new token."""

    def __init__(self, window):
        self.window = window
        self.k = []  # (position, key) pairs, in order

    def append(self, start, ks):
        keys = (self.k if self.window is None else self.k[-self.window:]) + [(start + i, k) for i, k in enumerate(ks)]
        self.k = keys if self.window is None else keys[-self.window:]
        return keys


def _visible_ref(keys, qpos, window):
    """What the attention of model.py:208-229 lets a query at qpos see."""
    return {p for p, _ in keys if p <= qpos and (window is None or p > qpos - window)}


@pytest.mark.parametrize("window", [None, 3, 5])
def test_device_kv_buffer_matches_reference_semantics(window):
    g = torch.Generator().manual_seed(0)
    heads, dim = 2, 4
    chunks = [1, 3, 1, 1, 2, 1, 1, 1, 4, 1, 1]
    buf = DeviceKVBuffer(heads, dim, capacity=32 if window is None else window + 4, window=window, device="cpu")
    ref = _RefKV(window)
    pos = 0
    for T in chunks:
        k = torch.randn(T, heads, dim, generator=g)
        v = torch.randn(T, heads, dim, generator=g)
        keys_ref = ref.append(pos, [k[i] for i in range(T)])
        kk, vv, slot_pos = buf.append(k, v, torch.tensor([pos]))
        assert int(buf.end) == pos + T
        qpos = torch.arange(pos, pos + T)
        mask = buf.visible(qpos)
        for t in range(T):
            seen = {int(slot_pos[s]) for s in range(buf.capacity) if mask[t, s]}
            assert seen == _visible_ref(keys_ref, pos + t, window), (T, pos, t)
            for s in range(buf.capacity):  # the slot holding a position holds its key and value
                if mask[t, s]:
                    p = int(slot_pos[s])
                    kref = dict(keys_ref)[p]
                    assert torch.equal(kk[s], kref)
        pos += T
    # truncation forgets later positions (the engine's prefix reuse)
    buf.truncate(pos - 2)
    assert int(buf.end) == pos - 2
    assert int(buf.slot_pos.max()) <= pos - 3


def test_device_kv_buffer_rejects_bad_sizes():
    with pytest.raises(ValueError):
        DeviceKVBuffer(2, 4, capacity=3, window=3, device="cpu")
    buf = DeviceKVBuffer(2, 4, capacity=5, window=3, device="cpu")
    with pytest.raises(ValueError):
        buf.append(torch.zeros(3, 2, 4), torch.zeros(3, 2, 4))  # more than the ring holds beside the window
    with pytest.raises(ValueError):
        buf.append(torch.zeros(1, 3, 4), torch.zeros(1, 3, 4))


def test_new_device_state_layout():
    st = new_device_state([True, False, True], heads=4, head_dim=8, kv_heads=2, partitions=3, window=5, capacity=16,
                          device="cpu")
    assert [lay.shared is not None for lay in st.layers] == [True, False, True]
    h = st.layers[0]
    assert tuple(h.shared.shape) == (4, 8, 8) and tuple(h.partitions.shape) == (3, 4, 8, 8)
    assert h.kv.window == 5 and h.kv.capacity == 6 and st.layers[1].kv.window is None
    assert st.layers[1].kv.capacity == 16
    h.shared.fill_(1.0)
    st.next_token.fill_(9)
    st.position.fill_(3)
    st.reset(4)
    assert float(h.shared.abs().sum()) == 0.0 and int(st.position) == 0 and int(st.next_token) == 4
    st.record(torch.tensor([7, 8]))
    assert st.tokens[:3].tolist() == [7, 8, 0]


# ---------------------------------------------------------------------------
# the hybrid-layer decode step with its state on the GPU, against the oracle
# ---------------------------------------------------------------------------
W8_TOL = 1e-3


def _cols(N, name, cap=48):
    """One output channel per sampled 16-row tile, plus the last."""
    rng = np.random.default_rng(sum(map(ord, name)))
    starts = np.arange(0, N, 16)
    if len(starts) > cap:
        starts = np.unique(np.linspace(0, len(starts) - 1, cap).astype(int)) * 16
    return np.unique(np.append(np.minimum(starts + rng.integers(0, 16, len(starts)), N - 1), N - 1))


def _check_taps(taps, orc, fmt, what):
    """Every projection of the step on its own (device) input against the
    oracle on sampled output channels: int8 rel-L2 <= 1e-3, int8-dyn
    bit-exact (the activation parameters of the whole input)."""
    assert len(taps) > 0
    for name, (x, y) in taps.items():
        q, s = orc.q[name]
        cols = _cols(q.shape[0], name)
        xn = x.float().cpu().numpy().reshape(1, -1)
        got = y.reshape(1, -1)[:, torch.from_numpy(cols).to(y.device)].float().cpu().numpy()
        if fmt == "int8":
            ref = oracle.int8_linear(xn, q[cols], s[cols])
            assert oracle.rel_l2(got, ref) <= W8_TOL, (what, name)
        else:
            ref = oracle.dyn_linear(xn, q[cols], s[cols])
            np.testing.assert_array_equal(got, ref, err_msg=f"{what} {name}")


@pytest.fixture(scope="module")
def hybrid_weights():
    from hybrid_decoder import Dims, make_weights, oracle_weights

    dm = Dims()
    w, emb = make_weights(dm)
    return dm, w, emb, oracle_weights(w, emb)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int8", "int8-dyn"])
def test_hybrid_decode_device_state_vs_oracle(dev, hybrid_weights, fmt):
    """The hybrid layer's launch pattern (fused reads-x group, grouped lora
    chain and output pair, fused gate+up, lm_head with the fused greedy
    token) with every state tensor on the GPU.
      * eager steps: every projection checked against the oracle on the
        device's own inputs;
      * one step captured in a HIP graph and replayed per token from the
        reset state: the same tokens and bit-identical logits as the eager
        steps, and every projection of every replay (the graph's own
        buffers) against the oracle again;
      * the same decode with its state on the CPU and every projection the
        oracle's (the reference's placement; teacher-forced with the
        device's tokens): logits within rel-L2 1e-3 (int8) / 2e-2 (int8-dyn:
        the non-projection math runs on another device, and a one-ulp
        difference in an input can move activations across a quantization
        step), and the same greedy token wherever the CPU logits' top-2
        margin exceeds twice the largest logit difference."""
    from hybrid_decoder import HybridDecoder, OracleLinears, SbqLinears

    dm, w, emb, qw = hybrid_weights
    orc = OracleLinears(fmt, w, emb, qw)
    announce(f"hybrid device-state decode fmt={fmt}: building the HIP modules")
    gpu = HybridDecoder(SbqLinears(fmt, w, emb, dm, dev), emb, dm, dev)
    steps, first = 6, 11
    eager_logits, eager_tok = [], []
    with torch.no_grad():
        gpu.reset(first)
        for t in range(steps):
            announce(f"hybrid fmt={fmt} eager step {t}")
            eager_logits.append(gpu.step().clone())
            eager_tok.append(int(gpu.state.next_token.item()))
            _check_taps(gpu.lin.taps, orc, fmt, f"eager step {t}")
        assert int(gpu.state.position.item()) == steps
        # one step captured (the warm-up creates the argmax state and workspaces)
        announce(f"hybrid fmt={fmt} graph capture")
        gpu.reset(first)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            gpu.step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            logits = gpu.step()
        gpu.reset(first)
        for t in range(steps):
            announce(f"hybrid fmt={fmt} graph replay {t}")
            g.replay()
            torch.cuda.synchronize()
            assert int(gpu.state.next_token.item()) == eager_tok[t], t
            np.testing.assert_array_equal(logits.cpu().numpy(), eager_logits[t].cpu().numpy())
            _check_taps(gpu.lin.taps, orc, fmt, f"graph replay {t}")
        assert int(gpu.state.position.item()) == steps
        del g
    # the reference's placement, every projection the oracle's
    cpu = HybridDecoder(orc, emb, dm, "cpu")
    cpu.reset(first)
    tol = W8_TOL if fmt == "int8" else 2e-2
    for t in range(4):
        announce(f"hybrid fmt={fmt} oracle step {t} (state on the CPU)")
        inp = torch.tensor([first if t == 0 else eager_tok[t - 1]])
        lc = cpu.step(inp)[0]
        ld = eager_logits[t][0].cpu()
        assert lc.device.type == "cpu"
        assert oracle.rel_l2(ld.numpy(), lc.numpy()) <= tol, t
        diff = float((ld - lc).abs().max())
        top2 = torch.topk(lc, 2).values
        if float(top2[0] - top2[1]) > 2 * diff:
            assert int(torch.argmax(lc)) == eager_tok[t], t
