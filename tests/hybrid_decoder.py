"""A decoder with the hybrid layer's projection pattern, for the
device-resident state tests and the matching bench line.

This build's own toy, not the reference model (paths relative to the
reference repository): its numerics (a delta-rule recurrence with a shared
and routed partition states, window attention, full attention, a gated MLP,
RMS norms without weights, no rotary) are simplified stand-ins.  What it
reproduces is how the quantized linears are called, at the real checkpoint's
dimensions by default (hidden 2560, FFN 9728, 32 heads of 128, 8 kv heads,
lora 128, 4 router partitions, vocab 151936; config.py:16-21):

* hybrid layer (model.py:284-301,317-329,355-371): the eleven projections of
  the normed input (sse_q, sse_k, sse_v, lora_q[0], lora_k[0], sse_a, sse_b,
  sse_e, swa_q, swa_k, swa_v) as the parts of one fused launch, the lora
  chain lora_q[0] -> lora_q[1] and lora_k[0] -> lora_k[1] as one grouped
  launch, sse_o and swa_o of the two branch outputs as one grouped launch;
* softmax layer (model.py:250-270): q, k, v fused, o;
* every layer's MLP (model.py:235-240): gate and up fused, down;
* lm_head (model.py:410,447) quantized from the embedding (loader.py:89-95),
  with the greedy token (engine.py:30-31).

The state is sbq.state's (KV buffers with a window for the hybrid layers,
shared and partition recurrent states, position, token ids) on the device
the decoder is built for, so with the state on the GPU a step has static
shapes and can be captured in a HIP graph.  The projections go through a
backend: `SbqLinears` (the HIP modules, make_linear / fuse_linears /
grouped_forward / forward_greedy) or `OracleLinears` (the CPU oracle on the
same weights).  `taps` records every projection's input and output of the
last step (under a graph capture: the graph's own buffers, which every
replay rewrites).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from sbq import quant
from sbq.state import new_device_state

READS_X = ("sse_q", "sse_k", "sse_v", "lora_q0", "lora_k0", "sse_a", "sse_b", "sse_e", "swa_q", "swa_k", "swa_v")


class Dims:
    def __init__(self, H=2560, F=9728, heads=32, kv=8, d=128, parts=4, window=16, V=151936, kinds="hsh",
                 emb_scale=0.02):
        self.H, self.F, self.heads, self.kv, self.d = H, F, heads, kv, d
        self.parts, self.window, self.V = parts, window, V
        self.hybrid = [c == "h" for c in kinds]
        # the token's embedding enters the residual stream scaled down, so that
        # the layers (not the tied lm_head's echo of the input) pick the token
        self.emb_scale = emb_scale


def layer_shapes(dm: Dims, i: int) -> dict:
    """(N, K) of every projection of layer i, keyed by name."""
    H, F, h, kv, d = dm.H, dm.F, dm.heads, dm.kv, dm.d
    out = {}
    if dm.hybrid[i]:
        for n, N in zip(READS_X, (h * d, h * d, h * d, d, d, 2 * h, 2 * h, dm.parts, h * d, kv * d, kv * d)):
            out[n] = (N, H)
        out.update(lora_q1=(h * d, d), lora_k1=(h * d, d), sse_o=(H, h * d), swa_o=(H, h * d))
    else:
        out.update(q=(h * d, H), k=(kv * d, H), v=(kv * d, H), o=(H, h * d))
    out.update(gate=(F, H), up=(F, H), down=(H, F))
    return out


def make_weights(dm: Dims, seed=7, std=0.02):
    """bf16 CPU weights (as the checkpoint holds them) and the embedding."""
    g = torch.Generator().manual_seed(seed)
    w = {}
    for i in range(len(dm.hybrid)):
        for n, (N, K) in layer_shapes(dm, i).items():
            w[f"{i}.{n}"] = (torch.randn(N, K, generator=g) * std).to(torch.bfloat16)
    emb = torch.randn(dm.V, dm.H, generator=g).to(torch.bfloat16)
    return w, emb


class SbqLinears:
    """The HIP path: make_linear modules, the same-input groups fused
    (FusedLinear parts as drop-ins), independent pairs grouped, the lm_head
    with the fused greedy token."""

    def __init__(self, fmt, weights, emb, dm: Dims, device):
        self.mods = {n: quant.make_linear(fmt, w.to(device)) for n, w in weights.items()}
        self.lm_head = quant.make_linear(fmt, emb.to(device))
        self.parts = {}
        for i in range(len(dm.hybrid)):
            groups = [READS_X] if dm.hybrid[i] else [("q", "k", "v")]
            for grp in groups + [("gate", "up")]:
                fused = quant.fuse_linears([self.mods[f"{i}.{n}"] for n in grp])
                for j, n in enumerate(grp):
                    self.parts[f"{i}.{n}"] = fused.part(j)
        self.taps = {}

    def group(self, names, x):
        ys = [self.parts[n](x) for n in names]  # one launch, each part a drop-in module
        for n, y in zip(names, ys):
            self.taps[n] = (x, y)
        return ys

    def pair(self, names, xs):
        ys = quant.grouped_forward([(self.mods[n], x) for n, x in zip(names, xs)])
        for n, x, y in zip(names, xs, ys):
            self.taps[n] = (x, y)
        return ys

    def single(self, name, x):
        y = self.mods[name](x)
        self.taps[name] = (x, y)
        return y

    def head(self, x):
        if x.is_cuda:
            logits, tok = self.lm_head.forward_greedy(x)
        else:  # the reference's placement: CPU logits, the token by argmax there
            logits = self.lm_head(x)
            tok = torch.argmax(logits, dim=-1)
        self.taps["lm_head"] = (x, logits)
        return logits, tok


def oracle_weights(weights, emb):
    """The oracle's (q, scale) of every weight and of the lm_head."""
    import oracle  # the checker, loaded only by the tests that use it

    q = {n: oracle.quantize_per_channel(w.float().numpy()) for n, w in weights.items()}
    q["lm_head"] = oracle.quantize_per_channel(emb.float().numpy())
    return q


class OracleLinears:
    """The CPU oracle on the same weights: each projection is the oracle's
    int8_linear (quant.py:41-53) or dyn_linear (quant.py:63-66) of its own
    input, the weights quantized by the oracle's quantize_per_channel; the
    greedy token is torch.argmax of the logits on the CPU (engine.py:30-31).
    `q` holds every weight's (q, scale) for the per-projection checks."""

    def __init__(self, fmt, weights, emb, q=None):
        self.fmt = fmt
        self.q = q if q is not None else oracle_weights(weights, emb)
        self.taps = {}

    def apply(self, name, x: np.ndarray) -> np.ndarray:
        import oracle

        q, s = self.q[name]
        return oracle.int8_linear(x, q, s) if self.fmt == "int8" else oracle.dyn_linear(x, q, s)

    def _run(self, name, x):
        y = torch.from_numpy(self.apply(name, x.float().numpy()))
        self.taps[name] = (x, y)
        return y

    def group(self, names, x):
        return [self._run(n, x) for n in names]

    def pair(self, names, xs):
        return [self._run(n, x) for n, x in zip(names, xs)]

    def single(self, name, x):
        return self._run(name, x)

    def head(self, x):
        logits = self._run("lm_head", x)
        return logits, torch.argmax(logits, dim=-1)


def _norm(t):
    return t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + 1e-6)


def _l2(t):
    return t / torch.sqrt(t.pow(2).sum(-1, keepdim=True) + 1e-6)


class HybridDecoder:
    def __init__(self, lin, emb, dm: Dims, device, capacity=64):
        self.lin, self.dm = lin, dm
        self.dev = torch.device(device)
        self.emb = emb.to(self.dev)
        self.state = new_device_state(dm.hybrid, dm.heads, dm.d, dm.kv, dm.parts, dm.window, capacity, self.dev)
        self.scale = dm.d ** -0.5

    def reset(self, token: int):
        self.state.reset(token)

    def _attend(self, q, kv, mask):
        """q [heads, d] against the buffer's keys [slots, kv, d] (GQA: head h
        reads kv head h // (heads / kv)), masked to the visible slots."""
        dm = self.dm
        rep = dm.heads // dm.kv
        k = kv.k.transpose(0, 1).repeat_interleave(rep, 0)  # [heads, slots, d]
        v = kv.v.transpose(0, 1).repeat_interleave(rep, 0)
        s = torch.matmul(k, q.unsqueeze(-1)).squeeze(-1) * self.scale  # [heads, slots]
        s = s.masked_fill(~mask, float("-inf"))
        return torch.matmul(torch.softmax(s, -1).unsqueeze(1), v).reshape(1, dm.heads * dm.d)

    def _delta(self, S, q, k, v, decay, beta):
        """One delta-rule update of S [heads, d, d] with k, v [heads, d];
        returns S^T q after the update."""
        pred = torch.matmul(k.unsqueeze(1), S).squeeze(1)  # [heads, d]
        S.mul_(decay[:, None, None])
        S.add_(k.unsqueeze(-1) * (beta[:, None] * (v - pred)).unsqueeze(1))
        return torch.matmul(q.unsqueeze(1), S).squeeze(1)

    def step(self, tok=None):
        """One decode step from token ids tok [1] (default: the state's next
        token); returns the logits [1, V] and stores the greedy token."""
        dm, st, P = self.dm, self.state, self.lin
        tok = st.next_token if tok is None else tok.to(self.dev)
        st.record(tok)
        pos = st.position
        x = self.emb.index_select(0, tok).float() * dm.emb_scale  # [1, H]
        h_, d = dm.heads, dm.d
        for i, layer in enumerate(st.layers):
            p = f"{i}."
            h = _norm(x)
            if dm.hybrid[i]:
                sq, sk, sv, lq0, lk0, a, b, e, wq, wk, wv = P.group([p + n for n in READS_X], h)
                lq1, lk1 = P.pair([p + "lora_q1", p + "lora_k1"], [lq0, lk0])
                v = F.silu(sv).view(h_, d)
                q1, k1 = _l2(F.silu(sq).view(h_, d)) * self.scale, _l2(F.silu(sk).view(h_, d))
                q2, k2 = _l2(F.silu(sq + lq1).view(h_, d)) * self.scale, _l2(F.silu(sk + lk1).view(h_, d))
                decay = torch.exp(-F.softplus(a.view(-1)[:h_]))
                beta = torch.sigmoid(b.view(-1)[:h_])
                eta = torch.softmax(e.view(-1), -1)  # router weights of the partitions
                o = self._delta(layer.shared, q1, k1, v, decay, beta)
                for j in range(dm.parts):
                    o = o + eta[j] * self._delta(layer.partitions[j], q2, k2, v, decay, beta * eta[j])
                sse_in = _norm(o).reshape(1, h_ * d)
                layer.kv.append(wk.view(1, dm.kv, d), wv.view(1, dm.kv, d), pos)
                swa_in = self._attend(wq.view(h_, d), layer.kv, layer.kv.visible(pos)[0])
                so, wo = P.pair([p + "sse_o", p + "swa_o"], [sse_in, swa_in])
                x = x + (_norm(so) + _norm(wo)) * 0.5
            else:
                q, k, v = P.group([p + "q", p + "k", p + "v"], h)
                layer.kv.append(k.view(1, dm.kv, d), v.view(1, dm.kv, d), pos)
                att = self._attend(q.view(h_, d), layer.kv, layer.kv.visible(pos)[0])
                x = x + P.single(p + "o", att)
            h = _norm(x)
            g, u = P.group([p + "gate", p + "up"], h)
            x = x + P.single(p + "down", F.silu(g) * u)
        logits, nxt = P.head(_norm(x))
        st.next_token.copy_(nxt.reshape(1).to(st.next_token.device))
        st.advance(1)
        return logits
