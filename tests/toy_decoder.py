"""A small decoder over the quantized linears, for the device-resident model
state tests and the matching bench line.

It is this build's own toy, not the reference model: embedding, blocks of
q/k/v/o projections around causal attention over a KV cache and a gated MLP
(the projection pattern of model.py:240-270, paths relative to the reference
repository), an RMS norm, and the lm_head tied to the embedding
(loader.py:89-95).  Every linear comes from make_linear, as loader.py:46-51
builds them.

Its state (KV cache, position, the next token's id) lives on `state_device`:
  * "cpu": where the reference model keeps it (KVBuffer model.py:66-67,82-83,
    LayerState model.py:420-421, token ids model.py:440); every projection
    then copies its input to the GPU and its output back, and the greedy token
    is torch.argmax on the CPU logits (engine.py:30-31);
  * the GPU: every tensor stays in HBM, the lm_head picks the greedy token in
    the same launch (forward_greedy), and the token feeds the next step's
    embedding lookup on the device.  The shapes are static (a max_len cache
    with a position mask), so one step can be captured in a HIP graph and
    replayed once per token with no host work in between.
"""
from __future__ import annotations

import torch

from sbq import quant


def toy_weights(H, F, blocks, V, seed=4, std=0.02):
    g = torch.Generator().manual_seed(seed)
    shapes = {"q": (H, H), "k": (H, H), "v": (H, H), "o": (H, H), "gate": (F, H), "up": (F, H), "down": (H, F)}
    weights = {f"{b}.{n}": torch.randn(*s, generator=g) * std for b in range(blocks) for n, s in shapes.items()}
    emb = torch.randn(V, H, generator=g)
    return weights, emb


class ToyDecoder:
    def __init__(self, fmt, weights, emb, heads, max_len, state_device):
        self.lin = {n: quant.make_linear(fmt, w) for n, w in weights.items()}
        self.lm_head = quant.make_linear(fmt, emb)
        self.blocks = len({n.split(".")[0] for n in weights})
        self.V, self.H = emb.shape
        self.heads, self.d = heads, self.H // heads
        self.max_len = max_len
        dev = torch.device(state_device)
        self.dev = dev
        self.emb = emb.to(dev)
        self.kc = torch.zeros(self.blocks, heads, max_len, self.d, device=dev)
        self.vc = torch.zeros(self.blocks, heads, max_len, self.d, device=dev)
        self.pos = torch.zeros((1,), dtype=torch.long, device=dev)
        self.ar = torch.arange(max_len, device=dev)
        self.tok = torch.zeros((1,), dtype=torch.long, device=dev)

    def reset(self, token: int):
        self.kc.zero_()
        self.vc.zero_()
        self.pos.zero_()
        self.tok.fill_(token)

    @staticmethod
    def _norm(t):
        return t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + 1e-6)

    def hidden(self, tok):
        """One decode step up to the lm_head input, for token ids `tok` [1]."""
        heads, d, H = self.heads, self.d, self.H
        x = self.emb.index_select(0, tok)  # [1, H]
        for b in range(self.blocks):
            h = self._norm(x)
            q, k, v = (self.lin[f"{b}.{p}"](h).view(heads, 1, d) for p in ("q", "k", "v"))
            self.kc[b].index_copy_(1, self.pos, k)
            self.vc[b].index_copy_(1, self.pos, v)
            s = (self.kc[b] @ q.transpose(1, 2).contiguous()).squeeze(-1) / d ** 0.5  # [heads, max_len]
            s = s.masked_fill(self.ar > self.pos, float("-inf"))
            att = torch.softmax(s, dim=-1).unsqueeze(1) @ self.vc[b]  # [heads, 1, d]
            x = x + self.lin[f"{b}.o"](att.reshape(1, H))
            h = self._norm(x)
            x = x + self.lin[f"{b}.down"](torch.nn.functional.silu(self.lin[f"{b}.gate"](h)) * self.lin[f"{b}.up"](h))
        self.pos += 1
        return self._norm(x)

    def step_cpu_state(self, tok=None):
        """The reference's placement: logits on the CPU, the token by
        torch.argmax there.  `tok` overrides the stored token (teacher
        forcing); returns the CPU logits [V] and stores the greedy token."""
        t = self.tok if tok is None else tok
        logits = self.lm_head(self.hidden(t))[0]
        self.tok.copy_(torch.argmax(logits).view(1))
        return logits

    def step_device(self, tok=None):
        """Everything on the GPU: logits [V] and the greedy token from one
        lm_head launch; the token is stored for the next step on the device."""
        t = self.tok if tok is None else tok
        logits, nxt = self.lm_head.forward_greedy(self.hidden(t))
        self.tok.copy_(nxt)
        return logits[0]
