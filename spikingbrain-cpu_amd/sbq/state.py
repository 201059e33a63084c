"""Device-resident decode state for the callers of the quantized linears.

The reference model keeps its inference state on the CPU (paths relative to
the reference repository):

* ``KVBuffer`` (model.py:61-85) grows CPU key / value tensors, or keeps the
  last ``window`` positions of a sliding-window layer;
* ``LayerState`` (model.py:94-97) adds a hybrid layer's shared [H, K, V] and
  partition [P, H, K, V] recurrent states;
* ``new_state`` (model.py:412-424) zero-initialises one of them per layer;
* ``forward_tokens`` builds the token ids as a CPU tensor (model.py:440) and
  the engine picks the next token on the CPU logits (engine.py:29-31).

With the linears on the GPU every projection then pays a host round trip.
The classes here hold the same state in HBM with fixed capacities: every
tensor keeps its address from step to step, positions are device tensors, a
key / value append is an ``index_copy_`` at slots computed on the device,
and which keys a query sees is given by the position each slot holds (a mask
for the attention) rather than by slicing.  A whole decode step, the token
feeding the next step included, can therefore be captured in a HIP graph and
replayed once per token with no host work in between.

Capacity: a full-attention buffer holds ``capacity`` positions (slot =
position).  A sliding-window buffer is a ring of ``capacity`` slots (slot =
position mod capacity); it must hold the window plus the tokens appended by
one call, so that no key a query of that call sees is overwritten.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch


def _as_pos(p, device: torch.device) -> torch.Tensor:
    if isinstance(p, torch.Tensor):
        return p.reshape(1).to(device=device, dtype=torch.long)
    return torch.tensor([int(p)], dtype=torch.long, device=device)


class DeviceKVBuffer:
    """model.py:61-85 KVBuffer with its storage in device memory.

    ``append(k, v)`` stores [T, heads, dim] keys / values at the positions
    ``end .. end + T - 1`` and returns ``(keys, values, slot_pos)``: the whole
    storage [slots, heads, dim] and the position each slot holds (-1 for an
    empty slot).  ``visible(q_pos)`` is the attention mask of queries at
    positions ``q_pos`` [T]: the slots holding a position <= the query's
    and, for a window, > the query's position - window, which are the keys the
    reference's ``append`` returns together with the mask its ``attention``
    (model.py:208-229) applies to them."""

    def __init__(self, heads: int, dim: int, capacity: int, window: int | None = None,
                 device: torch.device | str | None = None, dtype: torch.dtype = torch.float32):
        if capacity < 1 or (window is not None and (window < 1 or capacity < window + 1)):
            raise ValueError("DeviceKVBuffer: capacity must be >= 1, and >= window + 1 for a window")
        self.heads, self.dim, self.window, self.capacity = heads, dim, window, capacity
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.k = torch.zeros(capacity, heads, dim, dtype=dtype, device=dev)
        self.v = torch.zeros(capacity, heads, dim, dtype=dtype, device=dev)
        self.slot_pos = torch.full((capacity,), -1, dtype=torch.long, device=dev)
        self.end = torch.zeros((1,), dtype=torch.long, device=dev)  # next position to write

    @property
    def device(self) -> torch.device:
        return self.k.device

    def reset(self) -> None:
        self.k.zero_()
        self.v.zero_()
        self.slot_pos.fill_(-1)
        self.end.zero_()

    def append(self, k: torch.Tensor, v: torch.Tensor, start=None):
        """Store k, v [T, heads, dim] at positions start .. start + T - 1
        (default: after the last append); start may be an int or a device
        tensor (graph capture).  With a window, T must be <= capacity -
        window (the ring keeps every key the new queries see)."""
        T = k.shape[0]
        if tuple(k.shape[1:]) != (self.heads, self.dim) or k.shape != v.shape:
            raise ValueError(f"DeviceKVBuffer.append: expected [T, {self.heads}, {self.dim}] keys and values")
        if self.window is not None and T > self.capacity - self.window:
            raise ValueError("DeviceKVBuffer.append: more tokens than the ring holds beside the window")
        s = self.end if start is None else _as_pos(start, self.device)
        pos = s + torch.arange(T, device=self.device)
        slots = pos % self.capacity if self.window is not None else pos
        self.k.index_copy_(0, slots, k.to(self.k.dtype))
        self.v.index_copy_(0, slots, v.to(self.v.dtype))
        self.slot_pos.index_copy_(0, slots, pos)
        self.end.copy_(s + T)
        return self.k, self.v, self.slot_pos

    def visible(self, q_pos: torch.Tensor) -> torch.Tensor:
        """Boolean [T, slots]: which stored keys queries at q_pos [T] attend to."""
        kp = self.slot_pos[None, :]
        qp = q_pos.reshape(-1, 1)
        ok = (kp >= 0) & (kp <= qp)
        if self.window is not None:
            ok &= kp > qp - self.window
        return ok

    def truncate(self, length) -> None:
        """Forget positions >= length (the engine's prefix reuse restores a
        shorter length, model.py:119-127); length may be a device tensor."""
        n = _as_pos(length, self.device)
        self.slot_pos.masked_fill_(self.slot_pos >= n, -1)
        self.end.copy_(torch.minimum(self.end, n))


@dataclass
class DeviceLayerState:
    """model.py:94-97 LayerState: the layer's key / value buffer and, for a
    hybrid layer, its shared [H, K, V] and partition [P, H, K, V] states."""

    kv: DeviceKVBuffer
    shared: torch.Tensor | None = None
    partitions: torch.Tensor | None = None

    def reset(self) -> None:
        self.kv.reset()
        if self.shared is not None:
            self.shared.zero_()
            self.partitions.zero_()


@dataclass
class DeviceInferenceState:
    """model.py:99-103 InferenceState on the device: ``position`` is the next
    token's position (device long [1]), ``tokens`` the ids fed so far
    (device long [capacity], written at their positions) and ``next_token``
    the id the next decode step embeds (the greedy token of the last one)."""

    layers: list[DeviceLayerState]
    position: torch.Tensor
    tokens: torch.Tensor
    next_token: torch.Tensor = field(default=None)

    def reset(self, token: int | None = None) -> None:
        for layer in self.layers:
            layer.reset()
        self.position.zero_()
        self.tokens.zero_()
        if token is not None:
            self.next_token.fill_(int(token))

    def record(self, token_ids: torch.Tensor) -> None:
        """Write the ids of the tokens about to be fed at the current position."""
        T = token_ids.numel()
        idx = self.position + torch.arange(T, device=self.position.device)
        self.tokens.index_copy_(0, idx.clamp_(max=self.tokens.numel() - 1), token_ids.reshape(-1).long())

    def advance(self, T: int) -> None:
        self.position += T


def new_device_state(hybrid: list[bool], heads: int, head_dim: int, kv_heads: int, partitions: int,
                     window: int, capacity: int, device: torch.device | str | None = None,
                     ring_extra: int = 1) -> DeviceInferenceState:
    """model.py:412-424 new_state on the device: per layer a key / value
    buffer (windowed, a ring of window + ring_extra slots, for hybrid layers;
    `capacity` positions for softmax layers) and, for hybrid layers, zeroed
    shared [heads, head_dim, head_dim] and partition [partitions, heads,
    head_dim, head_dim] fp32 states.  ring_extra is the most tokens one call
    appends (1 for decode; the prefill chunk otherwise)."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    layers = []
    for is_hybrid in hybrid:
        if is_hybrid:
            layers.append(DeviceLayerState(
                kv=DeviceKVBuffer(kv_heads, head_dim, window + ring_extra, window, dev),
                shared=torch.zeros(heads, head_dim, head_dim, device=dev),
                partitions=torch.zeros(partitions, heads, head_dim, head_dim, device=dev)))
        else:
            layers.append(DeviceLayerState(kv=DeviceKVBuffer(kv_heads, head_dim, capacity, None, dev)))
    return DeviceInferenceState(layers=layers, position=torch.zeros((1,), dtype=torch.long, device=dev),
                                tokens=torch.zeros((capacity,), dtype=torch.long, device=dev),
                                next_token=torch.zeros((1,), dtype=torch.long, device=dev))
