"""Decode-time lattice state kept between forward calls: the prefix cache.

Interface of model/prefix_cache.py: `enabled` (:47-55), `budget_bytes` (:58-60), `state_bytes`
(:63-70), `describe` (:73-77), `affordable` (:80-97) and `PrefixCache` (:100-168), with the same
names, arguments and semantics:

* a layer's slot holds its fp32 lattice state [batch, K, d_e, d_m], or None before the layer has
  run (the mixer then starts from zeros);
* the size is fixed per sequence -- K * d_e * d_m floats per layer -- whatever the context length,
  so a byte ceiling limits the batch, and a cache over the ceiling is refused, never trimmed
  (the state summarises every token so far; no part of it belongs to an oldest token);
* `put` stores a detached tensor, so no autograd graph lives across decode calls;
* `len(cache)` is the number of tokens absorbed, `cache.layers` the number of slots.

The switch and the ceiling come from `mira_amd.config.INFERENCE`, read at call time.

One addition: `in_place`. When it is True a single-token mixer step overwrites the held state
tensor instead of returning a new one (no allocation per step, so a decode step can be captured
in a HIP graph and replayed on the same memory). A caller that keeps references to earlier
states must leave it False, the default, which keeps the reference's contract that `put` swaps in
a new tensor and earlier ones stay unchanged. `mira_amd.generate` owns its cache and sets it.
"""
from __future__ import annotations

import torch

from . import config

DTYPE = torch.float32        # the scan's state is fp32 whatever the model's dtype
BYTES = 4
GIB = float(1 << 30)


def enabled() -> bool:
    """Whether inference paths may carry a prefix cache (INFERENCE["prefix_cache"])."""
    return bool(int(config.INFERENCE.get("prefix_cache", 0)))


def budget_bytes() -> int:
    """The configured ceiling in bytes (INFERENCE["prefix_cache_size"] GiB), 0 for none."""
    return int(float(config.INFERENCE.get("prefix_cache_size", 0)) * GIB)


def state_bytes(layers, batch, order, channels, memory) -> int:
    """Bytes one cache of this geometry holds once every layer has run; there is no sequence
    length in it."""
    count = 1
    for extent in (layers, batch, order, channels, memory):
        count *= int(extent)
    return count * BYTES


def describe(layers, batch, order, channels, memory) -> str:
    """A one-line account of a geometry and its size."""
    total = state_bytes(layers, batch, order, channels, memory)
    per_layer = total / max(int(layers), 1)
    return (f"prefix cache: {layers} layers, batch {batch}, K={order}, d_e={channels}, "
            f"d_m={memory}: {total / GIB:.3f} GiB in all, {per_layer / 1024:.0f} KiB a layer")


def affordable(layers, batch, order, channels, memory, budget=None):
    """(True, "") when a cache of this geometry fits the ceiling (`budget` bytes, or the
    configured one when None; 0 means no ceiling), else (False, reason)."""
    need = state_bytes(layers, batch, order, channels, memory)
    ceiling = budget_bytes() if budget is None else int(budget)
    if not ceiling or need <= ceiling:
        return True, ""
    return False, (f"{describe(layers, batch, order, channels, memory)} exceeds the "
                   f"{ceiling / GIB:.3f} GiB ceiling (INFERENCE['prefix_cache_size']); only a "
                   f"smaller batch fits -- the state is the same size at any context length")


class PrefixCache:
    """Per-layer lattice state between forward calls (see the module docstring)."""

    def __init__(self, layers, budget=None):
        self.layers = int(layers)
        self.budget = budget_bytes() if budget is None else int(budget)
        self.state = [None for _ in range(self.layers)]
        self.tokens = 0
        self.key_valid = None        # [B, tokens so far] bool history of real tokens, or None
        self.in_place = False

    def __len__(self):
        return self.tokens

    def get(self, layer):
        return self.state[int(layer)]

    def put(self, layer, state):
        held = state.detach() if state is not None else None
        self.state[int(layer)] = held
        return held

    def advance(self, tokens):
        self.tokens = self.tokens + int(tokens)

    def clear_states(self):
        """Forget every layer's state, the token count and the mask history."""
        self.state = [None for _ in range(self.layers)]
        self.tokens = 0
        self.key_valid = None

    def reset(self, model):
        """Let `model` clear the slots (its reset_states), then forget the count and history."""
        model.reset_states(self.state)
        self.tokens = 0
        self.key_valid = None

    def nbytes(self) -> int:
        return sum(held.numel() * held.element_size() for held in self.state if held is not None)

    def within_budget(self):
        """(True, "") when what is held fits the ceiling, else (False, reason)."""
        held = self.nbytes()
        if not self.budget or held <= self.budget:
            return True, ""
        return False, (f"prefix cache holds {held / GIB:.3f} GiB, over its "
                       f"{self.budget / GIB:.3f} GiB ceiling")
