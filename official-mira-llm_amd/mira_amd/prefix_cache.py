"""The inference-only decode state the mixer carries between calls (model/prefix_cache.py:100-168).

One float32 [B, K, d_e, d_m] slot per layer; `put` detaches; nothing is trimmed; the byte budget
is checked, never enforced by truncation. `tokens` counts the tokens the state has absorbed,
which is also the `pos` a conv ring buffer needs.
"""
from __future__ import annotations

import torch

DTYPE = torch.float32
BYTES = 4
GIB = 1024 ** 3


def state_bytes(layers, batch, order, channels, memory):
    """Bytes of one cache of this geometry; independent of sequence length
    (model/prefix_cache.py:67-73)."""
    return int(layers) * int(batch) * int(order) * int(channels) * int(memory) * BYTES


def affordable(layers, batch, order, channels, memory, budget=0):
    """(fits?, why not) (model/prefix_cache.py:83-97)."""
    need = state_bytes(layers, batch, order, channels, memory)
    if budget and need > budget:
        return False, (f"the prefix cache needs {need / GIB:.3f} GiB but the budget allows "
                       f"{budget / GIB:.3f} GiB; reduce the batch -- the state does not shrink "
                       f"with a shorter context")
    return True, ""


class PrefixCache:
    """Per-layer lattice state, carried between forward passes (model/prefix_cache.py:100-168)."""

    def __init__(self, layers, budget=0):
        self.layers = int(layers)
        self.state = [None] * self.layers
        self.budget = int(budget)
        self.tokens = 0
        self.key_valid = None

    def __len__(self):
        return self.tokens

    def get(self, layer):
        return self.state[int(layer)]

    def put(self, layer, state):
        self.state[int(layer)] = None if state is None else state.detach()
        return self.state[int(layer)]

    def advance(self, tokens):
        self.tokens += int(tokens)

    def clear_states(self):
        self.state = [None] * self.layers
        self.tokens = 0
        self.key_valid = None

    def nbytes(self):
        return sum(0 if s is None else s.numel() * s.element_size() for s in self.state)

    def within_budget(self):
        held = self.nbytes()
        if self.budget and held > self.budget:
            return False, (f"the prefix cache holds {held / GIB:.3f} GiB against a "
                           f"{self.budget / GIB:.3f} GiB ceiling")
        return True, ""
