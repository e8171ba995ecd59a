"""Autoregressive decoding through the prefix cache: the reference's streaming consumer
(mirachat.py:753-849), batched.

The prompt goes through the model in one forward that leaves every layer's lattice state in a
PrefixCache; each new token is then one T = 1 step per layer, the state updated in place (the
loop owns its cache and sets PrefixCache.in_place, so mira_amd.mixer's single-token call
overwrites the held state through matrix_lattice_step). Sampling follows the
reference's rule (mirachat.py:824-838): greedy at temperature <= 0, else logits / temperature,
top-k masking, softmax, top-p truncation that always keeps the most likely token, and one draw.

With graph=True the single-token forward is captured once as a HIP graph (torch.cuda.CUDAGraph)
and replayed for every further token: the token ids go in through a static buffer, the states
are updated in place, and sampling runs outside the graph on the replayed logits. A captured
step launches nothing but the recorded kernels, which is what a decode loop at small batch needs.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .prefix_cache import PrefixCache


def sample(logits, temperature=0.0, top_k=0, top_p=1.0, generator=None):
    """Next token per row of logits [B, V] (mirachat.py:824-838)."""
    logits = logits.float()
    if temperature <= 0:
        return logits.argmax(dim=-1)
    logits = logits / temperature
    if top_k > 0:
        threshold = torch.topk(logits, min(top_k, logits.shape[-1]), dim=-1).values[:, -1:]
        logits = logits.masked_fill(logits < threshold, float("-inf"))
    probs = F.softmax(logits, dim=-1)
    if 0 < top_p < 1:
        sorted_probs, order = torch.sort(probs, dim=-1, descending=True)
        keep = (torch.cumsum(sorted_probs, dim=-1) - sorted_probs) <= top_p
        sorted_probs = sorted_probs * keep
        probs = torch.zeros_like(probs).scatter(-1, order, sorted_probs)
        probs = probs / probs.sum(dim=-1, keepdim=True).clamp_min(1e-9)
    return torch.multinomial(probs, 1, generator=generator)[:, 0]


class _CapturedStep:
    """One single-token forward of `model` on `cache`, captured as a HIP graph."""

    def __init__(self, model, cache, batch, device):
        self.ids = torch.zeros(batch, 1, dtype=torch.long, device=device)
        self.graph = torch.cuda.CUDAGraph()
        # the capture runs the step once on throwaway values: keep the states it would change
        saved = [None if s is None else s.clone() for s in cache.state]
        tokens = cache.tokens
        side = torch.cuda.Stream(device=device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            model(self.ids, cache=cache)                 # warm-up outside the capture
        torch.cuda.current_stream(device).wait_stream(side)
        with torch.cuda.graph(self.graph, stream=side):      # the warm-up's stream
            self.logits = model(self.ids, cache=cache).logits[:, -1]
        for held, keep in zip(cache.state, saved):
            if held is not None:
                held.copy_(keep)
        cache.tokens = tokens

    def __call__(self, ids, cache):
        self.ids.copy_(ids.view(-1, 1))
        self.graph.replay()
        cache.advance(1)
        return self.logits


@torch.no_grad()
def generate(model, prompt_ids, max_new, temperature=0.0, top_k=0, top_p=1.0, eos_id=None,
             generator=None, graph=False, on_token=None):
    """Tokens [B, n <= max_new] following prompt_ids [B, T]. A row that emits eos_id keeps
    emitting it; decoding stops when every row has. `on_token(tokens so far)` is called after
    every step."""
    if prompt_ids.dim() != 2 or prompt_ids.shape[1] < 1:
        raise ValueError("prompt_ids must be [batch, tokens] with at least one token")
    if model.training:
        raise ValueError("generate decodes through the prefix cache, which needs model.eval()")
    batch = prompt_ids.shape[0]
    cache = PrefixCache(len(model.blocks))
    cache.in_place = True                # this loop owns the cache and keeps no earlier states
    logits = model(prompt_ids, cache=cache).logits[:, -1]
    step = None
    out = []
    done = torch.zeros(batch, dtype=torch.bool, device=prompt_ids.device)
    for i in range(max_new):
        token = sample(logits, temperature, top_k, top_p, generator)
        if eos_id is not None:
            token = torch.where(done, torch.full_like(token, eos_id), token)
            done |= token == eos_id
        out.append(token)
        if on_token is not None:
            on_token(torch.stack(out, dim=1))
        if i + 1 == max_new or (eos_id is not None and bool(done.all())):
            break
        if graph:
            if step is None:
                step = _CapturedStep(model, cache, batch, prompt_ids.device)
            logits = step(token, cache)
        else:
            logits = model(token.view(-1, 1), cache=cache).logits[:, -1]
    return torch.stack(out, dim=1)
