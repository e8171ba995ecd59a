"""MiraLLM on the MI355X plugin: token embedding, n_layer MiraBlocks, the final RMSNorm (with
bias) and the vocabulary head tied to the embedding (model/mira_llm.py:20-157, 283-299, 345-351).

Kept from the reference: the constructor's geometry keywords, weight tying, the initialisation
(every Linear and the embedding N(0, 0.02^2), biases zero, then each block's residual-output
projections at 0.02 / sqrt(2 n_layer)), the forward over a PrefixCache (the cache advances by the
step's tokens after the last block), and `Output.logits`. The reference takes unnamed geometry
from its config scheme; here the defaults are the mira-s ratios (d_e = 2 d, d_r = d / 16,
d_m = 16, K = 2, FFN 4 d). Not built, being outside the scan's hot path: mixture-of-experts
layers, masked-token substitution (mask_positions / mask_gate / sub_ids), multi-device layer
sharding, activation checkpointing and vocabulary resizing.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .block import MiraBlock, RMSNorm


class Output:
    """.logits of a forward (model/mira_llm.py:13-17)."""

    def __init__(self, logits, mask_logit=None):
        self.logits = logits
        self.mask_logit = mask_logit


class MiraLLM(nn.Module):
    def __init__(self, vocab_size, n_layer=12, n_embd=512, dropout=0.0, ffn_hidden=None,
                 lattice_order=2, lattice_d_e=None, coefficient_bottleneck=None,
                 memory_dimension=16, arch="cauchy_x_hyperbolic", lattice_positive_poles=False,
                 lattice_initializer="W_uniform_b_jeffreys", lattice_init_horizon=None,
                 moe_total_experts=1, **unused):
        super().__init__()
        if int(moe_total_experts or 1) > 1:
            raise ValueError("mixture-of-experts layers are not built on the MI355X path")
        n_embd = int(n_embd)
        self.cfg = dict(vocab_size=int(vocab_size), n_layer=int(n_layer), n_embd=n_embd,
                        lattice_order=int(lattice_order),
                        lattice_d_e=int(lattice_d_e or 2 * n_embd),
                        coefficient_bottleneck=int(coefficient_bottleneck or max(1, n_embd // 16)),
                        memory_dimension=int(memory_dimension),
                        ffn_hidden=int(ffn_hidden or 4 * n_embd), arch=arch)
        self.tok = nn.Embedding(vocab_size, n_embd)
        # the reference's masked-token embedding (model/mira_llm.py:136): kept so a reference
        # state_dict loads as is; masked-token substitution itself is not built here
        self.mask_embed = nn.Parameter(torch.zeros(n_embd))
        self.drop = nn.Dropout(dropout)
        self.blocks = nn.ModuleList([
            MiraBlock(n_embd, dropout=dropout, lattice_order=self.cfg["lattice_order"],
                      d_e=self.cfg["lattice_d_e"],
                      coefficient_bottleneck=self.cfg["coefficient_bottleneck"],
                      memory_dimension=self.cfg["memory_dimension"],
                      ffn_hidden=self.cfg["ffn_hidden"],
                      positive_poles=bool(lattice_positive_poles),
                      lattice_initializer=lattice_initializer,
                      lattice_init_horizon=lattice_init_horizon, arch=arch)
            for _ in range(int(n_layer))])
        self.lnf = RMSNorm(n_embd, eps=1e-8, bias=True)
        self.head = nn.Linear(n_embd, vocab_size, bias=False)
        self.tok.weight = self.head.weight
        self.apply(self._init)
        for block in self.blocks:
            block.post_init(n_layer)

    @staticmethod
    def _init(m):
        if isinstance(m, nn.Linear):
            nn.init.normal_(m.weight, mean=0.0, std=0.02)
            if m.bias is not None:
                nn.init.zeros_(m.bias)
        elif isinstance(m, nn.Embedding):
            nn.init.normal_(m.weight, mean=0.0, std=0.02)

    def reset_states(self, lattice_states=None):
        """Empty every slot of a PrefixCache's state list (model/mira_llm.py:311-315): the next
        forward starts each layer from zeros."""
        if lattice_states is not None:
            for layer in range(len(lattice_states)):
                lattice_states[layer] = None

    def hidden_states(self, input_ids, attention_mask=None, cache=None):
        """The trunk's output (B, T, n_embd) before the head."""
        x = self.drop(self.tok(input_ids.to(self.tok.weight.device)))
        if cache is not None and (attention_mask is not None or cache.key_valid is not None):
            # the mask the blocks see is the full history of which tokens are real; a step with
            # no mask after a masked one adds real tokens (model/mira_llm.py:259-283)
            current = (attention_mask[:, -x.shape[1]:].bool() if attention_mask is not None else
                       torch.ones(x.shape[0], x.shape[1], dtype=torch.bool, device=x.device))
            past = cache.key_valid
            if past is None and len(cache):
                past = torch.ones(x.shape[0], len(cache), dtype=torch.bool, device=x.device)
            cache.key_valid = current if past is None else torch.cat([past, current], dim=1)
            attention_mask = cache.key_valid
        for i, block in enumerate(self.blocks):
            x = block(x, attention_mask, cache, i)
        if cache is not None:
            cache.advance(x.shape[1])
        return self.lnf(x)

    def forward(self, input_ids=None, attention_mask=None, cache=None, **unused):
        return Output(self.head(self.hidden_states(input_ids, attention_mask, cache)))
