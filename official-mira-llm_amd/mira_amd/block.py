"""MiraBlock on the MI355X plugin: one MIRA layer, RMSNorm -> MiraMixer on the residual stream,
RMSNorm -> feed-forward on the residual stream (model/mira_block.py:156-205).

The constructor and forward keep the reference's signatures, so a MiraLLM assembled from these
blocks is called as the reference's is. The mixer is mira_amd.mixer.MiraMixer, whose scan runs on
the HIP library; the norms and the feed-forward are PyTorch (their GEMMs go to hipBLASLt), except
that in inference the feed-forward's up projection, bias and SiLU run as one GEMM of the library
(mira_amd.mira.linear_silu).
Mixture-of-experts feed-forwards (model/mira_block.py:51-145) are not part of the scan's hot path
and are not built: a `moe` argument raises.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import mira as plugin
from .mixer import MiraMixer, _plain_linear


def _global_hooks():
    from torch.nn.modules import module as module_globals

    return bool(module_globals._global_forward_pre_hooks or module_globals._global_forward_hooks)


class RMSNorm(nn.Module):
    """x / sqrt(mean(x^2) + eps) * weight (+ bias), computed in float32 and returned in the
    input's dtype (model/mira_block.py:21-35)."""

    def __init__(self, width: int, eps: float = 1e-8, bias: bool = False):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(int(width)))
        self.bias = nn.Parameter(torch.zeros(int(width))) if bias else None
        self.eps = float(eps)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.bias is None and x.dtype == torch.bfloat16 and self.weight.dtype == x.dtype:
            # one fused kernel that computes in float32 and rounds once to bf16 (2.7 ms of a
            # 40 ms cfg5 forward saved). Its float32 sum runs in another order than the steps
            # below, so a few bf16 outputs in 10^5 land one bf16 ulp away; float32 rows would
            # differ by an ulp in a third of the outputs, so float32 takes the steps.
            return F.rms_norm(x, (x.shape[-1],), self.weight, self.eps)
        z = x.float()
        z = z * torch.rsqrt(z.square().mean(dim=-1, keepdim=True) + self.eps) * self.weight.float()
        if self.bias is not None:
            z = z + self.bias.float()
        return z.to(x.dtype)


class FeedForward(nn.Module):
    """down(SiLU(up(x))) with biases; hidden width 4 x width unless given
    (model/mira_block.py:38-48). Not SwiGLU."""

    def __init__(self, width: int, dropout: float = 0.0, hidden: int = None):
        super().__init__()
        hidden = int(hidden) if hidden else 4 * int(width)
        self.up = nn.Linear(width, hidden)
        self.down = nn.Linear(hidden, width)
        self.dropout = nn.Dropout(dropout)

    def forward(self, x):
        hidden = None
        if self._fused(x):
            # inference on the GPU: the up projection with bias and SiLU as one GEMM
            hidden = plugin.linear_silu(x, self.up.weight, self.up.bias)
        if hidden is None:
            hidden = F.silu(self.up(x))
        return self.dropout(self.down(hidden))

    def _fused(self, x):
        """The fused up projection serves this call: no gradients, bf16 on the GPU, a plain
        unhooked nn.Linear with a bias, rows that fit, and the HIP library loaded."""
        up = self.up
        return (not torch.is_grad_enabled() and x.is_cuda and x.dtype == torch.bfloat16
                and type(x) is torch.Tensor and up.bias is not None
                and up.weight.dtype == torch.bfloat16 and _plain_linear(up)
                and not _global_hooks() and x.numel() // max(x.shape[-1], 1) < 2 ** 31
                and plugin.status(x.device.index)[0])


class MiraBlock(nn.Module):
    def __init__(self, width: int, dropout: float = 0.0, lattice_order: int = 2, d_e: int = None,
                 coefficient_bottleneck: int = None, memory_dimension: int = 16,
                 ffn_hidden: int = None, positive_poles: bool = False,
                 lattice_initializer: str = "W_uniform_b_jeffreys", lattice_init_horizon=None,
                 arch: str = "cauchy_x_hyperbolic", moe: dict = None):
        super().__init__()
        if moe:
            raise ValueError("mixture-of-experts feed-forwards are not built on the MI355X path")
        width = int(width)
        d_e = 2 * width if d_e is None else int(d_e)
        coefficient_bottleneck = (max(1, width // 16) if coefficient_bottleneck is None
                                  else int(coefficient_bottleneck))
        self.rn1 = RMSNorm(width)
        self.mixer = MiraMixer(width, lattice_order, d_e, coefficient_bottleneck, memory_dimension,
                               dropout=dropout, positive_poles=positive_poles,
                               lattice_initializer=lattice_initializer,
                               lattice_init_horizon=lattice_init_horizon, arch=arch)
        self.rn2 = RMSNorm(width)
        self.ffn = FeedForward(width, dropout, hidden=ffn_hidden)

    def post_init(self, n_layer: int):
        """The residual-output projections drawn with std 0.02 / sqrt(2 n_layer)
        (model/mira_block.py:193-201). The reference also places the lattice poles here
        (model/mira_initializer.py); that initializer is not built, so the coefficient
        projection keeps the model-wide initialisation."""
        std = 0.02 / math.sqrt(2 * int(n_layer))
        nn.init.normal_(self.mixer.out_proj.weight, mean=0.0, std=std)
        nn.init.normal_(self.ffn.down.weight, mean=0.0, std=std)
        return self

    def forward(self, x, attn_mask=None, cache=None, layer=None):
        x = x + self.mixer(self.rn1(x), attn_mask, cache, layer)
        return x + self.ffn(self.rn2(x))
