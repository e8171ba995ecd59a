"""MiraMixer on the MI355X plugin: the reference host caller with its constructor and forward
signature (model/mira_mixer.py:544-856), so model/mira_block.py can use it unchanged.

Parameter layout (model/mira_mixer.py:593-627): input_projection d -> d_e + d_m (no bias),
to_control d -> d_r, to_gate d -> d_e, coefficient_projection d_r -> alpha | beta | rho | nu
(d_e K + d_e K + d_e (K+1) + (K+1) d_m), out_proj d_e -> d (no bias). The forward projects,
splits the fused projections into strided views (no copies, model/mira_mixer.py:807-813), takes
s = SiLU(raw write), and hands everything to mira_amd.mira.matrix_lattice_iir with the prefix
cache's state; with gradients it also hands over the two projection outputs those views come
from, so the plugin's backward writes into them whole. An uncached, gradient-free forward hands
the scan the d_r-wide control and coefficient_projection instead
(mira_amd.mira.matrix_lattice_iir_control, which forms alpha, beta and rho inside the scan where
it can; model/mira_mixer.py:739-760). There is no PyTorch fallback: a declined call raises, as in
the reference (model/mira_mixer.py:822-824).

The reference's lattice initializer (model/mira_initializer.py, Jeffreys-prior pole placement)
is out of scope here; parameters use torch's default nn.Linear initialisation.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import mira as plugin
from . import prefix_cache

ARCHES = tuple(plugin.ARCH_STAGE)
# tokens from which the inference input projection runs as two GEMMs instead of one
SPLIT_ROWS = 1024


def _declined(signal, order, memory_dimension):
    batch, tokens, channels = signal.shape
    ok, detail = plugin.status()
    return (f"the mira_amd kernel declined [B,T,C]=[{batch},{tokens},{channels}] "
            f"d_m={memory_dimension} K={order} dtype={signal.dtype}: {detail}. "
            f"MIRA does not fall back to a PyTorch scan -- build the library with "
            f"python official-mira-llm_amd/build.py")


def _plain_linear(module):
    return (type(module) is nn.Linear and not module._forward_pre_hooks
            and not module._forward_hooks and "forward" not in module.__dict__)


def _packing_signature(normalized_x, projections):
    """The key of the packed input-projection weight, or None when packing would bypass
    something a module call does (a tensor subclass, a global or module hook, a subclassed or
    patched Linear, a parameter that is not a plain nn.Parameter)."""
    from torch.nn.modules import module as module_globals

    if type(normalized_x) is not torch.Tensor:
        return None
    if module_globals._global_forward_pre_hooks or module_globals._global_forward_hooks:
        return None
    if not all(_plain_linear(p) for p in projections):
        return None
    parameters = [t for p in projections for t in (p.weight, p.bias) if t is not None]
    if not all(type(t) is nn.Parameter for t in parameters):
        return None
    return tuple((id(t), t.data_ptr(), t._version, t.dtype, t.device, tuple(t.shape),
                  tuple(t.stride())) for t in parameters)


def _used_on_this_stream(kept, reference):
    """Tell the caching allocator that the kept weight tensors are read on the current stream
    (once per stream; not while a graph is being captured, whose launches own no memory), so
    that memory they free on a rebuild is not handed out again while that stream may still
    read it. The weights are kept across streams instead of being rebuilt per stream: a
    rebuild inside a graph capture would replay its copies at every step."""
    if not reference.is_cuda or torch.cuda.is_current_stream_capturing():
        return
    stream = torch.cuda.current_stream(reference.device)
    if stream.cuda_stream in kept["streams"]:
        return
    for tensor in kept["tensors"]:
        tensor.record_stream(stream)
    kept["streams"].add(stream.cuda_stream)


class MiraMixer(nn.Module):
    def __init__(self, width, lattice_order=2, d_e=1536, coefficient_bottleneck=48,
                 memory_dimension=16, dropout=0.0, positive_poles=False,
                 lattice_initializer="W_uniform_b_jeffreys", lattice_init_horizon=None,
                 arch="cauchy_x_hyperbolic"):
        super().__init__()
        if arch not in ARCHES:
            raise ValueError(f"arch must be one of {ARCHES}, not {arch!r}")
        if not 1 <= int(lattice_order) <= 16:
            raise ValueError("lattice_order must be in [1,16]")
        self.width = int(width)
        self.order = self.lattice_order = int(lattice_order)
        self.inner = int(d_e)
        self.coefficient_bottleneck = int(coefficient_bottleneck)
        self.memory_dimension = int(memory_dimension)
        self.positive_poles = bool(positive_poles)
        self.arch = arch
        self.lattice_initializer = lattice_initializer
        self.lattice_init_horizon = lattice_init_horizon
        if self.positive_poles and self.order != 1:
            raise ValueError("positive_poles requires lattice_order=1")
        if self.positive_poles and self.arch != "cauchy_x_mobius":
            raise ValueError("positive_poles requires arch='cauchy_x_mobius'")
        if min(self.inner, self.coefficient_bottleneck, self.memory_dimension) < 1:
            raise ValueError("d_e, coefficient_bottleneck, and memory_dimension must be positive")
        channels, order = self.inner, self.order
        self.input_projection = nn.Linear(self.width, channels + self.memory_dimension, bias=False)
        self.to_control = nn.Linear(self.width, self.coefficient_bottleneck)
        self.to_gate = nn.Linear(self.width, channels)
        alpha_size = beta_size = channels * order
        rho_size = channels * (order + 1)
        read_size = (order + 1) * self.memory_dimension
        self.coefficient_projection = nn.Linear(
            self.coefficient_bottleneck, alpha_size + beta_size + rho_size + read_size)
        self.signal_span = (0, channels)
        self.write_span = (channels, channels + self.memory_dimension)
        self.alpha_span = (0, alpha_size)
        self.beta_span = (alpha_size, 2 * alpha_size)
        self.rho_span = (2 * alpha_size, 2 * alpha_size + rho_size)
        self.read_span = (2 * alpha_size + rho_size, 2 * alpha_size + rho_size + read_size)
        self.out_proj = nn.Linear(channels, self.width, bias=False)
        self.dropout = nn.Dropout(dropout)

    def state_values(self):
        return self.order * self.inner * self.memory_dimension

    def residual_out(self):
        return self.out_proj

    def project_recurrence_inputs(self, normalized_x, coefficients=True):
        """(input projection, coefficient projection, gamma) of the normalised input, or with
        coefficients=False (input projection, control, gamma) (model/mira_mixer.py:657-712).

        In inference the three input projections run as one GEMM on a packed weight kept
        between calls, so a decode step reads the weights once instead of concatenating them
        every time. That shortcut calls no module, so it is taken only when calling the modules
        would do exactly the same: a plain torch.Tensor input, no global module hooks, and three
        plain nn.Linear projections with no hooks, no replaced forward and plain nn.Parameter
        weights. The packed weight is rebuilt whenever any parameter's identity, storage,
        version, dtype, device, shape or strides change; it serves every stream. Otherwise (and
        with gradients) the three modules are called."""
        return self._project(normalized_x, self._packed_weights(normalized_x), coefficients)

    def _project(self, normalized_x, packed, coefficients):
        """project_recurrence_inputs on the packed weights `packed` (None: the modules)."""
        finish = self.coefficient_projection if coefficients else (lambda control: control)
        if packed is None:
            control = F.silu(self.to_control(normalized_x))
            return (self.input_projection(normalized_x), finish(control),
                    self.to_gate(normalized_x))
        projections = (self.input_projection, self.to_gate, self.to_control)
        projected = F.linear(normalized_x, packed["weight"], packed["bias"])
        projected_input, gamma, raw_control = projected.split(
            tuple(p.out_features for p in projections), dim=-1)
        control = F.silu(raw_control)
        return projected_input, finish(control), gamma

    def _packed_weights(self, normalized_x):
        """The inference weights kept between calls, or None where the modules must be called
        (see project_recurrence_inputs): the three input projections packed as one matrix, and
        the same rows regrouped as [signal | gate] and [write | control]."""
        if self.training or torch.is_grad_enabled():
            return None
        projections = (self.input_projection, self.to_gate, self.to_control)
        signature = _packing_signature(normalized_x, projections)
        if signature is None:
            return None
        packed = self.__dict__.get("_packed_projection")
        if packed is None or packed["signature"] != signature:
            weight = torch.cat([p.weight for p in projections])
            bias = torch.cat([p.bias if p.bias is not None else p.weight.new_zeros(p.out_features)
                              for p in projections])
            channels, memory = self.inner, self.memory_dimension
            gate_rows = slice(channels + memory, 2 * channels + memory)
            wide = (torch.cat([weight[:channels], weight[gate_rows]]),
                    torch.cat([bias[:channels], bias[gate_rows]]))
            narrow = (torch.cat([weight[channels:channels + memory], weight[2 * channels + memory:]]),
                      torch.cat([bias[channels:channels + memory], bias[2 * channels + memory:]]))
            packed = {"signature": signature, "weight": weight, "bias": bias, "wide": wide,
                      "narrow": narrow, "tensors": (weight, bias) + wide + narrow,
                      "streams": set()}
            self.__dict__["_packed_projection"] = packed
        _used_on_this_stream(packed, normalized_x)
        return packed

    def _padded_coefficient_weights(self, control):
        """coefficient_projection with its rows padded by zeros to a multiple of 256, kept
        between calls (rebuilt on the same rules as the packed input weights), or None where the
        module must be called. The GEMM library runs that many output columns 1.6x faster at
        d_r = 128 (8,192 rows x 14,528 columns: 114 us, padded to 14,592: 73 us on MI355X); the
        scan reads the real columns through strided views."""
        signature = _packing_signature(control, (self.coefficient_projection,))
        if signature is None:
            return None
        padded = self.__dict__.get("_padded_coefficients")
        if padded is None or padded["signature"] != signature:
            module = self.coefficient_projection
            extra = (-module.out_features) % 256
            weight = torch.cat([module.weight, module.weight.new_zeros(extra, module.in_features)])
            bias = torch.cat([module.bias, module.bias.new_zeros(extra)])
            padded = {"signature": signature, "tensors": (weight, bias), "streams": set()}
            self.__dict__["_padded_coefficients"] = padded
        _used_on_this_stream(padded, control)
        return padded["tensors"]

    def _recurrence_inputs(self, normalized_x, coefficients=True):
        """(signal, raw write, coefficient rows or control, gamma, input projection) for the
        forward. Inference takes the packed weights: for at least SPLIT_ROWS tokens as two GEMMs,
        [signal | gate] (2 d_e columns, a multiple of the GEMM tiles at the mixer's widths) and
        the narrow [write | control] (8,192 tokens at d_e 2048: 123 us against 160 us for the
        4,288-column GEMM on MI355X), fewer tokens as the one packed GEMM (a decode step is
        launch-bound); and the coefficient projection on its padded weight, whose output rows
        are wider than the coefficients by up to 255 zero columns. The input projection is
        returned whole only where it exists as one tensor (None after the two GEMMs). Below
        SPLIT_ROWS tokens the modules' own weights serve (decode steps: there the padded
        coefficient GEMM was slower)."""
        channels, memory = self.inner, self.memory_dimension
        packed = self._packed_weights(normalized_x)
        rows = normalized_x.numel() // max(normalized_x.shape[-1], 1)
        if packed is None or rows < SPLIT_ROWS:
            input_projection, finished, gamma = self._project(normalized_x, packed, False)
            signal, raw_write = input_projection.split((channels, memory), dim=-1)
            control = finished
        else:
            input_projection = None
            both = F.linear(normalized_x, *packed["wide"])
            signal, gamma = both.split((channels, channels), dim=-1)
            narrow = F.linear(normalized_x, *packed["narrow"])
            raw_write, raw_control = narrow.split((memory, self.coefficient_bottleneck), dim=-1)
            control = F.silu(raw_control)
        if not coefficients:
            return signal, raw_write, control, gamma, input_projection
        if packed is not None and rows >= SPLIT_ROWS:
            padded = self._padded_coefficient_weights(control)
            if padded is not None:
                return signal, raw_write, F.linear(control, *padded), gamma, input_projection
        return signal, raw_write, self.coefficient_projection(control), gamma, input_projection

    def _forms_coefficients_in_scan(self, normalized_x, cache):
        """Whether this call takes the coefficient-forming scan (model/mira_mixer.py:739-760):
        an uncached, gradient-free forward whose coefficient_projection is a plain, unhooked
        nn.Linear, no positive-pole remapping, and a geometry the scan has a kernel for (else
        the forward projects the coefficients itself, on the padded weight)."""
        if not (normalized_x.is_cuda and cache is None and not self.positive_poles
                and not torch.is_grad_enabled() and _plain_linear(self.coefficient_projection)):
            return False
        batch, tokens, _ = normalized_x.shape
        return plugin.control_scan_serves(batch, tokens, self.inner, self.order,
                                          self.memory_dimension, self.coefficient_bottleneck,
                                          normalized_x.dtype, normalized_x.device.index)

    def forward(self, normalized_x, attn_mask=None, cache=None, layer=None):
        if cache is not None and not (prefix_cache.enabled() and layer is not None
                                      and not self.training and hasattr(cache, "get")):
            raise ValueError("streaming cache is not wired into mira-dsp")
        batch, tokens, _ = normalized_x.shape
        channels, order, memory = self.inner, self.order, self.memory_dimension
        if self._forms_coefficients_in_scan(normalized_x, cache):
            signal, raw_write, control, gamma, _ = self._recurrence_inputs(
                normalized_x, coefficients=False)
            valid = None if attn_mask is None else attn_mask[:, -tokens:].bool()
            projection = self.coefficient_projection
            mixed = plugin.matrix_lattice_iir_control(
                signal, control, projection.weight, projection.bias,
                (self.alpha_span, self.beta_span, self.rho_span, self.read_span), gamma,
                F.silu(raw_write).contiguous(), valid=valid, arch=self.arch)
            if mixed is None:
                raise RuntimeError(_declined(signal, order, memory))
            output = self.out_proj(self.dropout(mixed))
            if valid is not None:
                output = torch.where(valid.unsqueeze(-1), output, torch.zeros_like(output))
            return output
        alpha_size = channels * order
        rho_size = channels * (order + 1)
        read_size = (order + 1) * memory
        if torch.is_grad_enabled() and cache is None:
            # training: the module outputs themselves, which the backward fills whole
            input_projection, coefficients, gamma = self.project_recurrence_inputs(normalized_x)
            signal, raw_write = input_projection.split((channels, memory), dim=-1)
        else:
            signal, raw_write, coefficients, gamma, input_projection = self._recurrence_inputs(
                normalized_x)
        raw_alpha, raw_beta, raw_rho, memory_read = coefficients[..., :self.read_span[1]].split(
            (alpha_size, alpha_size, rho_size, read_size), dim=-1)
        if self.positive_poles:
            value = raw_alpha.float()
            safe = torch.where(value == 0.0, torch.full_like(value, 1.0e-6), value)
            raw_alpha = torch.where(value.abs() < 1.0, safe.reciprocal(), value).to(raw_alpha.dtype)
            if torch.is_grad_enabled() and cache is None:
                # the remapped alpha must live in the packed storage the backward writes into
                coefficients = torch.cat((raw_alpha, raw_beta, raw_rho, memory_read), dim=-1)
                raw_alpha, raw_beta, raw_rho, memory_read = coefficients.split(
                    (alpha_size, alpha_size, rho_size, read_size), dim=-1)
        memory_write = F.silu(raw_write)
        raw_alpha = raw_alpha.view(batch, tokens, channels, order)
        raw_beta = raw_beta.view(batch, tokens, channels, order)
        raw_rho = raw_rho.view(batch, tokens, channels, order + 1)
        memory_read = memory_read.view(batch, tokens, order + 1, memory)
        valid = None if attn_mask is None else attn_mask[:, -tokens:].bool()
        held = None if cache is None else cache.get(layer)
        if tokens == 1 and held is not None:
            # a decode step on a held state; a cache that opted in (in_place) has it overwritten,
            # so the step allocates no state and a captured step replays on the same tensor
            result = plugin.matrix_lattice_step(
                signal, raw_alpha, raw_rho, gamma, memory_write.contiguous(), memory_read,
                raw_beta, held, valid=valid, arch=self.arch,
                inplace=bool(getattr(cache, "in_place", False)))
        else:
            # training hands the plugin the two projection outputs the views come from, so the
            # backward writes its gradients into them whole (model/mira_mixer.py:814-821)
            packed = ((input_projection, coefficients)
                      if torch.is_grad_enabled() and cache is None else None)
            result = plugin.matrix_lattice_iir(
                signal, raw_alpha, raw_rho, gamma, memory_write.contiguous(), memory_read,
                raw_beta=raw_beta, valid=valid, state=held,
                return_state=cache is not None, packed=packed, arch=self.arch)
        if result is None:
            raise RuntimeError(_declined(signal, order, memory))
        if cache is None:
            mixed = result
        else:
            mixed, final = result
            cache.put(layer, final)
            fits, why = cache.within_budget()
            if not fits:
                raise ValueError(why)
        output = self.out_proj(self.dropout(mixed))
        if valid is not None:
            output = torch.where(valid.unsqueeze(-1), output, torch.zeros_like(output))
        return output
