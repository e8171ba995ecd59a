"""The MI355X operator plugin for the Mira mixer scan (gfx950 HIP kernels behind a C-ABI).

Drop-in for the reference's `kernel/cuda/mira_dspv2/mira.py`: same entry points, same argument
meaning, same decline / error behaviour, selected by the mixer the way the reference selects its
CUDA package (model/mira_mixer.py:191-218):

  matrix_lattice_iir(x, raw_alpha, raw_rho, gamma, memory_write, memory_read, raw_beta=None,
                     valid=None, state=None, return_state=False, packed=None, arch=...)
                                               -- mira.py:1439-1563
  matrix_lattice_iir_control(x, control, coefficient_weight, coefficient_bias, spans, gamma,
                             memory_write, valid=None, state=None, return_state=False, arch=...)
                                               -- mira.py:1840-1894 (coefficients formed inside
                                                  the scan where served, else GEMM + scan)
  status(device=None) -> (bool, str)           -- mira.py:336-345
  usage() -> dict                              -- mira.py:348-349
  report(index=None)                           -- mira.py:352

plus the BASELINE-literal scans, which have no reference counterpart:
  diag_conv_scan / diag_conv_step              -- depthwise causal conv + diagonal decay scan
  gla_chunked / gla_step                       -- GLA matrix state, prefill and decode

A call the kernels do not serve returns None, exactly as the reference plugin does, and the
mixer raises; a malformed state or mask raises ValueError; a failed launch raises RuntimeError.
Every launch is asynchronous on torch's current stream of the tensors' device. A call under
autograd without return_state keeps a graph (the _LatticeScan Function: the forward at the
backward's chunk length, mira_lattice_backward in the backward, gradients written into the
packed projections when the mixer passes them); a (K, d_m) without backward kernels declines.
"""
from __future__ import annotations

import math
import os
import threading

import torch

from . import _lib

ORDERS = (1, 2, 4, 8)
MEMORY_DIMENSIONS = (1, 2, 4, 8, 16, 32, 64, 128)
ORDER_MEMORIES = {order: MEMORY_DIMENSIONS for order in ORDERS}
ARCH_STAGE = {"cauchy_x_mobius": 3, "cauchy_x_hyperbolic": 6, "cauchy_x_identity": 7,
              "gaussian_x_mobius": 8, "gaussian_x_hyperbolic": 9, "gaussian_x_identity": 10,
              "expexp_x_mobius": 11, "expexp_x_hyperbolic": 12, "expexp_x_identity": 13,
              "expsoftplus_x_mobius": 14, "expsoftplus_x_hyperbolic": 15,
              "expsoftplus_x_identity": 16,
              "hill_x_mobius": 17, "hill_x_hyperbolic": 18, "hill_x_identity": 19}
DTYPE = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}
CONV_WIDTH = 4
GLA_DIM = 128
USED = {"forward": 0, "backward": 0, "step": 0, "control": 0, "diag": 0, "gla": 0,
        "linear_silu": 0}
REPORTED = set()
_WORKSPACES = {}
_WORKSPACE_LOCK = threading.Lock()      # autograd / DataParallel threads may launch


def _row_stride(tensor, tokens):
    """Row stride of a [B,T,C] view with unit channel stride and batch stride T*row, or None
    (mira.py:315-321). With one token the batch stride is the row stride (torch may give a
    size-1 axis any stride)."""
    if tensor.stride(2) != 1:
        return None
    if tokens == 1:
        return int(tensor.stride(0))
    row = int(tensor.stride(1))
    if int(tensor.stride(0)) != tokens * row:
        return None
    return row


def dense_tail_row_stride(tensor, tokens):
    """Row stride of a view whose axes after the token axis are dense, or None (mira.py:324-333)."""
    expected = 1
    for axis in range(tensor.dim() - 1, 1, -1):
        if int(tensor.stride(axis)) != expected:
            return None
        expected *= int(tensor.shape[axis])
    if tokens == 1:
        return int(tensor.stride(0))
    row = int(tensor.stride(1))
    if int(tensor.stride(0)) != tokens * row:
        return None
    return row


def status(device=None):
    """(True, library path) when the HIP library loads and a GPU is visible, else (False, why)."""
    if not torch.cuda.is_available():
        return False, "no HIP device is visible"
    if _lib.library() is None:
        return False, _lib.why()
    return True, _lib.LIBRARY


def usage():
    return dict(USED)


def report(index=None):
    """Print once per device how a mixer call maps onto blocks, lanes and chunks."""
    if os.environ.get("MIRALLM_CUDA_REPORT", "1") == "0":
        return False
    if not torch.cuda.is_available():
        return False
    index = torch.cuda.current_device() if index is None else int(index)
    if index in REPORTED:
        return False
    REPORTED.add(index)
    props = torch.cuda.get_device_properties(index)
    lib = _lib.require()
    print(f"mira_amd on {props.name} ({getattr(props, 'gcnArchName', '?')}, "
          f"{props.multi_processor_count} CUs): {lib.mira_version().decode()}; "
          f"lattice block 256 threads = channels x lanes, lanes = fewest keeping <= 32 state "
          f"floats per lane; token chunks from mira_lattice_plan_chunk", flush=True)
    return True


def _stream(device):
    return ctypes_stream(torch.cuda.current_stream(device))


def ctypes_stream(stream):
    return int(stream.cuda_stream)


def _ptr(tensor):
    return None if tensor is None else int(tensor.data_ptr())


def workspace(kind, device, nbytes, zero=False):
    """A per-(kind, device, stream) device buffer of at least `nbytes`, grown on demand; `zero`
    fills it with zeros when it is (re)allocated. Calls on one stream reuse it in order."""
    if nbytes <= 0:
        return None
    stream = torch.cuda.current_stream(device).cuda_stream
    key = (kind, device.index, stream)
    with _WORKSPACE_LOCK:
        buffer = _WORKSPACES.get(key)
        if buffer is None or buffer.numel() < nbytes:
            size = max(int(nbytes), 1 << 20)
            buffer = (torch.zeros if zero else torch.empty)(size, dtype=torch.uint8, device=device)
            _WORKSPACES[key] = buffer
    return buffer


# --------------------------------------------------------------------------------------------
# the reference operator
# --------------------------------------------------------------------------------------------
def matrix_lattice_iir(x, raw_alpha, raw_rho, gamma, memory_write, memory_read, raw_beta=None,
                       valid=None, state=None, return_state=False, packed=None,
                       arch="cauchy_x_hyperbolic", chunk=None):
    """The K-stage lattice scan (model/mira_mixer.py:246-387) on the GPU. Acceptance rules of
    mira.py:1444-1517; returns the output [B,T,C] in x.dtype, (output, final state) with
    return_state, or None when declined. `chunk` forces the token chunk (tests); None lets the
    library choose."""
    if arch not in ARCH_STAGE:
        raise ValueError(f"arch must be one of {tuple(ARCH_STAGE)}, not {arch!r}")
    if not (x.dim() == 3 and gamma.dim() == 3 and raw_alpha.dim() == 4 and raw_rho.dim() == 4
            and memory_write.dim() == 3 and memory_read.dim() == 4):
        return None
    batch, tokens, channels = x.shape
    if not batch or not tokens or not channels:
        raise ValueError("mira-dsp requires nonempty batch, token and channel axes")
    order = int(raw_alpha.shape[-1])
    memory = int(memory_write.shape[-1])
    if order not in ORDERS or memory not in ORDER_MEMORIES[order]:
        return None
    if raw_alpha.shape != (batch, tokens, channels, order):
        return None
    if raw_rho.shape != (batch, tokens, channels, order + 1):
        return None
    if gamma.shape != x.shape or memory_write.shape != (batch, tokens, memory):
        return None
    if memory_read.shape != (batch, tokens, order + 1, memory):
        return None
    tensors = (x, raw_alpha, raw_rho, gamma, memory_write, memory_read)
    if not all(tensor.is_cuda for tensor in tensors):
        return None
    if len({tensor.device for tensor in tensors}) != 1 or len({t.dtype for t in tensors}) != 1:
        return None
    if DTYPE.get(x.dtype) is None or not memory_write.is_contiguous():
        return None
    if not (raw_beta is not None and raw_beta.shape == raw_alpha.shape
            and raw_beta.dtype == raw_alpha.dtype and raw_beta.device == x.device):
        return None
    row = _row_stride(x, tokens)
    gamma_row = _row_stride(gamma, tokens)
    if row is None or row < channels or gamma_row is None or gamma_row < channels:
        return None
    alpha_row = dense_tail_row_stride(raw_alpha, tokens)
    beta_row = dense_tail_row_stride(raw_beta, tokens)
    rho_row = dense_tail_row_stride(raw_rho, tokens)
    read_row = dense_tail_row_stride(memory_read, tokens)
    if None in (alpha_row, beta_row, rho_row, read_row):
        return None
    if not status(x.device.index)[0]:
        return None
    if valid is not None:
        if valid.shape != (batch, tokens) or valid.device != x.device or valid.dtype != torch.bool:
            raise ValueError("mira-dsp mask must be a boolean [batch, tokens] CUDA tensor")
        valid = valid.contiguous()
    if state is not None:
        if (state.shape != (batch, order, channels, memory) or state.device != x.device
                or state.dtype != torch.float32):
            raise ValueError("mira-dsp state must be FP32 [batch, order, channels, memory]")
        if state.requires_grad:
            raise ValueError("mira-dsp cached state is inference-only")
        if not return_state:
            raise ValueError("mira-dsp initial state requires return_state=True")
        state = state.contiguous()
    if packed is not None:
        _check_packed(packed, x, raw_alpha, raw_beta, raw_rho, memory_read, row,
                      (alpha_row, beta_row, rho_row, read_row))
    # a retained graph (gradients wanted, no state handed back) runs the training path; with
    # return_state the scan serves a cache and carries no gradient (mira.py:1518-1563)
    train = (not return_state and torch.is_grad_enabled() and any(
        t.requires_grad for t in tensors + (raw_beta,) + (() if packed is None else tuple(packed))))
    if train:
        lib = _lib.require()
        if not lib.mira_lattice_backward_chunk(order, memory):
            return None                      # no backward kernel for this (K, d_m)
        rows = (row, alpha_row, beta_row, rho_row, gamma_row, read_row)
        if packed is not None:
            x, raw_alpha, raw_beta, raw_rho, memory_write, memory_read = (
                t.detach() for t in (x, raw_alpha, raw_beta, raw_rho, memory_write, memory_read))
            packed_input, packed_coefficients = packed
        else:
            packed_input = packed_coefficients = None
        output = _LatticeScan.apply(x, raw_alpha, raw_beta, raw_rho, gamma, memory_write,
                                    memory_read, packed_input, packed_coefficients, valid, rows,
                                    arch)
        USED["forward"] += 1
        return output
    if return_state:
        with torch.no_grad():
            return _lattice_inference(x, raw_alpha, raw_beta, raw_rho, gamma, memory_write,
                                      memory_read, valid, state, True, arch, chunk,
                                      (row, alpha_row, beta_row, rho_row, gamma_row, read_row))
    return _lattice_inference(x, raw_alpha, raw_beta, raw_rho, gamma, memory_write, memory_read,
                              valid, state, False, arch, chunk,
                              (row, alpha_row, beta_row, rho_row, gamma_row, read_row))


def _check_packed(packed, x, raw_alpha, raw_beta, raw_rho, memory_read, row, coefficient_rows):
    """The packed projections of a training forward must be the storage the views come from
    (mira.py:1518-1537): [B,T,C+M] input projection with x at its start, and the
    [B,T,C(3K+1)+(K+1)M] coefficient projection holding alpha, beta, rho and nu in that order."""
    batch, tokens, channels = x.shape
    order = int(raw_alpha.shape[-1])
    memory = int(memory_read.shape[-1])
    packed_input, packed_coefficients = packed
    width = channels * (3 * order + 1) + (order + 1) * memory
    if (packed_input.shape != (batch, tokens, channels + memory)
            or packed_coefficients.shape != (batch, tokens, width)
            or not packed_input.is_contiguous() or not packed_coefficients.is_contiguous()
            or any(t.device != x.device or t.dtype != x.dtype for t in packed)):
        raise ValueError("mira-dsp packed projections have incompatible layout")
    base, element = packed_coefficients.data_ptr(), x.element_size()
    if (x.data_ptr() != packed_input.data_ptr() or raw_alpha.data_ptr() != base
            or raw_beta.data_ptr() != base + channels * order * element
            or raw_rho.data_ptr() != base + 2 * channels * order * element
            or memory_read.data_ptr() != base + channels * (3 * order + 1) * element
            or row != channels + memory or any(r != width for r in coefficient_rows)):
        raise ValueError("mira-dsp packed views do not match their projection storage")


def _lattice_inference(x, raw_alpha, raw_beta, raw_rho, gamma, memory_write, memory_read, valid,
                       state, return_state, arch, chunk, rows):
    """The forward without a retained graph: summary / combine / replay, or one launch."""
    row, alpha_row, beta_row, rho_row, gamma_row, read_row = rows
    batch, tokens, channels = x.shape
    order = int(raw_alpha.shape[-1])
    memory = int(memory_write.shape[-1])
    dtype = DTYPE[x.dtype]
    lib = _lib.require()
    output = torch.empty(batch, tokens, channels, device=x.device, dtype=x.dtype)
    final = (torch.empty(batch, order, channels, memory, device=x.device, dtype=torch.float32)
             if return_state else None)
    with torch.cuda.device(x.device):
        if chunk is None:
            chunk = lib.mira_lattice_plan_chunk(batch, tokens, channels, order, memory)
        chunk = max(1, min(int(chunk), tokens))
        need = lib.mira_lattice_workspace_bytes(batch, tokens, channels, order, memory, chunk)
        space = workspace("lattice", x.device, need)
        code = lib.mira_lattice_forward(
            _ptr(x), row, _ptr(raw_alpha), alpha_row, _ptr(raw_beta), beta_row, _ptr(raw_rho),
            rho_row, _ptr(gamma), gamma_row, _ptr(memory_write), _ptr(memory_read), read_row,
            _ptr(valid), _ptr(state), _ptr(final), _ptr(output), batch, tokens, channels, order,
            memory, dtype, ARCH_STAGE[arch], chunk, _ptr(space), 0 if space is None else
            space.numel(), _stream(x.device))
    if _lib.check(code, "mira_lattice_forward") is None:
        return None
    USED["forward"] += 1
    return (output, final) if return_state else output


class _LatticeScan(torch.autograd.Function):
    """The scan with a retained graph: the forward runs at the backward's chunk length and keeps
    its workspace (every chunk's transition and entering state: the checkpoints the backward
    replays from, mira.py:1165-1170); the backward launches mira_lattice_backward
    (mira.py:1295-1433). With packed projections the gradients land in two packed buffers, the
    raw write's through SiLU', and flow to the projections that made them."""

    @staticmethod
    def forward(ctx, x, raw_alpha, raw_beta, raw_rho, gamma, memory_write, memory_read,
                packed_input, packed_coefficients, valid, rows, arch):
        row, alpha_row, beta_row, rho_row, gamma_row, read_row = rows
        batch, tokens, channels = x.shape
        order, memory = int(raw_alpha.shape[-1]), int(memory_write.shape[-1])
        lib = _lib.require()
        chunk = lib.mira_lattice_backward_chunk(order, memory)
        output = torch.empty(batch, tokens, channels, device=x.device, dtype=x.dtype)
        need = lib.mira_lattice_workspace_bytes(batch, tokens, channels, order, memory, chunk)
        space = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
        with torch.cuda.device(x.device):
            code = lib.mira_lattice_forward(
                _ptr(x), row, _ptr(raw_alpha), alpha_row, _ptr(raw_beta), beta_row,
                _ptr(raw_rho), rho_row, _ptr(gamma), gamma_row, _ptr(memory_write),
                _ptr(memory_read), read_row, _ptr(valid), None, None, _ptr(output), batch,
                tokens, channels, order, memory, DTYPE[x.dtype], ARCH_STAGE[arch], chunk,
                _ptr(space), need, _stream(x.device))
        _lib.check(code, "mira_lattice_forward")
        ctx.save_for_backward(x, raw_alpha, raw_beta, raw_rho, gamma, memory_write, memory_read,
                              space, valid, packed_input)
        ctx.meta = (rows, arch, need, packed_coefficients is not None)
        return output

    @staticmethod
    def backward(ctx, grad_output):
        (x, raw_alpha, raw_beta, raw_rho, gamma, memory_write, memory_read, space, valid,
         packed_input) = ctx.saved_tensors
        rows, arch, forward_bytes, packed = ctx.meta
        row, alpha_row, beta_row, rho_row, gamma_row, read_row = rows
        batch, tokens, channels = x.shape
        order, memory = int(raw_alpha.shape[-1]), int(memory_write.shape[-1])
        grad_output = grad_output.to(x.dtype).contiguous()
        io = dict(device=x.device, dtype=x.dtype)
        if packed:
            width = channels * (3 * order + 1) + (order + 1) * memory
            grad_input = torch.empty(batch, tokens, channels + memory, **io)
            grad_coefficients = torch.empty(batch, tokens, width, **io)
            element = x.element_size()
            base = grad_coefficients.data_ptr()
            pointers = (grad_input.data_ptr(), channels + memory,
                        base, width, base + channels * order * element, width,
                        base + 2 * channels * order * element, width)
            write_pointer = grad_input.data_ptr() + channels * element
            read_pointer = base + channels * (3 * order + 1) * element
            write_rows, read_rows = channels + memory, width
            raw_write = packed_input.data_ptr() + channels * element
            raw_rows = channels + memory
        else:
            grad_input = grad_coefficients = None
            grads = [torch.empty(batch, tokens, channels, **io),
                     torch.empty(batch, tokens, channels, order, **io),
                     torch.empty(batch, tokens, channels, order, **io),
                     torch.empty(batch, tokens, channels, order + 1, **io),
                     torch.empty(batch, tokens, memory, **io),
                     torch.empty(batch, tokens, order + 1, memory, **io)]
            pointers = (grads[0].data_ptr(), channels, grads[1].data_ptr(), channels * order,
                        grads[2].data_ptr(), channels * order, grads[3].data_ptr(),
                        channels * (order + 1))
            write_pointer, read_pointer = grads[4].data_ptr(), grads[5].data_ptr()
            write_rows, read_rows = memory, (order + 1) * memory
            raw_write, raw_rows = None, 0
        grad_gamma = torch.empty(batch, tokens, channels, **io)
        lib = _lib.require()
        need = lib.mira_lattice_backward_workspace_bytes(batch, tokens, channels, order, memory)
        scratch = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
        with torch.cuda.device(x.device):
            code = lib.mira_lattice_backward(
                _ptr(x), row, _ptr(raw_alpha), alpha_row, _ptr(raw_beta), beta_row,
                _ptr(raw_rho), rho_row, _ptr(gamma), gamma_row, _ptr(memory_write),
                _ptr(memory_read), read_row, _ptr(valid), None, _ptr(grad_output),
                pointers[0], pointers[1], pointers[2], pointers[3], pointers[4], pointers[5],
                pointers[6], pointers[7], _ptr(grad_gamma), channels, write_pointer, write_rows,
                raw_write, raw_rows, read_pointer, read_rows, batch, tokens, channels, order,
                memory, DTYPE[x.dtype], ARCH_STAGE[arch], _ptr(space), forward_bytes,
                _ptr(scratch), need, _stream(x.device))
        _lib.check(code, "mira_lattice_backward")
        USED["backward"] += 1
        if packed:
            return (None, None, None, None, grad_gamma, None, None, grad_input, grad_coefficients,
                    None, None, None)
        wanted = ctx.needs_input_grad
        values = (grads[0], grads[1], grads[2], grads[3], grad_gamma, grads[4], grads[5])
        return tuple(v if wanted[i] else None for i, v in enumerate(values)) + (None,) * 5


def matrix_lattice_step(x, raw_alpha, raw_rho, gamma, memory_write, memory_read, raw_beta,
                        state, valid=None, arch="cauchy_x_hyperbolic", out=None, inplace=False):
    """The T=1 decode step: the reference launches mira_matrix_step_k{K}_m{M} for one token
    (mira.py:1192,1254-1276). Shapes as matrix_lattice_iir with T = 1; returns (output, state).
    With inplace=True the state tensor is updated in place (no new allocation)."""
    batch, tokens, channels = x.shape
    order, memory = int(raw_alpha.shape[-1]), int(memory_write.shape[-1])
    if tokens != 1:
        raise ValueError("matrix_lattice_step takes one token")
    dtype = DTYPE.get(x.dtype)
    if dtype is None or order not in ORDERS or memory not in ORDER_MEMORIES[order]:
        return None
    if state.shape != (batch, order, channels, memory) or state.dtype != torch.float32:
        raise ValueError("mira-dsp state must be FP32 [batch, order, channels, memory]")
    rows = (_row_stride(x, 1), dense_tail_row_stride(raw_alpha, 1),
            dense_tail_row_stride(raw_beta, 1), dense_tail_row_stride(raw_rho, 1),
            _row_stride(gamma, 1), dense_tail_row_stride(memory_read, 1))
    if None in rows or not memory_write.is_contiguous() or not state.is_contiguous():
        return None
    if valid is not None:
        valid = valid.contiguous()
    lib = _lib.require()
    output = out if out is not None else torch.empty_like(x, memory_format=torch.contiguous_format)
    final = state if inplace else torch.empty_like(state)
    code = lib.mira_lattice_step(
        _ptr(x), rows[0], _ptr(raw_alpha), rows[1], _ptr(raw_beta), rows[2], _ptr(raw_rho),
        rows[3], _ptr(gamma), rows[4], _ptr(memory_write), _ptr(memory_read), rows[5],
        _ptr(valid), _ptr(state), _ptr(final), _ptr(output), batch, channels, order, memory,
        dtype, ARCH_STAGE[arch], _stream(x.device))
    if _lib.check(code, "mira_lattice_step") is None:
        return None
    USED["step"] += 1
    return output, final


def _control_plan(x, control, weight, bias, gamma, memory_write, order, memory):
    """None, or (x row, gamma row) when the coefficient-forming scan serves this call
    (mira.py:1642-1672): inference, bf16 throughout, a (K, d_m, d_r) the library has, one token
    chunk, and layouts it reads in place."""
    tensors = (x, control, weight, gamma, memory_write)
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors + (bias,)
                                       if t is not None):
        return None
    if not all(t.is_cuda for t in tensors) or len({t.device for t in tensors}) != 1:
        return None
    if any(t.dtype != torch.bfloat16 for t in tensors):
        return None
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.device != x.device
                             or bias.dim() != 1 or bias.stride(0) != 1):
        return None
    if weight.dim() != 2 or weight.stride(1) != 1 or control.dim() != 3:
        return None
    batch, tokens, channels = x.shape
    rank = int(control.shape[-1])
    if control.shape[:2] != (batch, tokens) or weight.shape[1] != rank:
        return None
    if not status(x.device.index)[0]:
        return None
    lib = _lib.require()
    if not lib.mira_lattice_control_serves(batch, tokens, channels, order, memory, rank,
                                           _lib.BF16):
        return None
    row, gamma_row = _row_stride(x, tokens), _row_stride(gamma, tokens)
    if row is None or gamma_row is None or row < channels or gamma_row < channels:
        return None
    # the kernel reads control rows as 16-byte pieces and weight rows as 8-byte pieces
    # (mira_lattice_control_forward declines otherwise); such a call takes GEMM + scan instead
    if (control.contiguous().data_ptr() % 16 or weight.data_ptr() % 8
            or weight.stride(0) % 4):
        return None
    return row, gamma_row


def control_scan_serves(batch, tokens, channels, order, memory, rank, dtype, device_index=None):
    """Whether the coefficient-forming scan has a kernel for this geometry (bf16 only); a
    caller that holds the coefficient weights can then take the GEMM + scan route itself when
    it does not (mira_lattice_control_serves)."""
    if dtype != torch.bfloat16 or not status(device_index)[0]:
        return False
    return bool(_lib.require().mira_lattice_control_serves(batch, tokens, channels, order, memory,
                                                           rank, _lib.BF16))


def matrix_lattice_iir_control(x, control, coefficient_weight, coefficient_bias, spans, gamma,
                               memory_write, valid=None, state=None, return_state=False,
                               arch="cauchy_x_hyperbolic"):
    """The mixer forward from the d_r-wide control (mira.py:1840-1894). Where the
    coefficient-forming scan serves the call (_control_plan) alpha, beta and rho are formed
    inside the scan on the matrix cores from the control and coefficient_projection's rows
    (mira_lattice_control_forward) and only memory_read is projected here; otherwise the
    coefficient projection runs as one GEMM (hipBLASLt through torch), then the scan, bit for
    bit the materialised path (mira.py:1693-1704)."""
    import torch.nn.functional as F

    if arch not in ARCH_STAGE:
        raise ValueError(f"arch must be one of {tuple(ARCH_STAGE)}, not {arch!r}")
    alpha_span, beta_span, rho_span, read_span = spans
    batch, tokens, channels = x.shape
    order = (alpha_span[1] - alpha_span[0]) // channels
    memory = int(memory_write.shape[-1])
    plan = _control_plan(x, control, coefficient_weight, coefficient_bias, gamma, memory_write,
                         order, memory)
    if plan is not None:
        return _control_scan(x, control, coefficient_weight, coefficient_bias, spans, gamma,
                             memory_write, valid, state, return_state, arch, order, memory, plan)
    coefficients = F.linear(control, coefficient_weight, coefficient_bias)
    raw_alpha, raw_beta, raw_rho, memory_read = coefficients.split(
        tuple(hi - lo for lo, hi in spans), dim=-1)
    return matrix_lattice_iir(
        x, raw_alpha.view(batch, tokens, channels, order),
        raw_rho.view(batch, tokens, channels, order + 1), gamma, memory_write,
        memory_read.view(batch, tokens, order + 1, memory),
        raw_beta=raw_beta.view(batch, tokens, channels, order), valid=valid, state=state,
        return_state=return_state, arch=arch)


def _control_scan(x, control, weight, bias, spans, gamma, memory_write, valid, state,
                  return_state, arch, order, memory, plan):
    """The coefficient-forming scan (mira.py:1705-1741): memory_read projected here, alpha, beta
    and rho formed inside the kernel."""
    import torch.nn.functional as F

    row, gamma_row = plan
    batch, tokens, channels = x.shape
    (alpha_lo, alpha_hi), (beta_lo, beta_hi), (rho_lo, rho_hi), (read_lo, read_hi) = spans
    if (alpha_hi - alpha_lo != channels * order or beta_hi - beta_lo != channels * order
            or rho_hi - rho_lo != channels * (order + 1)
            or read_hi - read_lo != (order + 1) * memory):
        raise ValueError("mira-dsp: the coefficient spans must hold C K, C K, C (K+1) and "
                         "(K+1) d_m rows")
    if valid is not None:
        if valid.shape != (batch, tokens) or valid.device != x.device or valid.dtype != torch.bool:
            raise ValueError("mira-dsp mask must be a boolean [batch, tokens] CUDA tensor")
        valid = valid.contiguous()
    if state is not None:
        if (state.shape != (batch, order, channels, memory) or state.device != x.device
                or state.dtype != torch.float32):
            raise ValueError("mira-dsp state must be FP32 [batch, order, channels, memory]")
        if not return_state:
            raise ValueError("mira-dsp initial state requires return_state=True")
        state = state.contiguous()
    control = control.contiguous()
    memory_write = memory_write.contiguous()
    read_bias = None if bias is None else bias[read_lo:read_hi]
    memory_read = F.linear(control, weight[read_lo:read_hi], read_bias).contiguous()
    lib = _lib.require()
    output = torch.empty(batch, tokens, channels, device=x.device, dtype=x.dtype)
    final = (torch.empty(batch, order, channels, memory, device=x.device, dtype=torch.float32)
             if return_state else None)
    with torch.cuda.device(x.device):
        code = lib.mira_lattice_control_forward(
            _ptr(x), row, _ptr(control), _ptr(weight), int(weight.stride(0)),
            int(weight.shape[0]), _ptr(bias), alpha_lo, beta_lo, rho_lo, _ptr(gamma), gamma_row,
            _ptr(memory_write), _ptr(memory_read), (order + 1) * memory, _ptr(valid),
            _ptr(state), _ptr(final), _ptr(output), batch, tokens, channels, order, memory,
            int(control.shape[-1]), _lib.BF16, ARCH_STAGE[arch], _stream(x.device))
    if _lib.check(code, "mira_lattice_control_forward") is None:
        return None
    USED["forward"] += 1
    USED["control"] += 1
    return (output, final) if return_state else output


# --------------------------------------------------------------------------------------------
# BASELINE-literal: depthwise causal conv + diagonal decay scan
# --------------------------------------------------------------------------------------------
def _diag_check(x, a, w, bias, dims):
    if x.shape != a.shape or x.dim() != dims or x.dtype != a.dtype or x.dtype not in DTYPE:
        raise ValueError("diag: x and a must share one shape and a float dtype")
    if not (x.is_cuda and a.is_cuda):
        raise ValueError("diag: x and a must be device tensors")
    D = x.shape[-1]
    if w.shape != (D, CONV_WIDTH) or w.dtype != torch.float32:
        raise ValueError(f"diag: w must be float32 [D, {CONV_WIDTH}]")
    if bias is not None and (bias.shape != (D,) or bias.dtype != torch.float32):
        raise ValueError("diag: bias must be float32 [D]")


def diag_conv_scan(x, a, w, bias=None, h0=None, ring=None, pos=0, return_state=False,
                   ring_out=None):
    """Prefill of u = causal_conv(x) (width 4, ring history) then h_t = a_t h_(t-1) +
    (1-a_t) u_t. x, a [B,T,D]; w [D,4] float32; h0 [B,D] float32; ring [B,D,3] x.dtype with
    `pos` tokens absorbed before. Returns y = h [B,T,D], or (y, h_T, ring_out) with
    return_state (ring_out is the ring updated in place when `ring` is given, else None)."""
    _diag_check(x, a, w, bias, 3)
    B, T, D = x.shape
    x, a, w = x.contiguous(), a.contiguous(), w.contiguous()
    if h0 is not None:
        if h0.shape != (B, D) or h0.dtype != torch.float32:
            raise ValueError("diag: h0 must be float32 [B, D]")
        h0 = h0.contiguous()
    if ring is not None and (ring.shape != (B, D, CONV_WIDTH - 1) or ring.dtype != x.dtype
                             or not ring.is_contiguous()):
        raise ValueError("diag: ring must be a contiguous [B, D, 3] tensor of x's dtype")
    lib = _lib.require()
    y = torch.empty_like(x)
    hT = torch.empty(B, D, device=x.device, dtype=torch.float32) if return_state else None
    if ring_out is None and return_state:
        ring_out = ring
    with torch.cuda.device(x.device):
        need = lib.mira_diag_workspace_bytes(B, T, D, DTYPE[x.dtype])
        space = workspace("diag", x.device, need, zero=True)
        code = lib.mira_diag_conv_scan(
            _ptr(x), _ptr(a), _ptr(w), _ptr(bias), _ptr(h0), _ptr(ring), _ptr(ring_out),
            int(pos), _ptr(y), _ptr(hT), B, T, D, CONV_WIDTH, DTYPE[x.dtype], _ptr(space),
            space.numel(), _stream(x.device))
    if _lib.check(code, "mira_diag_conv_scan") is None:
        return None
    USED["diag"] += 1
    return (y, hT, ring_out) if return_state else y


def diag_conv_step(x, a, w, bias, h, ring, pos, out=None):
    """One decode token: x, a [B,D]; h [B,D] float32 and ring [B,D,3] updated in place."""
    _diag_check(x, a, w, bias, 2)
    B, D = x.shape
    if h.shape != (B, D) or h.dtype != torch.float32 or not h.is_contiguous():
        raise ValueError("diag: h must be a contiguous float32 [B, D] state")
    if ring is not None and (ring.shape != (B, D, CONV_WIDTH - 1) or ring.dtype != x.dtype
                             or not ring.is_contiguous()):
        raise ValueError("diag: ring must be a contiguous [B, D, 3] tensor of x's dtype")
    lib = _lib.require()
    y = out if out is not None else torch.empty_like(x)
    code = lib.mira_diag_conv_step(_ptr(x.contiguous()), _ptr(a.contiguous()), _ptr(w),
                                   _ptr(bias), _ptr(h), _ptr(ring), int(pos), _ptr(y), B, D,
                                   CONV_WIDTH, DTYPE[x.dtype], _stream(x.device))
    if _lib.check(code, "mira_diag_conv_step") is None:
        return None
    USED["step"] += 1
    return y


def diag_workspace_error(device=None):
    """The look-back watchdog word of this stream's diag workspace (synchronous): 0 = every
    prefill wait on it ended normally."""
    import ctypes

    device = torch.device("cuda", torch.cuda.current_device() if device is None else device)
    key = ("diag", device.index, torch.cuda.current_stream(device).cuda_stream)
    buffer = _WORKSPACES.get(key)
    if buffer is None:
        return 0
    value = ctypes.c_uint(0)
    torch.cuda.synchronize(device)
    _lib.check(_lib.require().mira_diag_workspace_error(_ptr(buffer), buffer.numel(),
                                                        ctypes.byref(value)), "watchdog")
    return int(value.value)


# --------------------------------------------------------------------------------------------
# BASELINE-literal: GLA matrix state
# --------------------------------------------------------------------------------------------
def _gla_check(q, k, v, g, dims):
    if q.dim() != dims or k.shape != q.shape or v.shape[:-1] != q.shape[:-1]:
        raise ValueError("gla: q, k [.., H, d_k] and v [.., H, d_v] must agree")
    if q.dtype not in DTYPE or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("gla: q, k, v must share a float dtype")
    if g.shape != q.shape[:-1] or g.dtype != torch.float32:
        raise ValueError("gla: g must be float32 with q's leading shape")


def gla_chunked(q, k, v, g, state=None, return_state=False):
    """Prefill: S_t = exp(g_t) S_(t-1) + k_t v_t^T, o_t = S_t^T q_t. q, k [B,T,H,d_k],
    v [B,T,H,d_v], g [B,T,H] float32; state [B,H,d_v,d_k] float32. Returns o [B,T,H,d_v], or
    (o, S_T) with return_state."""
    _gla_check(q, k, v, g, 4)
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    if state is not None and (state.shape != (B, H, dv, dk) or state.dtype != torch.float32):
        raise ValueError("gla: state must be float32 [B, H, d_v, d_k]")
    lib = _lib.require()
    q, k, v, g = q.contiguous(), k.contiguous(), v.contiguous(), g.contiguous()
    state = None if state is None else state.contiguous()
    o = torch.empty(B, T, H, dv, device=q.device, dtype=q.dtype)
    final = torch.empty(B, H, dv, dk, device=q.device, dtype=torch.float32) if return_state else None
    with torch.cuda.device(q.device):
        need = lib.mira_gla_workspace_bytes(B, T, H, dk, dv)
        space = workspace("gla", q.device, need)
        code = lib.mira_gla_chunked(_ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(state), _ptr(final),
                                    _ptr(o), B, T, H, dk, dv, DTYPE[q.dtype], _ptr(space),
                                    0 if space is None else space.numel(), _stream(q.device))
    if _lib.check(code, "mira_gla_chunked") is None:
        return None
    USED["gla"] += 1
    return (o, final) if return_state else o


def gla_step(q, k, v, g, state, out=None):
    """One decode token: q, k [B,H,d_k], v [B,H,d_v], g [B,H]; state [B,H,d_v,d_k] float32
    updated in place. Returns o [B,H,d_v]."""
    _gla_check(q, k, v, g, 3)
    B, H, dk = q.shape
    dv = v.shape[-1]
    if (state.shape != (B, H, dv, dk) or state.dtype != torch.float32
            or not state.is_contiguous()):
        raise ValueError("gla: state must be a contiguous float32 [B, H, d_v, d_k] tensor")
    lib = _lib.require()
    o = out if out is not None else torch.empty(B, H, dv, device=q.device, dtype=q.dtype)
    code = lib.mira_gla_step(_ptr(q.contiguous()), _ptr(k.contiguous()), _ptr(v.contiguous()),
                             _ptr(g.contiguous()), _ptr(state), _ptr(o), B, H, dk, dv,
                             DTYPE[q.dtype], _stream(q.device))
    if _lib.check(code, "mira_gla_step") is None:
        return None
    USED["step"] += 1
    return o


def linear_silu(x, weight, bias):
    """SiLU(x W^T + b) of the MiraBlock feed-forward's first projection (model/mira_block.py:
    38-48) as one hipBLASLt GEMM with a bias + SiLU epilogue (mira_linear_silu): bf16 x [..., in],
    weight [out, in], bias [out], all contiguous, on one GPU. None where the library declines
    (no algorithm for the shape); ValueError for arguments it cannot take."""
    tensors = (x, weight, bias)
    if any(t.dtype != torch.bfloat16 or not t.is_cuda for t in tensors):
        raise ValueError("linear_silu: x, weight and bias must be bf16 tensors on the GPU")
    if len({t.device for t in tensors}) != 1:
        raise ValueError("linear_silu: x, weight and bias must be on one device")
    if weight.dim() != 2 or bias.shape != (weight.shape[0],) or x.shape[-1] != weight.shape[1]:
        raise ValueError("linear_silu: shapes must be x [..., in], weight [out, in], bias [out]")
    x = x.contiguous()
    weight, bias = weight.contiguous(), bias.contiguous()
    rows = x.numel() // x.shape[-1]
    out = torch.empty(*x.shape[:-1], weight.shape[0], device=x.device, dtype=x.dtype)
    lib = _lib.require()
    code = lib.mira_linear_silu(_ptr(x), _ptr(weight), _ptr(bias), _ptr(out), rows,
                                int(weight.shape[1]), int(weight.shape[0]), _stream(x.device))
    if _lib.check(code, "mira_linear_silu") is None:
        return None
    USED["linear_silu"] += 1
    return out
