"""The backward of the lattice scan on the GPU (mira_lattice_backward through the autograd
Function of mira_amd.mira), against:
  * the reference's own autograd gradients (tests/golden/grad_*.npz: all 15 stage maps at K=2
    d_m=16 with a mask, and K/d_m 1/8, 4/8, 2/32, 2/64, 8/16), fp32, at the reference harness's
    bound (scaled error <= 3e-4, kernel/cuda/mira_dspv2/check.py:92);
  * the fp64 oracle backward (oracle/lattice.py lattice_backward) over several chunks, with masks
    and row-strided views, in fp32 (3e-4) and bf16 (1.5e-2, inputs rounded as the kernel sees
    them);
  * the packed-projection contract (gradients written into the projections' storage, the raw
    write's through SiLU') against the unpacked call;
  * a MiraLLM training step (loss.backward) against the same modules on the CPU in float64 whose
    scan is the oracle's forward and backward.
"""
import os

import numpy as np
import pytest

from _util import FP32_SCALED, golden_files, rounded, scaled, to_device, to_numpy
from oracle import lattice as L

pytestmark = pytest.mark.gpu

GRAD_NAMES = ("x", "alpha", "beta", "rho", "gamma", "write", "read")
INPUT_NAMES = ("x", "alpha", "rho", "gamma", "write", "read", "beta")
BF16_SCALED = 1.5e-2


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available()
    return torch


@pytest.fixture(scope="module")
def plugin():
    from mira_amd import _lib, mira

    assert _lib.library() is not None, _lib.why()
    return mira


def _run(torch, plugin, inputs, dy, valid, arch, dtype, strided=False):
    """Forward and backward through the plugin; returns (y, grads by GRAD_NAMES)."""
    kind = getattr(torch, dtype)
    tensors = []
    for i, value in enumerate(inputs):
        t = to_device(value, kind)
        if strided and i in (0, 3):                 # x and gamma as row-strided views
            B, T, C = t.shape
            base = torch.zeros(B, T, 2 * C + 3, device="cuda", dtype=kind)
            base[:, :, C + 1:2 * C + 1] = t
            t = base[:, :, C + 1:2 * C + 1]
        tensors.append(t.detach().requires_grad_(True))
    x, alpha, rho, gamma, write, read, beta = tensors
    mask = None if valid is None else torch.tensor(valid, device="cuda")
    y = plugin.matrix_lattice_iir(x, alpha, rho, gamma, write, read, raw_beta=beta, valid=mask,
                                  arch=arch)
    assert y is not None and y.requires_grad
    (y.float() * to_device(dy)).sum().backward()
    grads = dict(x=x.grad, alpha=alpha.grad, beta=beta.grad, rho=rho.grad, gamma=gamma.grad,
                 write=write.grad, read=read.grad)
    return to_numpy(y), {k: to_numpy(v) for k, v in grads.items()}


@pytest.mark.parametrize("path", golden_files("grad_"), ids=os.path.basename)
def test_gradients_match_reference_autograd(torch_mod, plugin, path):
    f = np.load(path, allow_pickle=False)
    valid = f["valid"] if "valid" in f.files else None
    inputs = [f[n] for n in INPUT_NAMES]
    y, grads = _run(torch_mod, plugin, inputs, f["dy"], valid, str(f["arch"]), "float32")
    assert scaled(y, f["y"]) <= FP32_SCALED
    for name in GRAD_NAMES:
        error = scaled(grads[name], f["d" + name])
        assert error <= FP32_SCALED, f"d{name}: scaled error {error:.3e}"


CASES = [(2, 16, "cauchy_x_hyperbolic"), (2, 64, "expsoftplus_x_mobius"),
         (1, 8, "hill_x_identity"), (4, 32, "gaussian_x_hyperbolic"), (8, 8, "expexp_x_mobius"),
         (2, 8, "cauchy_x_mobius"), (4, 64, "cauchy_x_identity"), (1, 16, "expexp_x_hyperbolic")]


@pytest.mark.parametrize("K,M,arch", CASES)
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_gradients_match_the_oracle_over_chunks(torch_mod, plugin, K, M, arch, dtype):
    """T = 100 spans several backward chunks (and ends in a partial one); a padding mask, an
    inner masked token and row-strided x / gamma views."""
    torch = torch_mod
    rng = np.random.default_rng(K * 100 + M)
    B, T, C = 2, 100, 37
    inputs = L.random_inputs(rng, B, T, C, K, M)
    valid = rng.random((B, T)) > 0.2
    valid[0, :3] = False
    dy = rng.standard_normal((B, T, C)).astype(np.float32)
    kind = getattr(torch, dtype)
    seen = [rounded(v, kind) for v in inputs] if dtype != "float32" else inputs
    want = L.lattice_backward(*seen, rounded(dy, kind) if dtype != "float32" else dy,
                              valid=valid, arch=arch)
    dy_in = rounded(dy, kind) if dtype != "float32" else dy
    _, grads = _run(torch, plugin, inputs, dy_in, valid, arch, dtype, strided=True)
    bound = FP32_SCALED if dtype == "float32" else BF16_SCALED
    for name, value in zip(GRAD_NAMES, want):
        error = scaled(grads[name], value)
        assert error <= bound, f"d{name}: scaled error {error:.3e}"


def test_short_sequences_and_one_token(torch_mod, plugin):
    """T below one chunk (no adjoint summary or combine) and T = 1."""
    torch = torch_mod
    for T in (1, 5, 16, 17):
        rng = np.random.default_rng(T)
        inputs = L.random_inputs(rng, 3, T, 9, 2, 16)
        dy = rng.standard_normal((3, T, 9)).astype(np.float32)
        want = L.lattice_backward(*inputs, dy, arch="cauchy_x_hyperbolic")
        _, grads = _run(torch, plugin, inputs, dy, None, "cauchy_x_hyperbolic", "float32")
        for name, value in zip(GRAD_NAMES, want):
            assert scaled(grads[name], value) <= FP32_SCALED, f"T={T} d{name}"


def test_packed_projections_receive_the_gradients(torch_mod, plugin):
    """With packed=(input projection, coefficient projection) the gradients land in those two
    tensors whole -- x and the raw write (through SiLU') in the first, alpha, beta, rho and nu in
    the second -- and equal the unpacked call's (mira.py:1518-1537,1346-1361)."""
    torch = torch_mod
    import torch.nn.functional as F

    rng = np.random.default_rng(5)
    B, T, C, K, M = 2, 40, 24, 2, 16
    width = C * (3 * K + 1) + (K + 1) * M
    packed_input = torch.tensor(rng.standard_normal((B, T, C + M)) * 0.3, dtype=torch.float32,
                                device="cuda", requires_grad=True)
    packed_coefficients = torch.tensor(rng.standard_normal((B, T, width)) * 0.3,
                                       dtype=torch.float32, device="cuda", requires_grad=True)
    gamma = torch.tensor(rng.standard_normal((B, T, C)) * 0.5, dtype=torch.float32,
                         device="cuda", requires_grad=True)
    dy = torch.tensor(rng.standard_normal((B, T, C)), dtype=torch.float32, device="cuda")

    def views(pi, pc):
        x, raw_write = pi.split((C, M), dim=-1)
        a, b, r, n = pc.split((C * K, C * K, C * (K + 1), (K + 1) * M), dim=-1)
        return (x, a.view(B, T, C, K), b.view(B, T, C, K), r.view(B, T, C, K + 1),
                n.view(B, T, K + 1, M), raw_write)

    x, a, b, r, n, raw_write = views(packed_input, packed_coefficients)
    y = plugin.matrix_lattice_iir(x, a, r, gamma, F.silu(raw_write).contiguous(), n, raw_beta=b,
                                  packed=(packed_input, packed_coefficients))
    (y * dy).sum().backward()
    # the same function, unpacked: autograd chains SiLU and the views itself
    pi2 = packed_input.detach().clone().requires_grad_(True)
    pc2 = packed_coefficients.detach().clone().requires_grad_(True)
    g2 = gamma.detach().clone().requires_grad_(True)
    x2, a2, b2, r2, n2, w2 = views(pi2, pc2)
    y2 = plugin.matrix_lattice_iir(x2.contiguous(), a2.contiguous(), r2.contiguous(), g2,
                                   F.silu(w2).contiguous(), n2.contiguous(), raw_beta=b2.contiguous())
    (y2 * dy).sum().backward()
    torch.testing.assert_close(y, y2)
    for got, want in ((packed_input.grad, pi2.grad), (packed_coefficients.grad, pc2.grad),
                      (gamma.grad, g2.grad)):
        assert scaled(to_numpy(got), to_numpy(want)) <= 1e-5
    with pytest.raises(ValueError, match="packed"):
        plugin.matrix_lattice_iir(x, a, r, gamma, F.silu(raw_write).contiguous(), n, raw_beta=b,
                                  packed=(packed_input, packed_coefficients[:, :, 1:]))


def _oracle_scan_function(torch):
    """A CPU float64 scan for torch autograd: forward and backward are the oracle's."""

    class Scan(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x, alpha, rho, gamma, write, read, beta, valid, arch):
            arrays = [t.detach().numpy() for t in (x, alpha, rho, gamma, write, read, beta)]
            mask = None if valid is None else valid.numpy()
            y, _ = L.lattice_scan_sequential(*arrays, valid=mask, arch=arch, dtype=np.float64)
            ctx.saved = (arrays, mask, arch)
            return torch.from_numpy(y)

        @staticmethod
        def backward(ctx, dy):
            arrays, mask, arch = ctx.saved
            g = L.lattice_backward(*arrays, dy.numpy(), valid=mask, arch=arch)
            dx, dalpha, dbeta, drho, dgamma, dwrite, dread = (torch.from_numpy(v) for v in g)
            return dx, dalpha, drho, dgamma, dwrite, dread, dbeta, None, None

    def matrix_lattice_iir(x, raw_alpha, raw_rho, gamma, memory_write, memory_read,
                           raw_beta=None, valid=None, state=None, return_state=False,
                           packed=None, arch="cauchy_x_hyperbolic", **unused):
        assert state is None and not return_state
        return Scan.apply(x, raw_alpha, raw_rho, gamma, memory_write, memory_read, raw_beta,
                          valid, arch)

    return matrix_lattice_iir


@pytest.mark.parametrize("arch,positive", [("cauchy_x_hyperbolic", False),
                                           ("cauchy_x_mobius", True)])
def test_llm_training_step_matches_float64_oracle_autograd(torch_mod, plugin, monkeypatch, arch,
                                                           positive):
    """loss.backward() of a 2-layer MiraLLM on the GPU in float32 (the mixer's training path:
    packed projections, the plugin's backward) against the same modules on the CPU in float64
    with the oracle's scan; every parameter's gradient within 3e-4 scaled."""
    torch = torch_mod
    from mira_amd import mixer as mixer_module
    from mira_amd.llm import MiraLLM

    order = 1 if positive else 2
    cfg = dict(vocab_size=53, n_layer=2, n_embd=32, lattice_d_e=24, lattice_order=order,
               coefficient_bottleneck=8, memory_dimension=16, ffn_hidden=48, arch=arch,
               lattice_positive_poles=positive)
    torch.manual_seed(3)
    gpu = MiraLLM(**cfg)
    with torch.no_grad():
        for name, value in gpu.named_parameters():
            if value.dim() == 2:
                value.normal_(0.0, 1.0 / np.sqrt(value.shape[1]))
            elif name.endswith("bias"):
                value.normal_(0.0, 0.1)
    cpu = MiraLLM(**cfg).double()
    cpu.load_state_dict({k: v.double() for k, v in gpu.state_dict().items()})
    gpu = gpu.cuda().train()
    rng = np.random.default_rng(4)
    ids = rng.integers(0, cfg["vocab_size"], (2, 37))
    valid = np.ones((2, 37), bool)
    valid[0, :4] = False
    targets = torch.tensor(rng.integers(0, cfg["vocab_size"], (2, 37)))

    def loss_of(model, device):
        logits = model(torch.tensor(ids, device=device),
                       attention_mask=torch.tensor(valid, device=device)).logits
        return torch.nn.functional.cross_entropy(logits.reshape(-1, cfg["vocab_size"]).double(),
                                                 targets.to(device).reshape(-1))

    loss_of(gpu, "cuda").backward()
    assert plugin.usage()["backward"] > 0
    monkeypatch.setattr(mixer_module.plugin, "matrix_lattice_iir", _oracle_scan_function(torch))
    loss_of(cpu.train(), "cpu").backward()
    monkeypatch.undo()
    for (name, p_gpu), (_, p_cpu) in zip(gpu.named_parameters(), cpu.named_parameters()):
        if p_cpu.grad is None:
            assert p_gpu.grad is None or float(p_gpu.grad.abs().max()) == 0.0, name
            continue
        error = scaled(to_numpy(p_gpu.grad), p_cpu.grad.numpy())
        assert error <= FP32_SCALED, f"{name}: scaled error {error:.3e}"
