"""The layer stack on the GPU: mira_amd.llm.MiraLLM (embedding, MiraBlocks whose mixer scans on
the HIP library, final norm, tied head) against oracle/stack.py in float64 on the same weights,
in float32 and bfloat16 (the oracle rounding to bf16 wherever the bf16 model stores a tensor),
with a padding mask; and a prompt followed by single-token steps through
a PrefixCache against the one-shot forward (the kv_cache.check invariant of
helpers/kv_cache.py:196-233 applied to the whole model)."""
import os

import numpy as np
import pytest

from _util import FP32_SCALED, HALF_SCALED, golden_files, max_abs, scaled
from oracle import stack as St

pytestmark = pytest.mark.gpu

CFG = dict(vocab_size=97, n_layer=2, n_embd=64, lattice_d_e=96, lattice_order=2,
           coefficient_bottleneck=16, memory_dimension=32, ffn_hidden=160,
           arch="cauchy_x_hyperbolic")


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available()
    return torch


@pytest.fixture(scope="module")
def model_cls():
    from mira_amd import _lib
    from mira_amd.llm import MiraLLM

    assert _lib.library() is not None, _lib.why()
    return MiraLLM


def _model(torch, MiraLLM, seed, dtype):
    torch.manual_seed(seed)
    model = MiraLLM(**CFG)
    with torch.no_grad():
        # weights large enough that every block changes the residual stream visibly
        for name, value in model.named_parameters():
            if name.endswith("weight") and value.dim() == 2:
                value.normal_(0.0, 1.0 / np.sqrt(value.shape[1]))
            elif name.endswith("bias"):
                value.normal_(0.0, 0.05)
    return model.to(device="cuda", dtype=dtype).eval()


def _params(model):
    return {k: v.detach().double().cpu().numpy() for k, v in model.state_dict().items()}


def _rounding(torch, dtype):
    """Where a half-precision model stores a tensor, the oracle rounds to the same type."""
    if dtype == "float32":
        return None
    kind = getattr(torch, dtype)
    return lambda a: torch.from_numpy(np.asarray(a, np.float64)).to(kind).double().numpy()


@pytest.mark.parametrize("dtype,bound", [("float32", FP32_SCALED), ("bfloat16", HALF_SCALED)])
def test_llm_matches_the_oracle(torch_mod, model_cls, dtype, bound):
    torch = torch_mod
    model = _model(torch, model_cls, 0, getattr(torch, dtype))
    rng = np.random.default_rng(7)
    ids = rng.integers(0, CFG["vocab_size"], (2, 37))
    valid = np.ones((2, 37), bool)
    valid[0, :5] = False                       # left padding of the first sequence
    valid[1, 20] = False
    mask = torch.tensor(valid, device="cuda")
    with torch.no_grad():
        got = model(torch.tensor(ids, device="cuda"), attention_mask=mask).logits
    want, _ = St.llm_forward(ids, _params(model), CFG, valid=valid, rnd=_rounding(torch, dtype))
    error = scaled(got.float().cpu().numpy(), want)
    assert error <= bound, f"{dtype}: scaled error {error:.3e}"


@pytest.mark.parametrize("dtype,bound", [("float32", FP32_SCALED), ("bfloat16", HALF_SCALED)])
def test_split_and_padded_projections_match_the_oracle(torch_mod, model_cls, monkeypatch, dtype,
                                                       bound):
    """The long-input projections -- [signal | gate] and [write | control] as two GEMMs, and
    the coefficient projection on weights padded to 1,024 rows (d_e 100: 796 coefficients) --
    against the oracle, with a padding mask."""
    torch = torch_mod
    from mira_amd import mixer as mixer_module

    monkeypatch.setattr(mixer_module, "SPLIT_ROWS", 1)
    cfg = dict(CFG, lattice_d_e=100)
    torch.manual_seed(3)
    model = model_cls(**cfg)
    with torch.no_grad():
        for name, value in model.named_parameters():
            if name.endswith("weight") and value.dim() == 2:
                value.normal_(0.0, 1.0 / np.sqrt(value.shape[1]))
            elif name.endswith("bias"):
                value.normal_(0.0, 0.05)
    model = model.to(device="cuda", dtype=getattr(torch, dtype)).eval()
    rng = np.random.default_rng(8)
    ids = rng.integers(0, cfg["vocab_size"], (2, 41))
    valid = np.ones((2, 41), bool)
    valid[1, :3] = False
    with torch.no_grad():
        got = model(torch.tensor(ids, device="cuda"),
                    attention_mask=torch.tensor(valid, device="cuda")).logits
    mixer = model.blocks[0].mixer
    assert mixer.__dict__["_padded_coefficients"]["tensors"][0].shape[0] == 1024
    want, _ = St.llm_forward(ids, _params(model), cfg, valid=valid, rnd=_rounding(torch, dtype))
    error = scaled(got.float().cpu().numpy(), want)
    assert error <= bound, f"{dtype}: scaled error {error:.3e}"


@pytest.mark.parametrize("rows,width,hidden", [(37, 64, 160), (8192, 2048, 8192)])
def test_fused_feed_forward_projection(torch_mod, model_cls, rows, width, hidden):
    """The inference feed-forward's up projection, bias and SiLU as one GEMM (mira_linear_silu)
    against the unfused torch steps, at a small shape and the cfg5 one (bf16: one rounding
    against two, so a few outputs land one bf16 ulp away)."""
    torch = torch_mod
    from mira_amd import mira
    from mira_amd.block import FeedForward

    torch.manual_seed(4)
    ffn = FeedForward(width, hidden=hidden).to(device="cuda", dtype=torch.bfloat16).eval()
    x = torch.randn(1, rows, width, device="cuda", dtype=torch.bfloat16)
    before = mira.USED["linear_silu"]
    with torch.no_grad():
        fused = mira.linear_silu(x, ffn.up.weight, ffn.up.bias)
        steps = torch.nn.functional.silu(ffn.up(x))
        whole = ffn(x)
    assert mira.USED["linear_silu"] == before + 2
    assert fused.shape == steps.shape
    error = scaled(fused.float().cpu().numpy(), steps.float().cpu().numpy())
    assert error <= 1e-2, f"fused SiLU(up): scaled error {error:.3e}"
    torch.testing.assert_close(whole, ffn.down(fused), rtol=0, atol=0)


def test_prompt_then_steps_equals_one_shot(torch_mod, model_cls):
    torch = torch_mod
    from mira_amd.prefix_cache import PrefixCache

    model = _model(torch, model_cls, 1, torch.float32)
    ids = torch.tensor(np.random.default_rng(8).integers(0, CFG["vocab_size"], (3, 26)),
                       device="cuda")
    with torch.no_grad():
        full = model(ids).logits
        cache = PrefixCache(CFG["n_layer"])
        parts = [model(ids[:, :17], cache=cache).logits]
        for t in range(17, 26):
            parts.append(model(ids[:, t:t + 1], cache=cache).logits)
    assert len(cache) == 26
    error = scaled(torch.cat(parts, dim=1).cpu().numpy(), full.cpu().numpy())
    assert error <= 1e-5, f"stepped vs one-shot: scaled error {error:.3e}"


STACK_FIXTURES = golden_files("stack_")


@pytest.mark.parametrize("path", STACK_FIXTURES, ids=os.path.basename)
def test_hip_stack_matches_the_reference_fixtures(torch_mod, model_cls, path):
    """The reference's own MiraMixer, MiraBlock and 2-layer MiraLLM outputs (CPU, float32, written
    by tests/golden/make_golden.py) against mira_amd's modules on the GPU in float32 with the
    same state_dict: the mixer with a padding mask, the block, the LLM logits, and prompt-then-
    steps through a PrefixCache. Bound: max abs error <= 1e-5 x max(1, largest magnitude)."""
    torch = torch_mod
    from mira_amd.prefix_cache import PrefixCache

    f = np.load(path, allow_pickle=False)
    cfg = dict(vocab_size=40, n_layer=2, n_embd=24, lattice_d_e=12, lattice_order=2,
               coefficient_bottleneck=6, memory_dimension=4, ffn_hidden=32, arch=str(f["arch"]))
    model = model_cls(**cfg)
    model.load_state_dict({k[2:]: torch.from_numpy(f[k].copy()) for k in f.files
                           if k.startswith("p.")}, strict=True)
    model = model.to("cuda").eval()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda")  # noqa: E731
    ids, mask, prompt = t(f["ids"]), t(f["mask"]), int(f["prompt"])
    with torch.no_grad():
        block = model.blocks[0]
        got = dict(mixer_out=block.mixer(block.rn1(t(f["hidden"])), mask),
                   block_out=block(t(f["hidden"]), mask),
                   llm_logits=model(ids, attention_mask=mask).logits)
        cache = PrefixCache(cfg["n_layer"], budget=0)
        parts = [model(ids[:, :prompt], cache=cache).logits]
        for i in range(prompt, ids.shape[1]):
            parts.append(model(ids[:, i:i + 1], cache=cache).logits)
        got["steps_logits"] = torch.cat(parts, dim=1)
    for name, value in got.items():
        want = f[name]
        error = max_abs(value.float().cpu().numpy(), want)
        assert error <= 1e-5 * max(1.0, float(np.abs(want).max())), f"{name}: {error:.3e}"


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_rms_norm_against_the_stepwise_form(torch_mod, dtype):
    """mira_amd.block.RMSNorm against the reference's stepwise float32 form
    (model/mira_block.py:28-35) on the GPU: float32 runs those steps, so it is bit-identical;
    bf16 runs PyTorch's fused rms_norm, whose sum of squares is ordered differently, so a few
    outputs in 10^4 may land one bf16 ulp away and none further."""
    torch = torch_mod
    from mira_amd.block import RMSNorm

    kind = getattr(torch, dtype)
    torch.manual_seed(11)
    for width in (24, 64, 2048, 4096):
        norm = RMSNorm(width).to("cuda", kind)
        with torch.no_grad():
            norm.weight.normal_(1.0, 0.2)
            x = (torch.randn(4, 33, width, device="cuda") * 3.0).to(kind)
            got = norm(x)
            z = x.float()
            stepwise = (z * torch.rsqrt(z.square().mean(dim=-1, keepdim=True) + norm.eps)
                        * norm.weight.float()).to(kind)
        if dtype == "float32":
            assert torch.equal(got, stepwise), f"width {width}"
            continue
        differ = got != stepwise
        ulp = torch.finfo(kind).eps * stepwise.float().abs().clamp_min(
            torch.finfo(kind).tiny)
        gap = (got.float() - stepwise.float()).abs()
        assert int(differ.sum()) <= max(1, differ.numel() // 10_000), f"width {width}"
        assert bool((gap <= ulp).all()), f"width {width}: a gap over one bf16 ulp"


def test_gradient_rules(torch_mod, model_cls):
    """Under autograd the scan keeps a graph only where the reference's does: with return_state
    (a cache) it runs without one and hands back outputs that carry no gradient
    (kernel/cuda/mira_dspv2/mira.py:1538-1563); a (K, d_m) without backward kernels declines
    (None, and the mixer raises) instead of dropping the gradient; a served one trains."""
    torch = torch_mod
    from mira_amd import mira
    from oracle import lattice as L

    rng = np.random.default_rng(9)
    values = [torch.tensor(v, device="cuda").requires_grad_() for v in L.random_inputs(rng, 1, 5, 8, 2, 16)]
    x, alpha, rho, gamma, write, read, beta = values
    state = torch.zeros(1, 2, 8, 16, device="cuda")
    y, final = mira.matrix_lattice_iir(x, alpha, rho, gamma, write, read, raw_beta=beta,
                                       state=state, return_state=True)
    assert not y.requires_grad and not final.requires_grad
    assert mira.matrix_lattice_iir(x, alpha, rho, gamma, write, read, raw_beta=beta).requires_grad
    wide = [torch.tensor(v, device="cuda").requires_grad_()
            for v in L.random_inputs(rng, 1, 5, 8, 2, 128)]
    assert mira.matrix_lattice_iir(*wide[:6], raw_beta=wide[6]) is None
    with torch.no_grad():
        assert mira.matrix_lattice_iir(*wide[:6], raw_beta=wide[6]) is not None
    model = _model(torch, model_cls, 3, torch.float32)
    ids = torch.tensor([[1, 2, 3]], device="cuda")
    model(ids).logits.sum().backward()
    assert model.blocks[0].mixer.coefficient_projection.weight.grad is not None
