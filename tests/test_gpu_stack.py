"""The layer stack on the GPU: mira_amd.llm.MiraLLM (embedding, MiraBlocks whose mixer scans on
the HIP library, final norm, tied head) against oracle/stack.py in float64 on the same weights,
in float32 and bfloat16 (the oracle rounding to bf16 wherever the bf16 model stores a tensor),
with a padding mask; and a prompt followed by single-token steps through
a PrefixCache against the one-shot forward (the kv_cache.check invariant of
helpers/kv_cache.py:196-233 applied to the whole model)."""
import numpy as np
import pytest

from _util import FP32_SCALED, HALF_SCALED, scaled
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


def test_gradients_are_refused_not_dropped(torch_mod, model_cls):
    """There is no backward for the scan: under autograd the plugin declines (even with a state,
    where the reference would return one with a gradient) and the mixer raises, instead of
    returning values that carry no gradient."""
    torch = torch_mod
    from mira_amd import mira
    from oracle import lattice as L

    rng = np.random.default_rng(9)
    values = [torch.tensor(v, device="cuda").requires_grad_() for v in L.random_inputs(rng, 1, 5, 8, 2, 16)]
    x, alpha, rho, gamma, write, read, beta = values
    state = torch.zeros(1, 2, 8, 16, device="cuda")
    assert mira.matrix_lattice_iir(x, alpha, rho, gamma, write, read, raw_beta=beta, state=state,
                                   return_state=True) is None
    model = _model(torch, model_cls, 3, torch.float32)
    ids = torch.tensor([[1, 2, 3]], device="cuda")
    with pytest.raises(RuntimeError, match="inference only"):
        model(ids)
    with torch.no_grad():
        assert model(ids).logits.shape == (1, 3, CFG["vocab_size"])
