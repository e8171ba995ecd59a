"""CPU checks of the layer stack around the scan: the oracle's RMSNorm / mixer / block / LLM
restatement (oracle/stack.py) pinned against closed forms and invariants, and the host modules
(mira_amd.block, mira_amd.llm) against the oracle where they need no GPU."""
import os

import numpy as np
import pytest

from _util import golden_files, scaled
from oracle import stack as St

STACK_FIXTURES = golden_files("stack_")
STACK_CFG = dict(vocab_size=40, n_layer=2, n_embd=24, lattice_d_e=12, lattice_order=2,
                 coefficient_bottleneck=6, memory_dimension=4, ffn_hidden=32)
# the oracle in float64 against the reference's float32 modules: a few float32 roundings apart
FIXTURE_SCALED = 1e-5


def _fixture(path):
    f = np.load(path, allow_pickle=False)
    params = {k[2:]: f[k].astype(np.float64) for k in f.files if k.startswith("p.")}
    return f, params, dict(STACK_CFG, arch=str(f["arch"]))


def _oracle_outputs(f, p, cfg):
    mask = f["mask"]
    hidden = f["hidden"].astype(np.float64)
    pre = "blocks.0."
    mixer, _ = St.mixer_forward(St.rmsnorm(hidden, p[pre + "rn1.weight"]), p, pre + "mixer.",
                                cfg["lattice_order"], cfg["lattice_d_e"],
                                cfg["memory_dimension"], cfg["arch"], valid=mask)
    block, _ = St.block_forward(hidden, p, pre, cfg, valid=mask)
    logits, _ = St.llm_forward(f["ids"], p, cfg, valid=mask)
    prompt = int(f["prompt"])
    ids = f["ids"]
    parts, states = [], None
    first, states = St.llm_forward(ids[:, :prompt], p, cfg)
    parts.append(first)
    for t in range(prompt, ids.shape[1]):
        step, states = St.llm_forward(ids[:, t:t + 1], p, cfg, states=states)
        parts.append(step)
    return dict(mixer_out=mixer, block_out=block, llm_logits=logits,
                steps_logits=np.concatenate(parts, axis=1))


@pytest.mark.parametrize("path", STACK_FIXTURES, ids=os.path.basename)
def test_oracle_matches_the_reference_stack(path):
    """The reference's MiraMixer, MiraBlock and 2-layer MiraLLM (model/mira_mixer.py:657-856,
    model/mira_block.py:21-48,203-205, model/mira_llm.py:225-351) on the CPU, with a nonzero
    coefficient projection, a padding mask and prompt-then-steps through its PrefixCache."""
    f, p, cfg = _fixture(path)
    for name, got in _oracle_outputs(f, p, cfg).items():
        error = scaled(got, f[name])
        assert error <= FIXTURE_SCALED, f"{name}: scaled error {error:.3e}"


def test_planted_stack_mistakes_are_caught(monkeypatch):
    """A control without its SiLU, or a final norm without its bias, misses the reference's
    logits by far more than the tolerance."""
    f, p, cfg = _fixture(STACK_FIXTURES[0])
    mask = f["mask"]
    monkeypatch.setattr(St, "control_activation", lambda x: x)
    no_silu, _ = St.llm_forward(f["ids"], p, cfg, valid=mask)
    monkeypatch.undo()
    assert scaled(no_silu, f["llm_logits"]) > 100 * FIXTURE_SCALED
    no_bias = dict(p, **{"lnf.bias": np.zeros_like(p["lnf.bias"])})
    dropped, _ = St.llm_forward(f["ids"], no_bias, cfg, valid=mask)
    assert scaled(dropped, f["llm_logits"]) > 100 * FIXTURE_SCALED
    untied = dict(p, **{"head.weight": p["head.weight"][::-1].copy()})
    wrong_head, _ = St.llm_forward(f["ids"], untied, cfg, valid=mask)
    assert scaled(wrong_head, f["llm_logits"]) > 100 * FIXTURE_SCALED


def test_host_model_loads_the_reference_state_dict():
    """A reference MiraLLM state_dict (names and shapes, the tied head and the unused mask
    embedding included) loads into mira_amd.llm.MiraLLM without a missing or extra key."""
    torch = pytest.importorskip("torch")
    from mira_amd.llm import MiraLLM

    f, _, cfg = _fixture(STACK_FIXTURES[0])
    model = MiraLLM(**cfg)
    state = {k[2:]: torch.from_numpy(f[k].copy()) for k in f.files if k.startswith("p.")}
    model.load_state_dict(state, strict=True)
    assert model.tok.weight is model.head.weight


def _params(rng, cfg, scale=0.3):
    """A parameter dict with mira_amd.llm.MiraLLM's state_dict names."""
    d, C, K, M, R = (cfg["n_embd"], cfg["lattice_d_e"], cfg["lattice_order"],
                     cfg["memory_dimension"], cfg["coefficient_bottleneck"])
    H, V = cfg["ffn_hidden"], cfg["vocab_size"]
    n = lambda *shape: rng.standard_normal(shape) * scale
    p = {"tok.weight": n(V, d), "lnf.weight": 1 + n(d) * 0.1, "lnf.bias": n(d) * 0.1}
    p["head.weight"] = p["tok.weight"]
    for i in range(cfg["n_layer"]):
        b = f"blocks.{i}."
        p.update({
            b + "rn1.weight": 1 + n(d) * 0.1, b + "rn2.weight": 1 + n(d) * 0.1,
            b + "mixer.input_projection.weight": n(C + M, d),
            b + "mixer.to_gate.weight": n(C, d), b + "mixer.to_gate.bias": n(C),
            b + "mixer.to_control.weight": n(R, d), b + "mixer.to_control.bias": n(R),
            b + "mixer.coefficient_projection.weight": n(2 * C * K + C * (K + 1) + (K + 1) * M, R),
            b + "mixer.coefficient_projection.bias": n(2 * C * K + C * (K + 1) + (K + 1) * M),
            b + "mixer.out_proj.weight": n(d, C),
            b + "ffn.up.weight": n(H, d), b + "ffn.up.bias": n(H),
            b + "ffn.down.weight": n(d, H), b + "ffn.down.bias": n(d),
        })
    return p


CFG = dict(vocab_size=40, n_layer=2, n_embd=24, lattice_d_e=12, lattice_order=2,
           coefficient_bottleneck=6, memory_dimension=4, ffn_hidden=32, arch="cauchy_x_hyperbolic")


def test_rmsnorm_rows_have_unit_rms():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 5, 16)) * 4
    z = St.rmsnorm(x, np.ones(16))
    assert np.allclose(np.sqrt(np.mean(z * z, axis=-1)), 1.0, atol=1e-12)
    w = rng.standard_normal(16)
    assert np.allclose(St.rmsnorm(x, w), z * w, atol=1e-12)
    row = np.full((1, 8), -2.5)
    assert np.allclose(St.rmsnorm(row, np.ones(8)), -1.0, atol=1e-12)


def test_zero_coefficient_projection_silences_the_mixer():
    rng = np.random.default_rng(1)
    p = _params(rng, CFG)
    pre = "blocks.0.mixer."
    p[pre + "coefficient_projection.weight"][:] = 0
    p[pre + "coefficient_projection.bias"][:] = 0
    out, _ = St.mixer_forward(rng.standard_normal((2, 7, 24)), p, pre, 2, 12, 4, CFG["arch"])
    assert np.array_equal(out, np.zeros_like(out))


def test_constant_coefficients_reduce_to_the_first_order_closed_form():
    """K=1, d_m=1, coefficients set through the projection bias alone (alpha, beta, rho0, rho1
    per channel, nu0, nu1): V_t = sum_j (-r sin)^(t-j) r cos x_j s_j, level1_t = r (sin x_t s_t +
    cos V_(t-1)), y_t = SiLU(g_t) (rho0 V_t nu0 + rho1 level1_t nu1), each product spelled out."""
    rng = np.random.default_rng(2)
    B, T, d, C = 2, 9, 10, 3
    cfg = dict(CFG, n_embd=d, lattice_d_e=C, lattice_order=1, memory_dimension=1,
               coefficient_bottleneck=4)
    p = _params(rng, cfg)
    pre = "blocks.0.mixer."
    alpha = np.array([0.3, -0.7, 1.4])
    beta = np.array([0.5, -1.2, 0.1])
    rho = np.array([[0.9, -0.4], [0.2, 1.1], [-0.6, 0.5]])
    nu = np.array([0.8, -1.3])
    p[pre + "coefficient_projection.weight"][:] = 0
    p[pre + "coefficient_projection.bias"][:] = np.concatenate([alpha, beta, rho.ravel(), nu])
    x = rng.standard_normal((B, T, d))
    out, final = St.mixer_forward(x, p, pre, 1, C, 1, "cauchy_x_mobius")
    signal = x @ p[pre + "input_projection.weight"][:C].T
    s = St.silu(x @ p[pre + "input_projection.weight"][C:].T)[..., 0]
    gate = St.silu(x @ p[pre + "to_gate.weight"].T + p[pre + "to_gate.bias"])
    r = 1 / (1 + beta ** 2)
    cos, sin = 2 * alpha / (1 + alpha ** 2), (1 - alpha ** 2) / (1 + alpha ** 2)  # mobius
    pole, gain = -r * sin, r * cos
    y = np.zeros((B, T, C))
    V_prev = np.zeros((B, C))
    for t in range(T):
        V_t = sum(pole ** (t - j) * gain * signal[:, j] * s[:, j, None] for j in range(t + 1))
        level1 = r * (sin * signal[:, t] * s[:, t, None] + cos * V_prev)
        y[:, t] = gate[:, t] * (rho[:, 0] * V_t * nu[0] + rho[:, 1] * level1 * nu[1])
        V_prev = V_t
    want = y @ p[pre + "out_proj.weight"].T
    assert np.allclose(out, want, atol=1e-10)
    assert np.allclose(final[:, 0, :, 0], V_prev, atol=1e-12)


def test_masked_token_is_invisible_downstream():
    rng = np.random.default_rng(3)
    p = _params(rng, CFG)
    ids = rng.integers(0, 40, (2, 8))
    valid = np.ones((2, 8), bool)
    valid[:, 3] = False
    logits, _ = St.llm_forward(ids, p, CFG, valid=valid)
    other = ids.copy()
    other[:, 3] = (ids[:, 3] + 7) % 40
    changed, _ = St.llm_forward(other, p, CFG, valid=valid)
    assert np.allclose(changed[:, 4:], logits[:, 4:], atol=1e-12)
    assert np.allclose(changed[:, :3], logits[:, :3], atol=1e-12)
    assert not np.allclose(changed[:, 3], logits[:, 3])
    # without the mask the token does reach later positions
    unmasked, _ = St.llm_forward(other, p, CFG)
    assert not np.allclose(unmasked[:, 4:], St.llm_forward(ids, p, CFG)[0][:, 4:])


def test_stepwise_through_the_carried_state_equals_one_shot():
    rng = np.random.default_rng(4)
    p = _params(rng, CFG)
    ids = rng.integers(0, 40, (2, 10))
    full, _ = St.llm_forward(ids, p, CFG)
    parts, states = [], None
    prompt, states = St.llm_forward(ids[:, :6], p, CFG, states=states)
    parts.append(prompt)
    for t in range(6, 10):
        step, states = St.llm_forward(ids[:, t:t + 1], p, CFG, states=states)
        parts.append(step)
    assert np.allclose(np.concatenate(parts, axis=1), full, atol=1e-12)


def test_planted_span_swap_is_caught():
    """The closed-form check above fails when alpha and beta trade places in the split."""
    rng = np.random.default_rng(5)
    cfg = dict(CFG, n_embd=6, lattice_d_e=2, lattice_order=1, memory_dimension=1,
               coefficient_bottleneck=3)
    p = _params(rng, cfg)
    pre = "blocks.0.mixer."
    p[pre + "coefficient_projection.weight"][:] = 0
    p[pre + "coefficient_projection.bias"][:] = [0.3, -0.7, 0.5, -1.2, 0.9, -0.4, 0.2, 1.1, 0.8, -1.3]
    x = rng.standard_normal((1, 5, 6))
    right, _ = St.mixer_forward(x, p, pre, 1, 2, 1, "cauchy_x_mobius")
    swapped = dict(p)
    bias = p[pre + "coefficient_projection.bias"].copy()
    bias[[0, 1, 2, 3]] = bias[[2, 3, 0, 1]]
    swapped[pre + "coefficient_projection.bias"] = bias
    wrong, _ = St.mixer_forward(x, swapped, pre, 1, 2, 1, "cauchy_x_mobius")
    assert not np.allclose(right, wrong, atol=1e-6)


# ---------------------------------------------------------------------------------------------
# host modules on the CPU (the mixer itself needs the GPU library)
# ---------------------------------------------------------------------------------------------
def test_norm_and_feed_forward_modules_match_the_oracle():
    torch = pytest.importorskip("torch")
    from mira_amd.block import FeedForward, RMSNorm

    torch.manual_seed(0)
    norm = RMSNorm(16, bias=True).double()
    with torch.no_grad():
        norm.weight.normal_()
        norm.bias.normal_()
    x = torch.randn(2, 5, 16, dtype=torch.float64) * 3
    want = St.rmsnorm(x.numpy(), norm.weight.detach().numpy(), norm.bias.detach().numpy())
    assert np.allclose(norm(x).detach().numpy(), want, atol=1e-12)
    ffn = FeedForward(16, hidden=24).double()
    p = {k: v.detach().numpy() for k, v in ffn.state_dict().items()}
    assert np.allclose(ffn(x).detach().numpy(), St.feed_forward(x.numpy(), p, ""), atol=1e-12)


def test_llm_ties_head_and_initialises_like_the_reference():
    torch = pytest.importorskip("torch")
    from mira_amd.llm import MiraLLM

    torch.manual_seed(0)
    model = MiraLLM(vocab_size=300, n_layer=4, n_embd=64, lattice_d_e=96, lattice_order=2,
                    coefficient_bottleneck=8, memory_dimension=16, ffn_hidden=128)
    assert model.tok.weight is model.head.weight
    names = set(model.state_dict())
    assert set(_params(np.random.default_rng(0), dict(
        CFG, n_layer=4, n_embd=64, lattice_d_e=96, coefficient_bottleneck=8,
        memory_dimension=16, ffn_hidden=128, vocab_size=300))) <= names
    block = model.blocks[0]
    assert abs(block.mixer.to_gate.weight.std().item() - 0.02) < 0.002
    assert abs(block.mixer.out_proj.weight.std().item() - 0.02 / np.sqrt(8)) < 0.001
    assert abs(block.ffn.down.weight.std().item() - 0.02 / np.sqrt(8)) < 0.001
    assert block.ffn.up.bias.abs().max().item() == 0.0
    with pytest.raises(ValueError):
        MiraLLM(vocab_size=10, n_layer=1, n_embd=16, moe_total_experts=4)
