"""CPU checks of the host mirror: the plugin's acceptance rules (kernel/cuda/mira_dspv2/mira.py:
1444-1517) decline on CPU tensors exactly as the reference plugin does, stride helpers, the
prefix cache, the device selector and the mixer's parameter layout."""
import numpy as np
import pytest
import torch

from mira_amd import config, hardware, mira, prefix_cache
from mira_amd import mixer as mixer_module
from mira_amd.llm import MiraLLM
from mira_amd.mixer import MiraMixer
from mira_amd.prefix_cache import PrefixCache, affordable, state_bytes
from oracle import lattice as L


def _inputs(B=1, T=4, C=3, K=2, M=16):
    return [torch.from_numpy(v) for v in L.random_inputs(np.random.default_rng(0), B, T, C, K, M)]


def test_cpu_tensors_decline():
    x, alpha, rho, gamma, write, read, beta = _inputs()
    assert mira.matrix_lattice_iir(x, alpha, rho, gamma, write, read, raw_beta=beta) is None


def test_shape_rules_decline_or_raise():
    x, alpha, rho, gamma, write, read, beta = _inputs()
    assert mira.matrix_lattice_iir(x, alpha, rho, gamma, write, read, raw_beta=None) is None
    assert mira.matrix_lattice_iir(x, alpha, rho[..., :2], gamma, write, read, raw_beta=beta) is None
    with pytest.raises(ValueError):
        mira.matrix_lattice_iir(x[:, :0], alpha[:, :0], rho[:, :0], gamma[:, :0], write[:, :0],
                                read[:, :0], raw_beta=beta[:, :0])
    with pytest.raises(ValueError):
        mira.matrix_lattice_iir(x, alpha, rho, gamma, write, read, raw_beta=beta, arch="nope")


def test_row_strides():
    base = torch.zeros(2, 5, 11)
    view = base[:, :, 3:7]
    assert mira._row_stride(view, 5) == 11
    assert mira._row_stride(base.transpose(1, 2), 11) is None
    coefficients = torch.zeros(2, 5, 30)
    alpha = coefficients[..., :8].view(2, 5, 4, 2)
    assert mira.dense_tail_row_stride(alpha, 5) == 30
    assert mira.dense_tail_row_stride(torch.zeros(2, 5, 4, 2).transpose(2, 3), 5) is None


def test_prefix_cache():
    cache = PrefixCache(3, budget=1000)
    assert cache.get(1) is None and len(cache) == 0
    t = torch.ones(1, 2, 3, 4, requires_grad=True)
    stored = cache.put(1, t * 2)
    assert not stored.requires_grad
    cache.advance(5)
    assert len(cache) == 5 and cache.nbytes() == 96
    assert cache.within_budget()[0]
    cache.put(0, torch.zeros(1, 2, 3, 40))
    fits, why = cache.within_budget()
    assert not fits and "ceiling" in why
    assert state_bytes(24, 4, 2, 2048, 64) == 24 * 4 * 2 * 2048 * 64 * 4
    assert affordable(1, 1, 1, 1, 1, budget=2)[0] is False
    cache.clear_states()
    assert cache.get(0) is None and len(cache) == 0


def test_hardware_selector():
    assert hardware.resolve("cpu").type == "cpu"
    if not torch.cuda.is_available():
        assert hardware.resolve("auto").type == "cpu"
        assert hardware.accelerator("cpu") is None
        with pytest.raises(RuntimeError):
            hardware.resolve("cuda")


def test_mixer_layout_and_cpu_refusal():
    mixer = MiraMixer(32, lattice_order=2, d_e=24, coefficient_bottleneck=8, memory_dimension=16)
    assert mixer.coefficient_projection.out_features == 24 * 2 * 2 + 24 * 3 + 3 * 16
    assert mixer.read_span[1] == mixer.coefficient_projection.out_features
    assert mixer.state_values() == 2 * 24 * 16
    with pytest.raises(RuntimeError, match="declined"):
        with torch.no_grad():
            mixer(torch.zeros(1, 3, 32))
    with pytest.raises(ValueError):
        MiraMixer(32, arch="nope")
    with pytest.raises(ValueError):
        mixer.train()(torch.zeros(1, 3, 32), cache=PrefixCache(1), layer=0)


def test_prefix_cache_switch_and_configured_budget(monkeypatch):
    """INFERENCE["prefix_cache"] = 0 makes the mixer refuse a cache (model/mira_mixer.py:726-729);
    the default ceiling is INFERENCE["prefix_cache_size"] GiB, read at call time
    (model/prefix_cache.py:47-64)."""
    monkeypatch.setitem(config.INFERENCE, "prefix_cache_size", 0.5)
    assert PrefixCache(2).budget == 1 << 29
    assert PrefixCache(2, budget=0).budget == 0
    assert affordable(1, 1, 1, 1 << 20, 256)[0] is False           # 1 GiB > 0.5 GiB
    assert affordable(1, 1, 1, 1 << 20, 64)[0] is True
    assert "GiB" in prefix_cache.describe(24, 4, 2, 2048, 64)
    mixer = MiraMixer(32, lattice_order=2, d_e=24, coefficient_bottleneck=8,
                      memory_dimension=16).eval()
    monkeypatch.setitem(config.INFERENCE, "prefix_cache", 0)
    assert not prefix_cache.enabled()
    with pytest.raises(ValueError, match="not wired"):
        with torch.no_grad():
            mixer(torch.zeros(1, 3, 32), cache=PrefixCache(1), layer=0)


def test_prefix_cache_reset_through_model():
    model = MiraLLM(vocab_size=17, n_layer=2, n_embd=16, lattice_d_e=8, memory_dimension=4)
    cache = PrefixCache(2)
    cache.put(0, torch.ones(1, 2, 8, 4))
    cache.advance(3)
    cache.key_valid = torch.ones(1, 3, dtype=torch.bool)
    cache.reset(model)
    assert cache.state == [None, None] and len(cache) == 0 and cache.key_valid is None


def test_prefix_cache_keeps_earlier_states_unless_in_place():
    """put() swaps in a new tensor; a caller holding an earlier state sees it unchanged. Only a
    cache that opts in (in_place) has its held tensor overwritten by single-token steps."""
    cache = PrefixCache(1)
    assert cache.in_place is False
    first = cache.put(0, torch.zeros(1, 1, 2, 2))
    second = cache.put(0, torch.ones(1, 1, 2, 2))
    assert first is not second and float(first.sum()) == 0.0


def _projection_mixer():
    torch.manual_seed(0)
    return MiraMixer(32, lattice_order=2, d_e=24, coefficient_bottleneck=8,
                     memory_dimension=16).eval()


def test_packed_projection_matches_module_calls():
    mixer = _projection_mixer()
    x = torch.randn(2, 5, 32)
    with torch.no_grad():
        packed = mixer.project_recurrence_inputs(x)
        assert "_packed_projection" in mixer.__dict__
    unpacked = (mixer.input_projection(x), mixer.coefficient_projection(
        torch.nn.functional.silu(mixer.to_control(x))), mixer.to_gate(x))
    for got, want in zip(packed, unpacked):
        torch.testing.assert_close(got, want.detach(), rtol=1e-5, atol=1e-6)


def test_packed_projection_respects_hooks_and_subclasses():
    """A forward hook on to_gate, a global hook or a Linear subclass must change what the
    inference projection returns exactly as calling the modules would (model/mira_mixer.py:
    664-672); the packed GEMM is skipped for them."""
    x = torch.randn(2, 5, 32)
    mixer = _projection_mixer()
    with torch.no_grad():
        base = mixer.project_recurrence_inputs(x)[2]
        handle = mixer.to_gate.register_forward_hook(lambda module, args, out: out * 3.0)
        hooked = mixer.project_recurrence_inputs(x)[2]
        handle.remove()
        torch.testing.assert_close(hooked, base * 3.0)
        handle = torch.nn.modules.module.register_module_forward_hook(
            lambda module, args, out: out + 1.0 if module is mixer.to_gate else None)
        try:
            globally = mixer.project_recurrence_inputs(x)[2]
        finally:
            handle.remove()
        torch.testing.assert_close(globally, base + 1.0)

    class Doubled(torch.nn.Linear):
        def forward(self, value):
            return 2.0 * super().forward(value)

    replacement = Doubled(32, mixer.to_gate.out_features)
    replacement.load_state_dict(mixer.to_gate.state_dict())
    mixer.to_gate = replacement
    with torch.no_grad():
        torch.testing.assert_close(mixer.project_recurrence_inputs(x)[2], base * 2.0)


def _module_inputs(mixer, x):
    """What the forward's projections must equal: the modules called one by one."""
    channels, memory = mixer.inner, mixer.memory_dimension
    signal, raw_write = mixer.input_projection(x).split((channels, memory), dim=-1)
    control = torch.nn.functional.silu(mixer.to_control(x))
    return signal, raw_write, control, mixer.coefficient_projection(control), mixer.to_gate(x)


@pytest.mark.parametrize("split_rows", [1, 10 ** 9])
def test_forward_projections_match_module_calls(monkeypatch, split_rows):
    """The forward's inference projections -- [signal | gate] and [write | control] as two
    GEMMs from SPLIT_ROWS tokens on, the packed GEMM below, and the coefficient projection on
    its zero-padded weight -- give the module calls' values; the padding columns are zero."""
    monkeypatch.setattr(mixer_module, "SPLIT_ROWS", split_rows)
    mixer = _projection_mixer()
    x = torch.randn(2, 7, 32)
    with torch.no_grad():
        signal, raw_write, coefficients, gamma, whole = mixer._recurrence_inputs(x)
        _, _, control, _, _ = mixer._recurrence_inputs(x, coefficients=False)
        want = _module_inputs(mixer, x)
    width = mixer.coefficient_projection.out_features
    if split_rows == 1:                        # long input: split GEMMs, padded coefficients
        assert coefficients.shape[-1] % 256 == 0 and coefficients.shape[-1] - width < 256
        assert torch.count_nonzero(coefficients[..., width:]) == 0
        assert whole is None
    else:                                      # short input: the packed GEMM, the module's weight
        assert coefficients.shape[-1] == width and whole is not None
    for got, expect in zip((signal, raw_write, control, coefficients[..., :width], gamma), want):
        torch.testing.assert_close(got, expect, rtol=1e-5, atol=1e-6)


def test_padded_coefficients_follow_the_module(monkeypatch):
    """The padded copy of coefficient_projection is rebuilt when its parameters change, and a
    hook on the module sends the forward back to calling it."""
    monkeypatch.setattr(mixer_module, "SPLIT_ROWS", 1)
    mixer = _projection_mixer()
    x = torch.randn(1, 3, 32)
    width = mixer.coefficient_projection.out_features
    with torch.no_grad():
        before = mixer._recurrence_inputs(x)[2][..., :width]
        mixer.coefficient_projection.weight.mul_(0.5)
        after = mixer._recurrence_inputs(x)[2][..., :width]
        assert not torch.equal(before, after)
        torch.testing.assert_close(after, _module_inputs(mixer, x)[3], rtol=1e-5, atol=1e-6)
        handle = mixer.coefficient_projection.register_forward_hook(lambda m, a, out: out * 2.0)
        try:
            hooked = mixer._recurrence_inputs(x)[2]
        finally:
            handle.remove()
    assert hooked.shape[-1] == width
    torch.testing.assert_close(hooked, 2.0 * after, rtol=1e-5, atol=1e-6)


def test_packed_projection_rebuilds_on_parameter_change():
    mixer = _projection_mixer()
    x = torch.randn(1, 3, 32)
    with torch.no_grad():
        before = mixer.project_recurrence_inputs(x)[2]
        mixer.to_gate.weight.mul_(0.5)                      # in place: _version moves
        mixer.to_gate.bias.zero_()
        after = mixer.project_recurrence_inputs(x)[2]
    assert not torch.equal(after, before)
    torch.testing.assert_close(after, mixer.to_gate(x))
