"""CPU checks of the host mirror: the plugin's acceptance rules (kernel/cuda/mira_dspv2/mira.py:
1444-1517) decline on CPU tensors exactly as the reference plugin does, stride helpers, the
prefix cache, the device selector and the mixer's parameter layout."""
import numpy as np
import pytest
import torch

from mira_amd import hardware, mira
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
