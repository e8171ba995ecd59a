"""GPU parity of the coefficient-forming scan (mira_lattice_control_forward, reached through
matrix_lattice_iir_control) against the materialised path (F.linear, then the lattice scan) and
the oracle.

Follows the reference harness's fused-scan check (kernel/cuda/mira_dspv2/check.py:1130-1261):
the same generators (weight ~ N(0, 1/d_r), bias ~ 0.3 N(0, 1), control = SiLU(N(0, 1)), x and
gamma as strided views of one packed tensor, write ~ N(0, 1)/4), the same bound (scaled error
<= 2e-2 against both the materialised path and the float reference, with at most 2 % of the bf16
outputs differing from the materialised path's: a formed coefficient may land one bf16 ulp away
because its d_r-term sum runs in another order), a split sequence that falls back to the
materialised path bit for bit, every stage map, and the mixer's eval forward. The reference's
shapes are kept where this library serves them in one token chunk; B=64 T=257 (chunked here)
becomes B=192 T=257.
"""
import numpy as np
import pytest

from _util import HALF_SCALED, scaled, to_numpy
from oracle import lattice as L

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    return torch


@pytest.fixture(scope="module")
def plugin():
    from mira_amd import _lib, mira

    assert _lib.library() is not None, _lib.why()
    return mira


def _inputs(torch, batch, tokens, channels, rank, order, memory, masked, with_state, seed):
    generator = torch.Generator(device="cuda").manual_seed(seed)

    def randn(*shape):
        return torch.randn(*shape, device="cuda", generator=generator)

    total = channels * (3 * order + 1) + (order + 1) * memory
    spans = ((0, channels * order), (channels * order, 2 * channels * order),
             (2 * channels * order, channels * (3 * order + 1)), (channels * (3 * order + 1), total))
    weight = (randn(total, rank) / rank ** 0.5).to(torch.bfloat16)
    bias = (0.3 * randn(total)).to(torch.bfloat16)
    control = torch.nn.functional.silu(randn(batch, tokens, rank)).to(torch.bfloat16)
    packed = randn(batch, tokens, 2 * channels + 3).to(torch.bfloat16)
    signal, gamma = packed[..., :channels], packed[..., channels:2 * channels]
    write = (randn(batch, tokens, memory) / 4).to(torch.bfloat16)
    valid = (torch.rand(batch, tokens, device="cuda", generator=generator) > 0.25) if masked else None
    state = randn(batch, order, channels, memory) if with_state else None
    return dict(weight=weight, bias=bias, control=control, signal=signal, gamma=gamma,
                write=write, valid=valid, state=state, spans=spans)


def _materialised(plugin, torch, v, order, memory, arch, with_state):
    import torch.nn.functional as F

    batch, tokens, channels = v["signal"].shape
    coefficients = F.linear(v["control"], v["weight"], v["bias"])
    alpha, beta, rho, read = coefficients.split(tuple(hi - lo for lo, hi in v["spans"]), dim=-1)
    views = (alpha.view(batch, tokens, channels, order), rho.view(batch, tokens, channels, order + 1),
             read.view(batch, tokens, order + 1, memory), beta.view(batch, tokens, channels, order))
    out = plugin.matrix_lattice_iir(
        v["signal"], views[0], views[1], v["gamma"], v["write"], views[2], raw_beta=views[3],
        valid=v["valid"], state=v["state"], return_state=with_state, arch=arch)
    return out, views


def _case(plugin, torch, batch, tokens, channels, rank, masked=False, with_state=False,
          arch="cauchy_x_mobius", order=2, memory=16, expect_fused=True, oracle=True, seed=0,
          zero_alpha=False):
    torch.manual_seed(20261011 + batch + tokens + channels + rank)
    v = _inputs(torch, batch, tokens, channels, rank, order, memory, masked, with_state,
                20261011 + batch + tokens + channels + rank + seed)
    if zero_alpha:                          # alpha = 0 exactly: the Moebius map's cos is 0
        lo, hi = v["spans"][0]
        v["weight"][lo:hi] = 0
        v["bias"][lo:hi] = 0
    before = plugin.usage()["control"]
    with torch.no_grad():
        got = plugin.matrix_lattice_iir_control(
            v["signal"], v["control"], v["weight"], v["bias"], v["spans"], v["gamma"], v["write"],
            valid=v["valid"], state=v["state"], return_state=with_state, arch=arch)
        fused = plugin.usage()["control"] > before
        want, views = _materialised(plugin, torch, v, order, memory, arch, with_state)
    assert got is not None and want is not None
    assert fused == expect_fused, f"fused path taken: {fused}, expected {expect_fused}"
    if with_state:
        (got, got_final), (want, want_final) = got, want
    torch.cuda.synchronize()
    if not expect_fused:
        assert torch.equal(got, want), "the fallback must be the materialised path bit for bit"
        if with_state:
            assert torch.equal(got_final, want_final)
        return 0.0, 0.0
    differing = float((got != want).float().mean())
    error = scaled(to_numpy(got), to_numpy(want))
    if oracle:
        seen = [to_numpy(t) for t in (v["signal"], views[0], views[1], v["gamma"], v["write"],
                                      views[2], views[3])]
        exact, exact_final = L.lattice_scan_sequential(
            *seen, valid=None if v["valid"] is None else to_numpy(v["valid"]).astype(bool),
            state=None if v["state"] is None else to_numpy(v["state"]), arch=arch,
            dtype=np.float64)
        error = max(error, scaled(to_numpy(got), exact))
        if with_state:
            error = max(error, scaled(to_numpy(got_final), exact_final))
    elif with_state:
        error = max(error, scaled(to_numpy(got_final), to_numpy(want_final)))
    assert error <= HALF_SCALED and differing <= 0.02, (
        f"B={batch} T={tokens} C={channels} d_r={rank} {arch}: scaled error {error:.3e}, "
        f"{differing:.2%} of outputs differ from the materialised path")
    return error, differing


@pytest.mark.parametrize("args", [
    (19, 5, 70, 48, False, False, "cauchy_x_mobius"),
    (19, 5, 70, 48, True, True, "cauchy_x_mobius"),
    (3, 4, 32, 16, True, False, "cauchy_x_hyperbolic"),
    (17, 3, 40, 32, False, True, "cauchy_x_identity"),
    (5, 16, 64, 64, True, True, "gaussian_x_mobius"),
    (9, 19, 48, 48, False, True, "cauchy_x_hyperbolic"),   # unmasked: runs of 6 tokens + 1
    (6, 32, 40, 32, False, True, "cauchy_x_identity"),    # 5 runs of 6 + 2
], ids=lambda a: f"B{a[0]}T{a[1]}C{a[2]}r{a[3]}{'m' if a[4] else ''}{'s' if a[5] else ''}")
def test_reference_cases(torch_mod, plugin, args):
    _case(plugin, torch_mod, *args)


@pytest.mark.parametrize("arch", ["cauchy_x_mobius", "cauchy_x_hyperbolic", "cauchy_x_identity"])
def test_exact_zero_alpha(torch_mod, plugin, arch):
    """Every alpha exactly 0 (a zero-initialised projection row): cos = 0 for the Moebius map,
    sin = 0 for the others, over 30 unmasked tokens with a carried-in state; the output and
    the final state stay finite and match the oracle."""
    _case(plugin, torch_mod, 6, 30, 40, 32, False, True, arch, zero_alpha=True)


@pytest.mark.parametrize("args", [(192, 257, 1536, 48, False, False, "cauchy_x_mobius"),
                                  (571, 33, 1536, 48, True, False, "cauchy_x_mobius")],
                         ids=["B192T257", "B571T33"])
def test_reference_geometry_at_batch(torch_mod, plugin, args):
    """The reference mira-s geometry (d_e 1536, d_m 16, d_r 48) at batches that fill the GPU
    in one token chunk: against the materialised path (the float oracle would take minutes)."""
    _case(plugin, torch_mod, *args, oracle=False)


@pytest.mark.parametrize("number,arch", list(enumerate(L.ARCH_STAGE)))
def test_every_arch(torch_mod, plugin, number, arch):
    rank = (16, 32, 48, 64)[number % 4]
    _case(plugin, torch_mod, 6 + number, 3 + number % 5, 64 + 32 * (number % 3), rank,
          number % 2 == 1, number % 3 == 0, arch)


@pytest.mark.parametrize("order,memory", [(1, 8), (1, 16), (2, 8), (4, 8)])
def test_orders_and_memories(torch_mod, plugin, order, memory):
    """The other served shapes beside the reference's one (K=2, d_m=16)."""
    _case(plugin, torch_mod, 9, 11, 48, 32, True, True, "cauchy_x_hyperbolic", order=order,
          memory=memory)


@pytest.mark.parametrize("order,memory", [(1, 8), (1, 16), (2, 8), (4, 8)])
@pytest.mark.parametrize("arch", list(L.ARCH_STAGE))
def test_every_map_at_every_served_shape(torch_mod, plugin, arch, order, memory):
    """The kernel is built once per stage map and served shape: every one of them runs, with a
    mask and a carried-in state, against the materialised path and the oracle."""
    _case(plugin, torch_mod, 7, 5, 40, 16, True, True, arch, order=order, memory=memory)


@pytest.mark.parametrize("order,memory", [(1, 32), (2, 32), (2, 64), (4, 16)])
def test_unserved_shapes_fall_back(torch_mod, plugin, order, memory):
    """(K, d_m) where the materialised path is the faster one: bit for bit that path."""
    _case(plugin, torch_mod, 9, 11, 48, 32, True, True, "cauchy_x_hyperbolic", order=order,
          memory=memory, expect_fused=False)


@pytest.mark.parametrize("args", [(64, 1, 64, 48, True, True), (40, 2, 96, 32, False, True)],
                         ids=["one_token", "two_tokens"])
def test_short_calls(torch_mod, plugin, args):
    """A single token (a cached step's shape) and two tokens, with carried state."""
    _case(plugin, torch_mod, *args, arch="cauchy_x_hyperbolic")


def test_fully_masked_rows_keep_the_state(torch_mod, plugin):
    """A sequence whose every token is masked writes zeros and hands its state back unchanged."""
    torch = torch_mod
    B, T, C, K, M, R = 6, 9, 48, 2, 16, 32
    v = _inputs(torch, B, T, C, R, K, M, True, True, 11)
    v["valid"][2] = False
    with torch.no_grad():
        out, final = plugin.matrix_lattice_iir_control(
            v["signal"], v["control"], v["weight"], v["bias"], v["spans"], v["gamma"], v["write"],
            valid=v["valid"], state=v["state"], return_state=True)
    torch.cuda.synchronize()
    assert torch.equal(out[2], torch.zeros_like(out[2]))
    assert torch.equal(final[2], v["state"][2])


def test_without_bias_and_with_a_strided_control(torch_mod, plugin):
    """coefficient_projection without a bias, and a control that is a column slice of a wider
    tensor (the wrapper makes it contiguous): still the fused path, still the materialised result."""
    import torch.nn.functional as F

    torch = torch_mod
    B, T, C, K, M, R = 20, 6, 64, 2, 16, 32
    v = _inputs(torch, B, T, C, R, K, M, True, True, 21)
    wide = torch.randn(B, T, R + 16, device="cuda").to(torch.bfloat16)
    wide[..., 8:8 + R] = v["control"]
    control = wide[..., 8:8 + R]
    assert not control.is_contiguous()
    before = plugin.usage()["control"]
    with torch.no_grad():
        got, got_final = plugin.matrix_lattice_iir_control(
            v["signal"], control, v["weight"], None, v["spans"], v["gamma"], v["write"],
            valid=v["valid"], state=v["state"], return_state=True)
        assert plugin.usage()["control"] == before + 1
        coefficients = F.linear(v["control"], v["weight"])
        alpha, beta, rho, read = coefficients.split(tuple(hi - lo for lo, hi in v["spans"]), dim=-1)
        want, want_final = plugin.matrix_lattice_iir(
            v["signal"], alpha.view(B, T, C, K), rho.view(B, T, C, K + 1), v["gamma"], v["write"],
            read.view(B, T, K + 1, M), raw_beta=beta.view(B, T, C, K), valid=v["valid"],
            state=v["state"], return_state=True)
    torch.cuda.synchronize()
    assert float((got != want).float().mean()) <= 0.02
    assert scaled(to_numpy(got), to_numpy(want)) <= HALF_SCALED
    assert scaled(to_numpy(got_final), to_numpy(want_final)) <= HALF_SCALED


@pytest.mark.parametrize("what", ["float32", "weight_columns_strided"])
def test_unserved_layouts_fall_back(torch_mod, plugin, what):
    """A float32 call, or a weight whose rows are not contiguous: the materialised path."""
    torch = torch_mod
    B, T, C, K, M, R = 4, 5, 32, 2, 16, 16
    v = _inputs(torch, B, T, C, R, K, M, False, False, 31)
    weight = v["weight"]
    args = [v["signal"], v["control"], weight, v["bias"], v["spans"], v["gamma"], v["write"]]
    if what == "float32":
        args = [t.float() if hasattr(t, "float") else t for t in args]
    else:
        args[2] = torch.empty(weight.shape[1], weight.shape[0], device="cuda",
                              dtype=weight.dtype).copy_(weight.t()).t()      # column-major view
        assert args[2].stride(1) != 1
    before = plugin.usage()["control"]
    with torch.no_grad():
        got = plugin.matrix_lattice_iir_control(*args)
    assert got is not None and plugin.usage()["control"] == before


def test_split_sequence_falls_back_bit_for_bit(torch_mod, plugin):
    _case(plugin, torch_mod, 1, 300, 1536, 48, expect_fused=False)


def test_unserved_rank_falls_back(torch_mod, plugin):
    _case(plugin, torch_mod, 4, 6, 64, 128, expect_fused=False)


def test_errors(torch_mod, plugin):
    torch = torch_mod
    v = _inputs(torch, 2, 3, 32, 16, 2, 16, False, False, 5)
    args = (v["signal"], v["control"], v["weight"], v["bias"], v["spans"], v["gamma"], v["write"])
    with torch.no_grad():
        with pytest.raises(ValueError):
            plugin.matrix_lattice_iir_control(*args, state=torch.zeros(2, 2, 32, 16, device="cuda"))
        with pytest.raises(ValueError):
            plugin.matrix_lattice_iir_control(*args, valid=torch.ones(2, 3, device="cuda"))
        (a0, a1), (b0, b1), (r0, r1), (n0, n1) = v["spans"]
        short_rho = ((a0, a1), (b0, b1), (r0, r1 - 1), (n0, n1))
        with pytest.raises(ValueError):
            plugin.matrix_lattice_iir_control(*args[:4], short_rho, *args[5:])


def test_mixer_eval_forward_takes_the_control_scan(torch_mod, plugin):
    """model/mira_mixer.py routes an uncached eval forward through matrix_lattice_iir_control; a
    forward hook on coefficient_projection sends it down the materialised path instead, as in
    the reference (model/mira_mixer.py:749-752)."""
    torch = torch_mod
    from mira_amd.mixer import MiraMixer

    torch.manual_seed(3)
    mixer = MiraMixer(768, lattice_order=2, d_e=1536, coefficient_bottleneck=48,
                      memory_dimension=16).cuda().to(torch.bfloat16).eval()
    x = torch.randn(8, 16, 768, device="cuda", dtype=torch.bfloat16)
    with torch.no_grad():
        before = plugin.usage()["control"]
        fused = mixer(x)
        assert plugin.usage()["control"] == before + 1, "the mixer did not reach the control scan"
        handle = mixer.coefficient_projection.register_forward_hook(lambda *a: None)
        try:
            plain = mixer(x)
        finally:
            handle.remove()
        assert plugin.usage()["control"] == before + 1
    error = scaled(to_numpy(fused), to_numpy(plain))
    assert error <= HALF_SCALED, f"fused vs materialised mixer forward: {error:.3e}"
