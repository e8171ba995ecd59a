"""GPU parity of the BASELINE GLA matrix state (mira_gla_chunked / mira_gla_step).

Anchors: oracle/baseline.py's recurrent and attention-form (quadratic) solutions in fp64; the
reference CPU mixer's output on the exact K=1 lattice realisation
(tests/golden/gla_cfg3_reduced.npz, through the lattice kernel since that fixture has d = 16);
decode-N == prefill; and BASELINE cfg3's full size on sampled heads.
Tolerances: float32 max abs <= 1e-5 relative to unit-scale outputs (o ~ |v| / (1 - e^g));
bf16 scaled <= 2e-2.
"""
import numpy as np
import pytest

from _util import GOLDEN, HALF_SCALED, max_abs, rounded, scaled, to_device, to_numpy
from oracle import baseline as Bl

pytestmark = pytest.mark.gpu


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


def _inputs(seed, B, T, H, d=128):
    rng = np.random.default_rng(seed)
    q, k, v, g = Bl.gla_inputs(rng, B, T, H, d, d)
    S0 = (rng.standard_normal((B, H, d, d)) * 0.1).astype(np.float32)
    return q, k, v, g, S0


def _fp32_ok(got, want, what):
    # outputs reach ~|v| / (1 - e^g) ~ 30: hold float32 to 1e-5 relative to the output scale
    scale = max(1.0, float(np.abs(want).max()))
    err = max_abs(got, want) / scale
    assert err <= 1e-5, f"{what}: max abs / scale {err:.3e}"


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_step_against_recurrence(torch_mod, plugin, dtype):
    torch = torch_mod
    td = getattr(torch, dtype)
    q, k, v, g, S0 = _inputs(1, 2, 1, 3)
    S = to_device(S0).clone()
    o = plugin.gla_step(to_device(q[:, 0], td), to_device(k[:, 0], td), to_device(v[:, 0], td),
                        to_device(g[:, 0]), S)
    want_o, want_S = Bl.gla_recurrent(rounded(q, td), rounded(k, td), rounded(v, td), g, S0)
    if dtype == "float32":
        _fp32_ok(to_numpy(o), want_o[:, 0], "o")
    else:
        assert scaled(to_numpy(o), want_o[:, 0]) <= HALF_SCALED
    assert max_abs(to_numpy(S), want_S) <= 1e-5


@pytest.mark.parametrize("T", [1, 63, 64, 65, 200])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_prefill_against_oracle(torch_mod, plugin, T, dtype):
    torch = torch_mod
    td = getattr(torch, dtype)
    q, k, v, g, S0 = _inputs(T, 1, T, 2)
    o, ST = plugin.gla_chunked(to_device(q, td), to_device(k, td), to_device(v, td), to_device(g),
                               state=to_device(S0), return_state=True)
    want_o, want_S = Bl.gla_recurrent(rounded(q, td), rounded(k, td), rounded(v, td), g, S0)
    if dtype == "float32":
        _fp32_ok(to_numpy(o), want_o, "o")
        _fp32_ok(to_numpy(ST), want_S, "S_T")
    else:
        assert scaled(to_numpy(o), want_o) <= HALF_SCALED
        assert scaled(to_numpy(ST), want_S) <= 1e-3
    if T <= 64:
        quad = Bl.gla_quadratic(rounded(q, td), rounded(k, td), rounded(v, td), g, S0)
        assert scaled(to_numpy(o), quad) <= (1e-5 if dtype == "float32" else HALF_SCALED)


def test_decode_equals_prefill(torch_mod, plugin):
    torch = torch_mod
    q, k, v, g, S0 = _inputs(5, 2, 24, 2)
    o, ST = plugin.gla_chunked(to_device(q), to_device(k), to_device(v), to_device(g),
                               state=to_device(S0), return_state=True)
    S = to_device(S0).clone()
    outs = [plugin.gla_step(to_device(q[:, t]), to_device(k[:, t]), to_device(v[:, t]),
                            to_device(g[:, t]), S) for t in range(24)]
    _fp32_ok(to_numpy(torch.stack(outs, 1)), to_numpy(o), "decode o")
    _fp32_ok(to_numpy(S), to_numpy(ST), "decode state")


def test_golden_reference_path_via_lattice(torch_mod, plugin):
    """The reference CPU mixer on the K=1 realisation (batch B*H, C = d_v, M = d_k = 16), run
    through the lattice kernel: y / 32 against the reference's y / 32."""
    d = np.load(f"{GOLDEN}/gla_cfg3_reduced.npz")
    lat = Bl.gla_as_lattice(d["q"], d["k"], d["v"], d["g"], d["S0"])
    out, final = plugin.matrix_lattice_iir(*[to_device(t) for t in lat[:6]],
                                           raw_beta=to_device(lat[6]), state=to_device(lat[7]),
                                           return_state=True)
    _fp32_ok(to_numpy(out) / 32.0, d["y"] / 32.0, "lattice realisation vs reference")
    _fp32_ok(to_numpy(final), d["final"], "state vs reference")


def test_cfg3_full_size_sampled_heads(torch_mod, plugin):
    """BASELINE cfg3 at full size (B=4, T=8192, H=16, d=128, bf16): two heads checked against the
    fp64 recurrence over all 8192 tokens."""
    torch = torch_mod
    gen = torch.Generator(device="cuda").manual_seed(3)
    B, T, H, d = 4, 8192, 16, 128
    q = torch.nn.functional.normalize(torch.randn(B, T, H, d, device="cuda", generator=gen), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, d, device="cuda", generator=gen), dim=-1)
    v = torch.randn(B, T, H, d, device="cuda", generator=gen)
    g = torch.rand(B, T, H, device="cuda", generator=gen) * -0.099 - 0.001
    q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    o, ST = plugin.gla_chunked(q, k, v, g, return_state=True)
    torch.cuda.synchronize()
    for b, h in ((0, 0), (3, 15)):
        want_o, want_S = Bl.gla_recurrent(to_numpy(q[b:b + 1, :, h:h + 1]),
                                          to_numpy(k[b:b + 1, :, h:h + 1]),
                                          to_numpy(v[b:b + 1, :, h:h + 1]),
                                          to_numpy(g[b:b + 1, :, h:h + 1]))
        assert scaled(to_numpy(o[b:b + 1, :, h:h + 1]), want_o) <= HALF_SCALED
        assert scaled(to_numpy(ST[b:b + 1, h:h + 1]), want_S) <= 1e-3


def test_prefill_bf16_grouped_heads(torch_mod, plugin):
    """B*H a multiple of 8 places a head's four value blocks on one XCD (the other block order):
    against the fp64 recurrence, with a ragged last chunk."""
    torch = torch_mod
    q, k, v, g, S0 = _inputs(11, 2, 130, 4)
    td = torch.bfloat16
    o, ST = plugin.gla_chunked(to_device(q, td), to_device(k, td), to_device(v, td), to_device(g),
                               state=to_device(S0), return_state=True)
    want_o, want_S = Bl.gla_recurrent(rounded(q, td), rounded(k, td), rounded(v, td), g, S0)
    assert scaled(to_numpy(o), want_o) <= HALF_SCALED
    assert scaled(to_numpy(ST), want_S) <= 1e-3


def test_prefill_bf16_unaligned_rows(torch_mod, plugin):
    """q, k, v that start 2 bytes off a 16-byte boundary take the per-row kernel; same answer."""
    torch = torch_mod
    q, k, v, g, S0 = _inputs(12, 1, 70, 2)
    td = torch.bfloat16

    def shifted(a):
        flat = torch.empty(a.size + 8, device="cuda", dtype=td)
        view = flat[1:1 + a.size].view(a.shape)
        view.copy_(to_device(a, td))
        assert view.data_ptr() % 16 != 0
        return view

    o, ST = plugin.gla_chunked(shifted(q), shifted(k), shifted(v), to_device(g),
                               state=to_device(S0), return_state=True)
    want_o, want_S = Bl.gla_recurrent(rounded(q, td), rounded(k, td), rounded(v, td), g, S0)
    assert scaled(to_numpy(o), want_o) <= HALF_SCALED
    assert scaled(to_numpy(ST), want_S) <= 1e-3


def test_decode_equals_prefill_bf16(torch_mod, plugin):
    """bf16: 70 decode steps against one chunked prefill over the same tokens."""
    torch = torch_mod
    td = torch.bfloat16
    q, k, v, g, S0 = _inputs(13, 1, 70, 2)
    qd, kd, vd, gd = to_device(q, td), to_device(k, td), to_device(v, td), to_device(g)
    o, ST = plugin.gla_chunked(qd, kd, vd, gd, state=to_device(S0), return_state=True)
    S = to_device(S0).clone()
    outs = [plugin.gla_step(qd[:, t], kd[:, t], vd[:, t], gd[:, t], S) for t in range(70)]
    assert scaled(to_numpy(torch.stack(outs, 1)), to_numpy(o)) <= HALF_SCALED
    assert scaled(to_numpy(S), to_numpy(ST)) <= 1e-3
