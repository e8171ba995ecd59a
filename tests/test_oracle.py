"""CPU pinning of the oracle: every oracle function is checked against something other than its
own formula -- textbook closed forms, special values, invariants, an independent formulation, or
the reference's own golden vectors -- chosen so that a dropped term, a wrong sign or index, or a
transposed operand fails at least one of them (see the planted-mistake tests at the end)."""
import os

import numpy as np
import pytest

from _util import GOLDEN, golden_files, max_abs, scaled
from oracle import baseline as Bl
from oracle import lattice as L

F64 = np.float64


# ---------------------------------------------------------------------------------------------
# stage maps (model/mira_mixer.py:56-155)
# ---------------------------------------------------------------------------------------------
ALPHAS = np.array([-50.0, -3.0, -1.0, -0.999, -0.3, 0.0, 0.3, 0.999, 1.0, 1.001, 3.0, 50.0])


def test_mobius_is_the_shifted_cayley_angle():
    # theta = pi/2 - 2 arctan(alpha): cos(theta) = sin(2 arctan a), sin(theta) = cos(2 arctan a)
    cos, sin = L.mobius_rotation(ALPHAS.astype(F64))
    theta = np.pi / 2 - 2 * np.arctan(ALPHAS)
    assert np.allclose(cos, np.cos(theta), atol=1e-14) and np.allclose(sin, np.sin(theta), atol=1e-14)
    c0, s0 = L.mobius_rotation(np.zeros(1))
    assert (c0[0], s0[0]) == (0.0, 1.0)


def test_hyperbolic_is_sech_tanh():
    cos, sin = L.hyperbolic_rotation(ALPHAS.astype(F64))
    assert np.allclose(cos, 1 / np.cosh(ALPHAS), rtol=1e-14, atol=1e-300)
    assert np.allclose(sin, np.tanh(ALPHAS), rtol=1e-14)
    c0, s0 = L.hyperbolic_rotation(np.zeros(1))
    assert (c0[0], s0[0]) == (1.0, 0.0)


def test_identity_is_cos_sin():
    cos, sin = L.identity_rotation(ALPHAS.astype(F64))
    assert np.array_equal(cos, np.cos(ALPHAS)) and np.array_equal(sin, np.sin(ALPHAS))


@pytest.mark.parametrize("rotation", ["mobius", "hyperbolic", "identity"])
def test_rotations_are_orthogonal_float32(rotation):
    alphas = np.linspace(-1e4, 1e4, 20001).astype(np.float32)
    cos, sin = L.ROTATIONS[rotation](alphas)
    assert np.all(np.isfinite(cos)) and np.all(np.isfinite(sin))
    assert np.abs(cos.astype(F64) ** 2 + sin.astype(F64) ** 2 - 1).max() < 1e-6


def test_radius_special_values_and_closed_forms():
    beta = np.array([-90.0, -3.0, -1.0, 0.0, 0.5, 1.0, 2.0, 81.0, 200.0])
    zero = np.zeros(1)
    assert L.cauchy_radius(zero)[0] == 1.0 and L.gaussian_radius(zero)[0] == 1.0
    assert L.expexp_radius(zero)[0] == np.exp(-1.0)
    assert L.expsoftplus_radius(zero)[0] == 0.5 and L.hill_radius(zero)[0] == 0.0
    assert np.allclose(L.cauchy_radius(beta), 1 / (1 + beta ** 2), rtol=1e-15)
    assert np.allclose(L.gaussian_radius(beta), np.exp(-beta ** 2), rtol=1e-15)
    assert np.allclose(L.expexp_radius(beta), np.exp(-np.exp(np.minimum(beta, 80))), rtol=1e-15)
    assert np.allclose(L.expsoftplus_radius(beta), np.exp(-np.logaddexp(0, beta)), rtol=1e-12,
                       atol=1e-300)
    assert np.allclose(L.hill_radius(beta), beta ** 2 / (1 + beta ** 2), rtol=1e-14)
    big = L.expexp_radius(np.array([1e4], np.float32))
    assert big[0] == 0.0 and np.isfinite(big).all()


def test_stage_maps_table():
    assert len(L.ARCH_STAGE) == 15
    for arch in L.ARCH_STAGE:
        rotation, radius = L.stage_maps(arch)
        assert rotation is L.ROTATIONS[arch.split("_x_")[1]]
        assert radius is L.RADII[arch.split("_x_")[0]]
    with pytest.raises(ValueError):
        L.stage_maps("cauchy_x_nothing")


# ---------------------------------------------------------------------------------------------
# the scan
# ---------------------------------------------------------------------------------------------
def _inputs(seed, B=2, T=23, C=4, K=2, M=8, **kw):
    return L.random_inputs(np.random.default_rng(seed), B, T, C, K, M, dtype=F64, **kw)


def test_k1_is_the_explicit_first_order_solution():
    """K=1: V_t = sum_j [prod_(j<i<=t) (-r_i sin_i)] (r_j cos_j) U_j + [prod (-r sin)] V_-1,
    level_1 = r (sin U + cos V_(t-1)); evaluated by products, not by a recurrence."""
    B, T, C, M = 2, 17, 3, 5
    x, alpha, rho, gamma, write, read, beta = _inputs(1, B, T, C, 1, M)
    state = np.random.default_rng(2).standard_normal((B, 1, C, M)) * 0.1
    cos, sin = L.hyperbolic_rotation(alpha[..., 0])
    r = L.cauchy_radius(beta[..., 0])
    pole, gain = -r * sin, r * cos                                     # [B,T,C]
    U = x[..., None] * write[:, :, None, :]                            # [B,T,C,M]
    y, final = L.lattice_scan_sequential(x, alpha, rho, gamma, write, read, beta, state=state,
                                         dtype=F64)
    gate = gamma / (1 + np.exp(-gamma))
    for t in range(T):
        V = np.prod(pole[:, :t + 1], axis=1)[..., None] * state[:, 0]
        for j in range(t + 1):
            V = V + (np.prod(pole[:, j + 1:t + 1], axis=1) * gain[:, j])[..., None] * U[:, j]
        prev = (np.prod(pole[:, :t], axis=1)[..., None] * state[:, 0] + sum(
            (np.prod(pole[:, j + 1:t], axis=1) * gain[:, j])[..., None] * U[:, j] for j in range(t)))
        level1 = r[:, t, :, None] * (sin[:, t, :, None] * U[:, t] + cos[:, t, :, None] * prev)
        want = gate[:, t] * (rho[:, t, :, 0] * (V * read[:, t, None, 0]).sum(-1)
                             + rho[:, t, :, 1] * (level1 * read[:, t, None, 1]).sum(-1))
        assert np.abs(y[:, t] - want).max() < 1e-13
    assert np.abs(final[:, 0] - V).max() < 1e-13


@pytest.mark.parametrize("K", [1, 2, 3, 4, 8])
def test_lossless_lattice_conserves_energy(K):
    """At r = 1 every stage is a rotation, so |V_t|^2 + level_K^2 = |V_(t-1)|^2 + U^2. level_K is
    read out alone (rho = e_K, nu = 1, SiLU(40) = 40 in float64) one token at a time."""
    rng = np.random.default_rng(3)
    B, C = 2, 3
    V = rng.standard_normal((B, K, C, 1))
    for t in range(9):
        x = rng.standard_normal((B, 1, C))
        alpha = rng.standard_normal((B, 1, C, K)) * 2
        beta = np.zeros((B, 1, C, K))                                  # cauchy radius: r = 1
        rho = np.zeros((B, 1, C, K + 1))
        rho[..., K] = 1.0
        gamma = np.full((B, 1, C), 40.0)
        y, V1 = L.lattice_scan_sequential(x, alpha, rho, gamma, np.ones((B, 1, 1)),
                                          np.ones((B, 1, K + 1, 1)), beta, state=V,
                                          arch="cauchy_x_mobius", dtype=F64)
        level_k = y[:, 0] / 40.0
        before = (V[..., 0] ** 2).sum(1) + x[:, 0] ** 2
        after = (V1[..., 0] ** 2).sum(1) + level_k ** 2
        assert np.abs(before - after).max() < 1e-12 * max(1.0, before.max())
        V = V1


@pytest.mark.parametrize("arch", list(L.ARCH_STAGE))
@pytest.mark.parametrize("K", [1, 2, 4])
def test_stage_loop_equals_batched_cumprod_form(arch, K):
    """The stage loop (model/mira_mixer.py:467-502) against the reference's own cumulative-
    product operators (model/mira_mixer.py:336-349), masked and with an initial state."""
    x, alpha, rho, gamma, write, read, beta = _inputs(5, K=K, alpha_bias=0.4)
    alpha[0, :3] *= 6.0
    state = np.random.default_rng(6).standard_normal((2, K, 4, 8)) * 0.1
    valid = np.random.default_rng(7).random((2, 23)) > 0.3
    a = L.lattice_scan_sequential(x, alpha, rho, gamma, write, read, beta, valid, state, arch,
                                  dtype=F64)
    b = L.lattice_scan_batched(x, alpha, rho, gamma, write, read, beta, valid, state, arch,
                               chunk=7, dtype=F64)
    assert max_abs(a[0], b[0]) < 1e-13 and max_abs(a[1], b[1]) < 1e-13


@pytest.mark.parametrize("K", [1, 2, 3, 8])
def test_stage_system_matches_stage_operators(K):
    alpha = np.random.default_rng(8).standard_normal((5, K)) * 2
    beta = np.random.default_rng(9).standard_normal((5, K))
    A, b, Cm, d = L.stage_system(alpha, beta, "cauchy_x_mobius")
    transition, coefficient = L.stage_operators(alpha, beta, "cauchy_x_mobius", F64)
    assert np.abs(Cm - transition).max() < 1e-14 and np.abs(d - coefficient).max() < 1e-14
    assert np.abs(A - transition[:, :K]).max() < 1e-14


@pytest.mark.parametrize("chunk", [1, 2, 5, 16, 100])
def test_chunked_composition_equals_sequential(chunk):
    x, alpha, rho, gamma, write, read, beta = _inputs(10, T=37)
    state = np.random.default_rng(11).standard_normal((2, 2, 4, 8)) * 0.1
    valid = np.random.default_rng(12).random((2, 37)) > 0.2
    want = L.lattice_scan_sequential(x, alpha, rho, gamma, write, read, beta, valid, state,
                                     dtype=F64)
    got = L.chunked_scan(x, alpha, rho, gamma, write, read, beta, valid, state, chunk=chunk)
    assert max_abs(got[0], want[0]) < 1e-12 and max_abs(got[1], want[1]) < 1e-12


def test_streaming_masks_linearity():
    x, alpha, rho, gamma, write, read, beta = _inputs(13, T=20)
    state = np.random.default_rng(14).standard_normal((2, 2, 4, 8)) * 0.1
    valid = np.ones((2, 20), bool)
    valid[0] = False
    one = L.lattice_scan_sequential(x, alpha, rho, gamma, write, read, beta, valid, state, dtype=F64)
    s = state
    parts = []
    for first, last in ((0, 7), (7, 8), (8, 20)):
        sl = lambda v: v[:, first:last]  # noqa: E731
        y, s = L.lattice_scan_sequential(sl(x), sl(alpha), sl(rho), sl(gamma), sl(write), sl(read),
                                         sl(beta), valid[:, first:last], s, dtype=F64)
        parts.append(y)
    assert max_abs(np.concatenate(parts, 1), one[0]) < 1e-14 and max_abs(s, one[1]) < 1e-14
    assert np.array_equal(one[1][0], state[0]) and np.all(one[0][0] == 0)
    nomask = L.lattice_scan_sequential(x, alpha, rho, gamma, write, read, beta, None, state)
    allmask = L.lattice_scan_sequential(x, alpha, rho, gamma, write, read, beta,
                                        np.ones((2, 20), bool), state)
    assert np.array_equal(nomask[0], allmask[0]) and np.array_equal(nomask[1], allmask[1])
    y1, _ = L.lattice_scan_sequential(x, alpha, rho, gamma, write, read, beta, dtype=F64)
    y3, _ = L.lattice_scan_sequential(3 * x, alpha, rho, gamma, write, read, beta, dtype=F64)
    assert max_abs(y3, 3 * y1) < 1e-14
    y0, s0 = L.lattice_scan_sequential(0 * x, alpha, rho, gamma, write, read, beta, dtype=F64)
    assert np.all(y0 == 0) and np.all(s0 == 0)


@pytest.mark.parametrize("path", golden_files("k"), ids=lambda p: os.path.basename(p)[:-4])
def test_oracle_matches_reference_golden_vectors(path):
    """The reference CPU mixer's own float32 output (written by tests/golden/make_golden.py)."""
    d = np.load(path)
    args = [d[k] for k in ("x", "alpha", "rho", "gamma", "write", "read", "beta")]
    valid = d["valid"] if "valid" in d else None
    state = d["state"] if "state" in d else None
    for form in (L.lattice_scan_sequential, L.lattice_scan_batched):
        y, final = form(*args, valid=valid, state=state, arch=str(d["arch"]))
        assert max_abs(y, d["y"]) <= 1e-6 and scaled(y, d["y"]) <= 1e-5
        assert max_abs(final, d["final"]) <= 1e-6


# ---------------------------------------------------------------------------------------------
# BASELINE closed forms
# ---------------------------------------------------------------------------------------------
def test_conv_impulse_response_and_ring():
    D = 3
    w = np.arange(12, dtype=F64).reshape(D, 4) + 1
    x = np.zeros((1, 8, D))
    x[0, 2] = 1.0
    u = Bl.causal_conv(x, w)
    assert np.array_equal(u[0, 2:6], w[:, ::-1].T)     # u_(2+k) = w[:, 3-k]
    assert np.all(u[0, :2] == 0) and np.all(u[0, 6:] == 0)
    rng = np.random.default_rng(0)
    xs = rng.standard_normal((2, 11, D))
    whole = Bl.causal_conv(xs, w)
    ring = np.zeros((2, D, 3))
    pieces = []
    pos = 0
    for n in (1, 2, 5, 3):
        pieces.append(Bl.causal_conv(xs[:, pos:pos + n], w, ring=ring, pos=pos))
        ring = Bl.ring_after(xs[:, pos:pos + n], ring, pos)
        pos += n
    assert max_abs(np.concatenate(pieces, 1), whole) < 1e-14
    for j in range(3):
        t = 11 - 3 + j
        assert np.array_equal(ring[:, :, t % 3], xs[:, t])


def test_diag_scan_closed_form_and_realisation():
    rng = np.random.default_rng(1)
    x, a, w, bias, h0 = Bl.diag_inputs(rng, 2, 30, 5, h0_scale=0.1)
    u = Bl.causal_conv(x, w, bias)
    h, hT = Bl.diag_scan(u, a, h0)
    assert max_abs(h, Bl.diag_scan_closed_form(u, a, h0)) < 1e-14
    lat = Bl.diag_as_lattice(u, a, h0, F64)
    y, st = L.lattice_scan_sequential(*lat[:7], state=lat[7], dtype=F64)
    assert max_abs(y / 32, h) < 1e-12 and max_abs(st[:, 0, :, 0], hT) < 1e-12


def test_diag_golden_reference_path():
    from _util import GOLDEN

    d = np.load(f"{GOLDEN}/diag_cfg1_reduced.npz")
    h, _ = Bl.diag_scan(Bl.causal_conv(d["x"], d["w"], d["bias"]), d["a"], d["h0"])
    assert max_abs(h, d["y"] / 32) <= 1e-6


def test_gla_three_forms_and_realisation():
    rng = np.random.default_rng(2)
    q, k, v, g = Bl.gla_inputs(rng, 2, 70, 2, 6, 5, dtype=F64)
    S0 = rng.standard_normal((2, 2, 5, 6)) * 0.1
    o1, S1 = Bl.gla_recurrent(q, k, v, g, S0)
    assert max_abs(o1, Bl.gla_quadratic(q, k, v, g, S0)) < 1e-12
    o3, S3 = Bl.gla_chunked(q, k, v, g, S0, chunk=16)
    assert max_abs(o1, o3) < 1e-12 and max_abs(S1, S3) < 1e-12
    lat = Bl.gla_as_lattice(q, k, v, g, S0, F64)
    y, st = L.lattice_scan_sequential(*lat[:7], state=lat[7], dtype=F64)
    assert max_abs(y.reshape(2, 2, 70, 5).transpose(0, 2, 1, 3) / 32, o1) < 1e-11
    assert max_abs(st.reshape(2, 2, 5, 6), S1) < 1e-12


def test_gla_golden_reference_path():
    from _util import GOLDEN

    d = np.load(f"{GOLDEN}/gla_cfg3_reduced.npz")
    o, S = Bl.gla_recurrent(d["q"], d["k"], d["v"], d["g"], d["S0"])
    B, T, H, dv = o.shape
    ref = (d["y"] / 32).reshape(B, H, T, dv).transpose(0, 2, 1, 3)
    assert max_abs(o, ref) <= 1e-5 * max(1.0, np.abs(ref).max())


# ---------------------------------------------------------------------------------------------
# planted mistakes: each plausible slip in the oracle fails a pinning check
# ---------------------------------------------------------------------------------------------
def _sequential_with(mistake):
    """A copy of the stage loop with one planted mistake (used only to show the checks bite)."""
    def scan(x, alpha, rho, gamma, write, read, beta, valid=None, state=None,
             arch="cauchy_x_hyperbolic", dtype=F64):
        B, T, C = x.shape
        K, M = alpha.shape[3], write.shape[2]
        rotation, radius_map = L.stage_maps(arch)
        cos, sin = rotation(alpha)
        r = radius_map(beta)
        gate = L.silu(gamma)
        V = np.zeros((B, K, C, M)) if state is None else state.copy()
        out = np.zeros((B, T, C))
        for t in range(T):
            U = x[:, t, :, None] * write[:, t, None, :]
            levels = [None] * (K + 1)
            for k in range(K, 0, -1):
                src = V[:, k - 1] if mistake != "index" else V[:, K - k]
                c, s, rr = cos[:, t, :, k - 1, None], sin[:, t, :, k - 1, None], r[:, t, :, k - 1, None]
                if mistake == "sign":
                    s = -s
                levels[k] = rr * (s * U + c * src)
                U = rr * (c * U - s * src) if mistake != "radius" else (c * U - s * src)
            levels[0] = U
            every = np.stack(levels, 1)
            comp = np.einsum("bkcm,bkm->bkc", every, read[:, t] if mistake != "transpose"
                             else read[:, t][:, ::-1])
            out[:, t] = (rho[:, t].transpose(0, 2, 1) * comp).sum(1) * gate[:, t]
            V = every[:, :K].copy()
        return out, V
    return scan


@pytest.mark.parametrize("mistake", ["sign", "index", "radius", "transpose"])
def test_planted_mistakes_are_caught(mistake):
    d = np.load(golden_files("k2m16_cauchy_x_hyperbolic")[0])
    args = [d[k].astype(F64) for k in ("x", "alpha", "rho", "gamma", "write", "read", "beta")]
    scan = _sequential_with(mistake)
    y, _ = scan(*args, valid=None, state=d["state"].astype(F64))
    ref, _ = L.lattice_scan_sequential(*args, valid=None, state=d["state"].astype(F64), dtype=F64)
    assert scaled(y, ref) > 1e-3, f"planted {mistake} went unnoticed"


# ---------------------------------------------------------------------------------------------
# the backward (gradients of the scan), pinned by the reference's own autograd and by fp64
# finite differences
# ---------------------------------------------------------------------------------------------
GRAD_NAMES = ("x", "alpha", "beta", "rho", "gamma", "write", "read")
GRAD_FIXTURES = golden_files("grad_")


def _grad_fixture(path):
    f = np.load(path, allow_pickle=False)
    valid = f["valid"] if "valid" in f.files else None
    inputs = [f[n] for n in ("x", "alpha", "rho", "gamma", "write", "read", "beta")]
    return f, inputs, valid


@pytest.mark.parametrize("path", GRAD_FIXTURES, ids=os.path.basename)
def test_backward_matches_reference_autograd(path):
    """Gradients of sum(dy * y) for every input against autograd through the reference's
    float32 matrix_lattice_iir (model/mira_mixer.py:246-387; tests/golden/grad_*.npz): all 15
    stage maps at K=2 d_m=16 with a mask, and K/d_m from 1/8 to 8/16."""
    f, inputs, valid = _grad_fixture(path)
    grads = L.lattice_backward(*inputs, f["dy"], valid=valid, arch=str(f["arch"]))
    for name, got in zip(GRAD_NAMES, grads):
        error = scaled(got, f["d" + name])
        assert error <= 2e-6, f"d{name}: scaled error {error:.3e}"


def _finite_difference(inputs, dy, valid, arch, index, h=1e-6):
    grad = np.zeros_like(inputs[index])
    for position in np.ndindex(grad.shape):
        values = []
        for sign in (1.0, -1.0):
            moved = [a.copy() for a in inputs]
            moved[index][position] += sign * h
            y, _ = L.lattice_scan_sequential(*moved, valid=valid, arch=arch, dtype=np.float64)
            values.append(float((y * dy).sum()))
        grad[position] = (values[0] - values[1]) / (2 * h)
    return grad


@pytest.mark.parametrize("arch,K,M", [("cauchy_x_hyperbolic", 2, 3), ("expsoftplus_x_mobius", 3, 2),
                                      ("hill_x_identity", 1, 2), ("expexp_x_mobius", 2, 1),
                                      ("gaussian_x_hyperbolic", 4, 1)])
def test_backward_matches_finite_differences(arch, K, M):
    """Central differences of the fp64 stage-loop forward, every element of every input."""
    rng = np.random.default_rng(K * 10 + M)
    inputs = [v.astype(np.float64) for v in L.random_inputs(rng, 2, 5, 3, K, M, scale=(0.5,) * 7)]
    valid = rng.random((2, 5)) > 0.3
    dy = rng.standard_normal((2, 5, 3))
    grads = dict(zip(GRAD_NAMES, L.lattice_backward(*inputs, dy, valid=valid, arch=arch)))
    for name, index in zip(("x", "alpha", "rho", "gamma", "write", "read", "beta"), range(7)):
        want = _finite_difference(inputs, dy, valid, arch, index)
        error = np.abs(grads[name] - want).max() / np.abs(want).max()
        assert error <= 1e-7, f"d{name}: relative error {error:.3e}"


def test_backward_planted_mistakes_fail(monkeypatch):
    """A sign slip in a rotation derivative, or sigmoid in place of SiLU's derivative, misses
    the reference's gradients by far more than the tolerance."""
    f, inputs, valid = _grad_fixture(os.path.join(GOLDEN, "grad_k2m16_cauchy_x_mobius.npz"))
    derivatives = L.stage_map_derivatives

    def flipped(alpha, beta, arch):
        cos, sin, r, dcos, dsin, dr = derivatives(alpha, beta, arch)
        return cos, sin, r, dcos, -dsin, dr

    monkeypatch.setattr(L, "stage_map_derivatives", flipped)
    grads = L.lattice_backward(*inputs, f["dy"], valid=valid, arch="cauchy_x_mobius")
    assert scaled(grads[1], f["dalpha"]) > 0.1
    monkeypatch.undo()
    monkeypatch.setattr(L, "silu_derivative", lambda g: 1.0 / (1.0 + np.exp(-g)))
    grads = L.lattice_backward(*inputs, f["dy"], valid=valid, arch="cauchy_x_mobius")
    assert scaled(grads[4], f["dgamma"]) > 0.01
