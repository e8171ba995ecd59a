"""CPU restatement of the reference lattice operator -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.

Restates, in numpy, the reference's PyTorch mixer scan (`model/mira_mixer.py`):
  * the rotation and radius stage maps             model/mira_mixer.py:56-155
  * `stage_system`, the per-token affine map        model/mira_mixer.py:169-188
  * `matrix_lattice_iir` (batched per-token form)   model/mira_mixer.py:246-387
  * `matrix_lattice_iir_sequential` (stage loop)    model/mira_mixer.py:390-518
  * the chunked (Phi, carry) emulation              kernel/cuda/mira_dspv2/check.py:885-1003

Every array may be float32 (the reference's own arithmetic) or float64 (brute force). Shapes are
the reference's: x, gamma [B,T,C]; alpha, beta [B,T,C,K]; rho [B,T,C,K+1]; write [B,T,M];
read [B,T,K+1,M]; valid [B,T] bool; state [B,K,C,M].

Pinning (tests/test_oracle.py): stage maps against textbook closed forms and special values;
K=1 against the explicit product-sum solution of the first-order recurrence; the stage loop
against the batched cumulative-product form and against `stage_system`; lossless (r=1)
energy conservation; chunked composition against the sequential scan; and, where the reference
could be imported in the build container, golden vectors of the reference's own fp32 output
(tests/golden/).
"""
from __future__ import annotations

import numpy as np

# The 15 stage-map archs and the reference kernel's mode numbers, kernel/cuda/mira_dspv2/mira.py:305-309.
ARCH_STAGE = {
    "cauchy_x_mobius": 3, "cauchy_x_hyperbolic": 6, "cauchy_x_identity": 7,
    "gaussian_x_mobius": 8, "gaussian_x_hyperbolic": 9, "gaussian_x_identity": 10,
    "expexp_x_mobius": 11, "expexp_x_hyperbolic": 12, "expexp_x_identity": 13,
    "expsoftplus_x_mobius": 14, "expsoftplus_x_hyperbolic": 15, "expsoftplus_x_identity": 16,
    "hill_x_mobius": 17, "hill_x_hyperbolic": 18, "hill_x_identity": 19,
}
EXPEXP_BETA_CEILING = 80.0          # model/mira_mixer.py:111


# --------------------------------------------------------------------------------------------
# stage maps: alpha -> (cos, sin), beta -> r           model/mira_mixer.py:56-155
# --------------------------------------------------------------------------------------------
def mobius_rotation(alpha):
    """cos, sin of theta = pi/2 - 2 arctan(alpha), rational, 1/alpha branch above |alpha| = 1
    (model/mira_mixer.py:56-79)."""
    f = alpha.dtype.type
    small = np.abs(alpha) <= f(1)
    bounded = np.where(small, alpha, f(0))
    with np.errstate(divide="ignore"):
        reciprocal = f(1) / np.where(small, f(1), alpha)
    square = bounded * bounded
    inv_square = reciprocal * reciprocal
    cosine = np.where(small, f(2) * bounded / (f(1) + square),
                      f(2) * reciprocal / (f(1) + inv_square))
    sine = np.where(small, (f(1) - square) / (f(1) + square),
                    (inv_square - f(1)) / (f(1) + inv_square))
    return cosine.astype(alpha.dtype), sine.astype(alpha.dtype)


def hyperbolic_rotation(alpha):
    """cos = sech(alpha) = 2e/(1+e^2) with e = exp(-|alpha|), sin = tanh(alpha)
    (model/mira_mixer.py:82-91)."""
    f = alpha.dtype.type
    decay = np.exp(-np.abs(alpha))
    cosine = f(2) * decay / (f(1) + decay * decay)
    return cosine.astype(alpha.dtype), np.tanh(alpha).astype(alpha.dtype)


def identity_rotation(alpha):
    """theta = alpha (model/mira_mixer.py:94-98)."""
    return np.cos(alpha).astype(alpha.dtype), np.sin(alpha).astype(alpha.dtype)


def cauchy_radius(beta):
    """r = 1/(1+beta^2) (model/mira_mixer.py:100-102)."""
    f = beta.dtype.type
    return (f(1) / (f(1) + beta * beta)).astype(beta.dtype)


def gaussian_radius(beta):
    """r = exp(-beta^2) (model/mira_mixer.py:105-107)."""
    return np.exp(-(beta * beta)).astype(beta.dtype)


def expexp_radius(beta):
    """r = exp(-exp(min(beta, 80))) (model/mira_mixer.py:113-121)."""
    f = beta.dtype.type
    return np.exp(-np.exp(np.minimum(beta, f(EXPEXP_BETA_CEILING)))).astype(beta.dtype)


def expsoftplus_radius(beta):
    """r = exp(-softplus(beta)) = sigmoid(-beta) (model/mira_mixer.py:124-133)."""
    f = beta.dtype.type
    with np.errstate(over="ignore"):
        return (f(1) / (f(1) + np.exp(beta))).astype(beta.dtype)


def hill_radius(beta):
    """r = q/(1+q), q = beta^2; 1 - 1/(1+q) above q = 1 (model/mira_mixer.py:136-145)."""
    f = beta.dtype.type
    square = beta * beta
    large = square > f(1)
    bounded = np.where(large, f(0), square)
    with np.errstate(over="ignore"):
        big = f(1) - f(1) / (f(1) + square)
    return np.where(large, big, bounded / (f(1) + bounded)).astype(beta.dtype)


ROTATIONS = {"mobius": mobius_rotation, "hyperbolic": hyperbolic_rotation,
             "identity": identity_rotation}
RADII = {"cauchy": cauchy_radius, "gaussian": gaussian_radius, "expexp": expexp_radius,
         "expsoftplus": expsoftplus_radius, "hill": hill_radius}


def stage_maps(arch):
    """(rotation, radius) of `arch` (model/mira_mixer.py:148-158)."""
    if arch not in ARCH_STAGE:
        raise ValueError(f"arch must be one of {tuple(ARCH_STAGE)}, not {arch!r}")
    radius, rotation = arch.split("_x_")
    return ROTATIONS[rotation], RADII[radius]


def silu(value):
    """x * sigmoid(x), as torch.nn.functional.silu on a float tensor."""
    f = value.dtype.type
    with np.errstate(over="ignore"):
        return (value / (f(1) + np.exp(-value))).astype(value.dtype)


def _cast(dtype, *arrays):
    return [None if a is None else np.asarray(a).astype(dtype) for a in arrays]


def _check_shapes(x, alpha, rho, gamma, write, read, beta, valid, state):
    """The reference's argument checks (model/mira_mixer.py:278-298, 311-317)."""
    if beta is None:
        raise ValueError("the canonical stage needs raw_beta, the radius coefficient")
    if x.ndim != 3:
        raise ValueError("x must have shape [B,T,C]")
    B, T, C = x.shape
    if alpha.ndim != 4:
        raise ValueError("raw_alpha must have shape [B,T,C,K]")
    K = alpha.shape[3]
    if alpha.shape != (B, T, C, K) or beta.shape != alpha.shape:
        raise ValueError("raw_alpha has an incompatible shape")
    if rho.shape != (B, T, C, K + 1):
        raise ValueError("raw_rho must have shape [B,T,C,K+1]")
    if gamma.shape != x.shape:
        raise ValueError("gamma must have the same shape as x")
    if write.ndim != 3 or write.shape[:2] != (B, T):
        raise ValueError("memory_write must have shape [B,T,M]")
    M = write.shape[2]
    if read.shape != (B, T, K + 1, M):
        raise ValueError("memory_read must have shape [B,T,K+1,M]")
    if valid is not None and valid.shape != (B, T):
        raise ValueError("valid must have shape [B,T]")
    if state is not None and state.shape != (B, K, C, M):
        raise ValueError(f"state must have shape [B,K,C,M] = {(B, K, C, M)}, got {state.shape}")
    return B, T, C, K, M


# --------------------------------------------------------------------------------------------
# the scan, stage loop form                              model/mira_mixer.py:390-518
# --------------------------------------------------------------------------------------------
def lattice_scan_sequential(x, alpha, rho, gamma, write, read, beta, valid=None, state=None,
                            arch="cauchy_x_hyperbolic", dtype=np.float32):
    """`matrix_lattice_iir_sequential`: for each token, k = K..1,
        level_k = r_k (sin_k U + cos_k V^(k-1)),   U <- r_k (cos_k U - sin_k V^(k-1)),
    level_0 = U, V^(0..K-1) <- level_(0..K-1), y = SiLU(gamma) sum_k rho_k (level_k . nu_k).
    A masked token keeps the state and emits 0. Returns (y [B,T,C] float, state [B,K,C,M])."""
    B, T, C, K, M = _check_shapes(x, alpha, rho, gamma, write, read, beta, valid, state)
    x, alpha, rho, gamma, write, read, beta, state = _cast(
        dtype, x, alpha, rho, gamma, write, read, beta, state)
    rotation, radius_map = stage_maps(arch)
    cosine, sine = rotation(alpha)
    radius = radius_map(beta)
    gate = silu(gamma)
    V = np.zeros((B, K, C, M), dtype) if state is None else state.copy()
    out = np.zeros((B, T, C), dtype)
    for t in range(T):
        U = x[:, t, :, None] * write[:, t, None, :]
        levels = [None] * (K + 1)
        for k in range(K, 0, -1):
            delayed = V[:, k - 1]
            c = cosine[:, t, :, k - 1, None]
            s = sine[:, t, :, k - 1, None]
            r = radius[:, t, :, k - 1, None]
            levels[k] = r * (s * U + c * delayed)
            U = r * (c * U - s * delayed)
        levels[0] = U
        every = np.stack(levels, axis=1)                              # [B, K+1, C, M]
        compressed = np.einsum("bkcm,bkm->bkc", every, read[:, t])
        mixed = (rho[:, t].transpose(0, 2, 1) * compressed).sum(axis=1) * gate[:, t]
        if valid is None:
            V = every[:, :K].copy()
        else:
            keep = np.asarray(valid[:, t], bool)
            V = np.where(keep[:, None, None, None], every[:, :K], V)
            mixed = np.where(keep[:, None], mixed, dtype(0))
        out[:, t] = mixed
    return out, V


# --------------------------------------------------------------------------------------------
# the scan, batched per-token form (the reference CPU mixer)   model/mira_mixer.py:319-387
# --------------------------------------------------------------------------------------------
def stage_operators(alpha, beta, arch, dtype=np.float32):
    """(transition [..,K+1,K], coefficient [..,K+1]) with D = r cos, E = r sin and
    G[i,j] = D^(i+1)..D^(j) (model/mira_mixer.py:336-349): V_t^(0..K) = transition V_{t-1} +
    coefficient U_t."""
    alpha, beta = _cast(dtype, alpha, beta)
    rotation, radius_map = stage_maps(arch)
    cosine, sine = rotation(alpha)
    radius = radius_map(beta)
    stage_d = radius * cosine
    stage_e = radius * sine
    K = alpha.shape[-1]
    one = np.ones(stage_d.shape[:-1] + (1,), dtype)
    d_with_one = np.concatenate([one, stage_d], axis=-1)
    e_with_one = np.concatenate([one, stage_e], axis=-1)
    upper = np.triu(np.ones((K + 1, K + 1), bool))
    strictly_upper = np.triu(upper, 1)
    products = np.cumprod(np.where(strictly_upper, d_with_one[..., None, :], dtype(1)),
                          axis=-1) * upper
    coefficient = e_with_one * products[..., K]
    shifted = np.zeros(stage_d.shape[:-1] + (K + 1, K), dtype)
    for i in range(1, K + 1):
        shifted[..., i, i - 1] = stage_d[..., i - 1]
    transition = (-e_with_one[..., None] * products[..., :K] * stage_e[..., None, :] + shifted)
    return transition.astype(dtype), coefficient.astype(dtype)


def lattice_scan_batched(x, alpha, rho, gamma, write, read, beta, valid=None, state=None,
                         arch="cauchy_x_hyperbolic", chunk=32, dtype=np.float32):
    """`matrix_lattice_iir`, the reference CPU mixer: per token one contraction of the stacked
    stage operators with the state (model/mira_mixer.py:351-386), in chunks of `chunk` tokens
    that thread the state. Returns (y, state)."""
    B, T, C, K, M = _check_shapes(x, alpha, rho, gamma, write, read, beta, valid, state)
    x, alpha, rho, gamma, write, read, beta, state = _cast(
        dtype, x, alpha, rho, gamma, write, read, beta, state)
    gate = silu(gamma)
    V = np.zeros((B, K, C, M), dtype) if state is None else state.copy()
    pieces = []
    for first in range(0, T, chunk):
        last = min(first + chunk, T)
        transition, coefficient = stage_operators(alpha[:, first:last], beta[:, first:last],
                                                  arch, dtype)
        for t in range(first, last):
            U = x[:, t, :, None] * write[:, t, None, :]
            levels = (np.einsum("bckj,bjcm->bkcm", transition[:, t - first], V)
                      + coefficient[:, t - first].transpose(0, 2, 1)[..., None] * U[:, None])
            compressed = np.einsum("bkcm,bkm->bkc", levels, read[:, t])
            mixed = (rho[:, t].transpose(0, 2, 1) * compressed).sum(axis=1) * gate[:, t]
            if valid is None:
                V = levels[:, :K].copy()
            else:
                keep = np.asarray(valid[:, t], bool)
                V = np.where(keep[:, None, None, None], levels[:, :K], V)
                mixed = np.where(keep[:, None], mixed, dtype(0))
            pieces.append(mixed)
    return np.stack(pieces, axis=1).astype(dtype), V


# --------------------------------------------------------------------------------------------
# per-token affine system and the chunked (Phi, carry) form
#     model/mira_mixer.py:169-188, kernel/cuda/mira_dspv2/check.py:885-1003
# --------------------------------------------------------------------------------------------
def stage_system(alpha, beta, arch, dtype=np.float64):
    """(A [..,K,K], b [..,K], Cm [..,K+1,K], d [..,K+1]): the K+1 basis inputs (the write, then
    V_{t-1}^(0..K-1)) pushed through the stage code (model/mira_mixer.py:169-188)."""
    alpha, beta = _cast(dtype, alpha, beta)
    rotation, radius_map = stage_maps(arch)
    K = alpha.shape[-1]
    lead = alpha.shape[:-1]
    eye = np.eye(K + 1, dtype=dtype)
    wave = np.broadcast_to(eye[0], lead + (K + 1,))
    delayed = [np.broadcast_to(eye[1 + j], lead + (K + 1,)) for j in range(K)]
    levels = [None] * (K + 1)
    for stage in range(K, 0, -1):
        cosine, sine = rotation(alpha[..., stage - 1:stage])
        radius = radius_map(beta[..., stage - 1:stage])
        levels[stage] = radius * (sine * wave + cosine * delayed[stage - 1])
        wave = radius * (cosine * wave - sine * delayed[stage - 1])
    levels[0] = wave
    maps = np.stack(levels, axis=-2)
    return maps[..., :K, 1:], maps[..., :K, 0], maps[..., :, 1:], maps[..., :, 0]


def token_maps(alpha, beta, valid, arch, dtype=np.float64):
    """stage_system with a masked token turned into the identity (check.py:885-894)."""
    A, b, Cm, d = stage_system(alpha, beta, arch, dtype)
    if valid is not None:
        keep = np.asarray(valid, bool)[:, :, None]
        eye = np.eye(A.shape[-1], dtype=dtype)
        A = np.where(keep[..., None, None], A, eye)
        b = np.where(keep[..., None], b, dtype(0))
    return A, b, Cm, d


def chunk_summary(A, b, u, first, last):
    """(Phi [B,C,K,K], carry [B,C,K,M]) of tokens [first, last) from a zero state
    (check.py:914-924, the p1 phase)."""
    B, _, C, K, _ = A.shape
    phi = np.broadcast_to(np.eye(K), (B, C, K, K)).copy()
    carry = np.zeros((B, C, K, u.shape[-1]))
    for t in range(first, last):
        phi = A[:, t] @ phi
        carry = A[:, t] @ carry + b[:, t, ..., None] * u[:, t, :, None, :]
    return phi, carry


def chunked_scan(x, alpha, rho, gamma, write, read, beta, valid=None, state=None,
                 arch="cauchy_x_hyperbolic", chunk=16):
    """The scan cut into chunks: summaries from zero, a serial composition
    S_(j+1) = Phi_j S_j + carry_j, and a replay of each chunk from its entering state
    (check.py:897-954), float64. Returns (y, state, entering_states)."""
    B, T, C, K, M = _check_shapes(x, alpha, rho, gamma, write, read, beta, valid, state)
    f64 = np.float64
    x, rho, gamma, write, read = _cast(f64, x, rho, gamma, write, read)
    A, b, Cm, d = token_maps(alpha, beta, valid, arch)
    u = x[..., None] * write[:, :, None, :]                      # [B,T,C,M]
    spans = [(s, min(T, s + chunk)) for s in range(0, T, chunk)]
    S = np.zeros((B, C, K, M)) if state is None else np.asarray(state, f64).transpose(0, 2, 1, 3)
    entering = []
    for first, last in spans:
        entering.append(S.copy())
        phi, carry = chunk_summary(A, b, u, first, last)
        S = phi @ S + carry
    gate = silu(gamma)
    out = np.zeros((B, T, C))
    for (first, last), S0 in zip(spans, entering):
        S = S0
        for t in range(first, last):
            levels = Cm[:, t] @ S + d[:, t, ..., None] * u[:, t, :, None, :]
            compressed = (levels * read[:, t, None]).sum(-1)           # [B,C,K+1]
            y = (rho[:, t] * compressed).sum(-1) * gate[:, t]
            if valid is not None:
                y = y * np.asarray(valid[:, t], f64)[:, None]
            out[:, t] = y
            S = A[:, t] @ S + b[:, t, ..., None] * u[:, t, :, None, :]
    return out, S.transpose(0, 2, 1, 3).copy(), entering


def random_inputs(rng, B, T, C, K, M, dtype=np.float32, scale=(0.15, 0.12, 0.15, 0.15, 0.12,
                                                                0.12, 0.12),
                  alpha_bias=0.0, beta_bias=0.0):
    """Seeded inputs of the reference harness's distribution (kernel/cuda/mira_dspv2/check.py:52-69):
    (x, alpha, rho, gamma, write, read, beta)."""
    shapes = ((B, T, C), (B, T, C, K), (B, T, C, K + 1), (B, T, C), (B, T, M), (B, T, K + 1, M),
              (B, T, C, K))
    values = [(rng.standard_normal(shape) * s).astype(dtype) for shape, s in zip(shapes, scale)]
    values[1] = (values[1] + dtype(alpha_bias)).astype(dtype)
    values[6] = (values[6] + dtype(beta_bias)).astype(dtype)
    return values


# --------------------------------------------------------------------------------------------
# the backward: gradients of the scan's output with respect to all seven inputs
#     what autograd returns through model/mira_mixer.py:246-387 (and the plugin's
#     MatrixLatticeIIR.backward, kernel/cuda/mira_dspv2/mira.py:1295-1433)
# --------------------------------------------------------------------------------------------
def stage_map_derivatives(alpha, beta, arch):
    """(cos, sin, r, dcos/dalpha, dsin/dalpha, dr/dbeta), float64, of the stage maps
    (model/mira_mixer.py:56-145), with the derivatives autograd forms there: the reciprocal
    branches of the rational maps give the same closed forms; hyperbolic's |alpha| has slope 0
    at 0 (so d sech = -sech tanh, also 0 there); expexp's ceiling stops the gradient above 80."""
    a = np.asarray(alpha, np.float64)
    b = np.asarray(beta, np.float64)
    radius_name, rotation_name = arch.split("_x_")
    if rotation_name == "mobius":
        denominator = 1.0 + a * a
        cos, sin = 2 * a / denominator, (1 - a * a) / denominator
        dcos, dsin = 2 * (1 - a * a) / denominator ** 2, -4 * a / denominator ** 2
    elif rotation_name == "hyperbolic":
        cos, sin = 1.0 / np.cosh(a), np.tanh(a)
        dcos, dsin = -cos * sin, cos * cos
    else:
        cos, sin = np.cos(a), np.sin(a)
        dcos, dsin = -sin, cos
    if radius_name == "cauchy":
        r = 1.0 / (1.0 + b * b)
        dr = -2 * b * r * r
    elif radius_name == "gaussian":
        r = np.exp(-b * b)
        dr = -2 * b * r
    elif radius_name == "expexp":
        capped = np.minimum(b, EXPEXP_BETA_CEILING)
        r = np.exp(-np.exp(capped))
        dr = np.where(b <= EXPEXP_BETA_CEILING, -np.exp(capped) * r, 0.0)
    elif radius_name == "expsoftplus":
        r = 1.0 / (1.0 + np.exp(b))
        dr = -r * (1 - r)
    else:
        q = b * b
        r = q / (1 + q)
        dr = 2 * b / (1 + q) ** 2
    return cos, sin, r, dcos, dsin, dr


def silu_derivative(value):
    """d/dx x sigmoid(x) = sigmoid(x) (1 + x (1 - sigmoid(x)))."""
    sigma = 1.0 / (1.0 + np.exp(-np.asarray(value, np.float64)))
    return sigma * (1.0 + value * (1.0 - sigma))


def lattice_backward(x, alpha, rho, gamma, write, read, beta, grad_out, valid=None,
                     arch="cauchy_x_hyperbolic"):
    """Gradients (dx, dalpha, dbeta, drho, dgamma, dwrite, dread) of sum(grad_out * y) for
    y = matrix_lattice_iir(...) from a zero state, in float64, by the explicit adjoint of the
    stage loop. With lambda the adjoint of the carried state V_t and
    Lambda_k = lambda_t[k] (k < K) + g rho_k nu_k dy (the readout's share), a token runs its
    stages backward (k = 1..K) from dU = Lambda_0:
        d rs_k += Lambda_k U_in - dU V_(t-1)[k-1],   d rc_k += Lambda_k V_(t-1)[k-1] + dU U_in,
        lambda_(t-1)[k-1] = rc_k Lambda_k - rs_k dU,  dU <- rs_k Lambda_k + rc_k dU,
    ending at dU = d(x s): dx = sum_m dU s, ds = sum_c dU x. rc = r cos and rs = r sin chain to
    alpha and beta through stage_map_derivatives. A masked token passes lambda through and gets
    zero gradients."""
    B, T, C, K, M = _check_shapes(x, alpha, rho, gamma, write, read, beta, valid, None)
    f64 = np.float64
    x, rho, gamma, write, read, dy = _cast(f64, x, rho, gamma, write, read, grad_out)
    cos, sin, r, dcos, dsin, dr = stage_map_derivatives(alpha, beta, arch)
    rc, rs = r * cos, r * sin                                    # [B,T,C,K], stage k at k-1
    gate = gamma / (1.0 + np.exp(-gamma))
    dgate = silu_derivative(gamma)
    keep = np.ones((B, T), bool) if valid is None else np.asarray(valid, bool)
    # forward, keeping the state entering every token
    entering = np.zeros((T, B, K, C, M))
    V = np.zeros((B, K, C, M))
    for t in range(T):
        entering[t] = V
        U = x[:, t, :, None] * write[:, t, None, :]
        levels = [None] * (K + 1)
        for k in range(K, 0, -1):
            delayed = V[:, k - 1]
            levels[k] = rs[:, t, :, k - 1, None] * U + rc[:, t, :, k - 1, None] * delayed
            U = rc[:, t, :, k - 1, None] * U - rs[:, t, :, k - 1, None] * delayed
        levels[0] = U
        V = np.where(keep[:, t, None, None, None], np.stack(levels[:K], axis=1), V)
    grads = dict(x=np.zeros((B, T, C)), alpha=np.zeros((B, T, C, K)), beta=np.zeros((B, T, C, K)),
                 rho=np.zeros((B, T, C, K + 1)), gamma=np.zeros((B, T, C)),
                 write=np.zeros((B, T, M)), read=np.zeros((B, T, K + 1, M)))
    lam = np.zeros((B, K, C, M))
    for t in range(T - 1, -1, -1):
        Vp = entering[t]
        U = x[:, t, :, None] * write[:, t, None, :]
        U_in = [None] * (K + 1)
        levels = [None] * (K + 1)
        for k in range(K, 0, -1):
            U_in[k] = U
            delayed = Vp[:, k - 1]
            levels[k] = rs[:, t, :, k - 1, None] * U + rc[:, t, :, k - 1, None] * delayed
            U = rc[:, t, :, k - 1, None] * U - rs[:, t, :, k - 1, None] * delayed
        levels[0] = U
        e = dy[:, t] * gate[:, t]                                             # [B,C]
        P = np.stack([(levels[k] * read[:, t, k, None, :]).sum(-1) for k in range(K + 1)], -1)
        weight = e[..., None] * rho[:, t]                                     # e rho_k, [B,C,K+1]
        Lam = [weight[..., k, None] * read[:, t, k, None, :]
               + (lam[:, k] if k < K else 0.0) for k in range(K + 1)]
        dU = Lam[0]
        drc, drs = np.zeros((B, C, K)), np.zeros((B, C, K))
        lam_new = np.zeros_like(lam)
        for k in range(1, K + 1):
            delayed = Vp[:, k - 1]
            drs[..., k - 1] = (Lam[k] * U_in[k] - dU * delayed).sum(-1)
            drc[..., k - 1] = (Lam[k] * delayed + dU * U_in[k]).sum(-1)
            lam_new[:, k - 1] = rc[:, t, :, k - 1, None] * Lam[k] - rs[:, t, :, k - 1, None] * dU
            dU = rs[:, t, :, k - 1, None] * Lam[k] + rc[:, t, :, k - 1, None] * dU
        on = keep[:, t]
        w = on[:, None].astype(f64)
        grads["x"][:, t] = w * (dU * write[:, t, None, :]).sum(-1)
        grads["write"][:, t] = on[:, None] * (dU * x[:, t, :, None]).sum(1)
        grads["rho"][:, t] = w[..., None] * e[..., None] * P
        grads["gamma"][:, t] = w * dy[:, t] * dgate[:, t] * (rho[:, t] * P).sum(-1)
        grads["read"][:, t] = on[:, None, None] * np.stack(
            [(weight[..., k, None] * levels[k]).sum(1) for k in range(K + 1)], 1)
        grads["alpha"][:, t] = w[..., None] * r[:, t] * (drc * dcos[:, t] + drs * dsin[:, t])
        grads["beta"][:, t] = w[..., None] * dr[:, t] * (drc * cos[:, t] + drs * sin[:, t])
        lam = np.where(on[:, None, None, None], lam_new, lam)
    return (grads["x"], grads["alpha"], grads["beta"], grads["rho"], grads["gamma"],
            grads["write"], grads["read"])
