"""CPU closed forms of the BASELINE-literal scans -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.

The reference has no convolution and no GLA operator (its mixer is the K-stage lattice of
model/mira_mixer.py:246-387). Both BASELINE scans are exact K=1 special cases of that lattice
after a reparameterisation of the inputs; `diag_as_lattice` and `gla_as_lattice` build those
lattice inputs so that the lattice oracle (oracle/lattice.py, the reference's algorithm) is the
parity anchor for the scans. The conv has no reference counterpart at all: its parity with the
reference is UNPINNED and only the closed form, brute force and invariants pin it.

Conventions (shared with the HIP kernels):
  * conv width W (4 in every config), weights w [D,W] float32, bias [D] float32;
    u_t[d] = sum_j w[d,j] x_(t-W+1+j)[d] + bias[d]; x before the first token comes from the
    ring, or is 0.
  * ring [B,D,W-1]: slot s holds x_t' for the t' = s (mod W-1) among the last W-1 tokens, where
    t' counts tokens from the start of the stream; `pos` is how many tokens the stream has
    absorbed before this call. A decode step therefore rewrites one slot.
  * diagonal scan h_t = a_t h_(t-1) + (1 - a_t) u_t, h float32 [B,D]; the output is h_t.
  * GLA: per (b, head) S_t = exp(g_t) S_(t-1) + k_t v_t^T, o_t = S_t^T q_t, with the state stored
    TRANSPOSED, [B,H,d_v,d_k], i.e. exactly the lattice state [B*H, 1, C=d_v, M=d_k].
"""
from __future__ import annotations

import numpy as np


# --------------------------------------------------------------------------------------------
# depthwise causal conv + diagonal decay scan
# --------------------------------------------------------------------------------------------
def conv_history(x, ring=None, pos=0):
    """x extended on the left by the W-1 tokens before it: [B, T+W-1, D] (ring order resolved).
    Slots never written (pos < W-1) hold zeros by construction of a zeroed ring."""
    B, T, D = x.shape
    if ring is None:
        return np.concatenate([np.zeros((B, 0, D), x.dtype), x], axis=1), 0
    Wm1 = ring.shape[2]
    past = np.stack([ring[:, :, (pos - Wm1 + j) % Wm1] for j in range(Wm1)], axis=1)  # [B,W-1,D]
    return np.concatenate([past.astype(x.dtype), x], axis=1), Wm1


def causal_conv(x, w, bias=None, ring=None, pos=0, dtype=np.float64):
    """u_t = sum_j w[:,j] x_(t-W+1+j) + bias, zero left pad or the ring's history."""
    B, T, D = x.shape
    W = w.shape[1]
    x = np.asarray(x, dtype)
    w = np.asarray(w, dtype)
    if ring is None:
        padded = np.concatenate([np.zeros((B, W - 1, D), dtype), x], axis=1)
    else:
        padded, _ = conv_history(x, np.asarray(ring, dtype), pos)
    u = np.zeros((B, T, D), dtype)
    for j in range(W):
        u += w[:, j] * padded[:, j:j + T]
    if bias is not None:
        u += np.asarray(bias, dtype)
    return u


def ring_after(x, ring, pos):
    """The ring after absorbing x [B,T,D] at position pos: the last W-1 tokens of the stream,
    each in slot (its stream index mod W-1)."""
    B, T, D = x.shape
    Wm1 = ring.shape[2]
    history, _ = conv_history(x, ring, pos)                    # stream tokens pos-W+1 .. pos+T-1
    out = np.array(ring, copy=True)
    for j in range(Wm1):
        t_stream = pos + T - Wm1 + j                           # one of the last W-1 tokens
        if t_stream < 0:
            continue
        out[:, :, t_stream % Wm1] = history[:, t_stream - pos + Wm1]
    return out


def diag_scan(u, a, h0=None, dtype=np.float64):
    """h_t = a_t h_(t-1) + (1 - a_t) u_t, returns (h [B,T,D], h_T [B,D])."""
    u = np.asarray(u, dtype)
    a = np.asarray(a, dtype)
    B, T, D = u.shape
    h = np.zeros((B, D), dtype) if h0 is None else np.asarray(h0, dtype).copy()
    out = np.empty((B, T, D), dtype)
    one = dtype(1)
    for t in range(T):
        h = a[:, t] * h + (one - a[:, t]) * u[:, t]
        out[:, t] = h
    return out, h


def diag_scan_closed_form(u, a, h0=None):
    """The same recurrence solved explicitly, float64, O(T^2):
    h_t = (prod_(i<=t) a_i) h0 + sum_(j<=t) (prod_(j<i<=t) a_i) (1 - a_j) u_j."""
    u = np.asarray(u, np.float64)
    a = np.asarray(a, np.float64)
    B, T, D = u.shape
    h0 = np.zeros((B, D)) if h0 is None else np.asarray(h0, np.float64)
    out = np.empty((B, T, D))
    for t in range(T):
        total = np.prod(a[:, :t + 1], axis=1) * h0
        for j in range(t + 1):
            total = total + np.prod(a[:, j + 1:t + 1], axis=1) * (1 - a[:, j]) * u[:, j]
        out[:, t] = total
    return out


def diag_conv_scan(x, a, w, bias=None, h0=None, ring=None, pos=0, dtype=np.float64):
    """The fused prefill: (h [B,T,D], h_T [B,D], ring_out or None)."""
    u = causal_conv(x, w, bias, ring, pos, dtype)
    h, hT = diag_scan(u, a, h0, dtype)
    return h, hT, (None if ring is None else ring_after(x, ring, pos))


# --------------------------------------------------------------------------------------------
# GLA matrix state
# --------------------------------------------------------------------------------------------
def gla_recurrent(q, k, v, g, S0=None, dtype=np.float64):
    """S_t = exp(g_t) S_(t-1) + k_t v_t^T, o_t = S_t^T q_t per (b, head); q,k,v [B,T,H,d],
    g [B,T,H]; state stored [B,H,d_v,d_k]. Returns (o [B,T,H,d_v], S_T [B,H,d_v,d_k])."""
    q, k, v, g = (np.asarray(t, dtype) for t in (q, k, v, g))
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    S = np.zeros((B, H, dv, dk), dtype) if S0 is None else np.asarray(S0, dtype).copy()
    o = np.empty((B, T, H, dv), dtype)
    for t in range(T):
        S = np.exp(g[:, t])[..., None, None] * S + v[:, t, :, :, None] * k[:, t, :, None, :]
        o[:, t] = np.einsum("bhvk,bhk->bhv", S, q[:, t])
    return o, S


def gla_quadratic(q, k, v, g, S0=None):
    """The attention-form solution, float64:
    o_t = sum_(j<=t) exp(G_t - G_j) (q_t . k_j) v_j + exp(G_t) S0 q_t, G_t = sum_(i<=t) g_i."""
    q, k, v, g = (np.asarray(t, np.float64) for t in (q, k, v, g))
    B, T, H, dk = q.shape
    G = np.cumsum(g, axis=1)                                           # [B,T,H]
    scores = np.einsum("bthd,bshd->bhts", q, k)
    decay = np.exp(G.transpose(0, 2, 1)[..., :, None] - G.transpose(0, 2, 1)[..., None, :])
    mask = np.tril(np.ones((T, T), bool))
    o = np.einsum("bhts,bshd->bthd", np.where(mask, scores * decay, 0.0), v)
    if S0 is not None:
        o = o + np.exp(G)[..., None] * np.einsum("bhvk,bthk->bthv", np.asarray(S0, np.float64), q)
    return o


def gla_chunked(q, k, v, g, S0=None, chunk=64):
    """The chunk form the MFMA kernel computes, float64: per chunk with in-chunk cumulative decay
    G, O = (Q K^T * D) V + (Q * e^G) S0^T, S_end = e^(G_L) S0 + sum_j e^(G_L - G_j) v_j k_j^T."""
    q, k, v, g = (np.asarray(t, np.float64) for t in (q, k, v, g))
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    S = np.zeros((B, H, dv, dk)) if S0 is None else np.asarray(S0, np.float64).copy()
    o = np.empty((B, T, H, dv))
    for first in range(0, T, chunk):
        last = min(T, first + chunk)
        Q, Kc, Vc = q[:, first:last], k[:, first:last], v[:, first:last]
        G = np.cumsum(g[:, first:last], axis=1).transpose(0, 2, 1)    # [B,H,L]
        L = last - first
        mask = np.tril(np.ones((L, L), bool))
        D = np.where(mask, np.exp(G[..., :, None] - G[..., None, :]), 0.0)
        A = np.einsum("bthd,bshd->bhts", Q, Kc) * D
        intra = np.einsum("bhts,bshv->bthv", A, Vc)
        inter = np.einsum("bhvk,bthk->bthv", S, Q) * np.exp(G).transpose(0, 2, 1)[..., None]
        o[:, first:last] = intra + inter
        tail = np.exp(G[..., -1:] - G)                                # [B,H,L]
        S = (np.exp(G[..., -1])[..., None, None] * S
             + np.einsum("bhs,bshv,bshk->bhvk", tail, Vc, Kc))
    return o, S


# --------------------------------------------------------------------------------------------
# exact K=1 realisations as reference-lattice inputs (cauchy_x_hyperbolic)
# --------------------------------------------------------------------------------------------
GAIN = 32.0   # SiLU(32) == 32 in float32: sigmoid(32) rounds to 1, so y = 32 h exactly.


def diag_as_lattice(u, a, h0=None, dtype=np.float32):
    """Lattice inputs whose K=1, M=1 scan is h_t = a_t h_(t-1) + (1 - a_t) u_t with y = 32 h:
    r = sqrt(a^2 + (1-a)^2), alpha = -atanh(a/r), beta = sqrt(1/r - 1), rho = (1, 0), nu = (1, 0),
    s = 1, gamma = 32. Coefficients derived in float64, then rounded to `dtype`.
    Returns (x, alpha, rho, gamma, write, read, beta, state)."""
    u = np.asarray(u, np.float64)
    a = np.asarray(a, np.float64)
    B, T, D = u.shape
    r = np.sqrt(a * a + (1 - a) ** 2)
    alpha = -np.arctanh(a / r)
    beta = np.sqrt(1.0 / r - 1.0)
    rho = np.zeros((B, T, D, 2))
    rho[..., 0] = 1.0
    read = np.zeros((B, T, 2, 1))
    read[:, :, 0, 0] = 1.0
    state = None if h0 is None else np.asarray(h0, np.float64).reshape(B, 1, D, 1)
    out = (u, alpha[..., None], rho, np.full((B, T, D), GAIN), np.ones((B, T, 1)), read,
           beta[..., None], state)
    return tuple(None if t is None else t.astype(dtype) for t in out)


def gla_as_lattice(q, k, v, g, S0=None, dtype=np.float32):
    """Lattice inputs (batch B*H, C = d_v, M = d_k) whose K=1 scan is the GLA recurrence with
    y = 32 o: beta = 0 (r = 1), alpha = -atanh(e^g) (sin = -e^g, cos = sqrt(1 - e^(2g))),
    x = v / sqrt(1 - e^(2g)), s = k, nu = (q, 0), rho = (1, 0), gamma = 32."""
    q, k, v, g = (np.asarray(t, np.float64) for t in (q, k, v, g))
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    fold = lambda t: t.transpose(0, 2, 1, 3).reshape(B * H, T, t.shape[-1])   # noqa: E731
    decay = np.exp(g).transpose(0, 2, 1).reshape(B * H, T)                    # [BH,T]
    cos = np.sqrt(1.0 - decay * decay)
    x = fold(v) / cos[..., None]
    alpha = np.broadcast_to((-np.arctanh(decay))[..., None, None], (B * H, T, dv, 1))
    beta = np.zeros((B * H, T, dv, 1))
    rho = np.zeros((B * H, T, dv, 2))
    rho[..., 0] = 1.0
    read = np.zeros((B * H, T, 2, dk))
    read[:, :, 0] = fold(q)
    state = None if S0 is None else np.asarray(S0, np.float64).reshape(B * H, 1, dv, dk)
    out = (x, alpha, rho, np.full((B * H, T, dv), GAIN), fold(k), read, beta, state)
    return tuple(None if t is None else np.ascontiguousarray(t).astype(dtype) for t in out)


def diag_inputs(rng, B, T, D, W=4, dtype=np.float32, h0_scale=0.0):
    """BASELINE cfg1/cfg2 synthetic inputs: x ~ N(0,1), a = sigmoid(U(2,6)), w ~ N(0, 0.5^2),
    bias 0, h0 ~ N(0, h0_scale^2) (or None when 0)."""
    x = rng.standard_normal((B, T, D)).astype(dtype)
    a = (1.0 / (1.0 + np.exp(-rng.uniform(2.0, 6.0, (B, T, D))))).astype(dtype)
    w = (rng.standard_normal((D, W)) * 0.5).astype(np.float32)
    bias = np.zeros(D, np.float32)
    h0 = None if h0_scale == 0 else (rng.standard_normal((B, D)) * h0_scale).astype(np.float32)
    return x, a, w, bias, h0


def gla_inputs(rng, B, T, H, dk, dv, dtype=np.float32):
    """BASELINE cfg3 synthetic inputs: q, k ~ N(0,1) L2-normalised per head, v ~ N(0,1),
    g ~ U(-0.1, -0.001)."""
    q = rng.standard_normal((B, T, H, dk))
    k = rng.standard_normal((B, T, H, dk))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, T, H, dv))
    g = rng.uniform(-0.1, -0.001, (B, T, H))
    return q.astype(dtype), k.astype(dtype), v.astype(dtype), g.astype(np.float32)
