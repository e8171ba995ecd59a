"""GPU parity of the lattice scan (mira_lattice_forward / mira_lattice_step) against the oracle
(oracle/lattice.py, the reference algorithm) and the reference's own golden vectors.

Follows the reference harness (kernel/cuda/mira_dspv2/check.py): values per arch x (K, d_m) x
dtype (`_case` :42-104), strided views, forced chunks (`_forward_case` :107-153), streaming ==
one shot with a masked sequence keeping its state bit-exact (`_state_case` :223-270), all-true
mask == no mask bit-exact (`_mask_dispatch_case` :320-343), plus decode-N == prefill.
Tolerances: float32 max abs <= 1e-5 and scaled <= 3e-4; bf16/f16 scaled <= 2e-2.
"""
import os

import numpy as np
import pytest

from _util import (FP32_ABS, FP32_SCALED, HALF_SCALED, golden_files, max_abs, rounded, scaled,
                   to_device, to_numpy)
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


DTYPES = {"float32": None, "bfloat16": None, "float16": None}


def _torch_dtype(torch, name):
    return getattr(torch, name)


def _run(plugin, torch, values, valid=None, state=None, arch="cauchy_x_hyperbolic", dtype="float32",
         chunk=None, strided=False):
    td = _torch_dtype(torch, dtype)
    x, alpha, rho, gamma, write, read, beta = [to_device(v, td) for v in values]
    if strided:
        B, T, C = x.shape
        base = torch.empty(B, T, 2 * C + 3, device="cuda", dtype=td)
        base[:, :, :C] = x
        x = base[:, :, :C]
        base2 = torch.empty(B, T, 2 * C + 3, device="cuda", dtype=td)
        base2[:, :, C:2 * C] = gamma
        gamma = base2[:, :, C:2 * C]
    out = plugin.matrix_lattice_iir(
        x, alpha, rho, gamma, write, read, raw_beta=beta,
        valid=None if valid is None else to_device(valid), state=to_device(state),
        return_state=True, arch=arch, chunk=chunk)
    assert out is not None, "the plugin declined a served shape"
    y, final = out
    torch.cuda.synchronize()
    return to_numpy(y), to_numpy(final)


def _oracle(values, valid, state, arch, dtype, torch):
    """fp64 oracle on the inputs the kernel sees (rounded to dtype)."""
    td = _torch_dtype(torch, dtype)
    seen = [rounded(v, td) for v in values]
    return L.lattice_scan_sequential(*seen, valid=valid, state=state, arch=arch, dtype=np.float64)


def _assert(got, want, dtype, what):
    if dtype == "float32":
        assert max_abs(got, want) <= FP32_ABS, f"{what}: max abs {max_abs(got, want):.3e}"
        assert scaled(got, want) <= FP32_SCALED, f"{what}: scaled {scaled(got, want):.3e}"
    else:
        assert scaled(got, want) <= HALF_SCALED, f"{what}: scaled {scaled(got, want):.3e}"


@pytest.mark.parametrize("path", golden_files("k"), ids=lambda p: os.path.basename(p)[:-4])
def test_golden_reference_vectors(torch_mod, plugin, path):
    """The reference CPU mixer's own float32 output on identical inputs."""
    d = np.load(path)
    values = [d[k] for k in ("x", "alpha", "rho", "gamma", "write", "read", "beta")]
    valid = d["valid"] if "valid" in d else None
    state = d["state"] if "state" in d else None
    y, final = _run(plugin, torch_mod, values, valid, state, str(d["arch"]))
    _assert(y, d["y"], "float32", "output")
    _assert(final, d["final"], "float32", "state")


CASES = [(1, 1), (1, 8), (1, 128), (2, 16), (2, 64), (4, 8), (4, 32), (8, 4), (8, 16), (2, 2)]


@pytest.mark.parametrize("order,memory", CASES)
@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_orders_memories_dtypes(torch_mod, plugin, order, memory, dtype):
    rng = np.random.default_rng(20260830 + memory + order)
    values = L.random_inputs(rng, 2, 45, 37, order, memory)
    state = (rng.standard_normal((2, order, 37, memory)) * 0.1).astype(np.float32)
    valid = rng.random((2, 45)) > 0.2
    y, final = _run(plugin, torch_mod, values, valid, state, "cauchy_x_mobius", dtype)
    want_y, want_state = _oracle(values, valid, state, "cauchy_x_mobius", dtype, torch_mod)
    _assert(y, want_y, dtype, "output")
    _assert(final, want_state, "float32" if dtype == "float32" else dtype, "state")


@pytest.mark.parametrize("arch", list(L.ARCH_STAGE))
def test_every_arch(torch_mod, plugin, arch):
    rng = np.random.default_rng(7)
    values = L.random_inputs(rng, 2, 33, 19, 2, 16, scale=(0.5, 1.2, 0.5, 0.8, 0.5, 0.5, 1.0),
                             beta_bias=0.3)
    values[1][0, :4] *= 8.0                     # |alpha| > 1: the reciprocal branches
    y, final = _run(plugin, torch_mod, values, None, None, arch)
    want_y, want_state = _oracle(values, None, None, arch, "float32", torch_mod)
    _assert(y, want_y, "float32", f"{arch} output")
    _assert(final, want_state, "float32", f"{arch} state")


@pytest.mark.parametrize("order,memory,chunk", [(2, 64, 32), (2, 16, 48), (4, 32, 48)],
                         ids=["k2m64_mfma_summary", "k2m16", "k4m32"])
@pytest.mark.parametrize("arch", list(L.ARCH_STAGE))
def test_every_arch_bf16_per_map_kernels(torch_mod, plugin, arch, order, memory, chunk):
    """bf16 at the mixer's shapes runs summary and replay kernels built for the one stage map of
    the call: every map, through the chunked path (summary, combine, replay), with a mask and a
    carried-in state, against the fp32 oracle on the bf16-rounded inputs."""
    rng = np.random.default_rng(60 + order + memory)
    values = L.random_inputs(rng, 2, 100, 40, order, memory, scale=(0.5, 1.2, 0.5, 0.8, 0.5, 0.5, 1.0),
                             beta_bias=0.3)
    values[1][0, :4] *= 8.0                     # |alpha| > 1: the reciprocal branches
    state = (rng.standard_normal((2, order, 40, memory)) * 0.1).astype(np.float32)
    valid = rng.random((2, 100)) > 0.15
    y, final = _run(plugin, torch_mod, values, valid, state, arch, "bfloat16", chunk=chunk)
    want_y, want_state = _oracle(values, valid, state, arch, "bfloat16", torch_mod)
    _assert(y, want_y, "bfloat16", f"{arch} output")
    assert max_abs(final, want_state) <= 1e-4, f"{arch} state: {max_abs(final, want_state):.3e}"


@pytest.mark.parametrize("order,memory", [(k, m) for k in (1, 2, 4) for m in (16, 32, 64, 128)])
@pytest.mark.parametrize("arch", list(L.ARCH_STAGE))
def test_per_map_kernels_every_shape(torch_mod, plugin, arch, order, memory):
    """Every (K, d_m) built per stage map in bf16 under every map, chunked (48-token chunks: the
    matrix summary at d_m >= 32, the per-slot one below), with a mask and a carried-in state."""
    rng = np.random.default_rng(90 + order + memory)
    values = L.random_inputs(rng, 2, 100, 24, order, memory)
    state = (rng.standard_normal((2, order, 24, memory)) * 0.1).astype(np.float32)
    valid = rng.random((2, 100)) > 0.15
    y, final = _run(plugin, torch_mod, values, valid, state, arch, "bfloat16", chunk=48)
    want_y, want_state = _oracle(values, valid, state, arch, "bfloat16", torch_mod)
    _assert(y, want_y, "bfloat16", f"{arch} K{order} d_m{memory} output")
    assert max_abs(final, want_state) <= 1e-4, f"state: {max_abs(final, want_state):.3e}"


@pytest.mark.parametrize("order,memory", [(1, 64), (2, 32), (2, 64), (2, 128)])
@pytest.mark.parametrize("arch", ["cauchy_x_hyperbolic", "cauchy_x_mobius", "cauchy_x_identity"])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_scaled_replay_special_coefficients(torch_mod, plugin, arch, order, memory, dtype):
    """The replay keeps K <= 2 state rows divided by per-channel scales built from the stage
    coefficients: exact zeros (alpha = 0 gives sin = 0 or, for the Moebius map, cos = 0), tiny
    radii (|beta| ~ 1e3 gives r ~ 1e-6), whole stretches of zeros (a zero-initialised
    projection), masked tokens and partial tiles must all match the fp64 oracle."""
    rng = np.random.default_rng(300 + 10 * order + memory)
    B, T, C = 2, 100, 24
    values = L.random_inputs(rng, B, T, C, order, memory)
    alpha, beta = values[1], values[6]
    alpha[rng.random(alpha.shape) < 0.25] = 0.0
    alpha[0, 40:72] = 0.0                       # every stage of every channel, 32 tokens
    beta[rng.random(beta.shape) < 0.05] = 1000.0
    beta[1, 10:14, :5] = -3000.0
    state = (rng.standard_normal((B, order, C, memory)) * 0.1).astype(np.float32)
    valid = rng.random((B, T)) > 0.1
    valid[0, 40:72] = True
    for chunk in (48, None):
        y, final = _run(plugin, torch_mod, values, valid, state, arch, dtype, chunk=chunk)
        want_y, want_state = _oracle(values, valid, state, arch, dtype, torch_mod)
        _assert(y, want_y, dtype, f"{arch} K{order} d_m{memory} chunk {chunk} output")
        assert max_abs(final, want_state) <= (FP32_ABS if dtype == "float32" else 1e-4), \
            f"state: {max_abs(final, want_state):.3e}"
        assert np.isfinite(y).all() and np.isfinite(final).all()


@pytest.mark.parametrize("chunk", [1, 5, 16, 17, 64, None, 1000])
def test_chunking_is_invisible(torch_mod, plugin, chunk):
    rng = np.random.default_rng(11)
    values = L.random_inputs(rng, 2, 129, 21, 2, 16)
    state = (rng.standard_normal((2, 2, 21, 16)) * 0.1).astype(np.float32)
    valid = rng.random((2, 129)) > 0.1
    y, final = _run(plugin, torch_mod, values, valid, state, chunk=chunk)
    want_y, want_state = _oracle(values, valid, state, "cauchy_x_hyperbolic", "float32", torch_mod)
    _assert(y, want_y, "float32", f"chunk {chunk} output")
    _assert(final, want_state, "float32", f"chunk {chunk} state")


def test_strided_views(torch_mod, plugin):
    rng = np.random.default_rng(3)
    values = L.random_inputs(rng, 2, 40, 24, 2, 16)
    y, _ = _run(plugin, torch_mod, values, strided=True)
    want_y, _ = _oracle(values, None, None, "cauchy_x_hyperbolic", "float32", torch_mod)
    _assert(y, want_y, "float32", "strided output")


def test_fused_projection_views(torch_mod, plugin):
    """alpha, beta, rho, nu as row-strided views of one coefficient projection (the mixer's
    split, model/mira_mixer.py:807-813)."""
    torch = torch_mod
    rng = np.random.default_rng(5)
    B, T, C, K, M = 2, 30, 12, 2, 16
    values = L.random_inputs(rng, B, T, C, K, M)
    x, alpha, rho, gamma, write, read, beta = values
    packed = np.concatenate([alpha.reshape(B, T, -1), beta.reshape(B, T, -1),
                             rho.reshape(B, T, -1), read.reshape(B, T, -1)], axis=-1)
    p = to_device(packed)
    a_, b_, r_, n_ = p.split((C * K, C * K, C * (K + 1), (K + 1) * M), dim=-1)
    out = plugin.matrix_lattice_iir(to_device(x), a_.view(B, T, C, K), r_.view(B, T, C, K + 1),
                                    to_device(gamma), to_device(write), n_.view(B, T, K + 1, M),
                                    raw_beta=b_.view(B, T, C, K))
    want, _ = _oracle(values, None, None, "cauchy_x_hyperbolic", "float32", torch)
    _assert(to_numpy(out), want, "float32", "packed views")


def test_streaming_equals_one_shot(torch_mod, plugin):
    rng = np.random.default_rng(20260830)
    values = L.random_inputs(rng, 2, 35, 3, 2, 16)
    initial = (rng.standard_normal((2, 2, 3, 16)) * 0.1).astype(np.float32)
    valid = np.ones((2, 35), bool)
    valid[0] = False
    valid[1, ::4] = False
    y, final = _run(plugin, torch_mod, values, valid, initial)
    state = initial
    parts = []
    first = 0
    for length in (1, 15, 1, 17, 1):
        sl = [v[:, first:first + length] for v in values]
        part, state = _run(plugin, torch_mod, sl, valid[:, first:first + length], state)
        parts.append(part)
        first += length
    streamed = np.concatenate(parts, axis=1)
    _assert(streamed, y, "float32", "streamed output")
    _assert(state, final, "float32", "streamed state")
    assert np.array_equal(state[0], initial[0]), "a fully masked sequence changed its state"
    want_y, want_state = _oracle(values, valid, initial, "cauchy_x_hyperbolic", "float32", torch_mod)
    _assert(y, want_y, "float32", "output")


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_all_true_mask_is_no_mask(torch_mod, plugin, dtype):
    rng = np.random.default_rng(20260919)
    values = L.random_inputs(rng, 2, 257, 193, 2, 16)
    initial = (rng.standard_normal((2, 2, 193, 16)) * 0.1).astype(np.float32)
    y0, s0 = _run(plugin, torch_mod, values, None, initial, dtype=dtype)
    y1, s1 = _run(plugin, torch_mod, values, np.ones((2, 257), bool), initial, dtype=dtype)
    assert np.array_equal(y0, y1) and np.array_equal(s0, s1)


@pytest.mark.parametrize("order,memory", [(2, 16), (1, 128), (4, 8)])
def test_decode_steps_equal_prefill(torch_mod, plugin, order, memory):
    torch = torch_mod
    rng = np.random.default_rng(17)
    B, N, C = 3, 12, 40
    values = L.random_inputs(rng, B, N, C, order, memory)
    initial = (rng.standard_normal((B, order, C, memory)) * 0.1).astype(np.float32)
    y, final = _run(plugin, torch, values, None, initial)
    state = to_device(initial)
    outs = []
    for t in range(N):
        step = [to_device(np.ascontiguousarray(v[:, t:t + 1])) for v in values]
        out, state = plugin.matrix_lattice_step(step[0], step[1], step[2], step[3], step[4],
                                                step[5], step[6], state, inplace=(t % 2 == 0))
        outs.append(to_numpy(out))
    torch.cuda.synchronize()
    _assert(np.concatenate(outs, axis=1), y, "float32", "decode outputs")
    _assert(to_numpy(state), final, "float32", "decode state")


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("order,memory", [(2, 64), (4, 32), (1, 8), (2, 128)])
def test_decode_step_kernel(torch_mod, plugin, order, memory, dtype):
    """T = 1 with K <= 4 and 8 <= d_m <= 128 runs the state-streaming step kernel: every dtype, a
    partial channel group (C = 300), a masked sequence, with and without a carried-in state,
    against the fp64 oracle on the inputs rounded to the dtype."""
    rng = np.random.default_rng(31 + order + memory)
    B, C = 5, 300
    values = L.random_inputs(rng, B, 1, C, order, memory)
    valid = np.array([True, False, True, True, False])[:, None]
    initial = (rng.standard_normal((B, order, C, memory)) * 0.1).astype(np.float32)
    for state in (initial, None):
        y, final = _run(plugin, torch_mod, values, valid, state, dtype=dtype)
        want_y, want_state = _oracle(values, valid, state, "cauchy_x_hyperbolic", dtype, torch_mod)
        _assert(y, want_y, dtype, f"step output (state {'in' if state is not None else 'none'})")
        _assert(final, want_state, "float32", "step state")
        if state is not None:
            assert np.array_equal(final[1], initial[1]) and np.array_equal(final[4], initial[4])


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("order,memory", [(2, 64), (1, 128)])
def test_decode_step_kernel_wide_blocks(torch_mod, plugin, order, memory, dtype):
    """A batch large enough that the step kernel runs 1,024-thread blocks (>= 2,048 of them):
    B = 256, a partial channel group (C = 1000), masked sequences, with and without a carried-in
    state, against the fp64 oracle."""
    rng = np.random.default_rng(41 + order + memory)
    B, C = 256, 1000
    values = L.random_inputs(rng, B, 1, C, order, memory)
    valid = (rng.random((B, 1)) > 0.1)
    initial = (rng.standard_normal((B, order, C, memory)) * 0.1).astype(np.float32)
    for state in (initial, None):
        y, final = _run(plugin, torch_mod, values, valid, state, dtype=dtype)
        want_y, want_state = _oracle(values, valid, state, "cauchy_x_hyperbolic", dtype, torch_mod)
        _assert(y, want_y, dtype, f"wide step output (state {'in' if state is not None else 'none'})")
        _assert(final, want_state, "float32", "wide step state")


def test_reference_geometry_bf16(torch_mod, plugin):
    """The reference mira-s mixer geometry (K=2, d_e=1536, d_m=16) in bf16 at 512 tokens."""
    rng = np.random.default_rng(23)
    values = L.random_inputs(rng, 2, 512, 1536, 2, 16)
    y, final = _run(plugin, torch_mod, values, None, None, dtype="bfloat16")
    td = torch_mod.bfloat16
    seen = [rounded(v, td) for v in values]
    want_y, want_state = L.lattice_scan_sequential(*seen, dtype=np.float32)
    _assert(y, want_y, "bfloat16", "output")
    assert max_abs(final, want_state) <= 1e-4


def test_decline_and_errors(torch_mod, plugin):
    torch = torch_mod
    rng = np.random.default_rng(1)
    values = [to_device(v) for v in L.random_inputs(rng, 1, 4, 3, 3, 16)]   # K = 3: not served
    assert plugin.matrix_lattice_iir(*values[:6], raw_beta=values[6]) is None
    values = [to_device(v) for v in L.random_inputs(rng, 1, 4, 3, 2, 16)]
    with pytest.raises(ValueError):
        plugin.matrix_lattice_iir(*values[:6], raw_beta=values[6],
                                  state=torch.zeros(1, 2, 3, 16, device="cuda"))  # no return_state
    with pytest.raises(ValueError):
        plugin.matrix_lattice_iir(*values[:6], raw_beta=values[6],
                                  valid=torch.ones(1, 4, device="cuda"))           # not bool
    assert plugin.matrix_lattice_iir(*values[:6], raw_beta=None) is None


def test_mixer_prefill_then_decode(torch_mod, plugin):
    """The host caller: MiraMixer with a PrefixCache, prompt then one token at a time, equals the
    uncached forward over the whole sequence (the kv_cache.check invariant, helpers/kv_cache.py:196)."""
    torch = torch_mod
    from mira_amd.mixer import MiraMixer
    from mira_amd.prefix_cache import PrefixCache

    torch.manual_seed(0)
    mixer = MiraMixer(64, lattice_order=2, d_e=96, coefficient_bottleneck=16,
                      memory_dimension=16).cuda().eval()
    x = torch.randn(2, 21, 64, device="cuda") * 0.5
    with torch.no_grad():
        full = mixer(x)
        cache = PrefixCache(1)
        parts = [mixer(x[:, :13], cache=cache, layer=0)]
        cache.advance(13)
        for t in range(13, 21):
            parts.append(mixer(x[:, t:t + 1], cache=cache, layer=0))
            cache.advance(1)
    streamed = torch.cat(parts, dim=1)
    assert max_abs(to_numpy(streamed), to_numpy(full)) <= 2e-5
    assert len(cache) == 21


@pytest.mark.parametrize("order,memory", [(1, 64), (2, 64), (4, 32), (2, 128)])
@pytest.mark.parametrize("chunk", [32, 48, 40])
def test_bf16_chunk_summaries(torch_mod, plugin, order, memory, chunk):
    """bf16 with several chunks: 16-token multiples take the matrix-core summary (backward scan of
    the stage maps + a GEMM of the injections with s), 40 takes the per-slot summary; both
    against the fp32 oracle on the bf16-rounded inputs, with a mask, a carried-in state and a
    partial channel group."""
    rng = np.random.default_rng(40 + order + memory + chunk)
    values = L.random_inputs(rng, 2, 200, 70, order, memory)
    state = (rng.standard_normal((2, order, 70, memory)) * 0.1).astype(np.float32)
    valid = rng.random((2, 200)) > 0.15
    y, final = _run(plugin, torch_mod, values, valid, state, "cauchy_x_hyperbolic", "bfloat16",
                    chunk=chunk)
    want_y, want_state = _oracle(values, valid, state, "cauchy_x_hyperbolic", "bfloat16", torch_mod)
    _assert(y, want_y, "bfloat16", f"chunk {chunk} output")
    # the state stays float32 through both summaries (the GEMM's left operand is split hi + lo)
    assert max_abs(final, want_state) <= 1e-4, f"chunk {chunk} state: {max_abs(final, want_state):.3e}"


@pytest.mark.parametrize("arch", list(L.ARCH_STAGE))
def test_stage_maps_against_fp64(torch_mod, plugin, arch):
    """The kernel's stage maps alone, for 8192 (alpha, beta) pairs per arch over the ranges the
    mixer feeds (|alpha| up to 12, beta up to 6): one decode step with K=1, x=0, state 1 reads
    r cos(theta) out through the readout (nu = (0, 1), rho = (0, 1), gamma = 32: y = 32 r cos) and
    -r sin(theta) as the new state. Against oracle/lattice.py's closed forms in float64."""
    torch = torch_mod
    rng = np.random.default_rng(99)
    C = 8192
    alpha = np.concatenate([rng.uniform(-12, 12, C // 2), rng.normal(0, 0.05, C // 2)]).astype(np.float32)
    beta = np.concatenate([rng.uniform(-6, 6, C // 2), rng.normal(0, 0.05, C // 2)]).astype(np.float32)
    x = np.zeros((1, 1, C), np.float32)
    rho = np.zeros((1, 1, C, 2), np.float32)
    rho[..., 1] = 1.0
    gamma = np.full((1, 1, C), 32.0, np.float32)
    write = np.ones((1, 1, 1), np.float32)
    read = np.zeros((1, 1, 2, 1), np.float32)
    read[:, :, 1, 0] = 1.0
    state = np.ones((1, 1, C, 1), np.float32)
    ins = [to_device(v) for v in (x, alpha.reshape(1, 1, C, 1), rho, gamma, write, read,
                                  beta.reshape(1, 1, C, 1))]
    out, final = plugin.matrix_lattice_step(*ins, to_device(state), arch=arch)
    torch.cuda.synchronize()
    rotation, radius = L.stage_maps(arch)
    cos, sin = rotation(alpha.astype(np.float64))
    r = radius(beta.astype(np.float64))
    got_rc = to_numpy(out).reshape(C) / 32.0
    got_rs = -to_numpy(final).reshape(C)
    assert max_abs(got_rc, r * cos) <= 1e-6, f"r cos: {max_abs(got_rc, r * cos):.3e}"
    assert max_abs(got_rs, r * sin) <= 1e-6, f"r sin: {max_abs(got_rs, r * sin):.3e}"
