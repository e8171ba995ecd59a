"""mira_lattice_forward_static, the allocation-free lattice forward (static device scratch), against
mira_lattice_forward with a caller's workspace, through the C-ABI: identical outputs and final
states, bit for bit, on two calls in a row (the second smaller, so it runs on what the first left
in the shared scratch), and a clear refusal when a call's chunk plan needs more scratch than the
static array holds."""
import ctypes

import numpy as np
import pytest

from _util import to_device
from oracle import lattice as L

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available()
    return torch


@pytest.fixture(scope="module")
def lib():
    from mira_amd import _lib

    assert _lib.library() is not None, _lib.why()
    return _lib


def _call(torch, lib, static, inputs, chunk, dtype):
    from mira_amd import mira

    x, alpha, rho, gamma, write, read, beta, valid, state = inputs
    B, T, C = x.shape
    K, M = alpha.shape[-1], write.shape[-1]
    out = torch.empty(B, T, C, device="cuda", dtype=dtype)
    final = torch.empty(B, K, C, M, device="cuda", dtype=torch.float32)
    ptr = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    common = (ptr(x), C, ptr(alpha), C * K, ptr(beta), C * K, ptr(rho), C * (K + 1), ptr(gamma),
              C, ptr(write), ptr(read), (K + 1) * M, ptr(valid), ptr(state), ptr(final), ptr(out),
              B, T, C, K, M, mira.DTYPE[dtype], mira.ARCH_STAGE["cauchy_x_hyperbolic"], chunk)
    handle = lib.require()
    if static:
        code = handle.mira_lattice_forward_static(*common, stream)
    else:
        need = handle.mira_lattice_workspace_bytes(B, T, C, K, M, chunk)
        space = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
        code = handle.mira_lattice_forward(*common, ptr(space), need, stream)
    lib.check(code, "static" if static else "workspace")
    return out, final


def _inputs(torch, seed, B, T, C, K, M, dtype):
    rng = np.random.default_rng(seed)
    values = L.random_inputs(rng, B, T, C, K, M)
    valid = rng.random((B, T)) > 0.2
    state = (rng.standard_normal((B, K, C, M)) * 0.1).astype(np.float32)
    return ([to_device(v, dtype) for v in values]
            + [to_device(valid.astype(np.uint8)), to_device(state)])


@pytest.mark.parametrize("dtype_name", ["float32", "bfloat16"])
def test_static_scratch_matches_the_workspace_entry_point(torch_mod, lib, dtype_name):
    torch = torch_mod
    dtype = getattr(torch, dtype_name)
    # first a large call (16 chunks over the static scratch), then a smaller one that reuses it
    for seed, (B, T, C, K, M, chunk) in enumerate([(4, 512, 256, 2, 64, 32),
                                                  (2, 100, 96, 2, 16, 16)]):
        inputs = _inputs(torch, seed, B, T, C, K, M, dtype)
        want, want_state = _call(torch, lib, False, inputs, chunk, dtype)
        got, got_state = _call(torch, lib, True, inputs, chunk, dtype)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {seed}: outputs differ"
        assert torch.equal(got_state, want_state), f"call {seed}: final states differ"


def test_static_scratch_refuses_oversized_calls(torch_mod, lib):
    torch = torch_mod
    B, T, C, K, M = 8, 4096, 2048, 2, 64
    need = lib.require().mira_lattice_workspace_bytes(B, T, C, K, M, 16)
    assert need > (64 << 20)
    inputs = _inputs(torch, 3, 1, 2, 8, K, M, torch.float32)
    x = inputs[0]
    handle = lib.require()
    ptr = ctypes.c_void_p(x.data_ptr())
    code = handle.mira_lattice_forward_static(
        ptr, C, ptr, C * K, ptr, C * K, ptr, C * (K + 1), ptr, C, ptr, ptr, (K + 1) * M, None,
        None, None, ptr, B, T, C, K, M, 0, 6, 16, None)
    assert code == lib.ERR_ARG
    assert "static scratch" in lib.last_error()
