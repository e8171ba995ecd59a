"""CPU checks of the C-ABI library: it loads without a GPU, exports every entry point that
include/mira_hip.h declares, and its host-only entry points (planning, workspace sizes, argument
validation) behave -- no kernel is launched here."""
import ctypes
import os
import re

import pytest

from _util import HERE

ROOT = os.path.dirname(HERE)
HEADER = os.path.join(ROOT, "include", "mira_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mira_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from mira_amd import _lib

    library = _lib.library()
    if library is None:
        pytest.fail(f"libmira_hip.so does not load: {_lib.why()}")
    return library


def test_every_declared_symbol_is_exported(lib):
    names = declared()
    assert len(names) >= 14
    missing = [name for name in names if not hasattr(lib, name)]
    assert not missing, f"declared in mira_hip.h but not exported: {missing}"


def test_binding_covers_the_header():
    from mira_amd import _lib

    assert sorted(_lib.SIGNATURES) == declared()


def test_version_and_support_table(lib):
    assert b"gfx950" in lib.mira_version()
    for K in (1, 2, 4, 8):
        for M in (1, 2, 4, 8, 16, 32, 64, 128):
            for dtype in (0, 1, 2):
                assert lib.mira_lattice_supported(K, M, dtype) == 1
    assert lib.mira_lattice_supported(3, 16, 0) == 0
    assert lib.mira_lattice_supported(2, 12, 0) == 0
    assert lib.mira_lattice_supported(2, 16, 3) == 0


def test_chunk_plan_and_workspace(lib):
    # one chunk for short or wide calls: no workspace
    assert lib.mira_lattice_plan_chunk(1, 16, 256, 2, 16) == 16
    assert lib.mira_lattice_workspace_bytes(1, 16, 256, 2, 16, 0) == 0
    chunk = lib.mira_lattice_plan_chunk(1, 8192, 64, 1, 128)
    assert 16 <= chunk < 8192 and chunk % 16 == 0
    chunks = -(-8192 // chunk)
    assert lib.mira_lattice_workspace_bytes(1, 8192, 64, 1, 128, chunk) == \
        4 * chunks * 64 * (1 + 128)
    assert lib.mira_diag_workspace_bytes(8, 4096, 2048, 1) > 0
    assert lib.mira_diag_workspace_bytes(0, 4096, 2048, 1) == 0


def test_argument_errors_without_a_launch(lib):
    """Validation happens before any HIP call: decline (1) or bad argument (2)."""
    null = None
    # K = 3 is not built: decline
    code = lib.mira_lattice_forward(null, 4, null, 12, null, 12, null, 16, null, 4, null, null, 64,
                                    null, null, null, null, 1, 8, 4, 3, 16, 0, 6, 0, null, 0, null)
    assert code == 1 and b"K=3" in lib.mira_last_error()
    # empty batch: bad argument
    code = lib.mira_lattice_forward(null, 4, null, 8, null, 8, null, 12, null, 4, null, null, 48,
                                    null, null, null, null, 0, 8, 4, 2, 16, 0, 6, 0, null, 0, null)
    assert code == 2
    # unknown arch mode
    fake = ctypes.c_void_p(16)
    code = lib.mira_lattice_forward(fake, 4, fake, 8, fake, 8, fake, 12, fake, 4, fake, fake, 48,
                                    null, null, null, fake, 1, 8, 4, 2, 16, 0, 5, 0, null, 0, null)
    assert code == 2 and b"arch" in lib.mira_last_error()
    # diag: width other than 4 declines, D not a multiple of 4 declines
    assert lib.mira_diag_conv_scan(fake, fake, fake, null, null, null, null, 0, fake, null,
                                   1, 8, 16, 3, 1, fake, 1 << 20, null) == 1
    assert lib.mira_diag_conv_scan(fake, fake, fake, null, null, null, null, 0, fake, null,
                                   1, 8, 6, 4, 1, fake, 1 << 20, null) == 1
    # gla: d = 64 declines
    assert lib.mira_gla_step(fake, fake, fake, fake, fake, fake, 1, 1, 64, 64, 1, null) == 1


def test_control_scan_plan_and_errors(lib):
    """mira_lattice_control_serves: bf16, the (K, d_m) where forming the coefficients in the scan
    is the faster path, d_r in {16, 32, 48, 64}, one token chunk; anything else declines before
    any HIP call, and coefficient rows outside the weight are a bad argument."""
    bf16, f32 = 1, 0
    served = {(1, 8), (1, 16), (2, 8), (2, 16), (4, 8)}
    for K in (1, 2, 4, 8):
        for M in (8, 16, 32, 64):
            want = int((K, M) in served)
            assert lib.mira_lattice_control_serves(8, 16, 256, K, M, 48, bf16) == want, (K, M)
    assert lib.mira_lattice_control_serves(8, 16, 256, 2, 16, 48, f32) == 0
    for rank in (8, 24, 80, 128):
        assert lib.mira_lattice_control_serves(8, 16, 256, 2, 16, rank, bf16) == 0
    # a call the chunk planner would split (one sequence of 300 tokens) declines
    assert lib.mira_lattice_plan_chunk(1, 300, 1536, 2, 16) < 300
    assert lib.mira_lattice_control_serves(1, 300, 1536, 2, 16, 48, bf16) == 0
    assert lib.mira_lattice_control_serves(1, 16, 1536, 2, 16, 48, bf16) == 1
    null, fake = None, ctypes.c_void_p(256)
    C, K, M, R = 32, 2, 16, 48
    rows = C * (3 * K + 1) + (K + 1) * M

    def call(alpha_first=0, weight_rows=rows, dtype=bf16, order=K):
        return lib.mira_lattice_control_forward(
            fake, C, fake, fake, R, weight_rows, null, alpha_first, C * K, 2 * C * K, fake, C,
            fake, fake, (K + 1) * M, null, null, null, fake, 2, 4, C, order, M, R, dtype, 6, null)

    assert call(dtype=f32) == 1
    assert call(order=8) == 1
    assert call(alpha_first=-1) == 2
    assert call(weight_rows=2 * C * K) == 2 and b"outside the weight" in lib.mira_last_error()


def test_backward_plan_and_errors(lib):
    """mira_lattice_backward_chunk: the chunk a training forward runs at (<= 16 tokens so a lane
    holds the chunk's states), 0 where (K, d_m) has no backward (the reference's ORDER_MEMORIES:
    K 1 and 8 at d_m 8, 16; K 2 and 4 at d_m 8..64); argument errors before any launch."""
    assert lib.mira_lattice_backward_chunk(2, 16) == 16
    assert lib.mira_lattice_backward_chunk(2, 64) == 16
    assert lib.mira_lattice_backward_chunk(1, 8) == 4
    for K, M in ((2, 128), (1, 32), (8, 32), (2, 1), (3, 16)):
        assert lib.mira_lattice_backward_chunk(K, M) == 0, (K, M)
    assert lib.mira_lattice_backward_workspace_bytes(2, 100, 64, 2, 16) > 0
    assert lib.mira_lattice_backward_workspace_bytes(2, 100, 64, 2, 128) == 0
    fake, null = ctypes.c_void_p(256), None
    args = [fake, 64, fake, 128, fake, 128, fake, 192, fake, 64, fake, fake, 48, null, null, fake]
    grads = [fake, 64, fake, 128, fake, 128, fake, 192, fake, 64, fake, 16, null, 0, fake, 48]
    tail = [2, 100, 64, 2, 16, 0, 6]
    # a missing gradient output: bad argument
    bad = list(grads)
    bad[4] = null
    assert lib.mira_lattice_backward(*args, *bad, *tail, fake, 1 << 30, fake, 1 << 30, null) == 2
    # no forward workspace over several chunks: bad argument
    assert lib.mira_lattice_backward(*args, *grads, *tail, null, 0, fake, 1 << 30, null) == 2
    assert b"forward" in lib.mira_last_error()
    # a workspace off a 16-byte boundary: bad argument (the reduce reads it 16 bytes at a time)
    assert lib.mira_lattice_backward(*args, *grads, *tail, fake, 1 << 30, ctypes.c_void_p(264),
                                     1 << 30, null) == 2
    assert b"aligned" in lib.mira_last_error()
    # a (K, d_m) without backward kernels declines
    tail_wide = [2, 100, 64, 2, 128, 0, 6]
    wide_args = list(args)
    wide_args[12] = 3 * 128
    wide_grads = list(grads)
    wide_grads[11], wide_grads[15] = 128, 3 * 128
    assert lib.mira_lattice_backward(*wide_args, *wide_grads, *tail_wide, fake, 1 << 30, fake,
                                     1 << 30, null) == 1
