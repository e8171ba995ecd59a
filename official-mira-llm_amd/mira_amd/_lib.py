"""ctypes binding of libmira_hip.so (include/mira_hip.h) -- replaces the reference's cubin loader.

The reference loads a fatbin through the CUDA driver API and launches by symbol name
(kernel/cuda/driver.py: module_for :328-344, launch_dims :910-934). Here the kernels live in one
HIP shared library built for gfx950 (official-mira-llm_amd/build.py) and are reached through the
C entry points below. The library is loaded once per process; a failure to load is remembered
and reported by `why()`, as the reference's driver remembers a refused cubin (driver.py:352-361).
There is no fallback: callers raise when `library()` is None.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "lib", "libmira_hip.so")

OK, DECLINE, ERR_ARG, ERR_HIP = 0, 1, 2, 3
F32, BF16, F16 = 0, 1, 2

_LOCK = threading.RLock()
_LIB = None
_WHY = ""

p, i64, i32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t

SIGNATURES = {
    "mira_last_error": ([], ctypes.c_char_p),
    "mira_version": ([], ctypes.c_char_p),
    "mira_lattice_supported": ([i32, i32, i32], i32),
    "mira_lattice_plan_chunk": ([i32, i32, i32, i32, i32], i32),
    "mira_lattice_workspace_bytes": ([i32, i32, i32, i32, i32, i32], sz),
    "mira_lattice_forward": ([p, i64, p, i64, p, i64, p, i64, p, i64, p, p, i64, p, p, p, p,
                              i32, i32, i32, i32, i32, i32, i32, i32, p, sz, p], i32),
    "mira_lattice_forward_static": ([p, i64, p, i64, p, i64, p, i64, p, i64, p, p, i64, p, p, p,
                                     p, i32, i32, i32, i32, i32, i32, i32, i32, p], i32),
    "mira_lattice_backward_chunk": ([i32, i32], i32),
    "mira_lattice_backward_workspace_bytes": ([i32, i32, i32, i32, i32], sz),
    "mira_lattice_backward": ([p, i64, p, i64, p, i64, p, i64, p, i64, p, p, i64, p, p, p,
                               p, i64, p, i64, p, i64, p, i64, p, i64, p, i64, p, i64, p, i64,
                               i32, i32, i32, i32, i32, i32, i32, p, sz, p, sz, p], i32),
    "mira_lattice_step": ([p, i64, p, i64, p, i64, p, i64, p, i64, p, p, i64, p, p, p, p,
                           i32, i32, i32, i32, i32, i32, p], i32),
    "mira_lattice_control_serves": ([i32, i32, i32, i32, i32, i32, i32], i32),
    "mira_lattice_control_forward": ([p, i64, p, p, i64, i64, p, i64, i64, i64, p, i64, p, p,
                                      i64, p, p, p, p, i32, i32, i32, i32, i32, i32, i32, i32,
                                      p], i32),
    "mira_diag_workspace_bytes": ([i32, i32, i32, i32], sz),
    "mira_diag_conv_scan": ([p, p, p, p, p, p, p, i64, p, p, i32, i32, i32, i32, i32, p, sz, p],
                            i32),
    "mira_diag_conv_step": ([p, p, p, p, p, p, i64, p, i32, i32, i32, i32, p], i32),
    "mira_diag_workspace_error": ([p, sz, ctypes.POINTER(ctypes.c_uint)], i32),
    "mira_gla_workspace_bytes": ([i32, i32, i32, i32, i32], sz),
    "mira_gla_chunked": ([p, p, p, p, p, p, p, i32, i32, i32, i32, i32, i32, p, sz, p], i32),
    "mira_gla_step": ([p, p, p, p, p, p, i32, i32, i32, i32, i32, p], i32),
    "mira_linear_silu": ([p, p, p, p, i64, i32, i32, p], i32),
}


def library():
    """The loaded library, or None (see why())."""
    global _LIB, _WHY
    with _LOCK:
        if _LIB is not None or _WHY:
            return _LIB
        path = os.environ.get("MIRA_HIP_LIBRARY", LIBRARY)
        if not os.path.exists(path):
            _WHY = (f"{path} is not built: run `python official-mira-llm_amd/build.py` "
                    f"(or __graft_entry__.build())")
            return None
        try:
            lib = ctypes.CDLL(path)
            for name, (args, result) in SIGNATURES.items():
                function = getattr(lib, name)
                function.argtypes = args
                function.restype = result
        except (OSError, AttributeError) as error:
            _WHY = f"loading {path} failed: {error}"
            return None
        expected = _source_hash()
        built = lib.mira_version().decode().rpartition("src:")[2]
        if expected is not None and built != expected:
            _WHY = (f"{path} was built from other sources (src:{built}, tree src:{expected}): "
                    f"rebuild with `python official-mira-llm_amd/build.py`")
            return None
        _LIB = lib
        return _LIB


def _source_hash():
    """The build's content hash of csrc/ and include/mira_hip.h (official-mira-llm_amd/build.py),
    or None when the sources are not beside the library."""
    import hashlib

    csrc = os.path.join(os.path.dirname(HERE), "csrc")
    header = os.path.join(os.path.dirname(os.path.dirname(HERE)), "include", "mira_hip.h")
    if not (os.path.isdir(csrc) and os.path.exists(header)):
        return None
    digest = hashlib.sha256()
    for path in sorted(os.path.join(csrc, n) for n in os.listdir(csrc)) + [header]:
        digest.update(os.path.basename(path).encode())
        with open(path, "rb") as handle:
            digest.update(handle.read())
    return digest.hexdigest()[:16]


def why():
    return _WHY


def require():
    """The library, or RuntimeError naming why it is missing (no silent fallback)."""
    lib = library()
    if lib is None:
        raise RuntimeError(f"mira_amd: the HIP library is unavailable: {why()}")
    return lib


def last_error():
    lib = library()
    return "" if lib is None else lib.mira_last_error().decode()


def check(code, what):
    """Map a C-ABI return code onto the reference plugin's conventions: DECLINE -> None,
    ERR_ARG -> ValueError, ERR_HIP -> RuntimeError (kernel/cuda/mira_dspv2/mira.py:513-519)."""
    if code == OK:
        return True
    if code == DECLINE:
        return None
    message = f"{what}: {last_error()}"
    if code == ERR_ARG:
        raise ValueError(message)
    raise RuntimeError(message)
