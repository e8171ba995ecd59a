"""Shared helpers for the parity tests: device transfer and the error metrics the reference
harness uses (kernel/cuda/mira_dspv2/check.py:36-39)."""
from __future__ import annotations

import glob
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")

# fp32: the north-star bound (max abs error <= 1e-5) and the reference harness's scaled bound
# (check.py:92); bf16/f16: <= 2e-2 relative to the largest reference magnitude.
FP32_ABS = 1e-5
FP32_SCALED = 3e-4
HALF_SCALED = 2e-2


def scaled(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    error = np.abs(got - ref).max() if got.size else 0.0
    return error / scale if scale > 0 else (0.0 if error == 0 else float("inf"))


def max_abs(got, ref):
    return float(np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64)).max())


def golden_files(prefix=""):
    return sorted(glob.glob(os.path.join(GOLDEN, f"{prefix}*.npz")))


def to_device(array, dtype=None, device="cuda"):
    import torch

    if array is None:
        return None
    tensor = torch.from_numpy(np.ascontiguousarray(array))
    if dtype is not None:
        tensor = tensor.to(dtype)
    return tensor.to(device)


def to_numpy(tensor):
    return tensor.detach().float().cpu().numpy()


def rounded(array, torch_dtype):
    """`array` rounded to torch_dtype and back to float32 (the inputs the kernel actually sees)."""
    import torch

    return torch.from_numpy(np.ascontiguousarray(array, np.float32)).to(torch_dtype).float().numpy()
