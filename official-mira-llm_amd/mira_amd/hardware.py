"""Device selection for the Mira mixer (kernel/hardware.py:1-52), HIP only.

On ROCm PyTorch the HIP device type is "cuda". The reference walks cuda -> npu -> mps -> cpu
(kernel/hardware.py:15-29); this build has one accelerator path, the gfx950 HIP library, so
`resolve` returns the HIP device when one is visible and the CPU otherwise, and `accelerator`
returns torch.cuda (HIP) or None. The mixer itself never runs the scan on the CPU.
"""
from __future__ import annotations

import os
import sys

import torch


def resolve(choice="auto"):
    """torch.device for `choice` ("auto", "cuda", "cuda:N", "cpu"). "cuda" without a visible
    HIP device raises, as the reference does (kernel/hardware.py:21-23)."""
    choice = str(choice)
    if choice in ("auto", "cuda"):
        if torch.cuda.is_available():
            return torch.device("cuda")
        if choice == "cuda":
            raise RuntimeError("no HIP accelerator is available")
        return torch.device("cpu")
    return torch.device(choice)


def accelerator(device=None):
    kind = resolve(os.environ.get("GPU", "auto")).type if device is None else torch.device(device).type
    return torch.cuda if kind == "cuda" else None


def count(choice="auto"):
    backend = accelerator(resolve(choice))
    return backend.device_count() if backend is not None else 1


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "count":
        print(count(sys.argv[2] if len(sys.argv) > 2 else "auto"))
    else:
        print(resolve(sys.argv[1] if len(sys.argv) > 1 else "auto").type)
