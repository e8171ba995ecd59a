"""Which device the Mira mixer runs on: the interface of kernel/hardware.py (resolve :15-29,
accelerator :32-40, count :43-45) with one accelerator, the gfx950 HIP library.

ROCm builds of PyTorch name the HIP device type "cuda", so "cuda" here means the MI355X. The
reference also probes Ascend NPUs and Apple MPS; neither exists on this path, so an explicit
request for a HIP device that is not there is an error, and "auto" settles on the CPU only when
no GPU is visible (the scan itself never runs on the CPU: the plugin declines there).
"""
from __future__ import annotations

import os

import torch

HIP_TYPE = "cuda"            # torch's device type for HIP devices on ROCm
AUTO = ("auto", HIP_TYPE)


def _hip_visible() -> bool:
    return bool(torch.cuda.is_available())


def resolve(choice="auto") -> torch.device:
    """The torch.device a setting such as the GPU environment variable names: "auto" is the HIP
    device when one is visible, else the CPU; "cuda" insists on the HIP device; anything else
    ("cpu", "cuda:1", ...) is passed to torch.device as given."""
    name = str(choice)
    if name not in AUTO:
        return torch.device(name)
    if _hip_visible():
        return torch.device(HIP_TYPE)
    if name == HIP_TYPE:
        raise RuntimeError(f"GPU={name!r} asks for the HIP device, but torch sees no HIP GPU "
                           f"(torch {torch.__version__}, HIP {torch.version.hip})")
    return torch.device("cpu")


def accelerator(device=None):
    """The torch device module (torch.cuda, which drives HIP here) for `device`, or None for a
    device with no accelerator module. Without an argument the GPU environment variable
    (default "auto") decides."""
    target = resolve(os.environ.get("GPU", "auto")) if device is None else torch.device(device)
    return torch.cuda if target.type == HIP_TYPE else None


def count(choice="auto") -> int:
    """Devices available to `choice`: the visible HIP devices, or 1 for the CPU."""
    module = accelerator(resolve(choice))
    return 1 if module is None else int(module.device_count())
