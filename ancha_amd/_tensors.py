"""Argument checks of the host mirror: every tensor handed to the C ABI must be device memory of
the expected dtype, on the expected device and of the expected size, because the kernels read
exactly the bytes the shape arguments describe. A mismatch raises ``ValueError`` before any
launch (the reference's ``assert!`` panics inside ``launch``, fused/attention.rs:262-269,
fused/gemm.rs:249-264): a host pointer or a short buffer handed to a kernel would fault the
GPU instead.
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch


def _index(device: torch.device) -> int:
    d = torch.device(device)
    return d.index if d.index is not None else torch.cuda.current_device()


def require(t: torch.Tensor, name: str, device: torch.device,
            shape: Optional[Sequence[int]] = None, dtype: torch.dtype = torch.float32) -> None:
    """Raise ValueError unless ``t`` is a ``dtype`` tensor on ``device`` (and of ``shape``)."""
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_cuda or torch.device(device).type != "cuda" or t.device.index != _index(device):
        raise ValueError(f"{name} must be on {device}, got {t.device}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


def require_optional(t: Optional[torch.Tensor], name: str, device: torch.device,
                     shape: Optional[Sequence[int]] = None) -> None:
    if t is not None:
        require(t, name, device, shape)
