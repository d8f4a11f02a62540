"""Argument validation shared by the decode and prefill entry points.

The reference entry points validate nothing (kernel.cu:982-1064, kernel.py:56-91);
here every tensor is checked before any launch so that a bad argument raises a
Python exception instead of reaching a kernel.
"""

from __future__ import annotations

import torch


def as_tensor(x, name: str):
    """torch tensors pass through; DLPack producers (e.g. tvm_ffi) are converted."""
    if x is None or isinstance(x, torch.Tensor):
        return x
    if hasattr(x, "__dlpack__"):
        return torch.from_dlpack(x)
    raise TypeError(f"{name}: expected a tensor, got {type(x).__name__}")


def check_tensor(t, name: str, dtype, shape, device) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected dtype {dtype}, got {t.dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}")
    if t.device != device:
        raise ValueError(f"{name}: expected device {device}, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")


def check_device(t, name: str) -> torch.device:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: the MI355X kernels need a GPU tensor, got device {t.device}")
    return t.device


def resolve_scale(scale, head_dim: int) -> float:
    """None or 0 selects 1/sqrt(head_dim), as the reference does."""
    if scale is None:
        return head_dim ** -0.5
    if isinstance(scale, torch.Tensor):
        scale = float(scale.item())
    scale = float(scale)
    if scale == 0.0:
        return head_dim ** -0.5
    return scale


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()
