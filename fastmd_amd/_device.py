"""Argument checks shared by the HIP wrappers (host side, before any launch)."""
from __future__ import annotations

import torch
from torch import Tensor

from fastmd_amd import _abi


def require_cuda(*tensors: Tensor | None) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"expected a GPU tensor, got one on {t.device} (the HIP kernels have no CPU path)")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"tensors on different devices: {device} and {t.device}")
    if device is None:
        raise ValueError("no tensor given")
    _abi.load()  # raises if the native library is missing
    return device


def require_dtype(t: Tensor | None, dtype: torch.dtype, name: str) -> None:
    if t is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")


def require_contiguous(t: Tensor | None, name: str) -> None:
    if t is not None and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def rows_view(t: Tensor) -> tuple[Tensor, int]:
    """(matrix, row stride) with unit column stride; copies only when needed."""
    if t.dim() != 2:
        raise ValueError(f"expected a 2-D tensor, got shape {tuple(t.shape)}")
    rows, width = t.shape
    if (t.stride(1) != 1 and width > 1) or (rows > 1 and t.stride(0) < width):
        t = t.contiguous()
    return t, (t.stride(0) if rows > 1 else width)


def stream() -> int:
    return _abi.stream_handle()
