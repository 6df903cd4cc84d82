"""Argument checks shared by the host entry points.

Every check runs before any HIP call. Shape, dtype and layout checks come before the
device check, so each error is raised the same way on a machine without a GPU.
"""
from __future__ import annotations

import torch


def tensor(name: str, t) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")


def on_gpu(name: str, t: torch.Tensor) -> None:
    tensor(name, t)
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a ROCm GPU device (got {t.device}); tilemaxsim_amd has no CPU path")


def same_device(**tensors: torch.Tensor) -> torch.device:
    devs = {name: t.device for name, t in tensors.items()}
    first = next(iter(devs.values()))
    for name, dev in devs.items():
        if dev != first:
            raise ValueError(f"all inputs must be on one device; {name} is on {dev}, expected {first}")
    return first


def embedding_dtype(name: str, t: torch.Tensor) -> None:
    if t.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"{name} must be float16, bfloat16 or float32 (got {t.dtype})")


def contiguous(name: str, t: torch.Tensor) -> None:
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous (row-major); call .contiguous() first")


def query_like(Q: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Queries are small: cast to the document dtype and make them contiguous on device."""
    if not Q.is_floating_point():
        raise TypeError(f"Q must be a floating-point tensor (got {Q.dtype})")
    if Q.dtype != dtype:
        Q = Q.to(dtype)
    return Q.contiguous()
