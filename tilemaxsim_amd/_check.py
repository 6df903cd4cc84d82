"""Argument checks shared by the host entry points.

Every check runs before any HIP call. Shape, dtype and layout checks come before the
device check, so each error is raised the same way on a machine without a GPU.
"""
from __future__ import annotations

import torch

from . import _lib


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


def query_for(Q: torch.Tensor, dtype: torch.dtype) -> tuple[torch.Tensor, int]:
    """The query as the kernels take it against documents (or a codebook) of ``dtype``,
    and the C dtype code to pass with it.

    A query of the documents' dtype is used as it is. Against fp32 documents any float
    query becomes fp32. Against fp16 / bf16 documents a query of another float dtype
    becomes fp32 (exactly, for a 16-bit query) and the code carries ``TMS_QUERY_F32``:
    the kernels then split each element into two 16-bit terms instead of rounding it to
    the documents' type, as the reference computes such a pair in fp32 / TF32
    (``src/flash_maxsim_v2.py:99,111,117``).
    """
    if not Q.is_floating_point():
        raise TypeError(f"Q must be a floating-point tensor (got {Q.dtype})")
    code = _lib.dtype_code(dtype)
    if Q.dtype == dtype:
        return Q.contiguous(), code
    Qf = Q.to(torch.float32).contiguous()
    if dtype == torch.float32:
        return Qf, code
    return Qf, code | _lib.TMS_QUERY_F32
