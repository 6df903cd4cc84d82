"""Top-k retrieval on the GPU: the per-query top-100 the reference takes with
``torch.topk(scores, k)`` after scoring (``src/cycle3_experiments.py:215``), here a HIP
kernel (``tms_topk``), plus ``maxsim_topk`` which scores and selects in one call.

Order: values descending; equal values by ascending index (deterministic, where
``torch.topk`` leaves ties unspecified); NaN ranks above +inf, as in ``torch.topk``.
"""
from __future__ import annotations

import functools

import torch

from . import _check, _lib
from .flash_maxsim_v2 import flash_maxsim_batched_queries, flash_maxsim_v2_multiquery

MAX_K = 1024


@functools.lru_cache(maxsize=256)
def _workspace_bytes(rows: int, n: int, k: int) -> int:
    return int(_lib.load().tms_topk_workspace_size(rows, n, k))


def topk(scores: torch.Tensor, k: int):
    """Largest ``k`` entries along the last dimension of a 1-D or 2-D fp32 score tensor.

    Returns ``(values, indices)`` shaped like ``torch.topk(scores, k)``: (k,) or (rows, k),
    float32 and int64.
    """
    _check.tensor("scores", scores)
    if scores.dim() not in (1, 2):
        raise ValueError(f"scores must be 1-D or 2-D, got shape {tuple(scores.shape)}")
    if scores.dtype != torch.float32:
        raise TypeError(f"scores must be float32, got {scores.dtype}")
    k = int(k)
    n = scores.shape[-1]
    if k < 0 or k > n:
        raise ValueError(f"k={k} out of range for rows of length {n}")
    if k > MAX_K:
        raise NotImplementedError(f"k={k} > {MAX_K} is not supported")
    _check.on_gpu("scores", scores)
    s2 = scores.reshape(1, n) if scores.dim() == 1 else scores
    s2 = s2.contiguous()
    rows = s2.shape[0]
    vals = torch.empty(rows, k, dtype=torch.float32, device=s2.device)
    idx = torch.empty(rows, k, dtype=torch.int64, device=s2.device)
    if rows > 0 and k > 0:
        lib = _lib.load()
        per_call = min(rows, 65535)  # grid-y limit per call
        ws_bytes = _workspace_bytes(per_call, n, k)
        # rows that fit one chunk need no workspace (the C entry point takes NULL then)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=s2.device) if ws_bytes > 0 else None
        ws_ptr = ws.data_ptr() if ws is not None else None
        with _lib.on_device(s2.device):
            stream = _lib.stream_of(s2)
            if rows == per_call:
                _lib.check(lib.tms_topk(s2.data_ptr(), rows, n, k, ws_ptr, ws_bytes, vals.data_ptr(),
                                        idx.data_ptr(), stream))
            else:
                for r0 in range(0, rows, per_call):
                    r1 = min(rows, r0 + per_call)
                    _lib.check(lib.tms_topk(s2[r0:r1].data_ptr(), r1 - r0, n, k, ws_ptr, ws_bytes,
                                            vals[r0:r1].data_ptr(), idx[r0:r1].data_ptr(), stream))
    if scores.dim() == 1:
        return vals[0], idx[0]
    return vals, idx


def maxsim_topk(Q: torch.Tensor, D: torch.Tensor, k: int):
    """Score ``Q`` against ``D`` (B, Nd, d) and return the top-``k`` documents.

    ``Q`` (Nq, d) gives ``(values (k,), indices (k,))``; ``Q`` (nQ, Nq, d) scores every
    query in shared passes over ``D`` and gives (nQ, k) results.
    """
    if Q.dim() == 3:
        return topk(flash_maxsim_batched_queries(Q, D), k)
    return topk(flash_maxsim_v2_multiquery(Q, D), k)
