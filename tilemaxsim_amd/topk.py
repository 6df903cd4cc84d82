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


_SCRATCH: dict = {}
# Documents' tokens (B x Nd) up to which one launch beats scoring, then ranking, for an
# eager call. The launch pays a device-scope ticket and an L2 write-back per workgroup
# (at most 256 of them) and ranks after the last one, so it saves the second call's host
# cost (about 10 us) while the GPU time stays below it. Measured on MI355X (32-token
# query, d = 128): every shape up to 160K tokens wins (1,000 x 128: 16.1 us against
# 19.3; 512 x 300: 17.2 against 19.5); 1,000 x 180 (180K) loses by 0.8 us and longer
# calls by 1-3 us. A HIP graph replays two launches without host cost, where one launch
# never wins by more than noise: captured calls take the two kernels.
ONE_LAUNCH_MAX_TOKENS = 160 * 1024


def _one_launch_workgroups(B: int, nd: int, d: int = 128, nq: int = 32) -> int:
    """Workgroups of tms_maxsim_topk's launch: 1, 2 or 4 waves per document (enough for
    about 2,048 waves, at most one per 16-token tile); 4, 8 or 16 waves a workgroup, the
    fewest that keep the launch within 256 workgroups (at most 8 at d = 128 with two
    32-token query blocks)."""
    tiles, wpd = (nd + 15) // 16, 1
    while wpd < 4 and B * wpd < 2048 and 2 * wpd <= tiles:
        wpd *= 2
    waves = B * wpd
    per = 4 if waves <= 1024 else (8 if waves <= 2048 else 16)
    if d == 128 and nq > 32:
        per = min(per, 8)
    return (waves + per - 1) // per


def _scratch(dev: torch.device, stream: int) -> tuple[int, int]:
    """Device addresses of the one-launch path's ticket counters and its B <= 1,024 scores,
    one buffer per device and stream: a launch leaves the counters zero and uses the
    scores only within itself, and launches on one stream never overlap."""
    key = (dev.index, stream)
    c = _SCRATCH.get(key)
    if c is None:
        words = _lib.TMS_MAXSIM_TOPK_COUNTER_WORDS
        # counters, then the scores; setdefault keeps one buffer when two threads race here
        c = _SCRATCH.setdefault(key, torch.zeros(words + 1024, dtype=torch.int32, device=dev))
    p = c.data_ptr()
    return p, p + 4 * _lib.TMS_MAXSIM_TOPK_COUNTER_WORDS


def _one_launch(Q: torch.Tensor, D: torch.Tensor, k: int):
    """``tms_maxsim_topk`` for the eager calls it takes (one query of at most 64 fp16 /
    bf16 tokens, d in {32, 64, 96, 128}, 1..1,024 contiguous documents, 1 <= k <= B,
    16-byte aligned, at most ONE_LAUNCH_MAX_TOKENS document tokens); None otherwise (the
    caller scores, then ranks)."""
    if not (isinstance(Q, torch.Tensor) and isinstance(D, torch.Tensor) and Q.dim() == 2 and D.dim() == 3):
        return None
    B, Nd, d = D.shape
    # the size checks first: a call beyond them costs the two-kernel path nothing more
    if not 1 <= B <= 1024 or not 1 <= k <= B or B * Nd > ONE_LAUNCH_MAX_TOKENS:
        return None
    Nq = Q.shape[0]
    if (d not in (32, 64, 96, 128) or not 1 <= Nq <= 64 or Q.shape[1] != d
            or D.dtype not in (torch.float16, torch.bfloat16) or not D.is_cuda or not D.is_contiguous()
            or Q.device != D.device or torch.cuda.is_current_stream_capturing()):
        return None
    Q2, code = _check.query_for(Q, D.dtype)
    if code not in (_lib.TMS_DTYPE_F16, _lib.TMS_DTYPE_BF16) or Q2.data_ptr() % 16 or D.data_ptr() % 16:
        return None
    vals = torch.empty(k, dtype=torch.float32, device=D.device)
    idx = torch.empty(k, dtype=torch.int64, device=D.device)
    lib = _lib.load()
    with _lib.on_device(D.device):
        stream = _lib.stream_of(D)
        counter, scores = _scratch(D.device, stream)
        _lib.check(lib.tms_maxsim_topk(Q2.data_ptr(), Nq, d, D.data_ptr(), B, Nd, code, k, scores, vals.data_ptr(),
                                       idx.data_ptr(), counter, stream))
    return vals, idx


def maxsim_topk(Q: torch.Tensor, D: torch.Tensor, k: int):
    """Score ``Q`` against ``D`` (B, Nd, d) and return the top-``k`` documents.

    ``Q`` (Nq, d) gives ``(values (k,), indices (k,))``; ``Q`` (nQ, Nq, d) scores every
    query in shared passes over ``D`` and gives (nQ, k) results. An eager reranking call
    (one query against a few hundred documents) scores and ranks in one launch
    (``tms_maxsim_topk``), with the same bits as scoring and then ranking.
    """
    if Q.dim() == 3:
        return topk(flash_maxsim_batched_queries(Q, D), k)
    one = _one_launch(Q, D, int(k))
    if one is not None:
        return one
    return topk(flash_maxsim_v2_multiquery(Q, D), k)
