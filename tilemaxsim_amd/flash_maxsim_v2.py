"""Fused dense MaxSim -- drop-in for the reference module ``src/flash_maxsim_v2.py``.

``flash_maxsim_v2_multiquery(Q, D)`` and ``flash_maxsim_v2(Q, D)`` keep the reference
signatures and return values; both run the gfx950 HIP kernel behind
``tms_maxsim_dense`` (``include/tilemaxsim.h``), which covers every embedding width
(the reference's d <= 128 kernel and its d-tiled kernel for d > 128).
"""
from __future__ import annotations

import torch

from . import _check, _lib


def _dense(Q: torch.Tensor, D: torch.Tensor, fn: str) -> torch.Tensor:
    _check.tensor("Q", Q)
    _check.tensor("D", D)
    if D.dim() != 3:
        raise ValueError(f"{fn}: D must be (B, Nd, d), got shape {tuple(D.shape)}")
    if Q.dim() != 2:
        raise ValueError(f"{fn}: Q must be (Nq, d), got shape {tuple(Q.shape)}")
    B, Nd, d = D.shape
    Nq = Q.shape[0]
    assert Q.shape[1] == d, f"{fn}: Q width {Q.shape[1]} != D width {d}"
    _check.embedding_dtype("D", D)
    _check.contiguous("D", D)
    _check.on_gpu("Q", Q)
    _check.on_gpu("D", D)
    _check.same_device(Q=Q, D=D)
    Q, code = _check.query_for(Q, D.dtype)
    scores = torch.empty(B, dtype=torch.float32, device=Q.device)
    if B == 0:
        return scores
    lib = _lib.load()
    with _lib.on_device(Q.device):
        _lib.check(lib.tms_maxsim_dense(Q.data_ptr(), Nq, d, D.data_ptr(), B, Nd, code, scores.data_ptr(),
                                        _lib.stream_of(Q)))
    return scores


def flash_maxsim_v2_multiquery(Q: torch.Tensor, D: torch.Tensor) -> torch.Tensor:
    """Fused MaxSim of one query against a batch of fixed-length documents.

    Drop-in for ``flash_maxsim_v2_multiquery`` (``src/flash_maxsim_v2.py:227-289``):
    ``scores[b] = sum_i max_j Q[i] . D[b, j]`` with fp32 accumulation. Unlike the
    reference, every d is accepted (the reference needs a power of two for d <= 128),
    D is read once for any Nq (the reference re-reads it per block of 32 query tokens
    and combines blocks with float atomics), and the result is deterministic.

    Args:
        Q: (Nq, d) query token embeddings. A query of another float dtype than D is
            scored at fp32 precision (split into two 16-bit terms against fp16 / bf16
            documents, never rounded to D's dtype).
        D: (B, Nd, d) document token embeddings, float16, bfloat16 or float32,
            contiguous (float32 is computed as bf16 hi + lo terms, relative error per
            product below 1e-4; the reference computes float32 with TF32 products).

    Returns:
        (B,) float32 scores on Q's device. A document with Nd == 0 scores -inf.
    """
    return _dense(Q, D, "flash_maxsim_v2_multiquery")


def flash_maxsim_v2(Q: torch.Tensor, D: torch.Tensor) -> torch.Tensor:
    """Drop-in for ``flash_maxsim_v2`` (``src/flash_maxsim_v2.py:193-224``).

    The reference runs a one-program-per-document VALU kernel; the scores are the
    same MaxSim, so this shares the MFMA kernel of :func:`flash_maxsim_v2_multiquery`.
    """
    return _dense(Q, D, "flash_maxsim_v2")


def flash_maxsim_batched_queries(Qs: torch.Tensor, D: torch.Tensor) -> torch.Tensor:
    """Score ``nQ`` queries against the same documents: ``Qs`` (nQ, Nq, d) -> (nQ, B).

    Equivalent to stacking ``flash_maxsim_v2_multiquery(Qs[i], D)`` over i, but two
    blocks of 32 query tokens share each pass over D. No reference counterpart.
    """
    _check.tensor("Qs", Qs)
    _check.tensor("D", D)
    if D.dim() != 3 or Qs.dim() != 3:
        raise ValueError("flash_maxsim_batched_queries: Qs must be (nQ, Nq, d) and D (B, Nd, d)")
    B, Nd, d = D.shape
    nQ, Nq, dq = Qs.shape
    assert dq == d, f"flash_maxsim_batched_queries: Q width {dq} != D width {d}"
    _check.embedding_dtype("D", D)
    _check.contiguous("D", D)
    _check.on_gpu("Qs", Qs)
    _check.on_gpu("D", D)
    _check.same_device(Qs=Qs, D=D)
    Qs, code = _check.query_for(Qs, D.dtype)
    out = torch.empty(nQ, B, dtype=torch.float32, device=Qs.device)
    if B == 0 or nQ == 0:
        return out
    lib = _lib.load()
    with _lib.on_device(Qs.device):
        _lib.check(lib.tms_maxsim_dense_batched(Qs.data_ptr(), nQ, Nq, d, D.data_ptr(), B, Nd, code, out.data_ptr(),
                                                _lib.stream_of(Qs)))
    return out
