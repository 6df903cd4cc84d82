"""PyTorch (CPU, fp32) restatement of the reference's scoring oracles -- TEST
INFRASTRUCTURE ONLY.

This is the CPU baseline ``bench.py`` times beside the GPU path: the reference's own
PyTorch formulation, restated (the reference module is not imported). Only ``tests/``
and the ``cpu_baseline`` leg of ``bench.py`` may import it; the product path never
calls it.

Reference functions restated (paths relative to the reference checkout):

* ``pytorch_maxsim_naive`` (``src/flash_maxsim_kernel.py:280-288``): materialise
  ``S = einsum('qd,bnd->bqn', Q.float(), D.float())``, ``max`` over document tokens,
  ``sum`` over query tokens -> :func:`maxsim_naive`.
* ``pytorch_maxsim_score`` (``src/e2e_retrieval_quality.py:105-110``): the same with
  padded document tokens ``masked_fill``-ed to -inf; variable-length documents are
  padded to the chunk's longest and masked, as that scorer's callers feed it ->
  :func:`maxsim_varlen_masked`.
* ``pytorch_pqsim_baseline`` (``src/flash_pqsim_kernel.py:283-313``): decompress the
  codes to fp32 vectors one subspace at a time, then the naive MaxSim ->
  :func:`pq_decompress_score`.

Callers chunk over documents to bound the materialised similarity tensor, as the
reference's callers chunk (``src/beir_evaluation.py:202``,
``src/e2e_retrieval_quality.py:267``).

Pinning: ``tests/test_oracle.py`` checks every function here against the numpy oracle
(``oracle/maxsim_oracle.py``, itself pinned by brute force, closed forms and the C
restatement) on the same inputs.
"""
from __future__ import annotations

import torch


def maxsim_naive(Q: torch.Tensor, D: torch.Tensor, chunk: int = 500) -> torch.Tensor:
    """Q (Nq, d), D (B, Nd, d) -> (B,) fp32 MaxSim, ``chunk`` documents at a time."""
    out = torch.empty(D.shape[0], dtype=torch.float32)
    Qf = Q.float()
    for b0 in range(0, D.shape[0], chunk):
        S = torch.einsum("qd,bnd->bqn", Qf, D[b0:b0 + chunk].float())
        out[b0:b0 + chunk] = S.max(dim=-1).values.sum(dim=-1)
    return out


def maxsim_varlen_masked(Q: torch.Tensor, D_flat: torch.Tensor, offsets: torch.Tensor,
                         chunk: int = 500) -> torch.Tensor:
    """Documents D_flat[offsets[b]:offsets[b+1]] (every one non-empty): each chunk is
    padded to its longest document, the padding masked to -inf before the max."""
    B = offsets.numel() - 1
    out = torch.empty(B, dtype=torch.float32)
    Qf = Q.float()
    d = D_flat.shape[1]
    for b0 in range(0, B, chunk):
        b1 = min(B, b0 + chunk)
        lens = offsets[b0 + 1:b1 + 1] - offsets[b0:b1]
        L = int(lens.max())
        pad = torch.zeros(b1 - b0, L, d, dtype=torch.float32)
        mask = torch.arange(L)[None, :] < lens[:, None]
        pad[mask] = D_flat[int(offsets[b0]):int(offsets[b1])].float()
        S = torch.einsum("qd,bnd->bqn", Qf, pad)
        S = S.masked_fill(~mask.unsqueeze(1), float("-inf"))
        out[b0:b1] = S.max(dim=-1).values.sum(dim=-1)
    return out


def pq_decompress_score(Q: torch.Tensor, codebook: torch.Tensor, codes: torch.Tensor,
                        chunk: int = 500) -> torch.Tensor:
    """Q (Nq, d), codebook (M, K, dsub), codes (B, Nd, M) -> (B,) fp32 scores of the
    decompressed documents."""
    M, K, dsub = codebook.shape
    B, Nd, _ = codes.shape
    out = torch.empty(B, dtype=torch.float32)
    Qf = Q.float()
    for b0 in range(0, B, chunk):
        c = codes[b0:b0 + chunk]
        Dc = torch.zeros(c.shape[0], Nd, M * dsub, dtype=torch.float32)
        for m in range(M):
            Dc[:, :, m * dsub:(m + 1) * dsub] = codebook[m][c[:, :, m].long()].float()
        S = torch.einsum("qd,bnd->bqn", Qf, Dc)
        out[b0:b0 + chunk] = S.max(dim=-1).values.sum(dim=-1)
    return out
