"""CPU oracle for the fused MaxSim / PQ-ADC scoring path -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the reference PyTorch computations that define what
the MaxSim scoring path must return. It is the checker for the HIP kernels in
``tilemaxsim_amd``: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it. The product path never calls it
and has no CPU fallback.

Reference files followed (paths relative to the reference checkout):

* ``src/flash_maxsim_kernel.py:280-288`` ``pytorch_maxsim_naive``: materialise
  ``S = einsum('qd,bnd->bqn', Q.float(), D.float())``, then ``max`` over doc tokens,
  ``sum`` over query tokens -> :func:`maxsim_naive` (fp32) and :func:`maxsim_f64`.
* ``src/flash_maxsim_kernel.py:291-303`` ``pytorch_maxsim_loop`` -> :func:`maxsim_loop`.
* ``src/flash_maxsim_v2.py:96-130,161-190`` kernel masking rules: invalid doc rows are
  -inf before the max (so a document with no tokens scores -inf), invalid query rows
  contribute 0 -> the ``Nd == 0`` handling in every dense function.
* ``src/e2e_retrieval_quality.py:105-110`` ``pytorch_maxsim_score`` (``masked_fill``
  with -inf of padded doc tokens) -> :func:`maxsim_masked`.
* ``src/flash_maxsim_kernel.py:248-273`` ``flash_maxsim_multi_doc`` (each document is
  scored over exactly ``D_flat[offsets[i]:offsets[i+1]]``) -> :func:`maxsim_varlen`.
* ``src/plaid_integration_benchmark.py:154-183`` ``flashmaxsim_score_packed`` (pad the
  packed documents, zero the padding, dense MaxSim) -> :func:`maxsim_packed_zero_padded`.
* ``src/flash_pqsim_kernel.py:31-67`` distance table ``T[q,m,k] = sum_j
  Q[q,m*dsub+j] * C[m,k,j]`` in fp32 -> :func:`pq_build_lut`.
* ``src/flash_pqsim_kernel.py:127-173`` + ``:250`` table gather, fp32 sum over ``m`` in
  ascending order, max over doc tokens, then ``sum`` over query tokens ->
  :func:`pq_score_lut`.
* ``src/flash_pqsim_kernel.py:283-313`` ``pytorch_pqsim_baseline`` (decompress the
  codes into fp32 vectors, then the naive MaxSim) -> :func:`pq_decompress_score`.

Pinning (what checks each function against something other than itself; the checks
live in ``tests/test_oracle.py``):

* dense / masked / varlen: pure-Python float64 brute force on tiny inputs, the
  closed forms ``Nq = Nd = 1`` (one dot product) and "documents that contain the
  normalised query tokens score ``Nq``", permutation / duplication / zero-padding /
  positive-scaling invariants, and the independent C restatement in
  ``oracle/maxsim_oracle.c`` (float64 loops) at mid sizes;
* PQ: the LUT equals a textbook per-subspace GEMM computed by brute force; LUT-gather
  scoring equals decompress-then-score (two different algorithms); ``K = 1`` reduces
  to dense MaxSim against a single fixed vector.

The reference ships no input/output vectors (its self-tests draw from the CUDA RNG),
so the golden fixtures under ``tests/golden/`` are generated from this module by
``tests/golden/make_golden.py`` after the checks above pass.
"""
from __future__ import annotations

import numpy as np

NEG_INF = np.float32(-np.inf)


def _as_f32(x: np.ndarray) -> np.ndarray:
    return np.asarray(x).astype(np.float32, copy=False)


def _dense_scores_from_sim(S: np.ndarray) -> np.ndarray:
    """``S`` is (B, Nd, Nq); returns max over Nd then sum over Nq (dtype of S).

    Nd == 0 gives -inf, as the reference kernels' running max starts at -inf
    (``src/flash_maxsim_v2.py:102``) and no tile updates it.
    """
    B, Nd, Nq = S.shape
    if Nd == 0:
        if Nq == 0:
            return np.zeros(B, dtype=S.dtype)
        return np.full(B, -np.inf, dtype=S.dtype)
    return S.max(axis=1).sum(axis=1, dtype=S.dtype)


def maxsim_naive(Q: np.ndarray, D: np.ndarray, chunk: int = 4096) -> np.ndarray:
    """fp32 materialise-then-reduce MaxSim (``src/flash_maxsim_kernel.py:280-288``).

    Q: (Nq, d); D: (B, Nd, d). Inputs are cast to fp32 (fp16 products are exact in
    fp32); the similarity block for ``chunk`` documents is materialised at a time, as
    the reference's callers chunk (``src/beir_evaluation.py:202``).
    Returns fp32 (B,).
    """
    Qf = _as_f32(Q)
    B, Nd, d = D.shape
    assert Qf.shape[1] == d
    out = np.empty(B, dtype=np.float32)
    QT = np.ascontiguousarray(Qf.T)
    for s in range(0, B, chunk):
        e = min(B, s + chunk)
        Dc = _as_f32(D[s:e]).reshape((e - s) * Nd, d)
        S = (Dc @ QT).reshape(e - s, Nd, Qf.shape[0])
        out[s:e] = _dense_scores_from_sim(S)
    return out


def maxsim_f64(Q: np.ndarray, D: np.ndarray, chunk: int = 2048) -> np.ndarray:
    """Same math as :func:`maxsim_naive` accumulated in float64 (high-precision oracle)."""
    Qd = np.asarray(Q, dtype=np.float64)
    B, Nd, d = D.shape
    out = np.empty(B, dtype=np.float64)
    QT = np.ascontiguousarray(Qd.T)
    for s in range(0, B, chunk):
        e = min(B, s + chunk)
        Dc = np.asarray(D[s:e], dtype=np.float64).reshape((e - s) * Nd, d)
        S = (Dc @ QT).reshape(e - s, Nd, Qd.shape[0])
        out[s:e] = _dense_scores_from_sim(S)
    return out


def maxsim_loop(Q: np.ndarray, D: np.ndarray) -> np.ndarray:
    """Loop over query tokens, adding each token's max into fp32 scores
    (``src/flash_maxsim_kernel.py:291-303``)."""
    Qf = _as_f32(Q)
    Df = _as_f32(D)
    B, Nd, d = Df.shape
    scores = np.zeros(B, dtype=np.float32)
    for i in range(Qf.shape[0]):
        sims = Df @ Qf[i]  # (B, Nd)
        scores += sims.max(axis=-1) if Nd else np.float32(-np.inf)
    return scores


def maxsim_masked(Q: np.ndarray, D: np.ndarray, D_mask: np.ndarray, f64: bool = False) -> np.ndarray:
    """Masked MaxSim: doc tokens with ``D_mask == False`` are -inf before the max
    (``src/e2e_retrieval_quality.py:105-110``). A document with no valid token
    scores -inf (when Nq > 0)."""
    dt = np.float64 if f64 else np.float32
    Qx = np.asarray(Q, dtype=dt)
    Dx = np.asarray(D, dtype=dt)
    B, Nd, d = Dx.shape
    S = np.einsum("bnd,qd->bnq", Dx, Qx)
    S = np.where(np.asarray(D_mask, dtype=bool)[:, :, None], S, -np.inf).astype(dt)
    return _dense_scores_from_sim(S)


def maxsim_varlen(Q: np.ndarray, D_flat: np.ndarray, offsets: np.ndarray, f64: bool = False) -> np.ndarray:
    """Variable-length MaxSim (``src/flash_maxsim_kernel.py:248-273``): document i
    is ``D_flat[offsets[i]:offsets[i+1]]``; an empty document scores -inf (the
    per-doc kernel's running max stays -inf, ``src/flash_maxsim_kernel.py:48,56``).

    Vectorised as one (T, Nq) similarity block plus a segmented max (``np.maximum
    .reduceat``), which is exact for a max."""
    dt = np.float64 if f64 else np.float32
    Qx = np.asarray(Q, dtype=dt)
    offsets = np.asarray(offsets, dtype=np.int64)
    B = offsets.shape[0] - 1
    Nq = Qx.shape[0]
    out = np.full(B, -np.inf if Nq else 0.0, dtype=dt)
    if B <= 0:
        return out[:0] if B < 0 else out
    lens = offsets[1:] - offsets[:-1]
    nonempty = np.nonzero(lens > 0)[0]
    if nonempty.size == 0 or Nq == 0:
        return out
    t0, t1 = int(offsets[0]), int(offsets[-1])
    S = np.asarray(D_flat[t0:t1], dtype=dt) @ Qx.T  # (T, Nq)
    starts = offsets[nonempty] - t0
    mx = np.maximum.reduceat(S, starts, axis=0)  # segment [starts[i], starts[i+1]) -> but trailing
    # reduceat's last segment runs to the end of S; trim it to the true doc end.
    last = nonempty[-1]
    mx[-1] = S[offsets[last] - t0: offsets[last + 1] - t0].max(axis=0)
    # a non-last segment ends at the next nonempty doc's start, which equals its own end
    # because the empty docs between them contribute no tokens.
    out[nonempty] = mx.sum(axis=1, dtype=dt)
    return out


def maxsim_packed_zero_padded(Q: np.ndarray, D_packed: np.ndarray, lengths: np.ndarray) -> np.ndarray:
    """The reference's PLAID drop-in (``src/plaid_integration_benchmark.py:160-183``):
    pad the packed documents to (B, max_len, d), multiply the padding by zero
    (``D_padded * D_mask``), then the plain MaxSim of ``flash_maxsim_v2_multiquery``.
    Computed literally (a materialised padded tensor), float64."""
    lengths = np.asarray(lengths, dtype=np.int64)
    B = lengths.shape[0]
    d = D_packed.shape[1]
    max_len = int(lengths.max()) if B else 0
    padded = np.zeros((B, max_len, d), dtype=np.float64)
    start = 0
    for b in range(B):
        padded[b, : lengths[b]] = np.asarray(D_packed[start: start + lengths[b]], dtype=np.float64)
        start += lengths[b]
    return maxsim_f64(Q, padded)


def pq_build_lut(Q: np.ndarray, codebook: np.ndarray) -> np.ndarray:
    """Distance table ``T[q,m,k] = sum_j Q[q, m*dsub+j] * C[m,k,j]`` in fp32
    (``src/flash_pqsim_kernel.py:31-67``). Q: (Nq, M*dsub); codebook (M, K, dsub).
    Returns fp32 (Nq, M, K)."""
    M, K, dsub = codebook.shape
    Qf = _as_f32(Q).reshape(Q.shape[0], M, dsub)
    C = _as_f32(codebook)
    return np.einsum("qmj,mkj->qmk", Qf, C).astype(np.float32)


def pq_score_lut(T: np.ndarray, codes: np.ndarray, chunk: int = 1024) -> np.ndarray:
    """PQ MaxSim by table gather (``src/flash_pqsim_kernel.py:127-173`` and ``:250``):
    ``scores[b] = sum_q max_t sum_{m ascending} T[q, m, codes[b,t,m]]`` in fp32.
    T: (Nq, M, K) fp32; codes: (B, Nd, M) integer. Returns fp32 (B,)."""
    Nq, M, K = T.shape
    B, Nd, Mc = codes.shape
    assert Mc == M
    T = _as_f32(T)
    out = np.empty(B, dtype=np.float32)
    for s in range(0, B, chunk):
        e = min(B, s + chunk)
        c = np.asarray(codes[s:e], dtype=np.int64)  # (b, Nd, M)
        acc = np.zeros((e - s, Nd, Nq), dtype=np.float32)
        for m in range(M):  # ascending m, fp32 adds, as the kernel's inner loop
            acc += T[:, m, :].T[c[:, :, m]]
        out[s:e] = _dense_scores_from_sim(acc)
    return out


def pq_decompress(codebook: np.ndarray, codes: np.ndarray, dtype=np.float32) -> np.ndarray:
    """Decompress (B, Nd, M) codes into (B, Nd, M*dsub) vectors by gathering codebook
    rows per subspace (``src/flash_pqsim_kernel.py:300-309``)."""
    M, K, dsub = codebook.shape
    B, Nd, _ = codes.shape
    C = np.asarray(codebook, dtype=dtype)
    c = np.asarray(codes, dtype=np.int64)
    out = np.empty((B, Nd, M * dsub), dtype=dtype)
    for m in range(M):
        out[:, :, m * dsub:(m + 1) * dsub] = C[m][c[:, :, m]]
    return out


def pq_decompress_score(Q: np.ndarray, codebook: np.ndarray, codes: np.ndarray, f64: bool = False,
                        chunk: int = 1024) -> np.ndarray:
    """Decompress-then-score PQ baseline (``src/flash_pqsim_kernel.py:283-313``)."""
    B = codes.shape[0]
    dt = np.float64 if f64 else np.float32
    out = np.empty(B, dtype=dt)
    for s in range(0, B, chunk):
        e = min(B, s + chunk)
        Dap = pq_decompress(codebook, codes[s:e], dtype=dt)
        out[s:e] = maxsim_f64(Q, Dap) if f64 else maxsim_naive(Q, Dap)
    return out


def topk(scores: np.ndarray, k: int):
    """Top-k (values descending, int64 indices) of a 1-D score vector, as the
    reference's callers take with ``torch.topk`` (``src/cycle3_experiments.py:215``).
    Ties are broken by the lower index; -0.0 and +0.0 are equal (a tie), and every NaN,
    whatever its sign bit, ranks above +inf, as ``torch.topk`` orders NaN."""
    s = np.asarray(scores)
    k = min(k, s.shape[0])
    s64 = s.astype(np.float64)
    nan = np.isnan(s64)
    # lexsort: last key first -- NaN first, then value descending, then index ascending
    order = np.lexsort((np.arange(s.shape[0]), -np.where(nan, 0.0, s64), ~nan))[:k]
    return s[order], order.astype(np.int64)
