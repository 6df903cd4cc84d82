"""Residual-compressed (ColBERTv2) documents: decompression and fused decode + MaxSim.

The reference's PLAID path (``src/plaid_integration_benchmark.py:154-183``, patched into
ColBERT at ``:328-333``) scores documents that ColBERT first decompresses from its
residual-compressed index. ColBERT is colbert-ai 0.2.22 (``:23``), whose codec
(``ResidualCodec``, ``colbert/indexing/codecs/residual.py`` in that package) stores each
token as a centroid id plus ``nbits`` bits per dimension, selecting one of ``2**nbits``
bucket weights. This module takes the index arrays as ColBERT holds them:

* ``codes`` (T,) centroid ids (int32; int64 is narrowed on the device);
* ``residuals`` (T, d * nbits / 8) uint8;
* ``centroids`` (C, d) and ``bucket_weights`` (2**nbits,), cast to fp16 as the codec's
  GPU path does;
* ``doc_offsets`` (ndocs + 1,) int64: document ``p`` is index rows
  ``[doc_offsets[p], doc_offsets[p+1])`` (ColBERT's ``doclens`` as a prefix sum).

:func:`decompress_residual` is the drop-in for ``ResidualCodec.decompress``.
:func:`flashmaxsim_score_residual` replaces "decompress the candidates, then
``flashmaxsim_score_packed``" with one kernel that decodes in registers and never
writes the decompressed tokens; :func:`flashmaxsim_score_residual_batched` does the same
for many queries over the same documents, decoding each tile once for all of them.
"""
from __future__ import annotations

import torch

from . import _check, _lib


def _prep_codec(codes, residuals, centroids, bucket_weights, nbits: int):
    for name, t in (("codes", codes), ("residuals", residuals), ("centroids", centroids),
                    ("bucket_weights", bucket_weights)):
        _check.tensor(name, t)
    if nbits not in (1, 2, 4):
        raise NotImplementedError(f"nbits={nbits} is not supported (1, 2 or 4)")
    if centroids.dim() != 2:
        raise ValueError(f"centroids must be (C, d), got {tuple(centroids.shape)}")
    d = centroids.shape[1]
    if codes.dim() != 1 or residuals.dim() != 2 or residuals.shape[0] != codes.shape[0]:
        raise ValueError(f"codes (T,) and residuals (T, d*nbits/8) disagree: {tuple(codes.shape)} vs "
                         f"{tuple(residuals.shape)}")
    if residuals.dtype != torch.uint8:
        raise TypeError(f"residuals must be uint8, got {residuals.dtype}")
    if residuals.shape[1] * 8 != d * nbits:
        raise ValueError(f"residual rows of {residuals.shape[1]} bytes do not hold d={d} at nbits={nbits}")
    if codes.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"codes must be int32 or int64, got {codes.dtype}")
    if bucket_weights.numel() != (1 << nbits):
        raise ValueError(f"bucket_weights must hold 2**nbits = {1 << nbits} values, got {bucket_weights.numel()}")
    if not centroids.is_floating_point() or not bucket_weights.is_floating_point():
        raise TypeError("centroids and bucket_weights must be floating point")
    _check.on_gpu("centroids", centroids)
    dev = _check.same_device(codes=codes, residuals=residuals, centroids=centroids, bucket_weights=bucket_weights)
    codes = codes.to(torch.int32).contiguous()
    residuals = residuals.contiguous()
    centroids = centroids.to(torch.float16).contiguous()
    bucket_weights = bucket_weights.reshape(-1).to(torch.float16).contiguous()
    return codes, residuals, centroids, bucket_weights, d, dev


def decompress_residual(codes: torch.Tensor, residuals: torch.Tensor, centroids: torch.Tensor,
                        bucket_weights: torch.Tensor, nbits: int) -> torch.Tensor:
    """Decompress T tokens: ``normalize(fp16(centroids[code] + bucket_weights[bucket]))``
    as (T, d) fp16, computed as the codec's GPU path computes it."""
    codes, residuals, centroids, bucket_weights, d, dev = _prep_codec(codes, residuals, centroids, bucket_weights,
                                                                      nbits)
    T = codes.shape[0]
    out = torch.empty(T, d, dtype=torch.float16, device=dev)
    if T == 0:
        return out
    lib = _lib.load()
    with _lib.on_device(dev):
        _lib.check(lib.tms_residual_decompress(codes.data_ptr(), residuals.data_ptr(), T, centroids.data_ptr(),
                                               centroids.shape[0], d, bucket_weights.data_ptr(), nbits,
                                               out.data_ptr(), _lib.stream_of(codes)))
    return out


def _prep_docs(fn: str, doc_offsets, pids, dev, T: int, padding: str, validate: bool):
    """Offsets, pids, B and pad_len for the MaxSim entry points (shared checks)."""
    if padding not in ("zeros", "mask"):
        raise ValueError(f"padding must be 'zeros' or 'mask', got {padding!r}")
    _check.tensor("doc_offsets", doc_offsets)
    if doc_offsets.dim() != 1 or doc_offsets.numel() < 1:
        raise ValueError("doc_offsets must be (ndocs + 1,)")
    if doc_offsets.dtype.is_floating_point or doc_offsets.dtype == torch.bool:
        raise TypeError(f"doc_offsets must be integer, got {doc_offsets.dtype}")
    offsets = doc_offsets.to(device=dev, dtype=torch.int64).contiguous()
    ndocs = offsets.numel() - 1
    if pids is not None:
        _check.tensor("pids", pids)
        if pids.dim() != 1 or pids.dtype.is_floating_point or pids.dtype == torch.bool:
            raise ValueError("pids must be a 1-D integer tensor")
        pids = pids.to(device=dev, dtype=torch.int64).contiguous()
        B = pids.numel()
    else:
        B = ndocs
    if B == 0:
        return offsets, pids, ndocs, B, 0
    if validate:
        bad = bool((offsets[1:] < offsets[:-1]).any()) or int(offsets[0]) < 0 or int(offsets[-1]) > T
        if pids is not None:
            bad = bad or bool(((pids < 0) | (pids >= ndocs)).any())
        if bad:
            raise ValueError(f"{fn}: doc_offsets must be non-decreasing within [0, T] and pids within [0, ndocs)")
    pad_len = 0
    if padding == "zeros" and ndocs > 0:  # the longest scored document (one host sync)
        lengths = offsets[1:] - offsets[:-1]
        if pids is not None:
            lengths = lengths[pids.clamp(0, ndocs - 1)]
        pad_len = max(int(lengths.max()), 0)
    return offsets, pids, ndocs, B, pad_len


def flashmaxsim_score_residual(Q: torch.Tensor, codes: torch.Tensor, residuals: torch.Tensor,
                               centroids: torch.Tensor, bucket_weights: torch.Tensor, nbits: int,
                               doc_offsets: torch.Tensor, pids: torch.Tensor | None = None,
                               padding: str = "zeros", validate: bool = True) -> torch.Tensor:
    """Score one query against residual-compressed documents in one kernel.

    Args:
        Q: (1, Nq, d) or (Nq, d) query (cast to fp16).
        codes, residuals, centroids, bucket_weights, nbits: the index, as above.
        doc_offsets: (ndocs + 1,) int64 prefix sums of the documents' token counts.
        pids: (B,) documents to score (PLAID's candidates); None scores all of them.
        padding: "zeros" -- the reference's PLAID drop-in semantics: documents are
            zero-padded to the longest scored one, so a shorter document's per-token max
            is at least 0 (``src/plaid_integration_benchmark.py:167-171``); "mask" --
            plain MaxSim, padding never wins (an empty document scores -inf).
        validate: check pids and offsets on the device first (one host sync); without
            it an invalid document scores NaN.

    Returns:
        (B,) float32 scores, equal to MaxSim over :func:`decompress_residual`'s output up
        to the fp16 rounding of the normalised tokens.
    """
    if padding not in ("zeros", "mask"):
        raise ValueError(f"padding must be 'zeros' or 'mask', got {padding!r}")
    _check.tensor("Q", Q)
    codes, residuals, centroids, bucket_weights, d, dev = _prep_codec(codes, residuals, centroids, bucket_weights,
                                                                      nbits)
    Q2 = Q.squeeze(0) if Q.dim() == 3 else Q
    if Q2.dim() != 2:
        raise ValueError(f"Q must be (1, Nq, d) or (Nq, d), got {tuple(Q.shape)}")
    assert Q2.shape[1] == d, f"flashmaxsim_score_residual: Q width {Q2.shape[1]} != centroid width {d}"
    T = codes.shape[0]
    offsets, pids, ndocs, B, pad_len = _prep_docs("flashmaxsim_score_residual", doc_offsets, pids, dev, T, padding,
                                                  validate)
    Q2 = _check.query_like(Q2.to(dev), torch.float16)
    scores = torch.empty(B, dtype=torch.float32, device=dev)
    if B == 0:
        return scores
    lib = _lib.load()
    with _lib.on_device(dev):
        _lib.check(lib.tms_maxsim_residual(Q2.data_ptr(), Q2.shape[0], d, centroids.data_ptr(), centroids.shape[0],
                                           bucket_weights.data_ptr(), nbits, codes.data_ptr(), residuals.data_ptr(),
                                           T, offsets.data_ptr(), ndocs,
                                           pids.data_ptr() if pids is not None else None, B, pad_len,
                                           scores.data_ptr(), _lib.stream_of(Q2)))
    return scores


def flashmaxsim_score_residual_batched(Qs: torch.Tensor, codes: torch.Tensor, residuals: torch.Tensor,
                                       centroids: torch.Tensor, bucket_weights: torch.Tensor, nbits: int,
                                       doc_offsets: torch.Tensor, pids: torch.Tensor | None = None,
                                       padding: str = "zeros", validate: bool = True) -> torch.Tensor:
    """Score ``nQ`` queries against the same residual-compressed documents:
    ``Qs`` (nQ, Nq, d) -> (nQ, B) float32.

    Arguments and semantics are those of :func:`flashmaxsim_score_residual`, query by
    query. Each tile of documents is decoded once per pass and shared by up to 32 query
    blocks of 32 tokens, so the decode cost is paid once for all the queries (exhaustive
    scoring of a compressed collection, or queries that share PLAID candidates). The
    decoded tokens are rounded to fp16 as the codec rounds them, so the scores equal
    MaxSim over :func:`decompress_residual`'s output up to the summation order.
    """
    if padding not in ("zeros", "mask"):
        raise ValueError(f"padding must be 'zeros' or 'mask', got {padding!r}")
    _check.tensor("Qs", Qs)
    codes, residuals, centroids, bucket_weights, d, dev = _prep_codec(codes, residuals, centroids, bucket_weights,
                                                                      nbits)
    if Qs.dim() != 3:
        raise ValueError(f"Qs must be (nQ, Nq, d), got {tuple(Qs.shape)}")
    assert Qs.shape[2] == d, f"flashmaxsim_score_residual_batched: Q width {Qs.shape[2]} != centroid width {d}"
    T = codes.shape[0]
    offsets, pids, ndocs, B, pad_len = _prep_docs("flashmaxsim_score_residual_batched", doc_offsets, pids, dev, T,
                                                  padding, validate)
    Qs = _check.query_like(Qs.to(dev), torch.float16)
    nQ, Nq = Qs.shape[0], Qs.shape[1]
    scores = torch.empty(nQ, B, dtype=torch.float32, device=dev)
    if B == 0 or nQ == 0:
        return scores
    lib = _lib.load()
    with _lib.on_device(dev):
        _lib.check(lib.tms_maxsim_residual_batched(Qs.data_ptr(), nQ, Nq, d, centroids.data_ptr(), centroids.shape[0],
                                                   bucket_weights.data_ptr(), nbits, codes.data_ptr(),
                                                   residuals.data_ptr(), T, offsets.data_ptr(), ndocs,
                                                   pids.data_ptr() if pids is not None else None, B, pad_len,
                                                   scores.data_ptr(), _lib.stream_of(Qs)))
    return scores
