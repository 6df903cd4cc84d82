"""MaxSim entry points of the reference module ``src/flash_maxsim_kernel.py``, plus
the masked scorer of ``src/e2e_retrieval_quality.py``.

* :func:`flash_maxsim_single` / :func:`flash_maxsim_batch` -- fixed-length documents
  (``tms_maxsim_dense``).
* :func:`flash_maxsim_multi_doc` -- variable-length documents in a flat token buffer
  with offsets, scored by one kernel launch with no padding (``tms_maxsim_varlen``);
  :func:`flash_maxsim_multi_doc_batched` scores many queries in one pass over them
  (``tms_maxsim_varlen_batched``).
* :func:`maxsim_score` -- padded documents with a token mask (``tms_maxsim_masked``).
"""
from __future__ import annotations

import torch

from . import _check, _lib
from .flash_maxsim_v2 import _dense


def flash_maxsim_single(Q: torch.Tensor, D: torch.Tensor) -> torch.Tensor:
    """MaxSim of one query against one document (``src/flash_maxsim_kernel.py:167-197``).

    Args:
        Q: (Nq, d) query token embeddings.
        D: (Nd, d) document token embeddings, float16, bfloat16 or float32.

    Returns:
        0-d float32 tensor (the reference returns ``out.sum()``).
    """
    _check.tensor("D", D)
    if D.dim() != 2:
        raise ValueError(f"flash_maxsim_single: D must be (Nd, d), got shape {tuple(D.shape)}")
    assert Q.shape[1] == D.shape[1], f"flash_maxsim_single: Q width {Q.shape[1]} != D width {D.shape[1]}"
    return _dense(Q, D.unsqueeze(0), "flash_maxsim_single").reshape(())


def flash_maxsim_batch(Q: torch.Tensor, D: torch.Tensor) -> torch.Tensor:
    """MaxSim of one query against a batch of documents (``src/flash_maxsim_kernel.py:200-245``).

    The reference expands Q to (B, Nq, d) and reduces per-token maxima in a second
    kernel; here the same scores come from the single fused kernel.

    Args:
        Q: (Nq, d); D: (B, Nd, d). Returns (B,) float32.
    """
    assert Q.dim() == 2 and D.dim() == 3 and Q.shape[1] == D.shape[2], "flash_maxsim_batch: Q (Nq, d) vs D (B, Nd, d)"
    return _dense(Q, D, "flash_maxsim_batch")


def flash_maxsim_multi_doc(Q: torch.Tensor, D_flat: torch.Tensor, doc_offsets: torch.Tensor,
                           validate: bool = True) -> torch.Tensor:
    """MaxSim for variable-length documents stored in a flat tensor
    (``src/flash_maxsim_kernel.py:248-273``).

    Document i is ``D_flat[doc_offsets[i]:doc_offsets[i+1]]`` and is scored over exactly
    its own tokens. The reference loops over documents in Python (two host syncs and
    two launches per document); here one launch scores all of them.

    Args:
        Q: (Nq, d) query embeddings.
        D_flat: (total_tokens, d) all document tokens, float16, bfloat16 or float32, contiguous.
        doc_offsets: (num_docs + 1,) integer start offsets (any device; moved to Q's
            device as int64).
        validate: check on the host that offsets are non-decreasing within
            [0, total_tokens] (one device-to-host copy); with ``validate=False`` a
            document with invalid offsets scores NaN instead of raising.

    Returns:
        (num_docs,) float32 scores; an empty document scores -inf.
    """
    _check.tensor("Q", Q)
    _check.tensor("D_flat", D_flat)
    _check.tensor("doc_offsets", doc_offsets)
    if D_flat.dim() != 2:
        raise ValueError(f"flash_maxsim_multi_doc: D_flat must be (total_tokens, d), got {tuple(D_flat.shape)}")
    if doc_offsets.dim() != 1 or doc_offsets.shape[0] < 1:
        raise ValueError("flash_maxsim_multi_doc: doc_offsets must be a 1-D tensor of num_docs + 1 entries")
    if doc_offsets.dtype.is_floating_point or doc_offsets.dtype == torch.bool:
        raise TypeError(f"flash_maxsim_multi_doc: doc_offsets must be integer, got {doc_offsets.dtype}")
    T, d = D_flat.shape
    Nq = Q.shape[0]
    assert Q.dim() == 2 and Q.shape[1] == d, f"flash_maxsim_multi_doc: Q width {Q.shape[1]} != D width {d}"
    _check.embedding_dtype("D_flat", D_flat)
    _check.contiguous("D_flat", D_flat)
    _check.on_gpu("Q", Q)
    _check.on_gpu("D_flat", D_flat)
    _check.same_device(Q=Q, D_flat=D_flat)
    Q, code = _check.query_for(Q, D_flat.dtype)
    offsets = doc_offsets.to(device=Q.device, dtype=torch.int64).contiguous()
    num_docs = offsets.shape[0] - 1
    if validate and num_docs > 0:
        bad = (offsets[0] < 0) | (offsets[-1] > T) | (offsets[1:] < offsets[:-1]).any()
        if bool(bad):
            raise ValueError("flash_maxsim_multi_doc: doc_offsets must be non-decreasing within [0, total_tokens]")
    scores = torch.empty(num_docs, dtype=torch.float32, device=Q.device)
    if num_docs == 0:
        return scores
    lib = _lib.load()
    with _lib.on_device(Q.device):
        _lib.check(lib.tms_maxsim_varlen(Q.data_ptr(), Nq, d, D_flat.data_ptr(), T, offsets.data_ptr(), num_docs,
                                         code, scores.data_ptr(), _lib.stream_of(Q)))
    return scores


def _varlen_batched(fn: str, Qs: torch.Tensor, D_flat: torch.Tensor, doc_offsets: torch.Tensor, validate: bool,
                    zero_pad: bool) -> torch.Tensor:
    _check.tensor("Qs", Qs)
    _check.tensor("D_flat", D_flat)
    _check.tensor("doc_offsets", doc_offsets)
    if Qs.dim() != 3 or D_flat.dim() != 2:
        raise ValueError(f"{fn}: Qs must be (nQ, Nq, d) and D_flat (total_tokens, d)")
    if doc_offsets.dim() != 1 or doc_offsets.shape[0] < 1:
        raise ValueError(f"{fn}: doc_offsets must be a 1-D tensor of num_docs + 1 entries")
    if doc_offsets.dtype.is_floating_point or doc_offsets.dtype == torch.bool:
        raise TypeError(f"{fn}: doc_offsets must be integer, got {doc_offsets.dtype}")
    T, d = D_flat.shape
    nQ, Nq = Qs.shape[0], Qs.shape[1]
    assert Qs.shape[2] == d, f"{fn}: Q width {Qs.shape[2]} != D width {d}"
    _check.embedding_dtype("D_flat", D_flat)
    _check.contiguous("D_flat", D_flat)
    _check.on_gpu("Qs", Qs)
    _check.on_gpu("D_flat", D_flat)
    _check.same_device(Qs=Qs, D_flat=D_flat)
    Qs, code = _check.query_for(Qs, D_flat.dtype)
    offsets = doc_offsets.to(device=Qs.device, dtype=torch.int64).contiguous()
    B = offsets.shape[0] - 1
    if (validate or zero_pad) and B > 0:
        bad = (offsets[0] < 0) | (offsets[-1] > T) | (offsets[1:] < offsets[:-1]).any()
        if bool(bad):
            raise ValueError(f"{fn}: doc_offsets must be non-decreasing within [0, total_tokens]")
    pad_len = int((offsets[1:] - offsets[:-1]).max()) if zero_pad and B > 0 else 0
    out = torch.empty(nQ, B, dtype=torch.float32, device=Qs.device)
    if B == 0 or nQ == 0:
        return out
    lib = _lib.load()
    with _lib.on_device(Qs.device):
        _lib.check(lib.tms_maxsim_varlen_batched(Qs.data_ptr(), nQ, Nq, d, D_flat.data_ptr(), T, offsets.data_ptr(), B,
                                                 pad_len, code, out.data_ptr(),
                                                 _lib.stream_of(Qs)))
    return out


def flash_maxsim_multi_doc_batched(Qs: torch.Tensor, D_flat: torch.Tensor, doc_offsets: torch.Tensor,
                                   validate: bool = True) -> torch.Tensor:
    """:func:`flash_maxsim_multi_doc` for ``nQ`` queries at once: ``Qs`` (nQ, Nq, d) ->
    (nQ, num_docs) float32.

    Up to 32 blocks of 32 query tokens share each pass over the documents (one tile
    load per workgroup, scored from LDS by all of them), which makes the call MFMA-bound
    instead of one HBM pass per query. Empty documents score -inf; with
    ``validate=False`` a document with invalid offsets scores NaN.
    No reference counterpart (the reference loops over queries).
    """
    return _varlen_batched("flash_maxsim_multi_doc_batched", Qs, D_flat, doc_offsets, validate, False)


def maxsim_score(Q: torch.Tensor, D: torch.Tensor, D_mask: torch.Tensor | None = None) -> torch.Tensor:
    """Masked MaxSim with the semantics of ``pytorch_maxsim_score(Q, D, D_mask)``
    (``src/e2e_retrieval_quality.py:105-110``): tokens with ``D_mask == False`` are -inf
    before the max, so padding never wins a max (a fully masked document scores -inf).

    Args:
        Q: (Nq, d); D: (B, Nd, d) float16/bfloat16/float32 contiguous; D_mask: (B, Nd) bool or
            integer (non-zero = real token), or None for no mask.

    Returns:
        (B,) float32 scores.
    """
    if D_mask is None:
        return _dense(Q, D, "maxsim_score")
    _check.tensor("Q", Q)
    _check.tensor("D", D)
    _check.tensor("D_mask", D_mask)
    if D.dim() != 3 or Q.dim() != 2:
        raise ValueError("maxsim_score: Q must be (Nq, d) and D (B, Nd, d)")
    B, Nd, d = D.shape
    if tuple(D_mask.shape) != (B, Nd):
        raise ValueError(f"maxsim_score: D_mask must be (B, Nd) = {(B, Nd)}, got {tuple(D_mask.shape)}")
    assert Q.shape[1] == d, f"maxsim_score: Q width {Q.shape[1]} != D width {d}"
    _check.embedding_dtype("D", D)
    _check.contiguous("D", D)
    _check.on_gpu("Q", Q)
    _check.on_gpu("D", D)
    _check.on_gpu("D_mask", D_mask)
    _check.same_device(Q=Q, D=D, D_mask=D_mask)
    Q, code = _check.query_for(Q, D.dtype)
    mask = D_mask
    if mask.dtype in (torch.bool, torch.int8):  # one byte per token: read as is (non-zero = real)
        mask = mask.view(torch.uint8)
    elif mask.dtype != torch.uint8:
        mask = (mask != 0).view(torch.uint8)
    mask = mask.contiguous()
    scores = torch.empty(B, dtype=torch.float32, device=Q.device)
    if B == 0:
        return scores
    lib = _lib.load()
    with _lib.on_device(Q.device):
        _lib.check(lib.tms_maxsim_masked(Q.data_ptr(), Q.shape[0], d, D.data_ptr(), mask.data_ptr(), B, Nd,
                                         code, scores.data_ptr(), _lib.stream_of(Q)))
    return scores
