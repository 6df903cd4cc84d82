"""PLAID / ColBERT packed-document scoring -- drop-in for the reference's
``flashmaxsim_score_packed`` (``src/plaid_integration_benchmark.py:154-183``), the
function the reference monkey-patches over ColBERT's ``colbert_score_packed``.

ColBERT hands the scorer a packed token buffer ``D_packed`` (T, d) plus per-document
lengths. The reference pads it to (B, max_len, d), multiplies the padding by zero and
runs its dense kernel, so a document shorter than ``max_len`` also sees zero vectors
(each query token's max is at least 0). Here the packed buffer is scored in place by
the variable-length kernel; ``padding="zeros"`` (default) reproduces the reference's
numbers exactly, and ``padding="mask"`` gives ColBERT's own masked semantics, where
padding never wins a max.
"""
from __future__ import annotations

import torch

from . import _check, _lib
from .flash_maxsim_kernel import _varlen_batched, flash_maxsim_multi_doc


def lengths_to_offsets(D_lengths: torch.Tensor, device: torch.device) -> torch.Tensor:
    """(B,) integer lengths -> (B + 1,) int64 offsets on ``device`` (computed on device)."""
    lengths = D_lengths.to(device=device, dtype=torch.int64)
    offsets = torch.zeros(lengths.numel() + 1, dtype=torch.int64, device=device)
    torch.cumsum(lengths, 0, out=offsets[1:])
    return offsets


def _to_configured_gpu(config, *tensors: torch.Tensor) -> tuple:
    """The reference's device step (``src/plaid_integration_benchmark.py:159-161``): with
    ``config.total_visible_gpus > 0`` every input is moved with ``.cuda()`` (to the
    current device; a no-op for a tensor already there). With no config, or a config
    that sees no GPU, the tensors stay where they are and the GPU check that follows
    rejects host tensors, since there is no CPU path."""
    if config is not None and getattr(config, "total_visible_gpus", 0) > 0:
        return tuple(t.cuda() for t in tensors)
    return tensors


def flashmaxsim_score_packed(Q: torch.Tensor, D_packed: torch.Tensor, D_lengths: torch.Tensor, config=None,
                             padding: str = "zeros") -> torch.Tensor:
    """Score one query against packed variable-length documents.

    Args:
        Q: (1, Nq, d) or (Nq, d) query embeddings (cast to half like the reference).
        D_packed: (T, d) all document tokens back to back.
        D_lengths: (B,) tokens per document; they must sum to at most T.
        config: ColBERT's run config, read as the reference reads it: when
            ``config.total_visible_gpus > 0``, host tensors are moved to the current GPU
            first. ``None`` leaves the tensors where they are (they must then be on the GPU).
        padding: "zeros" -- score as the reference does after zero-padding every
            document to the longest one; "mask" -- padding is -inf (ColBERT semantics).

    Returns:
        (B,) float32 scores on the GPU.
    """
    if padding not in ("zeros", "mask"):
        raise ValueError(f"padding must be 'zeros' or 'mask', got {padding!r}")
    _check.tensor("Q", Q)
    _check.tensor("D_packed", D_packed)
    _check.tensor("D_lengths", D_lengths)
    Q, D_packed, D_lengths = _to_configured_gpu(config, Q, D_packed, D_lengths)
    Q2 = Q.squeeze(0) if Q.dim() == 3 else Q
    if Q2.dim() != 2 or D_packed.dim() != 2 or D_lengths.dim() != 1:
        raise ValueError("flashmaxsim_score_packed: Q (1, Nq, d), D_packed (T, d), D_lengths (B,)")
    if D_lengths.dtype.is_floating_point or D_lengths.dtype == torch.bool:
        raise TypeError(f"D_lengths must be integer, got {D_lengths.dtype}")
    if D_packed.dtype != torch.float16:
        D_packed = D_packed.half()  # the reference scores .half() copies
    D_packed = D_packed.contiguous()
    _check.on_gpu("D_packed", D_packed)
    dev = D_packed.device
    Q2 = Q2.to(dev).half().contiguous()
    offsets = lengths_to_offsets(D_lengths, dev)
    if padding == "mask":
        return flash_maxsim_multi_doc(Q2, D_packed, offsets)
    B = offsets.numel() - 1
    T, d = D_packed.shape
    assert Q2.shape[1] == d, f"flashmaxsim_score_packed: Q width {Q2.shape[1]} != D width {d}"
    if B > 0 and (bool((offsets[1:] < offsets[:-1]).any()) or int(offsets[-1]) > T):
        raise ValueError("flashmaxsim_score_packed: D_lengths must be >= 0 and sum to at most D_packed.shape[0]")
    pad_len = int(D_lengths.max()) if B > 0 else 0
    scores = torch.empty(B, dtype=torch.float32, device=dev)
    if B == 0:
        return scores
    lib = _lib.load()
    with _lib.on_device(dev):
        _lib.check(lib.tms_maxsim_varlen_padded(Q2.data_ptr(), Q2.shape[0], d, D_packed.data_ptr(), T,
                                                offsets.data_ptr(), B, pad_len, _lib.TMS_DTYPE_F16,
                                                scores.data_ptr(), _lib.stream_of(Q2)))
    return scores


def flashmaxsim_score_packed_batched(Qs: torch.Tensor, D_packed: torch.Tensor, D_lengths: torch.Tensor,
                                     config=None, padding: str = "zeros") -> torch.Tensor:
    """:func:`flashmaxsim_score_packed` for ``nQ`` queries over the same packed documents:
    ``Qs`` (nQ, Nq, d) -> (nQ, B) float32, one pass over the tokens for up to 32 query
    blocks. ``config`` and ``padding`` as in :func:`flashmaxsim_score_packed`."""
    if padding not in ("zeros", "mask"):
        raise ValueError(f"padding must be 'zeros' or 'mask', got {padding!r}")
    _check.tensor("Qs", Qs)
    _check.tensor("D_packed", D_packed)
    _check.tensor("D_lengths", D_lengths)
    Qs, D_packed, D_lengths = _to_configured_gpu(config, Qs, D_packed, D_lengths)
    if D_lengths.dim() != 1 or D_lengths.dtype.is_floating_point or D_lengths.dtype == torch.bool:
        raise TypeError("flashmaxsim_score_packed_batched: D_lengths must be a 1-D integer tensor")
    if D_packed.dtype != torch.float16:
        D_packed = D_packed.half()
    D_packed = D_packed.contiguous()
    _check.on_gpu("D_packed", D_packed)
    offsets = lengths_to_offsets(D_lengths, D_packed.device)
    return _varlen_batched("flashmaxsim_score_packed_batched", Qs.to(D_packed.device).half(), D_packed, offsets,
                           True, padding == "zeros")
