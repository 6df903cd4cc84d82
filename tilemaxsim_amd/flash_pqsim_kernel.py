"""PQ / ADC MaxSim -- drop-in for ``TileMaxSimPQ`` of the reference module
``src/flash_pqsim_kernel.py``.

``build_distance_table`` runs ``tms_pq_build_lut``. ``score_batch`` runs the
codebook-gather MFMA kernel (``tms_pq_score``) whenever the shape allows it and the
reference's table-gather algorithm (``tms_pq_build_lut`` + ``tms_pq_score_lut_ex``)
otherwise; ``method=`` forces either one. uint8, int16 and int32 codes are read in place
at their own width (the reference makes an int32 copy of them first), and any K is
accepted, as in the reference.
"""
from __future__ import annotations

import torch

from . import _check, _lib


# Code element types read at their own width; other integer codes are converted to int32
# (the reference converts every code tensor to int32, src/flash_pqsim_kernel.py:233).
_CODE_FLAGS = {torch.uint8: 0, torch.int16: _lib.TMS_CODES_I16, torch.int32: _lib.TMS_CODES_I32}
_CODE_BYTES = {torch.uint8: 1, torch.int16: 2, torch.int32: 4}


class TileMaxSimPQ:
    """High-level PQ MaxSim scorer (``src/flash_pqsim_kernel.py:176-280``).

    Args:
        codebook: (M, K, dsub) PQ centroids, float16, bfloat16 or float32, on the GPU;
            any K. A float32 codebook, or one too large for the LDS (d * K 16-bit
            elements above 160 KiB), is scored by the table-gather kernel on an exact
            fp32 table (the MFMA kernel takes 16-bit centroids).
    """

    def __init__(self, codebook: torch.Tensor):
        _check.tensor("codebook", codebook)
        if codebook.dim() != 3:
            raise ValueError(f"codebook must be (M, K, dsub), got shape {tuple(codebook.shape)}")
        _check.embedding_dtype("codebook", codebook)
        _check.on_gpu("codebook", codebook)
        self.codebook = codebook.contiguous()
        self.M, self.K, self.dsub = codebook.shape
        self.d = self.M * self.dsub

    def _query(self, Q: torch.Tensor):
        """The query as the kernels take it, and its dtype code (an fp32 query against a
        16-bit codebook keeps its precision: ``TMS_QUERY_F32``)."""
        _check.tensor("Q", Q)
        if Q.dim() != 2:
            raise ValueError(f"Q must be (Nq, d), got shape {tuple(Q.shape)}")
        assert Q.shape[1] == self.d, f"Q width {Q.shape[1]} != M*dsub = {self.d}"
        _check.on_gpu("Q", Q)
        _check.same_device(Q=Q, codebook=self.codebook)
        return _check.query_for(Q, self.codebook.dtype)

    def _codes(self, codes: torch.Tensor, validate: bool) -> torch.Tensor:
        if codes.dtype.is_floating_point or codes.dtype == torch.bool:
            raise TypeError(f"codes must be an integer tensor, got {codes.dtype}")
        _check.on_gpu("codes", codes)
        _check.same_device(codes=codes, codebook=self.codebook)
        if validate and codes.numel() > 0 and (codes.dtype != torch.uint8 or self.K < 256):
            lo, hi = int(codes.min()), int(codes.max())
            if lo < 0 or hi >= self.K:
                raise ValueError(f"codes must lie in [0, K={self.K}), found [{lo}, {hi}]")
        if codes.dtype not in _CODE_FLAGS:
            codes = codes.to(torch.int32)
        return codes.contiguous()

    def _table(self, Q: torch.Tensor, qcode: int) -> torch.Tensor:
        Nq = Q.shape[0]
        table = torch.empty(Nq, self.M, self.K, dtype=torch.float32, device=Q.device)
        if table.numel() == 0:
            return table
        lib = _lib.load()
        with _lib.on_device(Q.device):
            _lib.check(lib.tms_pq_build_lut(Q.data_ptr(), Nq, self.codebook.data_ptr(), self.M, self.K, self.dsub,
                                            qcode, table.data_ptr(), _lib.stream_of(Q)))
        return table

    def build_distance_table(self, Q: torch.Tensor) -> torch.Tensor:
        """Query-centroid table ``T[q, m, k] = Q[q, m*dsub:(m+1)*dsub] . C[m, k]`` in fp32
        (``src/flash_pqsim_kernel.py:190-211``). Returns (Nq, M, K) float32. The query is
        used in its own precision (an fp32 query is not rounded to the codebook's type)."""
        Q, qcode = self._query(Q)
        return self._table(Q, qcode)

    def score_batch(self, Q: torch.Tensor, codes: torch.Tensor, method: str = "auto",
                    validate: bool = True) -> torch.Tensor:
        """Score a batch of PQ-compressed documents against a query
        (``src/flash_pqsim_kernel.py:213-252``).

        Args:
            Q: (Nq, d) query embeddings (an fp32 query against a 16-bit codebook is scored
                at fp32 precision, never rounded to the codebook's type).
            codes: (B, Nd, M) PQ codes: uint8, int16 or int32 (read in place at their
                width), or any other integer dtype (converted to int32), values < K.
            method: "auto" (MFMA kernel when the shape allows it, else the table path),
                "mfma" or "lut".
            validate: check that codes lie in [0, K) (one device-to-host copy; skipped
                for uint8 codes when K >= 256, where every byte is valid).

        Returns:
            (B,) float32 MaxSim scores; a document with Nd == 0 scores -inf.
        """
        _check.tensor("codes", codes)
        if codes.dim() != 3:
            raise ValueError(f"codes must be (B, Nd, M), got shape {tuple(codes.shape)}")
        B, Nd, M = codes.shape
        assert M == self.M, f"codes have M={M} subspaces, codebook has {self.M}"
        if method not in ("auto", "mfma", "lut"):
            raise ValueError(f"method must be 'auto', 'mfma' or 'lut', got {method!r}")
        Q, qcode = self._query(Q)
        codes = self._codes(codes, validate)
        Nq = Q.shape[0]
        scores = torch.empty(B, dtype=torch.float32, device=Q.device)
        if B == 0:
            return scores
        lib = _lib.load()
        with _lib.on_device(Q.device):
            stream = _lib.stream_of(Q)
            if method != "lut":
                # the C entry point refuses shapes the MFMA kernel does not take before any
                # device work; "auto" then scores through the table
                status = lib.tms_pq_score(Q.data_ptr(), Nq, self.codebook.data_ptr(), self.M, self.K, self.dsub,
                                          qcode | _CODE_FLAGS[codes.dtype], codes.data_ptr(), B, Nd,
                                          scores.data_ptr(), stream)
                if status == _lib.TMS_OK or method == "mfma" or status != _lib.TMS_ERR_UNSUPPORTED:
                    _lib.check(status)
                    return scores
            table = self._table(Q, qcode)
            _lib.check(lib.tms_pq_score_lut_ex(table.data_ptr(), Nq, self.M, self.K, codes.data_ptr(),
                                               _CODE_BYTES[codes.dtype], B, Nd, scores.data_ptr(), stream))
        return scores

    def score_batch_queries(self, Qs: torch.Tensor, codes: torch.Tensor, validate: bool = True) -> torch.Tensor:
        """Score ``nQ`` queries against the same PQ codes: ``Qs`` (nQ, Nq, d) -> (nQ, B).

        Equivalent to stacking :meth:`score_batch` over the queries. On the MFMA shapes
        (uint8 codes, a query of the codebook's type) each 16-token tile of codes is
        decoded once per pass through the codebook in LDS and shared by up to 32 query
        blocks of 32 tokens (``tms_pq_score_batched``); other inputs score query by query.
        No reference counterpart.
        """
        _check.tensor("Qs", Qs)
        _check.tensor("codes", codes)
        if Qs.dim() != 3:
            raise ValueError(f"Qs must be (nQ, Nq, d), got shape {tuple(Qs.shape)}")
        if codes.dim() != 3:
            raise ValueError(f"codes must be (B, Nd, M), got shape {tuple(codes.shape)}")
        B, Nd, M = codes.shape
        assert M == self.M, f"codes have M={M} subspaces, codebook has {self.M}"
        assert Qs.shape[2] == self.d, f"Q width {Qs.shape[2]} != M*dsub = {self.d}"
        _check.on_gpu("Qs", Qs)
        _check.same_device(Qs=Qs, codebook=self.codebook)
        Qs, qcode = _check.query_for(Qs, self.codebook.dtype)
        codes = self._codes(codes, validate)
        nQ, Nq = Qs.shape[0], Qs.shape[1]
        scores = torch.empty(nQ, B, dtype=torch.float32, device=Qs.device)
        if B == 0 or nQ == 0:
            return scores
        lib = _lib.load()
        with _lib.on_device(Qs.device):
            status = lib.tms_pq_score_batched(Qs.data_ptr(), nQ, Nq, self.codebook.data_ptr(), self.M, self.K,
                                              self.dsub, qcode | _CODE_FLAGS[codes.dtype], codes.data_ptr(), B, Nd,
                                              scores.data_ptr(), _lib.stream_of(Qs))
        if status == _lib.TMS_ERR_UNSUPPORTED:  # shapes without an MFMA path: the table, query by query
            for q in range(nQ):
                scores[q] = self.score_batch(Qs[q], codes, method="lut", validate=False)
            return scores
        _lib.check(status)
        return scores

    def score_single(self, Q: torch.Tensor, codes: torch.Tensor, method: str = "auto") -> torch.Tensor:
        """Score one PQ-compressed document (``src/flash_pqsim_kernel.py:254-280``).

        Args:
            Q: (Nq, d); codes: (Nd, M). Returns a 0-d float32 tensor.
        """
        if codes.dim() != 2:
            raise ValueError(f"codes must be (Nd, M), got shape {tuple(codes.shape)}")
        return self.score_batch(Q, codes.unsqueeze(0), method=method).reshape(())
