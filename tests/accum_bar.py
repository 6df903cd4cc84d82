"""The fp32-accumulation bar of the parity tests (test infrastructure, not product code).

Every MaxSim score here is a sum over query tokens of a max over document tokens of a
dot product. With 16-bit inputs each product is exact in fp32 (two 11- or 8-bit
significands fit fp32's 24 bits); with fp32 table entries (the PQ table path) each
product is rounded once. Accumulated in fp32 in any order, a dot product of d terms
is within gamma_d * sum_k |q_k d_k| of the exact value (gamma_n = n u / (1 - n u),
u = 2^-24), a max moves by no more than its arguments do, and the sum over Nq query
tokens adds gamma_Nq. With A = MaxSim(|Q|, |D|) -- the oracle on absolute values,
which bounds sum_i max_j sum_k |q_ik| |d_jk| -- a score is therefore within

    (d + Nq) * 2^-23 * A

of the exact one: twice fp32's unit roundoff per operation, a margin for the order
of the additions inside an MFMA. A float64 oracle is exact to far below that.

* fp32 queries against 16-bit documents are split into hi + lo terms of the
  documents' type (two MFMAs per product). The split leaves q - hi - lo within
  2^-22 |q| for fp16 terms (2^-16 |q| for bf16), and a dot product has 2d terms:
  ``(2d + Nq) * 2^-23 * A`` plus the split term.
* Against an fp32 restatement (a GPU GEMM), that restatement's own error, of the
  same form, is added.

On inputs whose products all round the same way, fp16 accumulation and bf16-rounded
products miss the bar by 24x and 68x for every document, and on L2-normalised Gaussian
inputs they miss it for most documents (``test_accum_bar.py`` restates both on the
CPU), so a kernel that stopped accumulating in fp32 fails the parity tests; the north
star's 1e-3 relative bar is checked beside it.
"""
from __future__ import annotations

import numpy as np

NORTH_STAR_RTOL = 1e-3
NORTH_STAR_ATOL = 1e-3
_SPLIT = {None: 0.0, "fp16": 2.0 ** -21, "bf16": 2.0 ** -15}


def rel(d: int, nq: int, qsplit: str | None = None, restated: bool = False) -> float:
    """The bar's factor on MaxSim(|Q|, |D|): ``qsplit`` names the 16-bit type fp32
    queries are split into (None: the query is used as it is); ``restated`` adds the
    error of an fp32 restatement used as the reference."""
    terms = 2 * d if qsplit else d
    r = (terms + nq) * 2.0 ** -23 + _SPLIT[qsplit]
    if restated:
        r += (d + nq) * 2.0 ** -23
    return r


def bound(absref, d: int, nq: int, qsplit: str | None = None, restated: bool = False) -> np.ndarray:
    """Largest |score - exact| fp32 accumulation allows, per score; ``absref`` is
    MaxSim(|Q|, |D|) per score (see :func:`rel`)."""
    absref = np.asarray(absref, np.float64)
    return rel(d, nq, qsplit, restated) * np.where(np.isfinite(absref), absref, 0.0) + 1e-30


def with_bound(fn, Q, X, *rest, qsplit: str | None = None, **kw):
    """``fn(Q, X, *rest)`` and the per-score bar for it, from ``fn(|Q|, |X|, *rest)``.
    ``Q`` is (Nq, d); ``X`` is what ``fn`` scores Q against (documents, or a PQ
    codebook whose rows the codes select)."""
    Q = np.asarray(Q)
    ref = fn(Q, X, *rest, **kw)
    absref = fn(np.abs(Q), np.abs(np.asarray(X)), *rest, **kw)
    return ref, bound(absref, Q.shape[-1], Q.shape[-2], qsplit)


def assert_scores(got, ref, lim=None, what: str = "") -> None:
    """-inf (and NaN) exactly where the reference has them; every finite score within
    the north star's 1e-3 relative bar and, when ``lim`` is given, within it too."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    inf = np.isinf(ref)
    assert np.array_equal(np.isinf(got), inf), f"{what}: -inf pattern differs"
    assert np.all(got[inf] == ref[inf]), f"{what}: infinite values differ"
    fin = ~inf
    np.testing.assert_allclose(got[fin], ref[fin], rtol=NORTH_STAR_RTOL, atol=NORTH_STAR_ATOL, err_msg=what)
    if lim is not None:
        lim = np.broadcast_to(np.asarray(lim, np.float64), ref.shape)[fin]
        err = np.abs(got[fin] - ref[fin])
        if err.size:
            worst = int(np.argmax(err - lim))
            assert np.all(err <= lim), (f"{what}: |delta| {err[worst]:.3e} above the fp32-accumulation bar "
                                        f"{lim[worst]:.3e}")
