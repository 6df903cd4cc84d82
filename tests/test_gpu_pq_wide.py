"""PQ codebooks beyond 256 centroids, int16 / int32 codes read at their own width, tables
tiled over m, and fp32 queries against 16-bit codebooks.

The reference's ``TileMaxSimPQ.score_batch`` takes "uint8 or int32" codes, converts them
with ``codes.to(torch.int32)`` and gathers ``Table[q, m, codes]`` with no K limit
(``src/flash_pqsim_kernel.py:219, 233, 161-165``); it builds the table from the query
loaded ``.to(tl.float32)`` (``:54-67``). Oracle: decompress-then-score in float64
(``pytorch_pqsim_baseline``, ``:283-313``), on the unrounded query.

Paths covered (the C entry point picks them from the shape):
* the MFMA kernel with int16 / int32 codes, and with K = 512 (a 128 KiB codebook, one
  workgroup per CU);
* the table-gather kernel with every code width: M * K <= 16384 (slices of query tokens),
  larger tables (slices tiled over m, per-token partial sums in registers), and K > 16384
  (gathered from the table in memory);
* fp32 queries (split into two 16-bit terms on MFMA; an fp32 table on the table path).

Bars: 1e-3 relative, and against the float64 oracle the fp32-accumulation bar of
``accum_bar.py`` (16-bit queries) or the split-product bar of ``test_gpu_fp32.py``
(fp32 queries).
"""
import numpy as np
import pytest

import accum_bar as bar
from oracle import maxsim_oracle as orc

from test_gpu_fp32 import _assert_fp32_scores, _coherent


def _gpu(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _check(got, ref, what, lim=None):
    bar.assert_scores(got, ref, lim, what)


def _pq_oracle(Q, C, codes):
    """Float64 decompress-then-score and its fp32-accumulation bar."""
    return bar.with_bound(orc.pq_decompress_score, Q, C, codes, f64=True)


def _mk(seed, M, K, dsub, Nq, B, Nd, code_dtype):
    rng = np.random.default_rng(seed)
    C = rng.standard_normal((M, K, dsub), dtype=np.float32).astype(np.float16)
    Q = rng.standard_normal((Nq, M * dsub), dtype=np.float32)
    Q = (Q / np.linalg.norm(Q, axis=-1, keepdims=True)).astype(np.float16)
    codes = rng.integers(0, K, size=(B, Nd, M)).astype(code_dtype)
    return Q, C, codes


# (M, K, dsub, code dtype, methods): MFMA-sized tables first, then the table path's three
# forms: query-token slices (M*K <= 16384), m-tiled slices, and the in-memory table.
CASES = [
    (16, 256, 8, np.int32, ("mfma", "lut")),     # int32 codes on the C5 shape
    (16, 256, 8, np.int16, ("mfma", "lut")),
    (16, 512, 8, np.int32, ("mfma", "lut")),     # 128 KiB codebook: MFMA, one workgroup per CU
    (16, 512, 8, np.int16, ("mfma", "lut")),
    (32, 300, 4, np.int32, ("mfma", "lut")),     # K not a power of two; 8 codes of 4 bytes per lane
    (64, 200, 2, np.int16, ("mfma", "lut")),     # 16 codes of 2 bytes per lane
    (12, 400, 8, np.int32, ("mfma", "lut")),     # 3 codes per lane (12-byte runs)
    (16, 1024, 8, np.int32, ("auto", "lut")),    # M*K = 16384: one query token per slice
    (32, 1024, 4, np.int32, ("auto", "lut")),    # M*K = 32768: m-tiled slices
    (128, 256, 1, np.uint8, ("auto", "lut")),    # dsub = 1, M*K = 32768: m-tiled, uint8 codes
    (64, 512, 2, np.int16, ("auto", "lut")),     # m-tiled, int16 codes
    (4, 20000, 8, np.int32, ("auto", "lut")),    # K > 16384: gathered from the table in memory
]


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,dsub,cdt,methods", CASES)
def test_pq_wide_codes_and_large_tables(cuda, M, K, dsub, cdt, methods):
    from tilemaxsim_amd import TileMaxSimPQ
    Q, C, codes = _mk(M * 7 + K + dsub, M, K, dsub, 32, 90, 41, cdt)
    pq = TileMaxSimPQ(_gpu(C))
    ref, lim = _pq_oracle(Q, C, codes)
    for method in methods:
        got = pq.score_batch(_gpu(Q), _gpu(codes), method=method).cpu().numpy()
        _check(got, ref, f"M={M} K={K} dsub={dsub} {np.dtype(cdt).name} {method}", lim)
    # the reference algorithm's own sum order (table gather, ascending m)
    _check(pq.score_batch(_gpu(Q), _gpu(codes), method="lut").cpu().numpy(),
           orc.pq_score_lut(orc.pq_build_lut(Q, C), codes), "lut vs table oracle")


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,dsub", [(32, 1024, 4), (128, 256, 1)])
def test_pq_mtile_ragged_shapes(cuda, M, K, dsub):
    """m-tiled table path: query lengths that leave partial query groups, a document run
    shorter than a workgroup's capacity, long documents (3000 tokens, one per run), no
    document tokens and invalid codes clamped into the table."""
    import torch
    from tilemaxsim_amd import TileMaxSimPQ
    for Nq, B, Nd in [(5, 33, 17), (70, 7, 3000), (1, 300, 1)]:
        Q, C, codes = _mk(Nq + B + Nd, M, K, dsub, Nq, B, Nd, np.int32)
        pq = TileMaxSimPQ(_gpu(C))
        got = pq.score_batch(_gpu(Q), _gpu(codes)).cpu().numpy()
        ref, lim = _pq_oracle(Q, C, codes)
        _check(got, ref, f"M={M} Nq={Nq} B={B} Nd={Nd}", lim)
    empty = pq.score_batch(_gpu(Q), torch.zeros(4, 0, M, dtype=torch.int32, device="cuda")).cpu().numpy()
    assert np.all(np.isneginf(empty))
    bad = codes.copy()
    bad[0, 0, 0] = K + 77
    bad[1, 0, 1] = -5
    with pytest.raises(ValueError):
        pq.score_batch(_gpu(Q), _gpu(bad))
    got = pq.score_batch(_gpu(Q), _gpu(bad), validate=False).cpu().numpy()
    clamped = np.where((bad < 0) | (bad >= K), K - 1, bad)  # negative int32 codes read as large unsigned
    ref, lim = _pq_oracle(Q, C, clamped)
    _check(got, ref, "clamped", lim)


@pytest.mark.gpu
def test_pq_wide_batched_queries_and_int64(cuda):
    """score_batch_queries with int32 codes and K = 512 (query by query on MFMA), and
    int64 codes (converted to int32, as the reference converts every code tensor)."""
    from tilemaxsim_amd import TileMaxSimPQ
    Q, C, codes = _mk(3, 16, 512, 8, 32, 120, 50, np.int32)
    rng = np.random.default_rng(4)
    Qs = np.stack([Q] + [rng.standard_normal(Q.shape, dtype=np.float32).astype(np.float16) for _ in range(3)])
    pq = TileMaxSimPQ(_gpu(C))
    got = pq.score_batch_queries(_gpu(Qs), _gpu(codes)).cpu().numpy()
    for q in range(4):
        ref, lim = _pq_oracle(Qs[q], C, codes)
        _check(got[q], ref, f"batched int32 K=512 q={q}", lim)
    got = pq.score_batch(_gpu(Q), _gpu(codes.astype(np.int64))).cpu().numpy()
    ref, lim = _pq_oracle(Q, C, codes)
    _check(got, ref, "int64 codes", lim)


@pytest.mark.gpu
@pytest.mark.parametrize("cb", ["fp16", "bf16"])
def test_pq_fp32_query_unrounded(cuda, cb):
    """fp32 queries against a 16-bit codebook: the table is built from the unrounded
    query (within dsub * 2^-23 of the float64 table, relative to |Q| . |C|), and both
    scoring paths match the float64 oracle on the unrounded query to the fp32 bar, which
    the query rounded to the codebook's type misses (``test_gpu_qsplit.py``)."""
    import torch
    from tilemaxsim_amd import TileMaxSimPQ
    tdt = torch.float16 if cb == "fp16" else torch.bfloat16
    rng = np.random.default_rng(12)
    M, K, dsub = 16, 256, 8
    Ct = torch.from_numpy(np.abs(rng.standard_normal((M, K, dsub), dtype=np.float32))).to(tdt)
    C = Ct.float().numpy()
    Q = _coherent(rng, (32, M * dsub), cb)
    codes = rng.integers(0, K, size=(150, 60, M)).astype(np.uint8)
    pq = TileMaxSimPQ(Ct.cuda())
    T = pq.build_distance_table(_gpu(Q)).cpu().numpy()
    T64 = np.einsum("qmj,mkj->qmk", Q.reshape(32, M, dsub).astype(np.float64), C.astype(np.float64))
    Tabs = np.einsum("qmj,mkj->qmk", np.abs(Q).reshape(32, M, dsub).astype(np.float64), np.abs(C).astype(np.float64))
    assert np.all(np.abs(T - T64) <= dsub * 2.0 ** -23 * Tabs)
    Qr = torch.from_numpy(Q).to(tdt).float().numpy()  # the rounded query's table misses that bar
    Tr = np.einsum("qmj,mkj->qmk", Qr.reshape(32, M, dsub).astype(np.float64), C.astype(np.float64))
    assert np.mean(np.abs(Tr - T64) > dsub * 2.0 ** -23 * Tabs) > 0.9
    ref = orc.pq_decompress_score(Q, C, codes, f64=True)
    absref = orc.pq_decompress_score(np.abs(Q), np.abs(C), codes, f64=True)
    for method in ("mfma", "lut"):
        got = pq.score_batch(_gpu(Q), _gpu(codes), method=method).cpu().numpy()
        _assert_fp32_scores(got, ref, absref, M * dsub, f"fp32 Q / {cb} codebook, {method}")
    Qs = np.stack([Q, _coherent(rng, (32, M * dsub), cb)])
    got = pq.score_batch_queries(_gpu(Qs), _gpu(codes)).cpu().numpy()
    for q in range(2):
        _assert_fp32_scores(got[q], orc.pq_decompress_score(Qs[q], C, codes, f64=True),
                            orc.pq_decompress_score(np.abs(Qs[q]), np.abs(C), codes, f64=True), M * dsub,
                            f"fp32 Q batched q={q}")
    # fp32 query with int32 codes: no MFMA form; "auto" takes the table
    got = pq.score_batch(_gpu(Q), _gpu(codes.astype(np.int32))).cpu().numpy()
    _assert_fp32_scores(got, ref, absref, M * dsub, "fp32 Q, int32 codes")
    with pytest.raises(NotImplementedError):
        pq.score_batch(_gpu(Q), _gpu(codes.astype(np.int32)), method="mfma")
