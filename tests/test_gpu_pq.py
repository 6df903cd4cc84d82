"""GPU parity of the PQ / ADC kernels (``TileMaxSimPQ``) against the CPU oracle.

Oracles: the reference's decompress-then-score baseline ``pytorch_pqsim_baseline``
(``src/flash_pqsim_kernel.py:283-313``) in float64, and the table-gather form
(``:127-173``). Bars: |score - oracle| <= 1e-3 relative, and the fp32-accumulation bar
(d + Nq) * 2^-23 * MaxSim(|Q|, |decoded tokens|) of ``accum_bar.py`` against the float64
oracle (the reference sums fp32 table entries, ``:154-167``, and the q-sum with
``torch.sum``, ``:250``); identical top-100 up to ties.
"""
import numpy as np
import pytest

import accum_bar as bar
from oracle import maxsim_oracle as orc

pytestmark = pytest.mark.gpu

RTOL = bar.NORTH_STAR_RTOL
ATOL = bar.NORTH_STAR_ATOL


def _mk(seed, M, K, dsub, Nq, B, Nd, normalize_q=True, dtype=np.float16):
    rng = np.random.default_rng(seed)
    C = rng.standard_normal((M, K, dsub), dtype=np.float32).astype(dtype)
    Q = rng.standard_normal((Nq, M * dsub), dtype=np.float32)
    if normalize_q:
        Q /= np.linalg.norm(Q, axis=-1, keepdims=True) + 1e-12
    Q = Q.astype(dtype)
    codes = rng.integers(0, K, size=(B, Nd, M), dtype=np.uint8) if K <= 256 else None
    return Q, C, codes


def _gpu(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _check(got, ref, what, lim=None):
    """The 1e-3 bar, and the fp32-accumulation bar ``lim`` against the float64 oracle."""
    bar.assert_scores(got, ref, lim, what)


def _pq_oracle(Q, C, codes):
    """Float64 decompress-then-score and its fp32-accumulation bar."""
    return bar.with_bound(orc.pq_decompress_score, Q, C, codes, f64=True)


@pytest.mark.parametrize("method", ["mfma", "lut"])
def test_reference_selftest_shape(cuda, method):
    """The reference self-test shape (src/flash_pqsim_kernel.py:320-332)."""
    from tilemaxsim_amd import TileMaxSimPQ
    Q, C, codes = _mk(42, 16, 256, 8, 32, 8, 128, normalize_q=False)
    pq = TileMaxSimPQ(_gpu(C))
    got = pq.score_batch(_gpu(Q), _gpu(codes), method=method).cpu().numpy()
    ref, lim = _pq_oracle(Q, C, codes)
    _check(got, ref, f"selftest {method}", lim)
    _check(got, orc.pq_score_lut(orc.pq_build_lut(Q, C), codes), f"selftest {method} vs lut oracle")


def test_build_distance_table(cuda):
    from tilemaxsim_amd import TileMaxSimPQ
    Q, C, _ = _mk(1, 16, 256, 8, 32, 1, 1, normalize_q=False)
    pq = TileMaxSimPQ(_gpu(C))
    T = pq.build_distance_table(_gpu(Q)).cpu().numpy()
    ref = np.einsum("qmj,mkj->qmk", Q.astype(np.float64).reshape(32, 16, 8), C.astype(np.float64))
    assert T.shape == (32, 16, 256) and T.dtype == np.float32
    np.testing.assert_allclose(T, ref, rtol=1e-5, atol=1e-5)


SHAPES = [
    # (M, K, dsub, Nq, B, Nd)
    (16, 256, 8, 32, 200, 128), (16, 256, 8, 1, 50, 1), (16, 256, 8, 33, 60, 17), (16, 256, 8, 64, 40, 70),
    (16, 256, 8, 100, 20, 33), (32, 256, 4, 32, 100, 40), (64, 256, 2, 32, 100, 40), (8, 256, 16, 32, 100, 40),
    (4, 256, 32, 32, 100, 40), (8, 256, 8, 32, 100, 40), (12, 256, 8, 32, 100, 40), (4, 256, 8, 32, 100, 40),
    (16, 16, 8, 32, 100, 40), (16, 100, 8, 20, 100, 50),
]


@pytest.mark.parametrize("method", ["auto", "lut"])
@pytest.mark.parametrize("M,K,dsub,Nq,B,Nd", SHAPES)
def test_pq_shapes(cuda, M, K, dsub, Nq, B, Nd, method):
    from tilemaxsim_amd import TileMaxSimPQ
    Q, C, codes = _mk(M * 1000 + K + dsub + Nq + B + Nd, M, K, dsub, Nq, B, Nd)
    pq = TileMaxSimPQ(_gpu(C))
    got = pq.score_batch(_gpu(Q), _gpu(codes), method=method).cpu().numpy()
    ref, lim = _pq_oracle(Q, C, codes)
    _check(got, ref, f"M={M} K={K} dsub={dsub} Nq={Nq} {method}", lim)


@pytest.mark.parametrize("M,dsub", [(16, 3), (40, 4), (10, 8), (48, 8)])
def test_pq_generic_shapes_take_lut_path(cuda, M, dsub):
    from tilemaxsim_amd import TileMaxSimPQ
    Q, C, codes = _mk(M + dsub, M, 64, dsub, 32, 50, 30)
    pq = TileMaxSimPQ(_gpu(C))
    got = pq.score_batch(_gpu(Q), _gpu(codes)).cpu().numpy()
    ref, lim = _pq_oracle(Q, C, codes)
    _check(got, ref, f"generic M={M} dsub={dsub}", lim)


def test_pq_bf16_int_codes_and_single(cuda):
    import torch
    from tilemaxsim_amd import TileMaxSimPQ
    rng = np.random.default_rng(8)
    C = torch.from_numpy(rng.standard_normal((16, 256, 8), dtype=np.float32)).to(torch.bfloat16)
    Q = torch.from_numpy(rng.standard_normal((32, 128), dtype=np.float32)).to(torch.bfloat16)
    codes = rng.integers(0, 256, size=(30, 64, 16)).astype(np.int32)
    pq = TileMaxSimPQ(C.cuda())
    ref, lim = _pq_oracle(Q.float().numpy(), C.float().numpy(), codes)
    for method in ("mfma", "lut"):
        got = pq.score_batch(Q.cuda(), _gpu(codes), method=method).cpu().numpy()
        _check(got, ref, f"bf16 {method}", lim)
    s = pq.score_single(Q.cuda(), _gpu(codes[4].astype(np.uint8)))
    assert s.dim() == 0
    _check(np.array([s.item()]), ref[4:5], "single", lim[4:5])


def test_pq_empty_and_invalid(cuda):
    import torch
    from tilemaxsim_amd import TileMaxSimPQ
    Q, C, _ = _mk(3, 16, 256, 8, 32, 1, 1)
    pq = TileMaxSimPQ(_gpu(C))
    e = torch.empty(4, 0, 16, dtype=torch.uint8, device="cuda")
    for method in ("mfma", "lut"):
        assert np.all(np.isneginf(pq.score_batch(_gpu(Q), e, method=method).cpu().numpy()))
    assert pq.score_batch(_gpu(Q), torch.empty(0, 5, 16, dtype=torch.uint8, device="cuda")).shape == (0,)
    pq16 = TileMaxSimPQ(_gpu(C[:, :16]))
    bad = torch.full((2, 3, 16), 20, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError):
        pq16.score_batch(_gpu(Q), bad)
    with pytest.raises(AssertionError):
        pq.score_batch(_gpu(Q), torch.zeros(2, 3, 8, dtype=torch.uint8, device="cuda"))


def test_pq_methods_agree_and_rank(cuda):
    """C5 shape at a bounded size: MFMA path vs table path (two algorithms) and the
    float64 oracle; top-100 identical up to ties within tolerance."""
    from tilemaxsim_amd import TileMaxSimPQ
    Q, C, codes = _mk(5, 16, 256, 8, 32, 6000, 128)
    pq = TileMaxSimPQ(_gpu(C))
    a = pq.score_batch(_gpu(Q), _gpu(codes), method="mfma").cpu().numpy()
    b = pq.score_batch(_gpu(Q), _gpu(codes), method="lut").cpu().numpy()
    ref, lim = _pq_oracle(Q, C, codes)
    _check(a, ref, "mfma", lim)
    _check(b, ref, "lut", lim)
    _check(a, b, "mfma vs lut")
    kth = np.sort(ref)[::-1][99]
    for got in (a, b):
        diff = set(orc.topk(got, 100)[1].tolist()) ^ set(orc.topk(ref, 100)[1].tolist())
        for i in diff:
            assert abs(ref[i] - kth) <= RTOL * abs(kth) + ATOL


# (M, K, dsub): every codeword width of the MFMA shapes, K < 256, d < 128
@pytest.mark.parametrize("M,K,dsub", [(16, 256, 8), (32, 256, 4), (64, 100, 2), (8, 256, 16), (4, 128, 32),
                                      (8, 256, 8), (12, 64, 8)])
def test_pq_batched_queries_formats(cuda, M, K, dsub):
    """tms_pq_score_batched: each tile decoded once and shared by the query blocks."""
    from tilemaxsim_amd import TileMaxSimPQ
    rng = np.random.default_rng(M * 1000 + K + dsub)
    Q, C, codes = _mk(M + dsub, M, K, dsub, 32, 700, 45)
    Qs = np.stack([Q] + [rng.standard_normal(Q.shape, dtype=np.float32).astype(np.float16) for _ in range(5)])
    pq = TileMaxSimPQ(_gpu(C))
    got = pq.score_batch_queries(_gpu(Qs), _gpu(codes)).cpu().numpy()
    assert got.shape == (6, 700)
    for q in range(6):
        ref, lim = _pq_oracle(Qs[q], C, codes)
        _check(got[q], ref, f"M={M} K={K} dsub={dsub} q={q}", lim)
    one = pq.score_batch(_gpu(Qs[5]), _gpu(codes)).cpu().numpy()
    _check(got[5], one, "batched vs one query")


# (nQ, Nq): 1 block per wave; 2 per wave; 4 per wave over two launches; 3 blocks per
# query; 4 blocks per query; 5 blocks per query (query by query); a single block
@pytest.mark.parametrize("nQ,nq", [(5, 32), (12, 32), (37, 32), (4, 70), (6, 128), (2, 150), (1, 32)])
def test_pq_batched_queries_shapes(cuda, nQ, nq):
    from tilemaxsim_amd import TileMaxSimPQ
    rng = np.random.default_rng(nQ * 100 + nq)
    _, C, codes = _mk(nQ + nq, 16, 256, 8, 1, 1500, 77)
    Qs = rng.standard_normal((nQ, nq, 128), dtype=np.float32)
    Qs = (Qs / np.linalg.norm(Qs, axis=-1, keepdims=True)).astype(np.float16)
    got = TileMaxSimPQ(_gpu(C)).score_batch_queries(_gpu(Qs), _gpu(codes)).cpu().numpy()
    for q in range(nQ):
        ref, lim = _pq_oracle(Qs[q], C, codes)
        _check(got[q], ref, f"nQ={nQ} nq={nq} q={q}", lim)


def test_pq_batched_queries_edges(cuda):
    import torch
    from tilemaxsim_amd import TileMaxSimPQ
    Q, C, codes = _mk(9, 16, 200, 8, 32, 300, 33)
    Qs = np.stack([Q, Q[::-1].copy(), Q * 2])
    pq = TileMaxSimPQ(_gpu(C))
    # codes >= K: rejected when validated, clamped into the table otherwise
    bad = codes.copy()
    bad[3, 5, 7] = 250
    with pytest.raises(ValueError):
        pq.score_batch_queries(_gpu(Qs), _gpu(bad))
    got = pq.score_batch_queries(_gpu(Qs), _gpu(bad), validate=False).cpu().numpy()
    for q in range(3):
        ref, lim = _pq_oracle(Qs[q], C, np.minimum(bad, 199))
        _check(got[q], ref, f"clamped q={q}", lim)
    # bf16 codebook and queries
    pqb = TileMaxSimPQ(_gpu(C).to(torch.bfloat16))
    got = pqb.score_batch_queries(_gpu(Qs).to(torch.bfloat16), _gpu(codes)).cpu().numpy()
    Cb = _gpu(C).to(torch.bfloat16).float().cpu().numpy()
    Qb = _gpu(Qs).to(torch.bfloat16).float().cpu().numpy()
    for q in range(3):
        ref, lim = _pq_oracle(Qb[q], Cb, codes)
        _check(got[q], ref, f"bf16 q={q}", lim)
    # no document tokens; no query tokens; no documents; no queries
    got = pq.score_batch_queries(_gpu(Qs), _gpu(codes[:, :0])).cpu().numpy()
    assert got.shape == (3, 300) and np.all(got == -np.inf)
    got = pq.score_batch_queries(_gpu(Qs[:, :0]), _gpu(codes)).cpu().numpy()
    assert np.all(got == 0.0)
    assert pq.score_batch_queries(_gpu(Qs), _gpu(codes[:0])).shape == (3, 0)
    assert pq.score_batch_queries(_gpu(Qs[:0]), _gpu(codes)).shape == (0, 300)
