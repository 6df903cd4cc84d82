"""CPU checks that pin the oracle (oracle/maxsim_oracle.py) to something other than itself.

The reference ships no input/output vectors for this path (its self-tests draw inputs
from the CUDA RNG and only print max |diff|), so each oracle function is pinned by
  * pure-Python float64 brute force on tiny inputs (a different code path),
  * closed forms and special cases the mathematics fixes,
  * invariants (permutation, duplication, zero padding, positive scaling, lengths),
  * the independent C restatement (oracle/maxsim_oracle.c) at mid sizes,
and the planted-mistake tests at the bottom show that those checks fail when a
plausible bug (dropped term, sum instead of max, wrong axis, off-by-one offset) is
put into an oracle copy.
"""
import itertools
import math

import numpy as np
import pytest

from oracle import c_oracle
from oracle import maxsim_oracle as orc


def _rng(s):
    return np.random.default_rng(s)


def _h(rng, shape, normalize=False):
    x = rng.standard_normal(shape, dtype=np.float32)
    if normalize:
        x /= np.linalg.norm(x, axis=-1, keepdims=True) + 1e-12
    return x.astype(np.float16)


# ---------------------------------------------------------------- brute force helpers
def brute_dense(Q, D, mask=None):
    Q = [[float(v) for v in row] for row in np.asarray(Q, np.float64)]
    out = []
    for b in range(D.shape[0]):
        rows = np.asarray(D[b], np.float64)
        total = 0.0
        for q in Q:
            best = -math.inf
            for j in range(rows.shape[0]):
                if mask is not None and not mask[b][j]:
                    continue
                s = 0.0
                for k in range(len(q)):
                    s += q[k] * float(rows[j, k])
                best = max(best, s)
            total += best
        out.append(total if Q else 0.0)
    return np.array(out)


def brute_pq(Q, C, codes):
    M, K, dsub = C.shape
    Qd = np.asarray(Q, np.float64)
    Cd = np.asarray(C, np.float64)
    out = []
    for b in range(codes.shape[0]):
        total = 0.0
        for i in range(Qd.shape[0]):
            best = -math.inf
            for t in range(codes.shape[1]):
                s = 0.0
                for m in range(M):
                    for j in range(dsub):
                        s += Qd[i, m * dsub + j] * Cd[m, codes[b, t, m], j]
                best = max(best, s)
            total += best
        out.append(total)
    return np.array(out)


# ---------------------------------------------------------------- dense
@pytest.mark.parametrize("Nq,Nd,d,B", [(1, 1, 1, 1), (3, 5, 7, 4), (4, 9, 16, 3), (2, 1, 8, 5)])
def test_dense_matches_brute_force(Nq, Nd, d, B):
    rng = _rng(Nq * 100 + Nd * 10 + d)
    Q, D = _h(rng, (Nq, d)), _h(rng, (B, Nd, d))
    ref = brute_dense(Q, D)
    np.testing.assert_allclose(orc.maxsim_f64(Q, D), ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(orc.maxsim_naive(Q, D), ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(orc.maxsim_loop(Q, D), ref, rtol=1e-5, atol=1e-5)


def test_single_token_is_a_dot_product():
    rng = _rng(1)
    q, d = _h(rng, (1, 64)), _h(rng, (1, 1, 64))
    expect = float(np.dot(q[0].astype(np.float64), d[0, 0].astype(np.float64)))
    assert orc.maxsim_f64(q, d)[0] == pytest.approx(expect, rel=1e-14)


def test_documents_containing_the_query_tokens():
    """If a document holds every (normalised) query token, each max is >= |q|^2 and
    <= |q| * max|d_j| (Cauchy-Schwarz), so the score is Nq up to fp16 rounding."""
    rng = _rng(2)
    Nq, d = 32, 128
    Q = _h(rng, (Nq, d), normalize=True)
    others = _h(rng, (1, 40, d), normalize=True)
    D = np.concatenate([others[:, :20], Q[None], others[:, 20:]], axis=1)
    s = orc.maxsim_f64(Q, D)[0]
    qn = np.linalg.norm(Q.astype(np.float64), axis=1)
    dn = np.linalg.norm(D[0].astype(np.float64), axis=1).max()
    assert (qn ** 2).sum() - 1e-9 <= s <= (qn * dn).sum() + 1e-9
    assert abs(s - Nq) < 0.05


def test_dense_invariants():
    rng = _rng(3)
    Q, D = _h(rng, (16, 48)), _h(rng, (6, 20, 48))
    base = orc.maxsim_f64(Q, D)
    # permuting doc tokens: each max is over the same set -> bit-identical
    assert np.array_equal(orc.maxsim_f64(Q, D[:, rng.permutation(20)]), base)
    # permuting query tokens: same terms, different sum order
    np.testing.assert_allclose(orc.maxsim_f64(Q[rng.permutation(16)], D), base, rtol=1e-13)
    # duplicating a doc token
    assert np.array_equal(orc.maxsim_f64(Q, np.concatenate([D, D[:, 3:4]], axis=1)), base)
    # zero-padding the embedding dimension
    pad = lambda x: np.concatenate([x, np.zeros(x.shape[:-1] + (80,), x.dtype)], axis=-1)
    np.testing.assert_allclose(orc.maxsim_f64(pad(Q), pad(D)), base, rtol=1e-13)
    # scaling the query by 2 (exact in fp16) scales the score by 2
    np.testing.assert_allclose(orc.maxsim_f64((Q.astype(np.float32) * 2).astype(np.float16), D), 2 * base, rtol=1e-13)
    # empty documents score -inf, no query tokens scores 0
    assert np.all(np.isneginf(orc.maxsim_f64(Q, D[:, :0])))
    assert np.all(orc.maxsim_naive(Q[:0], D) == 0)


def test_masked_and_varlen_pins():
    rng = _rng(4)
    Q = _h(rng, (8, 24))
    D = _h(rng, (5, 12, 24))
    mask = rng.random((5, 12)) < 0.5
    mask[0] = False
    mask[1] = True
    ref = brute_dense(Q, D, mask)
    np.testing.assert_allclose(orc.maxsim_masked(Q, D, mask, f64=True), ref, rtol=1e-12)
    np.testing.assert_allclose(orc.maxsim_masked(Q, D, mask), ref, rtol=1e-5)
    assert np.array_equal(orc.maxsim_masked(Q, D, np.ones((5, 12), bool), f64=True), orc.maxsim_f64(Q, D))
    # varlen over the compacted valid tokens == masked
    lens = mask.sum(1)
    offsets = np.concatenate([[0], np.cumsum(lens)])
    flat = np.concatenate([D[b][mask[b]] for b in range(5)], axis=0)
    np.testing.assert_allclose(orc.maxsim_varlen(Q, flat, offsets, f64=True), ref, rtol=1e-12)
    # varlen == per-document dense on each slice
    for b in range(5):
        if lens[b]:
            np.testing.assert_allclose(orc.maxsim_varlen(Q, flat, offsets, f64=True)[b],
                                       orc.maxsim_f64(Q, flat[offsets[b]:offsets[b + 1]][None])[0], rtol=1e-13)


def test_varlen_empty_docs_everywhere():
    rng = _rng(5)
    Q = _h(rng, (4, 8))
    lens = np.array([0, 3, 0, 0, 2, 1, 0])
    offsets = np.concatenate([[0], np.cumsum(lens)])
    flat = _h(rng, (int(offsets[-1]), 8))
    got = orc.maxsim_varlen(Q, flat, offsets, f64=True)
    for b in range(7):
        if lens[b] == 0:
            assert np.isneginf(got[b])
        else:
            assert got[b] == pytest.approx(brute_dense(Q, flat[offsets[b]:offsets[b + 1]][None])[0], rel=1e-12)


def test_c_restatement_agrees_at_mid_size():
    rng = _rng(6)
    Q = _h(rng, (32, 128), normalize=True)
    D = _h(rng, (200, 70, 128), normalize=True)
    np.testing.assert_allclose(c_oracle.maxsim_dense(Q, D), orc.maxsim_f64(Q, D), rtol=1e-12)
    mask = rng.random((200, 70)) < 0.3
    np.testing.assert_allclose(c_oracle.maxsim_masked(Q, D, mask), orc.maxsim_masked(Q, D, mask, f64=True), rtol=1e-12)
    lens = rng.integers(0, 50, size=300)
    offsets = np.concatenate([[0], np.cumsum(lens)])
    flat = _h(rng, (int(offsets[-1]), 128))
    np.testing.assert_allclose(c_oracle.maxsim_varlen(Q, flat, offsets), orc.maxsim_varlen(Q, flat, offsets, f64=True),
                               rtol=1e-12)


# ---------------------------------------------------------------- PQ
def test_pq_lut_is_the_subspace_gemm():
    rng = _rng(7)
    M, K, dsub = 4, 5, 3
    Q, C = _h(rng, (2, M * dsub)), _h(rng, (M, K, dsub))
    T = orc.pq_build_lut(Q, C)
    for q, m, k in itertools.product(range(2), range(M), range(K)):
        expect = sum(float(Q[q, m * dsub + j]) * float(C[m, k, j]) for j in range(dsub))
        assert T[q, m, k] == pytest.approx(expect, rel=1e-6, abs=1e-6)
    np.testing.assert_allclose(c_oracle.pq_build_lut(Q, C), T, rtol=1e-6, atol=1e-6)


def test_pq_score_matches_brute_force_and_both_algorithms_agree():
    rng = _rng(8)
    M, K, dsub = 4, 8, 2
    Q, C = _h(rng, (3, M * dsub)), _h(rng, (M, K, dsub))
    codes = rng.integers(0, K, size=(5, 6, M)).astype(np.uint8)
    ref = brute_pq(Q, C, codes)
    np.testing.assert_allclose(orc.pq_decompress_score(Q, C, codes, f64=True), ref, rtol=1e-12)
    np.testing.assert_allclose(orc.pq_decompress_score(Q, C, codes), ref, rtol=1e-5)
    np.testing.assert_allclose(orc.pq_score_lut(orc.pq_build_lut(Q, C), codes), ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(c_oracle.pq_score(Q, C, codes), ref, rtol=1e-12)


def test_pq_single_centroid_is_closed_form():
    """K = 1: every token decodes to the same vector v, so score = sum_q <q, v>."""
    rng = _rng(9)
    M, dsub = 16, 8
    Q, C = _h(rng, (32, M * dsub)), _h(rng, (M, 1, dsub))
    codes = np.zeros((3, 10, M), np.uint8)
    v = C[:, 0, :].reshape(-1).astype(np.float64)
    expect = float((Q.astype(np.float64) @ v).sum())
    np.testing.assert_allclose(orc.pq_decompress_score(Q, C, codes, f64=True), expect, rtol=1e-12)
    np.testing.assert_allclose(orc.pq_score_lut(orc.pq_build_lut(Q, C), codes), expect, rtol=1e-5)


def test_pq_mid_size_c_restatement():
    rng = _rng(10)
    M, K, dsub = 16, 256, 8
    Q, C = _h(rng, (32, 128), normalize=True), _h(rng, (M, K, dsub))
    codes = rng.integers(0, K, size=(40, 64, M)).astype(np.uint8)
    np.testing.assert_allclose(c_oracle.pq_score(Q, C, codes), orc.pq_decompress_score(Q, C, codes, f64=True),
                               rtol=1e-12)
    np.testing.assert_allclose(orc.pq_score_lut(orc.pq_build_lut(Q, C), codes),
                               orc.pq_decompress_score(Q, C, codes, f64=True), rtol=1e-5)


def test_topk_ties_break_by_index():
    v, i = orc.topk(np.array([1.0, 3.0, 3.0, 2.0]), 3)
    assert i.tolist() == [1, 2, 3] and v.tolist() == [3.0, 3.0, 2.0]


def _brute_topk(x, k):
    order = sorted(range(len(x)), key=lambda j: (-float(x[j]), j))[:k]
    return [float(x[j]) for j in order], order


@pytest.mark.parametrize("n,k", [(1, 1), (7, 7), (50, 10), (300, 100)])
def test_topk_matches_brute_force_and_sort(n, k):
    rng = _rng(n + k)
    x = np.round(rng.standard_normal(n) * 3).astype(np.float32)  # many exact ties
    x[rng.integers(0, n)] = np.inf
    x[rng.integers(0, n)] = -np.inf
    v, i = orc.topk(x, k)
    bv, bi = _brute_topk(x, k)
    assert i.tolist() == bi and v.tolist() == bv
    assert np.array_equal(v, np.sort(x)[::-1][:k])  # values: the library sort
    rest = np.delete(x, i)
    assert rest.size == 0 or rest.max() <= v.min()  # nothing left out beats what was kept


def test_topk_signed_zero_and_nan():
    """-0.0 ties with +0.0 (by index), and a NaN of either sign ranks above +inf."""
    neg_nan = np.array([0xFFC00000], dtype=np.uint32).view(np.float32)[0]
    x = np.array([1.0, -0.0, 0.0, -0.0, np.inf, neg_nan, -1.0, np.nan], dtype=np.float32)
    v, i = orc.topk(x, 8)
    assert i.tolist() == [5, 7, 4, 0, 1, 2, 3, 6]
    assert np.signbit(v[4]) and not np.signbit(v[5]) and np.signbit(v[6])  # values keep their bits
    # brute force over the same rule (NaN -> above +inf; -0.0 == 0.0)
    key = [(0 if np.isnan(t) else 1, -float(t) if not np.isnan(t) else 0.0, j) for j, t in enumerate(x)]
    assert [j for *_, j in sorted(key)] == i.tolist()


def test_planted_topk_mistakes_are_caught():
    x = np.array([2.0, 5.0, 5.0, 1.0, 5.0, 3.0], dtype=np.float32)
    bv, bi = _brute_topk(x, 4)
    ascending = np.argsort(x, kind="stable")[:4]
    ties_high_first = np.argsort(x, kind="stable")[::-1][:4]  # ties by the higher index
    assert ascending.tolist() != bi and ties_high_first.tolist() != bi
    assert orc.topk(x, 4)[1].tolist() == bi == [1, 2, 4, 5]


# ---------------------------------------------------------------- planted mistakes
# Each mutant is a plausible oracle bug; the pins above must reject it.
def _mut_sum_instead_of_max(Q, D):
    S = np.einsum("bnd,qd->bnq", D.astype(np.float64), Q.astype(np.float64))
    return S.sum(axis=1).sum(axis=1)


def _mut_drop_last_dim(Q, D):
    return orc.maxsim_f64(Q[:, :-1], D[:, :, :-1])


def _mut_max_over_queries(Q, D):
    S = np.einsum("bnd,qd->bnq", D.astype(np.float64), Q.astype(np.float64))
    return S.max(axis=2).sum(axis=1)


@pytest.mark.parametrize("mutant", [_mut_sum_instead_of_max, _mut_drop_last_dim, _mut_max_over_queries])
def test_planted_dense_mistakes_are_caught(mutant):
    rng = _rng(11)
    Q, D = _h(rng, (3, 5)), _h(rng, (4, 6, 5))
    assert not np.allclose(mutant(Q, D), brute_dense(Q, D), rtol=1e-3)


def test_planted_varlen_off_by_one_is_caught():
    rng = _rng(12)
    Q = _h(rng, (4, 8))
    lens = np.array([3, 5, 2])
    offsets = np.concatenate([[0], np.cumsum(lens)])
    flat = _h(rng, (10, 8))
    bad = offsets.copy()
    bad[1:-1] += 1  # each document starts one token late
    good = [brute_dense(Q, flat[offsets[b]:offsets[b + 1]][None])[0] for b in range(3)]
    assert not np.allclose(orc.maxsim_varlen(Q, flat, bad, f64=True), good, rtol=1e-3)
    np.testing.assert_allclose(orc.maxsim_varlen(Q, flat, offsets, f64=True), good, rtol=1e-12)


def test_planted_pq_transposed_codebook_is_caught():
    rng = _rng(13)
    M, K, dsub = 4, 4, 4
    Q, C = _h(rng, (2, M * dsub)), _h(rng, (M, K, dsub))
    codes = rng.integers(0, K, size=(3, 5, M)).astype(np.uint8)
    wrong = orc.pq_decompress_score(Q, np.ascontiguousarray(C.transpose(1, 0, 2)), codes, f64=True)
    assert not np.allclose(wrong, brute_pq(Q, C, codes), rtol=1e-3)


def test_packed_zero_padding_pins():
    """The PLAID drop-in's zero padding: a shorter document's per-token max is at least
    0; a document at the batch's max length is unaffected; an empty one scores 0."""
    rng = _rng(14)
    Q = _h(rng, (6, 16))
    lens = np.array([3, 7, 0, 7, 1])
    offsets = np.concatenate([[0], np.cumsum(lens)])
    flat = _h(rng, (int(offsets[-1]), 16))
    got = orc.maxsim_packed_zero_padded(Q, flat, lens)
    for b in range(5):
        rows = flat[offsets[b]:offsets[b + 1]].astype(np.float64)
        per_q = [max([float(np.dot(q.astype(np.float64), r)) for r in rows] + ([0.0] if lens[b] < 7 else []))
                 for q in Q]
        assert got[b] == pytest.approx(sum(per_q), rel=1e-12, abs=1e-12)
    full = orc.maxsim_varlen(Q, flat, offsets, f64=True)
    assert got[1] == pytest.approx(full[1], rel=1e-13) and got[3] == pytest.approx(full[3], rel=1e-13)
    assert got[2] == 0.0


# ---------------------------------------------------------------- torch restatement
def test_torch_restatement_matches_numpy_oracle():
    """oracle/torch_ref.py (the CPU baseline bench.py times) against the pinned numpy
    oracle: dense, variable-length (padded and masked) and PQ decompress-then-score."""
    import torch
    from oracle import torch_ref as tr
    rng = _rng(314)
    Q = rng.standard_normal((32, 64)).astype(np.float16)
    D = rng.standard_normal((70, 23, 64)).astype(np.float16)
    np.testing.assert_allclose(tr.maxsim_naive(torch.from_numpy(Q), torch.from_numpy(D), chunk=16).numpy(),
                               orc.maxsim_f64(Q, D), rtol=1e-5, atol=1e-5)
    lens = rng.integers(1, 40, size=55)
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    Df = rng.standard_normal((int(offs[-1]), 64)).astype(np.float16)
    got = tr.maxsim_varlen_masked(torch.from_numpy(Q), torch.from_numpy(Df), torch.from_numpy(offs), chunk=9)
    np.testing.assert_allclose(got.numpy(), orc.maxsim_varlen(Q, Df, offs, f64=True), rtol=1e-5, atol=1e-5)
    C = rng.standard_normal((8, 40, 8)).astype(np.float16)
    codes = rng.integers(0, 40, size=(33, 11, 8)).astype(np.uint8)
    got = tr.pq_decompress_score(torch.from_numpy(Q), torch.from_numpy(C), torch.from_numpy(codes), chunk=10)
    np.testing.assert_allclose(got.numpy(), orc.pq_decompress_score(Q, C, codes, f64=True), rtol=1e-5, atol=1e-5)
