"""GPU parity of the residual-compressed (ColBERTv2) path against oracle/residual_oracle.py.

* tms_residual_decompress: fp16 outputs equal to the oracle's restatement of the codec
  (same half add, fp32 norm, fp32 division) up to 1 fp16 ulp; only the fp32 summation
  order of the norm differs, and it can move a rounding boundary;
* tms_maxsim_residual: |score - oracle| <= 1e-3 relative + 1e-3 absolute, the scoring
  bar of every path; the oracle scores the decompressed fp16 tokens in float64;
* and, tighter, each kernel against its own arithmetic restated in float64
  (``residual_oracle.maxsim_residual_kernel_envelope``): the single-query kernel scores
  <q, v> / fp16(|v|) without rounding the normalised token to fp16, the batched kernel
  rounds x = fp16(v * fp32(1 / fp16(|v|))); where a token's fp16 norm can round either
  way (its fp32 sum of squares depends on the order) both are taken. The score must lie
  in that envelope widened by the fp32-accumulation bar ``accum_bar.bound``.
  Against the codec's decompress-then-score, a norm that rounds the other way rescales
  a whole token by one fp16 ulp, and the unrounded token differs from the codec's by up
  to half an ulp per element, so the seeded sweep's codec check adds 3 * 2^-11 *
  MaxSim(|Q|, |X|) to the 1e-3 bar (a one-token document whose 64 query maxima cancel
  to 0.08 moved by 1.1e-3 that way).
"""
import os

import numpy as np
import pytest

from oracle import maxsim_oracle as mo
from oracle import residual_oracle as ro

pytestmark = pytest.mark.gpu

RTOL = 1e-3
ATOL = 1e-3


@pytest.fixture(params=["default", "split", "whole"])
def fused_path(request):
    """The fused kernel's tests run at the default dispatch, with documents split over
    waves for every call small enough (tms_set_rerank_limit raised), and with every wave
    walking whole documents (limit 0)."""
    from tilemaxsim_amd import _lib
    limit = {"default": None, "split": 1 << 40, "whole": 0}[request.param]
    if limit is None:
        yield request.param
        return
    with _lib.rerank_limit(limit):
        yield request.param


def _index(rng, T, d, nbits, ncent):
    """A synthetic index: unit-norm fp16 centroids, random codes and residual buckets,
    bucket weights at the quantiles of a small residual distribution (as the codec fits
    them)."""
    C = rng.standard_normal((ncent, d)).astype(np.float32)
    C /= np.linalg.norm(C, axis=1, keepdims=True)
    codes = rng.integers(0, ncent, T).astype(np.int32)
    buckets = rng.integers(0, 1 << nbits, (T, d)).astype(np.uint8)
    w = np.sort(rng.normal(0, 0.05, 1 << nbits)).astype(np.float16)
    return C.astype(np.float16), codes, ro.pack_buckets(buckets, nbits), w


def _gpu(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _form(nQ, nq):
    """The kernel tms_maxsim_residual_batched takes: the batched one for at most 4 query
    blocks of 32 tokens per query and at least 2 blocks in all, else one query at a time."""
    nbq = (nq + 31) // 32
    return "batched" if nbq <= 4 and nQ * nbq >= 2 else "fused"


def _assert_kernel(got, Q, idx_np, offsets, pids, pad_len, form, what=""):
    """got within [lo, hi] of the kernel's own arithmetic, widened by the fp32-accumulation
    bar (two more roundings for the multiply by 1 / |v|)."""
    import accum_bar as bar
    codes, res, C, w, nbits = idx_np
    lo, hi, absref = ro.maxsim_residual_kernel_envelope(Q, codes, res, C, w, nbits, offsets, pids, pad_len, form=form)
    got = np.asarray(got, dtype=np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(lo)), f"{what}: NaN pattern differs"
    assert np.array_equal(np.isinf(got), np.isinf(lo)), f"{what}: inf pattern differs"
    assert np.all(got[np.isinf(lo)] == lo[np.isinf(lo)]), what
    fin = np.isfinite(lo)
    b = bar.bound(absref, Q.shape[1] + 2, Q.shape[0])
    below, above = got[fin] < lo[fin] - b[fin], got[fin] > hi[fin] + b[fin]
    assert not below.any() and not above.any(), (
        f"{what}: {int(below.sum() + above.sum())} scores outside the {form} envelope, worst "
        f"{float(np.max(np.maximum(lo[fin] - got[fin], got[fin] - hi[fin]) / b[fin])):.2f} x the bar")
    return absref


def _assert_scores(got, ref, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), f"{what}: NaN pattern differs"
    assert np.array_equal(np.isinf(got), np.isinf(ref)), f"{what}: inf pattern differs"
    fin = np.isfinite(ref)
    assert np.all(got[np.isinf(ref)] == ref[np.isinf(ref)]), what
    np.testing.assert_allclose(got[fin], ref[fin], rtol=RTOL, atol=ATOL, err_msg=what)


@pytest.mark.parametrize("nbits", [1, 2, 4])
@pytest.mark.parametrize("d", [32, 64, 96, 128])
def test_decompress_matches_codec(cuda, nbits, d):
    from tilemaxsim_amd import decompress_residual
    rng = np.random.default_rng(100 * nbits + d)
    T = 3001
    C, codes, res, w = _index(rng, T, d, nbits, 97)
    got = decompress_residual(_gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits).cpu().numpy()
    ref = ro.decompress(codes, res, C, w, nbits)
    assert got.shape == (T, d) and got.dtype == np.float16
    ulps = np.abs(got.view(np.int16).astype(np.int32) - ref.view(np.int16).astype(np.int32))
    assert ulps.max() <= 1, f"max ulp difference {ulps.max()}"
    assert (ulps == 0).mean() > 0.99
    # int64 codes take the same path
    got64 = decompress_residual(_gpu(codes.astype(np.int64)), _gpu(res), _gpu(C), _gpu(w), nbits).cpu().numpy()
    assert np.array_equal(got64, got)


# Residual rows written byte by byte, with each dimension's bucket derived by hand from
# the format (per dimension, bits 0..nbits-1 of the bucket, least significant first, enter
# one bit stream that fills each byte from its most significant bit), not by the oracle:
#   nbits=1: 0xA5 = 1010 0101 -> 1,0,1,0,0,1,0,1; 0x0F -> 0,0,0,0,1,1,1,1; 0x80 -> 1,0..0;
#            0x01 -> 0..0,1
#   nbits=2: 0xC9 = 11 00 10 01 -> 3,0,1,2; 0x1B = 00 01 10 11 -> 0,2,1,3; 0xFF -> 3,3,3,3;
#            0x80 -> 1,0,0,0; 0x40 -> 2,0,0,0; 0x01 -> 0,0,0,2; 0x02 -> 0,0,0,1
#   nbits=4: 0x3C = 0011 1100 -> 12,3; 0x81 -> 1,8; 0xF0 -> 15,0; 0x96 = 1001 0110 -> 9,6;
#            0x07 -> 0,14
_HAND_ROWS = {
    1: ([0xA5, 0x0F, 0x80, 0x01],
        [1, 0, 1, 0, 0, 1, 0, 1] + [0, 0, 0, 0, 1, 1, 1, 1] + [1] + [0] * 7 + [0] * 7 + [1]),
    2: ([0xC9, 0x1B, 0x00, 0xFF, 0x80, 0x40, 0x01, 0x02],
        [3, 0, 1, 2, 0, 2, 1, 3, 0, 0, 0, 0, 3, 3, 3, 3, 1, 0, 0, 0, 2, 0, 0, 0, 0, 0, 0, 2, 0, 0, 0, 1]),
    4: ([0x3C, 0x81, 0xF0, 0x96] + [0x00] * 11 + [0x07],
        [12, 3, 1, 8, 15, 0, 9, 6] + [0] * 22 + [0, 14]),
}
_HAND_WEIGHTS = {1: [-0.5, 0.25], 2: [-0.5, -0.125, 0.25, 1.0], 4: [(i - 7.5) / 8 for i in range(16)]}


@pytest.mark.parametrize("nbits", [1, 2, 4])
def test_decompress_hand_built_bytes(cuda, nbits):
    """tms_residual_decompress on residual bytes written by hand, against the closed form
    v = centroid[code] + weight[bucket] (every value exact in fp16), out = v / |v|."""
    from tilemaxsim_amd import decompress_residual
    d = 32
    row, buckets = _HAND_ROWS[nbits]
    assert len(row) == d * nbits // 8 and len(buckets) == d
    res = np.array([row, row], dtype=np.uint8)
    C = np.zeros((3, d), dtype=np.float16)
    C[2] = 0.25
    codes = np.array([0, 2], dtype=np.int32)
    w = np.array(_HAND_WEIGHTS[nbits], dtype=np.float16)
    got = decompress_residual(_gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits).cpu().numpy().astype(np.float64)
    wb = np.array([_HAND_WEIGHTS[nbits][b] for b in buckets], dtype=np.float64)
    for t, base in enumerate((0.0, 0.25)):
        v = base + wb
        expect = v / np.linalg.norm(v)
        # fp16 norm and fp16 output: within 2 fp16 ulps of the exact quotient
        np.testing.assert_allclose(got[t], expect, rtol=2 * 2.0 ** -10, atol=2.0 ** -24, err_msg=f"token {t}")


@pytest.mark.parametrize("nbits,d,nq", [(2, 128, 32), (1, 128, 32), (4, 128, 32), (2, 64, 20), (2, 32, 1),
                                        (2, 96, 33), (4, 128, 64), (2, 128, 100)])
@pytest.mark.parametrize("padding", ["zeros", "mask"])
def test_fused_maxsim_matches_oracle(cuda, fused_path, nbits, d, nq, padding):
    from tilemaxsim_amd import flashmaxsim_score_residual
    rng = np.random.default_rng(nbits * 1000 + d + nq)
    ndocs = 900
    lens = rng.integers(0, 160, ndocs)
    lens[::37] = 0
    lens[5] = 300
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(offsets[-1])
    C, codes, res, w = _index(rng, T, d, nbits, 517)
    Q = rng.standard_normal((nq, d)).astype(np.float32)
    Q /= np.linalg.norm(Q, axis=1, keepdims=True)
    Q = Q.astype(np.float16)
    got = flashmaxsim_score_residual(_gpu(Q), _gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits, _gpu(offsets),
                                     padding=padding).cpu().numpy()
    pad_len = int(lens.max()) if padding == "zeros" else 0
    ref = ro.maxsim_residual(Q, codes, res, C, w, nbits, offsets, None, pad_len)
    _assert_scores(got, ref, f"nbits={nbits} d={d} nq={nq} {padding}")
    _assert_kernel(got, Q, (codes, res, C, w, nbits), offsets, None, pad_len, "fused",
                   f"nbits={nbits} d={d} nq={nq} {padding}")


@pytest.mark.parametrize("nbits,d", [(1, 128), (2, 128), (4, 128), (2, 64), (4, 64), (1, 32), (2, 96)])
def test_fused_residual_offsets_alignment(cuda, fused_path, nbits, d):
    """A residuals view that starts nbits bytes into its buffer is aligned for one chunk
    but not for a lane's whole run of chunks, so the fused kernel reads it chunk by chunk;
    the aligned tensor takes one load per token. Both read the same bytes: bit-identical
    scores, and both within tolerance of the oracle."""
    import torch
    from tilemaxsim_amd import flashmaxsim_score_residual
    rng = np.random.default_rng(7 * nbits + d)
    lens = rng.integers(0, 120, 300)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(offsets[-1])
    C, codes, res, w = _index(rng, T, d, nbits, 129)
    Q = rng.standard_normal((32, d)).astype(np.float32)
    Q /= np.linalg.norm(Q, axis=1, keepdims=True)
    Q = Q.astype(np.float16)
    rb = res.shape[1]
    buf = torch.zeros(T * rb + nbits, dtype=torch.uint8, device="cuda")
    buf[nbits:] = _gpu(res.reshape(-1))
    shifted = buf[nbits:].view(T, rb)
    assert shifted.data_ptr() % nbits == 0 and shifted.data_ptr() % (2 * nbits) != 0
    args = (_gpu(C), _gpu(w), nbits, _gpu(offsets))
    got_a = flashmaxsim_score_residual(_gpu(Q), _gpu(codes), _gpu(res), *args, padding="mask").cpu().numpy()
    got_s = flashmaxsim_score_residual(_gpu(Q), _gpu(codes), shifted, *args, padding="mask").cpu().numpy()
    assert np.array_equal(got_a, got_s, equal_nan=True)
    _assert_scores(got_a, ro.maxsim_residual(Q, codes, res, C, w, nbits, offsets), f"nbits={nbits} d={d}")


def test_fused_candidates_match_packed_scoring(cuda, fused_path):
    """PLAID's flow: pick candidate pids, decompress their tokens, score them packed.
    The fused kernel must give the same scores without the decompressed copy."""
    import torch
    from tilemaxsim_amd import decompress_residual, flashmaxsim_score_packed, flashmaxsim_score_residual
    rng = np.random.default_rng(77)
    d, nbits, ndocs = 128, 2, 4000
    lens = rng.integers(20, 180, ndocs)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    C, codes, res, w = _index(rng, int(offsets[-1]), d, nbits, 1024)
    Q = rng.standard_normal((32, d)).astype(np.float32)
    Q = (Q / np.linalg.norm(Q, axis=1, keepdims=True)).astype(np.float16)
    pids = rng.choice(ndocs, 700, replace=False).astype(np.int64)
    pids[10] = pids[11]  # a duplicate candidate
    fused = flashmaxsim_score_residual(_gpu(Q), _gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits, _gpu(offsets),
                                       _gpu(pids)).cpu().numpy()
    rows = np.concatenate([np.arange(offsets[p], offsets[p + 1]) for p in pids])
    D = decompress_residual(_gpu(codes[rows]), _gpu(res[rows]), _gpu(C), _gpu(w), nbits)
    packed = flashmaxsim_score_packed(_gpu(Q), D, torch.from_numpy(lens[pids])).cpu().numpy()
    np.testing.assert_allclose(fused, packed, rtol=2e-4, atol=2e-4)
    ref = ro.maxsim_residual(Q, codes, res, C, w, nbits, offsets, pids, int(lens[pids].max()))
    _assert_scores(fused, ref, "candidates")
    assert fused[10] == fused[11]
    # top-100 identical except swaps within tolerance of the 100th score
    kth = np.sort(ref)[::-1][99]
    diff = set(np.argsort(-fused, kind="stable")[:100].tolist()) ^ set(mo.topk(ref, 100)[1].tolist())
    for i in diff:
        assert abs(ref[i] - kth) <= RTOL * abs(kth) + ATOL


def test_invalid_documents_and_codes(cuda, fused_path):
    from tilemaxsim_amd import flashmaxsim_score_residual
    rng = np.random.default_rng(5)
    d, nbits = 64, 2
    lens = np.array([5, 0, 7, 3])
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    C, codes, res, w = _index(rng, int(offsets[-1]), d, nbits, 11)
    Q = rng.standard_normal((8, d)).astype(np.float16)
    args = (_gpu(Q), _gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits, _gpu(offsets))
    pids = np.array([3, -1, 4, 1, 0], dtype=np.int64)
    with pytest.raises(ValueError):
        flashmaxsim_score_residual(*args, _gpu(pids))
    got = flashmaxsim_score_residual(*args, _gpu(pids), padding="mask", validate=False).cpu().numpy()
    ref = ro.maxsim_residual(Q, codes, res, C, w, nbits, offsets, pids, 0)
    assert np.isnan(got[1]) and np.isnan(got[2]) and got[3] == -np.inf
    _assert_scores(got, ref, "invalid pids")
    # centroid ids outside [0, C) are clamped to the table, never read out of bounds
    bad = codes.copy()
    bad[0], bad[3] = 11, -4
    clamped = np.clip(bad, 0, 10).astype(np.int32)
    got = flashmaxsim_score_residual(_gpu(Q), _gpu(bad), _gpu(res), _gpu(C), _gpu(w), nbits, _gpu(offsets),
                                     padding="mask").cpu().numpy()
    _assert_scores(got, ro.maxsim_residual(Q, clamped, res, C, w, nbits, offsets), "clamped codes")


@pytest.mark.parametrize("nbits,d,nq", [(2, 128, 32), (1, 64, 20), (4, 96, 70), (2, 32, 1)])
@pytest.mark.parametrize("B", [1, 3, 37, 700, 2047])
def test_split_documents_same_bits(cuda, nbits, d, nq, B):
    """Small candidate lists split each document over 2 or 4 waves (its tiles p, p + wpd,
    ...), whose maxima meet in LDS. The scores must be the bits of the whole-document walk
    (the same tile sums, exact maxima, the same summation order) and match the oracle, for
    both paddings, with duplicate, invalid and empty candidates."""
    from tilemaxsim_amd import _lib, flashmaxsim_score_residual
    rng = np.random.default_rng(B * 10 + nbits + d + nq)
    ndocs = 3000
    lens = rng.integers(1, 260, ndocs)
    lens[::29] = 0
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    C, codes, res, w = _index(rng, int(offsets[-1]), d, nbits, 333)
    Q = rng.standard_normal((nq, d)).astype(np.float32)
    Q = (Q / np.linalg.norm(Q, axis=1, keepdims=True)).astype(np.float16)
    pids = rng.integers(0, ndocs, B).astype(np.int64)
    if B > 3:
        pids[1] = pids[2]                       # a duplicate candidate
        pids[3] = int(np.nonzero(lens == 0)[0][0])  # an empty document
    args = (_gpu(Q), _gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits, _gpu(offsets), _gpu(pids))
    for padding in ("zeros", "mask"):
        with _lib.rerank_limit(1 << 40):
            split = flashmaxsim_score_residual(*args, padding=padding).cpu().numpy()
        with _lib.rerank_limit(0):
            whole = flashmaxsim_score_residual(*args, padding=padding).cpu().numpy()
        assert np.array_equal(split.view(np.uint32), whole.view(np.uint32)), f"B={B} {padding}"
        pad_len = int(lens[pids].max()) if padding == "zeros" else 0
        ref = ro.maxsim_residual(Q, codes, res, C, w, nbits, offsets, pids, pad_len)
        _assert_scores(split, ref, f"B={B} nbits={nbits} d={d} nq={nq} {padding}")
    if B > 3:  # invalid candidates score NaN on both paths
        bad = pids.copy()
        bad[0], bad[-1] = -5, ndocs + 2
        args = args[:-1] + (_gpu(bad),)
        with _lib.rerank_limit(1 << 40):
            split = flashmaxsim_score_residual(*args, padding="mask", validate=False).cpu().numpy()
        with _lib.rerank_limit(0):
            whole = flashmaxsim_score_residual(*args, padding="mask", validate=False).cpu().numpy()
        assert np.isnan(split[0]) and np.isnan(split[-1])
        assert np.array_equal(split.view(np.uint32), whole.view(np.uint32))


def test_edge_sizes(cuda, fused_path):
    import torch
    from tilemaxsim_amd import decompress_residual, flashmaxsim_score_residual
    rng = np.random.default_rng(9)
    d, nbits = 128, 2
    C, codes, res, w = _index(rng, 40, d, nbits, 3)
    Q = rng.standard_normal((32, d)).astype(np.float16)
    # one document of one token; every document empty; no query tokens; no documents
    one = np.array([0, 1], dtype=np.int64)
    got = flashmaxsim_score_residual(_gpu(Q), _gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits, _gpu(one))
    _assert_scores(got.cpu().numpy(), ro.maxsim_residual(Q, codes, res, C, w, nbits, one, None, 1), "one token")
    empty = np.zeros(6, dtype=np.int64)  # all empty: nothing to pad to, so -inf either way
    for padding in ("zeros", "mask"):
        got = flashmaxsim_score_residual(_gpu(Q), _gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits, _gpu(empty),
                                         padding=padding)
        assert np.all(got.cpu().numpy() == -np.inf)
    some = np.array([0, 0, 0, 3, 3], dtype=np.int64)  # empties beside a 3-token document
    got = flashmaxsim_score_residual(_gpu(Q), _gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits, _gpu(some))
    assert got.cpu().numpy()[[0, 1, 3]].tolist() == [0.0, 0.0, 0.0]  # zero padding: each max is 0
    _assert_scores(got.cpu().numpy(), ro.maxsim_residual(Q, codes, res, C, w, nbits, some, None, 3), "some")
    got = flashmaxsim_score_residual(_gpu(Q[:0]), _gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits,
                                     _gpu(np.array([0, 10, 40])))
    assert np.all(got.cpu().numpy() == 0.0)
    got = flashmaxsim_score_residual(_gpu(Q), _gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits,
                                     _gpu(np.array([0, 40])), pids=_gpu(np.zeros(0, np.int64)))
    assert got.shape == (0,)
    assert decompress_residual(_gpu(codes[:0]), _gpu(res[:0]), _gpu(C), _gpu(w), nbits).shape == (0, d)
    with pytest.raises(NotImplementedError):
        decompress_residual(_gpu(codes), _gpu(res), _gpu(C), _gpu(w), 3)
    with pytest.raises(ValueError):
        decompress_residual(_gpu(codes), _gpu(res[:, :16]), _gpu(C), _gpu(w), nbits)
    with pytest.raises(NotImplementedError):  # d not in {32, 64, 96, 128}
        Cw = torch.zeros(3, 256, dtype=torch.float16, device="cuda")
        decompress_residual(_gpu(codes), torch.zeros(40, 64, dtype=torch.uint8, device="cuda"), Cw, _gpu(w), nbits)


def _queries(rng, nQ, nq, d):
    Q = rng.standard_normal((nQ, nq, d)).astype(np.float32)
    Q /= np.linalg.norm(Q, axis=2, keepdims=True)
    return Q.astype(np.float16)


# (nQ, Nq): 1 block per wave with idle waves; 2 per wave; two queries of 2 blocks per
# wave over two launches; 4 per wave over two launches, the second partial; queries of
# 4 blocks (Nq not a multiple of 32); Nq = 130 (5 blocks: one query at a time); a single
# block (the one-query kernel)
@pytest.mark.parametrize("nQ,nq", [(2, 32), (5, 20), (12, 32), (9, 64), (37, 32), (3, 100), (2, 130), (1, 32)])
def test_batched_maxsim_matches_oracle(cuda, nQ, nq):
    from tilemaxsim_amd import flashmaxsim_score_residual, flashmaxsim_score_residual_batched
    rng = np.random.default_rng(nQ * 100 + nq)
    d, nbits, ndocs = 128, 2, 700
    lens = rng.integers(0, 200, ndocs)
    lens[::29] = 0
    lens[3] = 1
    lens[7] = 333
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    C, codes, res, w = _index(rng, int(offsets[-1]), d, nbits, 301)
    Qs = _queries(rng, nQ, nq, d)
    idx = (_gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits, _gpu(offsets))
    for padding in ("zeros", "mask"):
        got = flashmaxsim_score_residual_batched(_gpu(Qs), *idx, padding=padding).cpu().numpy()
        assert got.shape == (nQ, ndocs)
        pad_len = int(lens.max()) if padding == "zeros" else 0
        for q in range(nQ):
            ref = ro.maxsim_residual(Qs[q], codes, res, C, w, nbits, offsets, None, pad_len)
            _assert_scores(got[q], ref, f"batched nQ={nQ} nq={nq} q={q} {padding}")
            _assert_kernel(got[q], Qs[q], (codes, res, C, w, nbits), offsets, None, pad_len, _form(nQ, nq),
                           f"batched nQ={nQ} nq={nq} q={q} {padding}")
        one = flashmaxsim_score_residual(_gpu(Qs[nQ - 1]), *idx, padding=padding).cpu().numpy()
        _assert_scores(got[nQ - 1], one, "batched vs one query")


@pytest.mark.parametrize("nbits", [1, 2, 4])
@pytest.mark.parametrize("d", [32, 64, 96, 128])
def test_batched_maxsim_formats(cuda, nbits, d):
    """Every (d, nbits) instantiation; the decoded tiles are the codec's fp16 tokens, so
    the scores also match dense MaxSim over tms_residual_decompress's output (to 1e-4: a
    token whose fp16 norm rounds the other way in the other fp32 summation order moves
    by one fp16 ulp)."""
    import torch
    from tilemaxsim_amd import decompress_residual, flash_maxsim_multi_doc, flashmaxsim_score_residual_batched
    rng = np.random.default_rng(nbits * 10 + d)
    ndocs = 500
    lens = rng.integers(1, 120, ndocs)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    C, codes, res, w = _index(rng, int(offsets[-1]), d, nbits, 211)
    Qs = _queries(rng, 6, 32, d)
    got = flashmaxsim_score_residual_batched(_gpu(Qs), _gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits,
                                             _gpu(offsets), padding="mask").cpu().numpy()
    D = decompress_residual(_gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits)
    for q in range(6):
        ref = ro.maxsim_residual(Qs[q], codes, res, C, w, nbits, offsets)
        _assert_scores(got[q], ref, f"nbits={nbits} d={d} q={q}")
        dense = flash_maxsim_multi_doc(_gpu(Qs[q]), D, torch.from_numpy(offsets)).cpu().numpy()
        np.testing.assert_allclose(got[q], dense, rtol=1e-4, atol=1e-4)


def test_batched_candidates_invalid_and_edges(cuda):
    from tilemaxsim_amd import flashmaxsim_score_residual_batched
    rng = np.random.default_rng(12)
    d, nbits, ndocs = 64, 4, 300
    lens = rng.integers(0, 90, ndocs)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    C, codes, res, w = _index(rng, int(offsets[-1]), d, nbits, 50)
    codes[5], codes[9] = 50, -3  # out-of-range centroid ids are clamped
    clamped = np.clip(codes, 0, 49).astype(np.int32)
    Qs = _queries(rng, 7, 32, d)
    idx = (_gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits, _gpu(offsets))
    pids = rng.integers(0, ndocs, 257).astype(np.int64)
    pids[4] = pids[5]
    got = flashmaxsim_score_residual_batched(_gpu(Qs), *idx, pids=_gpu(pids)).cpu().numpy()
    pad_len = int(lens[pids].max())
    for q in range(7):
        _assert_scores(got[q], ro.maxsim_residual(Qs[q], clamped, res, C, w, nbits, offsets, pids, pad_len),
                       f"candidates q={q}")
    assert np.array_equal(got[:, 4], got[:, 5])
    bad = pids.copy()
    bad[[0, 100, 256]] = [-1, ndocs, 10 ** 9]
    with pytest.raises(ValueError):
        flashmaxsim_score_residual_batched(_gpu(Qs), *idx, pids=_gpu(bad))
    got = flashmaxsim_score_residual_batched(_gpu(Qs), *idx, pids=_gpu(bad), padding="mask",
                                             validate=False).cpu().numpy()
    for q in range(7):
        _assert_scores(got[q], ro.maxsim_residual(Qs[q], clamped, res, C, w, nbits, offsets, bad, 0), f"invalid q={q}")
    assert np.isnan(got[:, [0, 100, 256]]).all()
    # all documents empty; no query tokens; no queries; no documents
    empty = _gpu(np.zeros(70, dtype=np.int64))
    for padding in ("zeros", "mask"):
        got = flashmaxsim_score_residual_batched(_gpu(Qs), *idx[:5], empty, padding=padding).cpu().numpy()
        assert got.shape == (7, 69) and np.all(got == -np.inf)
    got = flashmaxsim_score_residual_batched(_gpu(Qs[:, :0]), *idx).cpu().numpy()
    assert got.shape == (7, ndocs) and np.all(got == 0.0)
    assert flashmaxsim_score_residual_batched(_gpu(Qs[:0]), *idx).shape == (0, ndocs)
    assert flashmaxsim_score_residual_batched(_gpu(Qs), *idx, pids=_gpu(np.zeros(0, np.int64))).shape == (7, 0)


N_RANDOM = int(os.environ.get("TMS_RANDOM_SEEDS", "160")) // 4


@pytest.mark.parametrize("seed", range(N_RANDOM))
def test_random_residual_case(cuda, seed):
    """Seeded sweep (``TMS_RANDOM_SEEDS=N`` runs N/4 seeds, default 40): nbits, width,
    query length, document count and lengths (with empty documents), centroid count,
    padding, candidate pids (repeats, unsorted) or all documents, and the entry point
    (one query at every fused dispatch, or several queries through the batched kernel),
    against the float64 oracle on the decompressed tokens."""
    from tilemaxsim_amd import _lib, flashmaxsim_score_residual, flashmaxsim_score_residual_batched
    rng = np.random.default_rng(90_000 + seed)
    nbits = int(rng.choice([1, 2, 4]))
    d = int(rng.choice([32, 64, 96, 128]))
    nq = int(rng.choice([1, 5, 20, 32, 33, 64, 70]))
    ndocs = int(rng.integers(1, 400))
    lens = rng.integers(0, int(rng.choice([2, 17, 64, 180, 300])), ndocs)
    lens[rng.random(ndocs) < 0.1] = 0
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = max(int(offsets[-1]), 1)
    ncent = int(rng.choice([1, 7, 300, 4096]))
    C, codes, res, w = _index(rng, T, d, nbits, ncent)
    padding = str(rng.choice(["zeros", "mask"]))
    pids = None
    if seed % 3 == 0:
        pids = rng.integers(0, ndocs, int(rng.integers(0, 2 * ndocs))).astype(np.int64)
    nQ = 1 if seed % 2 == 0 else int(rng.integers(2, 7))
    what = f"seed={seed} nbits={nbits} d={d} nq={nq} ndocs={ndocs} ncent={ncent} {padding} nQ={nQ} pids={pids is not None}"
    print(what, flush=True)
    Qs = _queries(rng, nQ, nq, d)
    idx = (_gpu(codes), _gpu(res), _gpu(C), _gpu(w), nbits, _gpu(offsets))
    pid_t = None if pids is None else _gpu(pids)
    rows = lens if pids is None else lens[pids]
    pad_len = int(rows.max()) if padding == "zeros" and len(rows) else 0
    refs = [ro.maxsim_residual(Qs[q], codes, res, C, w, nbits, offsets, pids, pad_len) for q in range(nQ)]
    idx_np = (codes, res, C, w, nbits)

    def check(got, q, form, label):
        absref = _assert_kernel(got, Qs[q], idx_np, offsets, pids, pad_len, form, label)
        ref = refs[q]
        fin = np.isfinite(ref)
        assert np.array_equal(np.isfinite(got), fin), label
        assert np.all((got[~fin] == ref[~fin]) | np.isnan(ref[~fin])), label
        slack = 1e-3 * np.abs(ref[fin]) + 1e-3 + 3 * 2.0 ** -11 * absref[fin]
        assert np.all(np.abs(got[fin] - ref[fin]) <= slack), f"{label}: codec check"

    if nQ == 1:
        for limit in (None, 1 << 40, 0):
            if limit is None:
                got = flashmaxsim_score_residual(_gpu(Qs[0]), *idx, pids=pid_t, padding=padding).cpu().numpy()
            else:
                with _lib.rerank_limit(limit):
                    got = flashmaxsim_score_residual(_gpu(Qs[0]), *idx, pids=pid_t, padding=padding).cpu().numpy()
            check(got, 0, "fused", f"{what} limit={limit}")
    else:
        got = flashmaxsim_score_residual_batched(_gpu(Qs), *idx, pids=pid_t, padding=padding).cpu().numpy()
        for q in range(nQ):
            check(got[q], q, _form(nQ, nq), f"{what} q={q}")
