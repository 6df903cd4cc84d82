"""float32 embeddings through the dense, masked, variable-length and PQ entry points.

The reference accepts float32 Q and D in the same kernels: its precision experiment
(``src/cycle6_rerun_scaling.py:96-106``) scores FP32, FP16 and BF16 inputs with
``flash_maxsim_v2_multiquery``, and its loads cast every element to fp32
(``src/flash_maxsim_v2.py:99,111``) before a TF32 ``tl.dot``.

Here each fp32 element is split into bf16 hi + lo terms and a product is
hi*hi + hi*lo + lo*hi (three bf16 MFMAs). Bar, per document:

    |score - oracle| <= (4 * 2^-16 + d * 2^-24) * MaxSim(|Q|, |D|) + 1e-6

with the oracle the float64 MaxSim of the same fp32 values and MaxSim(|Q|, |D|) (the
oracle on absolute values) bounding sum_i max_j sum_k |q_ik| |d_jk|: 3 * 2^-16 for the
split, 2^-16 of slack, d * 2^-24 for fp32 accumulation. ``_coherent`` inputs sit a
fifth of an fp16 (or bf16) unit in the last place above a representable value, all
positive, so rounding them down would bias every product the same way; the CPU test at
the end shows the bar then fails a kernel that cast its fp32 inputs to fp16 or bf16, and
the GPU test runs the same inputs through the fp32 path.
"""
import numpy as np
import pytest

from oracle import maxsim_oracle as orc


def _rng(seed):
    return np.random.default_rng(seed)


def _randn(rng, shape, normalize=False):
    x = rng.standard_normal(shape, dtype=np.float32)
    if normalize:
        x /= np.linalg.norm(x, axis=-1, keepdims=True) + 1e-12
    return x.astype(np.float32)


def _coherent(rng, shape, rounding):
    """Positive fp32 values x = h * (1 + 0.2 * 2^-p) with h representable in fp16
    (p = 10) or bf16 (p = 7): rounding x to that type returns h, one fifth of a unit in
    the last place low for every element, since half a unit is at least 0.25 * 2^-p of
    the value."""
    import torch
    v = np.abs(rng.standard_normal(shape, dtype=np.float32)) + 0.05
    v /= np.linalg.norm(v, axis=-1, keepdims=True)
    tdt, p = (torch.float16, 10) if rounding == "fp16" else (torch.bfloat16, 7)
    h = torch.from_numpy(v).to(tdt).float().numpy()
    x = (h * np.float32(1 + 0.2 * 2.0 ** -p)).astype(np.float32)
    assert np.array_equal(torch.from_numpy(x).to(tdt).float().numpy(), h)
    return x


def _bound(absmaxsim, d):
    return (4 * 2.0 ** -16 + d * 2.0 ** -24) * absmaxsim + 1e-6


def _assert_fp32_scores(got, ref, absref, d, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    inf_ref = np.isinf(ref)
    assert np.array_equal(np.isinf(got), inf_ref), f"{what}: -inf pattern differs"
    assert np.all(got[inf_ref] == ref[inf_ref]), f"{what}: infinite values differ"
    fin = ~inf_ref
    err = np.abs(got[fin] - ref[fin])
    lim = _bound(np.asarray(absref, dtype=np.float64)[fin], d)
    worst = int(np.argmax(err - lim)) if err.size else 0
    assert np.all(err <= lim), f"{what}: error {err[worst]:.3e} > bound {lim[worst]:.3e}"


def _gpu(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


FIXED = [
    # (Nq, Nd, d, B, normalise)
    (32, 128, 128, 300, True), (32, 70, 128, 64, False), (33, 17, 96, 50, True), (64, 40, 64, 40, True),
    (20, 30, 100, 20, False), (16, 40, 256, 30, True), (16, 20, 768, 12, False), (8, 10, 1024, 5, True),
    (1, 1, 32, 3, False), (70, 9, 136, 11, True),
]


@pytest.mark.gpu
@pytest.mark.parametrize("Nq,Nd,d,B,norm", FIXED)
def test_fp32_dense(cuda, Nq, Nd, d, B, norm):
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    rng = _rng(31 * Nq + Nd + 7 * d + B)
    Q = _randn(rng, (Nq, d), norm)
    D = _randn(rng, (B, Nd, d), norm)
    got = flash_maxsim_v2_multiquery(_gpu(Q), _gpu(D)).cpu().numpy()
    _assert_fp32_scores(got, orc.maxsim_f64(Q, D), orc.maxsim_f64(np.abs(Q), np.abs(D)), d,
                        f"fp32 Nq={Nq} Nd={Nd} d={d} B={B}")


@pytest.mark.gpu
@pytest.mark.parametrize("rounding", ["bf16", "fp16"])
def test_fp32_coherent_inputs(cuda, rounding):
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    rng = _rng(3)
    Q = _coherent(rng, (32, 128), rounding)
    D = _coherent(rng, (300, 128, 128), rounding)
    got = flash_maxsim_v2_multiquery(_gpu(Q), _gpu(D)).cpu().numpy()
    _assert_fp32_scores(got, orc.maxsim_f64(Q, D), orc.maxsim_f64(Q, D), 128, f"coherent {rounding}")


@pytest.mark.gpu
def test_fp32_misaligned_pointer_and_mixed_dtypes(cuda):
    import torch
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    rng = _rng(5)
    Q = _randn(rng, (32, 128))
    D = _randn(rng, (40, 30, 128))
    # D starting 4 bytes into a buffer: the element-wise (unaligned) load path
    buf = torch.zeros(D.size + 1, dtype=torch.float32, device="cuda")
    Dv = buf[1:].view(D.shape)
    Dv.copy_(torch.from_numpy(D))
    got = flash_maxsim_v2_multiquery(_gpu(Q), Dv).cpu().numpy()
    absref = orc.maxsim_f64(np.abs(Q), np.abs(D))
    _assert_fp32_scores(got, orc.maxsim_f64(Q, D), absref, 128, "misaligned fp32 D")
    # fp16 queries against fp32 documents: cast to fp32 exactly
    Qh = Q.astype(np.float16)
    got = flash_maxsim_v2_multiquery(_gpu(Qh), _gpu(D)).cpu().numpy()
    _assert_fp32_scores(got, orc.maxsim_f64(Qh, D), orc.maxsim_f64(np.abs(Qh), np.abs(D)), 128, "fp16 Q, fp32 D")


@pytest.mark.gpu
@pytest.mark.parametrize("nQ,nq,d", [(20, 32, 128), (6, 64, 64), (5, 40, 96), (3, 32, 32), (17, 64, 128)])
def test_fp32_shared_tiles(cuda, nQ, nq, d):
    """Several fp32 queries over the same fp32 documents: the shared-tile kernel (tiles
    split into bf16 hi + lo in the LDS ring, 1 or 2 query blocks per wave, up to 16 per
    pass), fixed-length and variable-length (empty documents, invalid offsets)."""
    from tilemaxsim_amd import flash_maxsim_batched_queries, flash_maxsim_multi_doc_batched
    rng = _rng(nQ * 100 + nq + d)
    Qs = _randn(rng, (nQ, nq, d), True)
    Dfix = _randn(rng, (70, 33, d), True)
    got = flash_maxsim_batched_queries(_gpu(Qs), _gpu(Dfix)).cpu().numpy()
    for q in range(nQ):
        _assert_fp32_scores(got[q], orc.maxsim_f64(Qs[q], Dfix), orc.maxsim_f64(np.abs(Qs[q]), np.abs(Dfix)), d,
                            f"fixed fp32 shared tiles q={q}")
    lens = rng.integers(0, 60, 90)
    lens[[0, 7, 89]] = 0
    lens[1] = 10
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    flat = _randn(rng, (int(offsets[-1]), d), True)
    got = flash_maxsim_multi_doc_batched(_gpu(Qs), _gpu(flat), _gpu(offsets)).cpu().numpy()
    for q in range(nQ):
        _assert_fp32_scores(got[q], orc.maxsim_varlen(Qs[q], flat, offsets, f64=True),
                            orc.maxsim_varlen(np.abs(Qs[q]), np.abs(flat), offsets, f64=True), d,
                            f"varlen fp32 shared tiles q={q}")
    bad = offsets.copy()
    bad[5] = bad[4] - 1  # document 4 ends before it starts (document 5 starts a row early)
    got = flash_maxsim_multi_doc_batched(_gpu(Qs), _gpu(flat), _gpu(bad), validate=False).cpu().numpy()
    assert np.all(np.isnan(got[:, 4]))
    assert not np.isnan(np.delete(got, 4, axis=1)).any()


@pytest.mark.gpu
@pytest.mark.parametrize("d", [128, 768])  # Q in VGPRs; Q in LDS above 80 KiB (8-wave workgroups)
def test_fp32_masked_varlen_and_batched(cuda, d):
    import torch
    from tilemaxsim_amd import (flash_maxsim_batched_queries, flash_maxsim_multi_doc,
                                flash_maxsim_multi_doc_batched, maxsim_score)
    rng = _rng(9 + d)
    B, Nmax = 120, 90
    lens = rng.integers(0, Nmax + 1, B)
    lens[:3] = 0
    Q = _randn(rng, (32, d), True)
    D = _randn(rng, (B, Nmax, d), True)
    mask = np.arange(Nmax)[None, :] < lens[:, None]
    ref = orc.maxsim_masked(Q, D, mask, f64=True)
    absref = orc.maxsim_masked(np.abs(Q), np.abs(D), mask, f64=True)
    got = maxsim_score(_gpu(Q), _gpu(D), _gpu(mask)).cpu().numpy()
    _assert_fp32_scores(got, ref, absref, d, "masked fp32")

    flat = np.concatenate([D[b, : lens[b]] for b in range(B)])
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    got = flash_maxsim_multi_doc(_gpu(Q), _gpu(flat), _gpu(offsets)).cpu().numpy()
    _assert_fp32_scores(got, ref, absref, d, "varlen fp32")

    Qs = np.stack([Q, _randn(rng, (32, d), True), _randn(rng, (32, d), True)])
    got = flash_maxsim_multi_doc_batched(_gpu(Qs), _gpu(flat), _gpu(offsets)).cpu().numpy()
    for q in range(3):
        _assert_fp32_scores(got[q], orc.maxsim_varlen(Qs[q], flat, offsets, f64=True),
                            orc.maxsim_varlen(np.abs(Qs[q]), np.abs(flat), offsets, f64=True), d,
                            f"varlen batched fp32 q={q}")

    Dfix = _randn(rng, (50, 40, d), True)
    got = flash_maxsim_batched_queries(_gpu(Qs), _gpu(Dfix)).cpu().numpy()
    for q in range(3):
        _assert_fp32_scores(got[q], orc.maxsim_f64(Qs[q], Dfix), orc.maxsim_f64(np.abs(Qs[q]), np.abs(Dfix)), d,
                            f"dense batched fp32 q={q}")
    del torch


@pytest.mark.gpu
def test_fp32_pq_codebook(cuda):
    import torch
    from tilemaxsim_amd import TileMaxSimPQ
    rng = _rng(21)
    M, K, dsub, B, Nd = 16, 256, 8, 300, 40
    C = rng.standard_normal((M, K, dsub), dtype=np.float32)
    codes = rng.integers(0, K, (B, Nd, M)).astype(np.uint8)
    Q = _randn(rng, (32, M * dsub), True)
    pq = TileMaxSimPQ(_gpu(C))
    # the table: fp32 products and sums, against float64
    T = pq.build_distance_table(_gpu(Q)).cpu().numpy()
    T64 = np.einsum("qmj,mkj->qmk", Q.reshape(32, M, dsub).astype(np.float64), C.astype(np.float64))
    Tabs = np.einsum("qmj,mkj->qmk", np.abs(Q).reshape(32, M, dsub).astype(np.float64), np.abs(C).astype(np.float64))
    assert np.all(np.abs(T - T64) <= dsub * 2.0 ** -23 * Tabs + 1e-30)
    # scores through the table-gather kernel (a float32 codebook has no MFMA path)
    ref = orc.pq_decompress_score(Q, C, codes, f64=True)
    got = pq.score_batch(_gpu(Q), _gpu(codes)).cpu().numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-4)
    np.testing.assert_array_equal(got, pq.score_batch(_gpu(Q), _gpu(codes), method="lut").cpu().numpy())
    with pytest.raises(NotImplementedError, match="dtype"):
        pq.score_batch(_gpu(Q), _gpu(codes), method="mfma")
    Qs = np.stack([Q, _randn(rng, (32, M * dsub), True)])
    got_b = pq.score_batch_queries(_gpu(Qs), _gpu(codes)).cpu().numpy()
    np.testing.assert_array_equal(got_b[0], got)
    np.testing.assert_allclose(got_b[1], orc.pq_decompress_score(Qs[1], C, codes, f64=True), rtol=1e-5, atol=1e-4)
    del torch


@pytest.mark.parametrize("rounding", ["bf16", "fp16"])
def test_fp32_bar_rejects_rounded_inputs(rounding):
    """The bar above is strict: on the coherent inputs, scoring their bf16- or
    fp16-rounded copies (what a kernel that cast its inputs down would compute) exceeds
    it for every document. Oracle-only, on the CPU."""
    import torch
    rng = _rng(3)
    Q = _coherent(rng, (32, 128), rounding)
    D = _coherent(rng, (300, 128, 128), rounding)
    tdt = torch.bfloat16 if rounding == "bf16" else torch.float16
    Qr = torch.from_numpy(Q).to(tdt).float().numpy()
    Dr = torch.from_numpy(D).to(tdt).float().numpy()
    ref = orc.maxsim_f64(Q, D)
    err = np.abs(orc.maxsim_f64(Qr, Dr) - ref)
    assert np.all(err > _bound(ref, 128))
