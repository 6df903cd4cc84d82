"""Queries of another float dtype than the documents, and embeddings wider than 1024.

The reference loads Q and D tiles with ``.to(tl.float32)`` and multiplies them with a
TF32 ``tl.dot`` (``src/flash_maxsim_v2.py:99,111,117,170-181``), so an fp32 query against
fp16 / bf16 documents keeps (at least) TF32's 11 significant bits, and a 16-bit query of
the other 16-bit type converts exactly. Here such a query is converted to fp32 (exact for
16-bit queries) and each element is split into two terms of the documents' type (fp16:
after a per-token power-of-two scale); a product takes two MFMAs. The bar is the fp32 bar
of ``test_gpu_fp32.py``:

    |score - oracle| <= (4 * 2^-16 + d * 2^-24) * MaxSim(|Q|, |D|) + 1e-6

against the float64 oracle on the unrounded query. ``test_q32_bar_rejects_rounded_query``
shows on the CPU that scoring the query rounded to the documents' dtype (what casting Q
down would compute) fails it on the coherent inputs used here.

Widths above 1024 (the reference's d-tiled kernel loops over any d, ``:168``) run with
the query fragments in LDS while they fit (16-bit below d = 2560, fp32 or split queries
below d = 1280), and read from memory with each tile beyond that.
"""
import numpy as np
import pytest

from oracle import maxsim_oracle as orc

from test_gpu_fp32 import _assert_fp32_scores, _bound, _coherent, _gpu, _randn, _rng


def _docs16(rng, shape, dt, normalize=True):
    """Documents exactly representable in the 16-bit type `dt`, returned as fp32 values
    (for the oracle) and as the 16-bit array (for the kernel)."""
    import torch
    x = _randn(rng, shape, normalize)
    t = torch.from_numpy(x).to(dt)
    return t.float().numpy(), t


def test_q32_bar_rejects_rounded_query():
    """On coherent fp32 queries (a fifth of a 16-bit ulp above a representable value,
    all positive) against exactly representable documents, the score of the query
    rounded to fp16 or bf16 misses the bar for every document. CPU only."""
    import torch
    rng = _rng(17)
    for rounding, dt in (("fp16", torch.float16), ("bf16", torch.bfloat16)):
        Q = _coherent(rng, (32, 128), rounding)
        D = np.abs(_docs16(rng, (200, 64, 128), dt)[0])
        Qr = torch.from_numpy(Q).to(dt).float().numpy()
        ref = orc.maxsim_f64(Q, D)
        err = np.abs(orc.maxsim_f64(Qr, D) - ref)
        assert np.all(err > _bound(ref, 128)), rounding


SHAPES = [
    # (Nq, Nd, d, B): Q in VGPRs (d <= 128), Q in LDS, unaligned width, long query
    (32, 128, 128, 200), (32, 40, 64, 64), (20, 30, 100, 20), (16, 40, 256, 30), (16, 20, 768, 12), (70, 9, 136, 11),
]


@pytest.mark.gpu
@pytest.mark.parametrize("ddt", ["fp16", "bf16"])
@pytest.mark.parametrize("Nq,Nd,d,B", SHAPES)
def test_q32_dense(cuda, ddt, Nq, Nd, d, B):
    import torch
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    dt = torch.float16 if ddt == "fp16" else torch.bfloat16
    rng = _rng(Nq * 7 + Nd + d + B)
    Q = _coherent(rng, (Nq, d), ddt)
    D, Dt = _docs16(rng, (B, Nd, d), dt)
    got = flash_maxsim_v2_multiquery(_gpu(Q), Dt.cuda()).cpu().numpy()
    _assert_fp32_scores(got, orc.maxsim_f64(Q, D), orc.maxsim_f64(np.abs(Q), np.abs(D)), d,
                        f"fp32 Q, {ddt} D, Nq={Nq} Nd={Nd} d={d}")


@pytest.mark.gpu
@pytest.mark.parametrize("ddt", ["fp16", "bf16"])
@pytest.mark.parametrize("d", [128, 384])
def test_q32_masked_varlen_batched(cuda, ddt, d):
    import torch
    from tilemaxsim_amd import (flash_maxsim_batched_queries, flash_maxsim_multi_doc,
                                flash_maxsim_multi_doc_batched, maxsim_score)
    dt = torch.float16 if ddt == "fp16" else torch.bfloat16
    rng = _rng(40 + d)
    B, Nmax = 90, 70
    lens = rng.integers(0, Nmax + 1, B)
    lens[:2] = 0
    Q = _coherent(rng, (32, d), ddt)
    D, Dt = _docs16(rng, (B, Nmax, d), dt)
    mask = np.arange(Nmax)[None, :] < lens[:, None]
    ref = orc.maxsim_masked(Q, D, mask, f64=True)
    absref = orc.maxsim_masked(np.abs(Q), np.abs(D), mask, f64=True)
    got = maxsim_score(_gpu(Q), Dt.cuda(), _gpu(mask)).cpu().numpy()
    _assert_fp32_scores(got, ref, absref, d, f"masked fp32 Q / {ddt}")

    flat = np.concatenate([D[b, : lens[b]] for b in range(B)])
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    flat_t = torch.from_numpy(flat).to(dt).cuda()
    got = flash_maxsim_multi_doc(_gpu(Q), flat_t, _gpu(offsets)).cpu().numpy()
    _assert_fp32_scores(got, ref, absref, d, f"varlen fp32 Q / {ddt}")

    Qs = np.stack([Q, _coherent(rng, (32, d), ddt), _coherent(rng, (32, d), ddt), _coherent(rng, (32, d), ddt)])
    got = flash_maxsim_multi_doc_batched(_gpu(Qs), flat_t, _gpu(offsets)).cpu().numpy()
    for q in range(4):
        _assert_fp32_scores(got[q], orc.maxsim_varlen(Qs[q], flat, offsets, f64=True),
                            orc.maxsim_varlen(np.abs(Qs[q]), np.abs(flat), offsets, f64=True), d,
                            f"varlen batched fp32 Q / {ddt} q={q}")
    Dfix, Dfix_t = _docs16(rng, (50, 40, d), dt)
    got = flash_maxsim_batched_queries(_gpu(Qs), Dfix_t.cuda()).cpu().numpy()
    for q in range(4):
        _assert_fp32_scores(got[q], orc.maxsim_f64(Qs[q], Dfix), orc.maxsim_f64(np.abs(Qs[q]), np.abs(Dfix)), d,
                            f"dense batched fp32 Q / {ddt} q={q}")


@pytest.mark.gpu
@pytest.mark.parametrize("ddt", ["fp16", "bf16"])
@pytest.mark.parametrize("nQ,nq,d", [(20, 64, 128), (9, 32, 64), (3, 50, 96)])
def test_q32_shared_tiles(cuda, ddt, nQ, nq, d):
    """Several fp32 queries over 16-bit documents share each tile (the shared-tile kernel
    with split query fragments, up to 16 blocks per pass: 40 blocks here take three
    passes). Some query tokens are scaled far outside fp16's range or deep into its
    subnormals, which the per-token power-of-two scale must absorb."""
    import torch
    from tilemaxsim_amd import flash_maxsim_batched_queries, flash_maxsim_multi_doc_batched
    dt = torch.float16 if ddt == "fp16" else torch.bfloat16
    rng = _rng(nQ * 31 + nq + d)
    Qs = np.stack([_coherent(rng, (nq, d), ddt) for _ in range(nQ)])
    Qs[0, 3] *= np.float32(2.0 ** 24)
    Qs[1, 0] *= np.float32(2.0 ** -40)
    D, Dt = _docs16(rng, (60, 37, d), dt)
    got = flash_maxsim_batched_queries(_gpu(Qs), Dt.cuda()).cpu().numpy()
    assert np.all(np.isfinite(got))
    for q in range(nQ):
        _assert_fp32_scores(got[q], orc.maxsim_f64(Qs[q], D), orc.maxsim_f64(np.abs(Qs[q]), np.abs(D)), d,
                            f"fixed, fp32 Q / {ddt} q={q}")
    lens = rng.integers(0, 50, 70)
    lens[[0, 33]] = 0
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    flat, flat_t = _docs16(rng, (int(offsets[-1]), d), dt)
    got = flash_maxsim_multi_doc_batched(_gpu(Qs), flat_t.cuda(), _gpu(offsets)).cpu().numpy()
    for q in range(nQ):
        _assert_fp32_scores(got[q], orc.maxsim_varlen(Qs[q], flat, offsets, f64=True),
                            orc.maxsim_varlen(np.abs(Qs[q]), np.abs(flat), offsets, f64=True), d,
                            f"varlen, fp32 Q / {ddt} q={q}")


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [2.0 ** 24, 2.0 ** -40])
def test_q32_fp16_docs_any_query_magnitude(cuda, scale):
    """fp32 queries far outside fp16's range (2^24 ~ 1.7e7 > 65504) or deep in its
    subnormals: the per-token power-of-two scale keeps every split term in range, so the
    scores are the float64 ones to the same relative bar (rounding such a query to fp16
    would give inf or 0)."""
    import torch
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    rng = _rng(77)
    Q = (_randn(rng, (32, 128), True) * np.float32(scale)).astype(np.float32)
    Q[5] *= np.float32(2.0 ** -12)  # one token much smaller than the rest
    D, Dt = _docs16(rng, (100, 50, 128), torch.float16)
    got = flash_maxsim_v2_multiquery(_gpu(Q), Dt.cuda()).cpu().numpy()
    ref = orc.maxsim_f64(Q, D)
    absref = orc.maxsim_f64(np.abs(Q), np.abs(D))
    assert np.all(np.isfinite(got))
    err = np.abs(got - ref)
    assert np.all(err <= (4 * 2.0 ** -16 + 128 * 2.0 ** -24) * absref), err.max()


@pytest.mark.gpu
def test_16bit_query_of_the_other_type(cuda):
    """fp16 queries against bf16 documents and bf16 queries against fp16 ones: converted
    to fp32 exactly and split, so the scores are those of the unrounded 16-bit query."""
    import torch
    from tilemaxsim_amd import flash_maxsim_multi_doc, flash_maxsim_v2_multiquery
    rng = _rng(8)
    for qdt, ddt in ((torch.float16, torch.bfloat16), (torch.bfloat16, torch.float16)):
        Qt = torch.from_numpy(_randn(rng, (32, 128), True)).to(qdt)
        Q = Qt.float().numpy()
        D, Dt = _docs16(rng, (120, 60, 128), ddt)
        got = flash_maxsim_v2_multiquery(Qt.cuda(), Dt.cuda()).cpu().numpy()
        _assert_fp32_scores(got, orc.maxsim_f64(Q, D), orc.maxsim_f64(np.abs(Q), np.abs(D)), 128, f"{qdt} Q / {ddt} D")
        offs = np.arange(0, 121 * 60, 60, dtype=np.int64)
        got = flash_maxsim_multi_doc(Qt.cuda(), Dt.reshape(-1, 128).cuda(), _gpu(offs)).cpu().numpy()
        _assert_fp32_scores(got, orc.maxsim_f64(Q, D), orc.maxsim_f64(np.abs(Q), np.abs(D)), 128,
                            f"varlen {qdt} Q / {ddt} D")


WIDE = [
    # (query dtype, document dtype, d): 16-bit in LDS below d = 2560 (8-wave workgroups
    # above 80 KiB); fp32 and split queries read from memory from d = 1280
    ("fp16", "fp16", 1536), ("fp16", "fp16", 2048), ("bf16", "bf16", 2560), ("fp16", "fp16", 3072),
    ("fp32", "fp32", 1280), ("fp32", "fp32", 1536), ("fp32", "fp32", 2048),
    ("fp32", "fp16", 1536), ("fp32", "bf16", 2048), ("fp32", "fp16", 4000),
]


@pytest.mark.gpu
@pytest.mark.parametrize("qdt,ddt,d", WIDE)
def test_wide_embeddings(cuda, qdt, ddt, d):
    import torch
    from tilemaxsim_amd import flash_maxsim_multi_doc, flash_maxsim_v2_multiquery
    tdt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
    rng = _rng(d + len(qdt) + 3 * len(ddt))
    Qt = torch.from_numpy(_randn(rng, (32, d), True)).to(tdt[qdt])
    Dt = torch.from_numpy(_randn(rng, (40, 33, d), True)).to(tdt[ddt])
    Q, D = Qt.float().numpy(), Dt.float().numpy()
    ref, absref = orc.maxsim_f64(Q, D), orc.maxsim_f64(np.abs(Q), np.abs(D))
    got = flash_maxsim_v2_multiquery(Qt.cuda(), Dt.cuda()).cpu().numpy()
    if qdt == ddt and ddt != "fp32":  # 16-bit products are exact: fp32 accumulation only
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    else:
        _assert_fp32_scores(got, ref, absref, d, f"{qdt} Q / {ddt} D, d={d}")
    # the same documents as a flat buffer with ragged lengths, an empty one included
    lens = rng.integers(0, 34, 40)
    lens[3] = 0
    flat = np.concatenate([D[b, : lens[b]] for b in range(40)])
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    got = flash_maxsim_multi_doc(Qt.cuda(), torch.from_numpy(flat).to(tdt[ddt]).cuda(), _gpu(offs)).cpu().numpy()
    vref = orc.maxsim_varlen(Q, flat, offs, f64=True)
    vabs = orc.maxsim_varlen(np.abs(Q), np.abs(flat), offs, f64=True)
    _assert_fp32_scores(got, vref, vabs, d, f"varlen {qdt} Q / {ddt} D, d={d}")
