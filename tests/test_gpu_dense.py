"""GPU parity of the dense / masked / variable-length MaxSim kernels against the CPU oracle.

Bars: |score - oracle| <= 1e-3 relative (the north star's), and within the
fp32-accumulation bar (d + Nq) * 2^-23 * MaxSim(|Q|, |D|) of ``accum_bar.py`` (the
reference accumulates in fp32: ``tl.dot`` at ``src/flash_maxsim_v2.py:117``); top-100
rankings identical except for swaps among scores within the 1e-3 tolerance.
The oracle is the float64 restatement of ``pytorch_maxsim_naive``
(``src/flash_maxsim_kernel.py:280-288``) on the same fp16/bf16 input values.
"""
import numpy as np
import pytest

import accum_bar as bar
from oracle import maxsim_oracle as orc

pytestmark = pytest.mark.gpu

RTOL = bar.NORTH_STAR_RTOL
ATOL = bar.NORTH_STAR_ATOL


@pytest.fixture(autouse=True, params=["default", "small_batch", "streaming"])
def dense_path(request):
    """Every test runs at the default dispatch, with the small-batch kernel taking every
    call it can (fp16 / bf16, d in {32, 64, 96, 128}, at most three query blocks), and
    with it off (the streaming kernels)."""
    from tilemaxsim_amd import _lib
    limit = {"default": None, "small_batch": 1 << 40, "streaming": 0}[request.param]
    if limit is None:
        yield request.param
        return
    with _lib.rerank_limit(limit):
        yield request.param


def _rng(seed):
    return np.random.default_rng(seed)


def _randn(rng, shape, normalize=False, dtype=np.float16):
    x = rng.standard_normal(shape, dtype=np.float32)
    if normalize:
        x /= np.linalg.norm(x, axis=-1, keepdims=True) + 1e-12
    return x.astype(dtype)


def _to_gpu(x, torch_dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x))
    if torch_dtype is not None:
        t = t.to(torch_dtype)
    return t.cuda()


def _oracle(fn, Q, X, *rest, what="", qsplit=None, **kw):
    """(float64 oracle scores, what, the fp32-accumulation bar) for ``_assert_scores``."""
    ref, lim = bar.with_bound(fn, Q, X, *rest, qsplit=qsplit, **kw)
    return ref, what, lim


def _assert_scores(got, ref, what="", lim=None):
    """The 1e-3 bar, and the fp32-accumulation bar ``lim`` when the reference is the
    float64 oracle (``bar.with_bound``); kernel-against-kernel checks pass no ``lim``."""
    bar.assert_scores(got, ref, lim, what)


# exp10 shape grid of the reference (src/run_all_experiments.py:617-626): (Nq, Nd, d, B)
EXP10_GRID = [
    (8, 32, 64, 100), (16, 64, 128, 100), (32, 128, 128, 100), (32, 128, 256, 100),
    (32, 256, 128, 100), (64, 128, 128, 100), (32, 128, 384, 50), (32, 128, 768, 20),
]


@pytest.mark.parametrize("Nq,Nd,d,B", EXP10_GRID)
def test_exp10_grid_unnormalised(cuda, Nq, Nd, d, B):
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    rng = _rng(1000 + Nq + Nd + d)
    Q = _randn(rng, (Nq, d))
    D = _randn(rng, (B, Nd, d))
    got = flash_maxsim_v2_multiquery(_to_gpu(Q), _to_gpu(D)).cpu().numpy()
    _assert_scores(got, *_oracle(orc.maxsim_f64, Q, D, what=f"exp10 Nq={Nq} Nd={Nd} d={d} B={B}"))


EDGE = [
    # (Nq, Nd, d, B)
    (1, 1, 128, 1), (1, 1, 32, 7), (32, 1, 128, 33), (32, 180, 128, 257), (33, 17, 128, 50),
    (100, 40, 128, 20), (200, 9, 64, 11), (32, 128, 32, 64), (32, 64, 96, 64), (32, 50, 80, 40),
    (32, 50, 200, 40), (20, 70, 1000, 9), (32, 33, 512, 30), (5, 300, 128, 3), (32, 31, 136, 17),
]


@pytest.mark.parametrize("Nq,Nd,d,B", EDGE)
def test_dense_edge_shapes(cuda, Nq, Nd, d, B):
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    rng = _rng(7 * Nq + 13 * Nd + d + B)
    Q = _randn(rng, (Nq, d), normalize=True)
    D = _randn(rng, (B, Nd, d), normalize=True)
    got = flash_maxsim_v2_multiquery(_to_gpu(Q), _to_gpu(D)).cpu().numpy()
    _assert_scores(got, *_oracle(orc.maxsim_f64, Q, D, what=f"Nq={Nq} Nd={Nd} d={d} B={B}"))


@pytest.mark.parametrize("d", [100, 130, 6])
def test_dense_unaligned_width(cuda, d):
    """d not a multiple of 8 takes the element-wise load path."""
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    rng = _rng(d)
    Q = _randn(rng, (32, d))
    D = _randn(rng, (40, 37, d))
    got = flash_maxsim_v2_multiquery(_to_gpu(Q), _to_gpu(D)).cpu().numpy()
    _assert_scores(got, *_oracle(orc.maxsim_f64, Q, D, what=f"d={d}"))


@pytest.mark.parametrize("dt,d,mode", [("fp16", 128, "fixed"), ("bf16", 64, "fixed"), ("fp16", 256, "fixed"),
                                       ("fp16", 128, "varlen"), ("fp32", 128, "fixed"), ("fp32", 256, "fixed"),
                                       ("fp32", 128, "varlen")])
def test_whole_line_loads_at_16_byte_offsets(cuda, dt, d, mode):
    """The whole-line document loads (16-bit rows at d % 64 == 0, fp32 rows at
    d % 32 == 0) from documents that start 16 bytes past a 128-byte line, so that every
    load straddles two lines: the scores equal, bit for bit, those of the same documents
    at an aligned address, and the oracle's within the bar."""
    import torch
    from tilemaxsim_amd import flash_maxsim_multi_doc, flash_maxsim_v2_multiquery
    tdt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[dt]
    rng = _rng(d + len(mode) + len(dt))
    Q = _randn(rng, (32, d), True, np.float32)
    if mode == "fixed":
        D = _randn(rng, (40, 45, d), True, np.float32)
        lens = None
    else:
        lens = rng.integers(0, 70, size=40)
        lens[3] = 0
        D = _randn(rng, (int(lens.sum()), d), True, np.float32)
    # the values each dtype holds, so that the oracle sees what the kernel reads
    Qt = torch.from_numpy(Q).to(tdt)
    Dt = torch.from_numpy(D).to(tdt)
    Qn, Dn = Qt.float().numpy(), Dt.float().numpy()
    pad = 16 // Dt.element_size()
    buf = torch.empty(Dt.numel() + pad, dtype=tdt, device="cuda")
    Dv = buf[pad:].view(Dt.shape)
    Dv.copy_(Dt)
    Da = Dt.cuda()
    assert Dv.data_ptr() % 128 == 16 and Da.data_ptr() % 128 == 0
    Qg = Qt.cuda()
    if mode == "fixed":
        got, ref_al = flash_maxsim_v2_multiquery(Qg, Dv), flash_maxsim_v2_multiquery(Qg, Da)
        fn = orc.maxsim_f64
    else:
        offs = torch.from_numpy(np.concatenate([[0], np.cumsum(lens)]).astype(np.int64))
        got, ref_al = flash_maxsim_multi_doc(Qg, Dv, offs), flash_maxsim_multi_doc(Qg, Da, offs)
        fn = lambda q, x: orc.maxsim_varlen(q, x, offs.numpy(), f64=True)  # noqa: E731
    assert torch.equal(got.view(torch.int32), ref_al.view(torch.int32)), f"{dt} d={d} {mode}"
    ref, absref = fn(Qn, Dn), fn(np.abs(Qn), np.abs(Dn))
    absref = np.where(np.isfinite(absref), absref, 0.0)
    # fp32: products of bf16 hi + lo terms, the fp32 bar of test_gpu_fp32.py
    lim = (4 * 2.0 ** -16 + d * 2.0 ** -24) * absref + 1e-6 if dt == "fp32" else bar.rel(d, 32) * absref + 1e-30
    _assert_scores(got.cpu().numpy(), ref, what=f"{dt} d={d} {mode}", lim=lim)


def test_dense_misaligned_pointer(cuda):
    """A contiguous view that starts 2 bytes into its storage (not 16-byte aligned)."""
    import torch
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    rng = _rng(5)
    Q = _randn(rng, (32, 128))
    D = _randn(rng, (30 * 20 * 128 + 1,))
    Dg = _to_gpu(D)[1:].view(30, 20, 128)
    assert Dg.data_ptr() % 16 != 0
    got = flash_maxsim_v2_multiquery(_to_gpu(Q), Dg).cpu().numpy()
    _assert_scores(got, *_oracle(orc.maxsim_f64, Q, D[1:].reshape(30, 20, 128), what="misaligned"))


def test_empty_documents_and_batch(cuda):
    import torch
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    Q = _to_gpu(np.ones((4, 64), np.float16))
    D0 = torch.empty(5, 0, 64, dtype=torch.float16, device="cuda")
    got = flash_maxsim_v2_multiquery(Q, D0).cpu().numpy()
    assert np.all(np.isneginf(got)) and got.shape == (5,)
    DB0 = torch.empty(0, 8, 64, dtype=torch.float16, device="cuda")
    assert flash_maxsim_v2_multiquery(Q, DB0).shape == (0,)
    Qe = torch.empty(0, 64, dtype=torch.float16, device="cuda")
    D = torch.ones(3, 8, 64, dtype=torch.float16, device="cuda")
    assert np.all(flash_maxsim_v2_multiquery(Qe, D).cpu().numpy() == 0.0)


def test_bf16_and_fp32_query(cuda):
    import torch
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    rng = _rng(11)
    Q = rng.standard_normal((32, 128), dtype=np.float32)
    D = rng.standard_normal((64, 70, 128), dtype=np.float32)
    Qb = torch.from_numpy(Q).to(torch.bfloat16)
    Db = torch.from_numpy(D).to(torch.bfloat16)
    got = flash_maxsim_v2_multiquery(Qb.cuda(), Db.cuda()).cpu().numpy()
    _assert_scores(got, *_oracle(orc.maxsim_f64, Qb.float().numpy(), Db.float().numpy(), what="bf16"))
    # fp32 queries against fp16 documents are scored unrounded (split into two fp16 terms)
    Dh = D.astype(np.float16)
    got = flash_maxsim_v2_multiquery(_to_gpu(Q), _to_gpu(Dh)).cpu().numpy()
    _assert_scores(got, *_oracle(orc.maxsim_f64, Q, Dh, what="fp32 Q", qsplit="fp16"))


def test_c1_ranking_parity(cuda):
    """Workload C1, the CPU-runnable case: 1 query x 1000 docs x Nd=128, d=128, L2-normalised fp16.
    Top-100 must match the oracle except swaps among scores within tolerance."""
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    rng = _rng(0)
    Q = _randn(rng, (32, 128), normalize=True)
    D = _randn(rng, (1000, 128, 128), normalize=True)
    got = flash_maxsim_v2_multiquery(_to_gpu(Q), _to_gpu(D)).cpu().numpy()
    ref, lim = bar.with_bound(orc.maxsim_f64, Q, D)
    _assert_scores(got, ref, "C1", lim)
    _assert_topk_equal(got, ref, 100)


def _assert_topk_equal(got, ref, k):
    """Top-k index sets agree except for documents whose oracle score is within
    tolerance of the k-th oracle score (ties within tolerance)."""
    ref = np.asarray(ref, np.float64)
    _, gi = orc.topk(got, k)
    _, ri = orc.topk(ref, k)
    kth = np.sort(ref)[::-1][k - 1]
    tol = RTOL * abs(kth) + ATOL
    diff = set(gi.tolist()) ^ set(ri.tolist())
    for i in diff:
        assert abs(ref[i] - kth) <= tol, f"doc {i} (score {ref[i]}) differs in top-{k}, kth={kth}"


def test_determinism(cuda):
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    rng = _rng(3)
    Q = _to_gpu(_randn(rng, (64, 128)))
    D = _to_gpu(_randn(rng, (2000, 50, 128)))
    a = flash_maxsim_v2_multiquery(Q, D).cpu().numpy()
    for _ in range(3):
        b = flash_maxsim_v2_multiquery(Q, D).cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("nq,Nd,d,dtype,B", [(32, 128, 128, "fp16", 6000), (64, 180, 128, "fp16", 6000),
                                             (20, 33, 96, "bf16", 60000), (70, 7, 64, "fp16", 300000),
                                             (32, 300, 32, "bf16", 6000)])
def test_scores_do_not_depend_on_the_batch(cuda, nq, Nd, d, dtype, B):
    """A wave walks a run of documents whose length depends on B (192 tokens' worth for
    large B, one document for small B), so the same document lands at a different place
    in a different wave's run. Its score must not depend on that: the first documents of
    a B-document call, scored again in calls of 1000, 300 and 37 documents, give the same
    bits, and match the oracle."""
    import torch
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    tdt = torch.float16 if dtype == "fp16" else torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(nq + Nd + d)
    Q = torch.nn.functional.normalize(torch.randn(nq, d, device="cuda", generator=g), dim=-1).to(tdt)
    D = torch.nn.functional.normalize(torch.randn(B, Nd, d, device="cuda", generator=g), dim=-1).to(tdt)
    big = flash_maxsim_v2_multiquery(Q, D).cpu().numpy()
    for b in (1000, 300, 37):
        small = flash_maxsim_v2_multiquery(Q, D[:b].contiguous()).cpu().numpy()
        assert np.array_equal(small.view(np.uint32), big[:b].view(np.uint32)), f"B={b}"
    _assert_scores(big[:37], *_oracle(orc.maxsim_f64, Q.float().cpu().numpy(), D[:37].float().cpu().numpy(),
                                      what="first 37 documents"))


def test_single_and_batch_entry_points(cuda):
    from tilemaxsim_amd import flash_maxsim_batch, flash_maxsim_single, flash_maxsim_v2
    rng = _rng(21)
    Q = _randn(rng, (32, 128))
    D = _randn(rng, (16, 128, 128))
    ref, lim = bar.with_bound(orc.maxsim_f64, Q, D)
    _assert_scores(flash_maxsim_batch(_to_gpu(Q), _to_gpu(D)).cpu().numpy(), ref, "batch", lim)
    _assert_scores(flash_maxsim_v2(_to_gpu(Q), _to_gpu(D)).cpu().numpy(), ref, "v2", lim)
    s = flash_maxsim_single(_to_gpu(Q), _to_gpu(D[3]))
    assert s.dim() == 0
    _assert_scores(np.array([s.item()]), ref[3:4], "single", lim[3:4])


@pytest.mark.parametrize("dist", ["uniform", "with_empty"])
def test_varlen(cuda, dist):
    import torch
    from tilemaxsim_amd import flash_maxsim_multi_doc
    rng = _rng(99 if dist == "uniform" else 98)
    B = 3000
    lens = rng.integers(32, 301, size=B)
    if dist == "with_empty":
        lens = rng.integers(0, 40, size=B)
        lens[rng.random(B) < 0.2] = 0
        lens[:3] = 0
        lens[-2:] = 0
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(offsets[-1])
    Q = _randn(rng, (32, 128), normalize=True)
    Dflat = _randn(rng, (T, 128), normalize=True)
    got = flash_maxsim_multi_doc(_to_gpu(Q), _to_gpu(Dflat), torch.from_numpy(offsets)).cpu().numpy()
    _assert_scores(got, *_oracle(orc.maxsim_varlen, Q, Dflat, offsets, f64=True, what=f"varlen {dist}"))


def test_varlen_equals_fixed(cuda):
    import torch
    from tilemaxsim_amd import flash_maxsim_multi_doc, flash_maxsim_v2_multiquery
    rng = _rng(17)
    Q = _to_gpu(_randn(rng, (32, 128), normalize=True))
    D = _to_gpu(_randn(rng, (500, 77, 128), normalize=True))
    offs = torch.arange(0, 501 * 77, 77, dtype=torch.int64)
    a = flash_maxsim_v2_multiquery(Q, D).cpu().numpy()
    b = flash_maxsim_multi_doc(Q, D.view(-1, 128), offs).cpu().numpy()
    assert np.array_equal(a, b)


def test_varlen_bad_offsets(cuda):
    import torch
    from tilemaxsim_amd import flash_maxsim_multi_doc
    Q = torch.ones(4, 64, dtype=torch.float16, device="cuda")
    D = torch.ones(10, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        flash_maxsim_multi_doc(Q, D, torch.tensor([0, 5, 3, 10]))
    with pytest.raises(ValueError):
        flash_maxsim_multi_doc(Q, D, torch.tensor([0, 5, 11]))
    got = flash_maxsim_multi_doc(Q, D, torch.tensor([0, 5, 3, 10]), validate=False).cpu().numpy()
    assert np.isnan(got[1]) and got[0] == 4 * 64 and got[2] == 4 * 64


# (nQ, Nq): 1 block per wave with idle waves; 2 per wave; 4 per wave over two launches;
# queries of 3 blocks; queries of 4 blocks; 2 blocks in all (the per-pass kernel);
# 5 blocks per query (the per-pass kernel)
@pytest.mark.parametrize("nQ,nq", [(5, 32), (12, 32), (37, 32), (4, 70), (6, 128), (2, 32), (3, 150)])
def test_varlen_batched(cuda, nQ, nq):
    import torch
    from tilemaxsim_amd import flash_maxsim_multi_doc, flash_maxsim_multi_doc_batched
    rng = _rng(nQ * 1000 + nq)
    B = 1500
    lens = rng.integers(0, 260, size=B)
    lens[rng.random(B) < 0.1] = 0
    lens[:2] = 0
    lens[5] = 1
    lens[-1] = 0
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(offsets[-1])
    Qs = _randn(rng, (nQ, nq, 128), normalize=True)
    Dflat = _randn(rng, (T, 128), normalize=True)
    got = flash_maxsim_multi_doc_batched(_to_gpu(Qs), _to_gpu(Dflat), torch.from_numpy(offsets)).cpu().numpy()
    assert got.shape == (nQ, B)
    for q in range(nQ):
        _assert_scores(got[q], *_oracle(orc.maxsim_varlen, Qs[q], Dflat, offsets, f64=True,
                                        what=f"varlen batched q={q}"))
    one = flash_maxsim_multi_doc(_to_gpu(Qs[-1]), _to_gpu(Dflat), torch.from_numpy(offsets)).cpu().numpy()
    _assert_scores(got[-1], one, "batched vs one query")


@pytest.mark.parametrize("d", [32, 64, 96, 80, 256])
def test_varlen_batched_widths_bf16_and_invalid(cuda, d):
    """Every k-step count of the batched kernel (d = 32 .. 128), widths it does not take
    (80, 256: the per-pass kernel), bf16 documents and invalid offsets (NaN)."""
    import torch
    from tilemaxsim_amd import flash_maxsim_multi_doc_batched
    rng = _rng(d)
    lens = rng.integers(0, 100, size=400)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(offsets[-1])
    Qs = _randn(rng, (9, 32, d), normalize=True)
    Dflat = _randn(rng, (T, d), normalize=True)
    for dt in (torch.float16, torch.bfloat16):
        D = _to_gpu(Dflat, dt)
        got = flash_maxsim_multi_doc_batched(_to_gpu(Qs), D, torch.from_numpy(offsets)).cpu().numpy()
        Dr = D.float().cpu().numpy()
        for q in range(9):  # fp32 queries are scored unrounded against 16-bit documents
            _assert_scores(got[q], *_oracle(orc.maxsim_varlen, Qs[q], Dr, offsets, f64=True, what=f"d={d} {dt} q={q}",
                                            qsplit="bf16" if dt == torch.bfloat16 else None))
    bad = offsets.copy()
    bad[10] = bad[11] + 5  # document 9 ends after document 10 starts, document 10 is reversed
    got = flash_maxsim_multi_doc_batched(_to_gpu(Qs), _to_gpu(Dflat), torch.from_numpy(bad),
                                         validate=False).cpu().numpy()
    assert np.isnan(got[:, 10]).all() and not np.isnan(np.delete(got, 10, axis=1)).any()
    with pytest.raises(ValueError):
        flash_maxsim_multi_doc_batched(_to_gpu(Qs), _to_gpu(Dflat), torch.from_numpy(bad))


def test_packed_batched_both_paddings(cuda):
    import torch
    from tilemaxsim_amd import flashmaxsim_score_packed, flashmaxsim_score_packed_batched
    rng = _rng(4242)
    lens = rng.integers(0, 150, size=900)
    lens[7] = 0
    T = int(lens.sum())
    Qs = _randn(rng, (20, 32, 128), normalize=True)
    Dp = _randn(rng, (T, 128), normalize=True)
    for padding in ("zeros", "mask"):
        got = flashmaxsim_score_packed_batched(_to_gpu(Qs), _to_gpu(Dp), torch.from_numpy(lens),
                                               padding=padding).cpu().numpy()
        offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        for q in (0, 11, 19):
            if padding == "zeros":
                ref, lim = bar.with_bound(orc.maxsim_packed_zero_padded, Qs[q], Dp, lens)
            else:
                ref, lim = bar.with_bound(orc.maxsim_varlen, Qs[q], Dp, offsets, f64=True)
            _assert_scores(got[q], ref, f"packed batched {padding} q={q}", lim)
            one = flashmaxsim_score_packed(_to_gpu(Qs[q][None]), _to_gpu(Dp), torch.from_numpy(lens),
                                           padding=padding).cpu().numpy()
            _assert_scores(got[q], one, "packed batched vs one query")
        assert got[:, 7].tolist() == ([0.0] * 20 if padding == "zeros" else [-np.inf] * 20)


def test_masked(cuda):
    import torch
    from tilemaxsim_amd import maxsim_score
    rng = _rng(23)
    B, Nd, d = 300, 90, 128
    Q = _randn(rng, (32, d), normalize=True)
    D = _randn(rng, (B, Nd, d), normalize=True)
    mask = rng.random((B, Nd)) < 0.6
    mask[0] = False
    mask[1, :] = False
    mask[1, -1] = True
    got = maxsim_score(_to_gpu(Q), _to_gpu(D), torch.from_numpy(mask).cuda()).cpu().numpy()
    _assert_scores(got, *_oracle(orc.maxsim_masked, Q, D, mask, f64=True, what="masked"))


@pytest.mark.parametrize("padding", ["zeros", "mask"])
def test_plaid_packed_dropin(cuda, padding):
    """flashmaxsim_score_packed (src/plaid_integration_benchmark.py:154-183): zero
    padding to the longest document, as the reference computes it, or ColBERT's mask."""
    import torch
    from tilemaxsim_amd import flashmaxsim_score_packed
    rng = _rng(41 if padding == "zeros" else 42)
    lens = rng.integers(0, 90, size=700)
    lens[5] = 0
    lens[9] = lens.max()
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    Q = _randn(rng, (1, 32, 128), normalize=True)
    # anti-aligned documents (negative similarities) make zero padding visible
    flat = -_randn(rng, (int(offsets[-1]), 128), normalize=True)
    flat[: int(offsets[-1]) // 2] *= -1
    got = flashmaxsim_score_packed(torch.from_numpy(Q).cuda(), _to_gpu(flat), torch.from_numpy(lens),
                                   config=None, padding=padding).cpu().numpy()
    if padding == "zeros":
        ref, lim = bar.with_bound(orc.maxsim_packed_zero_padded, Q[0], flat, lens)
        assert got[5] == 0.0
    else:
        ref, lim = bar.with_bound(orc.maxsim_varlen, Q[0], flat, offsets, f64=True)
    _assert_scores(got, ref, f"packed {padding}", lim)


def test_batched_queries(cuda):
    import torch
    from tilemaxsim_amd import flash_maxsim_batched_queries, flash_maxsim_v2_multiquery
    rng = _rng(31)
    # Batched kernel, 8 waves per workgroup holding 1, 2 or 4 blocks each:
    # (5, 32): 1 block per wave, 5 of 8 waves used; (12, 32): 2 per wave; (7, 64): 2 per
    # wave, one query each; (4, 70): 3 blocks per query, 3 per wave; (37, 32): 4 per
    # wave, two launches, the second partial; (6, 128): 4 blocks per query.
    # (3, 20): 3 blocks, the per-pass stream kernel.
    for nQ, Nq in [(5, 32), (12, 32), (7, 64), (3, 20), (4, 70), (37, 32), (6, 128)]:
        Qs = _to_gpu(_randn(rng, (nQ, Nq, 128), normalize=True))
        D = _to_gpu(_randn(rng, (400, 60, 128), normalize=True))
        got = flash_maxsim_batched_queries(Qs, D).cpu().numpy()
        for i in range(nQ):
            ref, lim = bar.with_bound(orc.maxsim_f64, Qs[i].cpu().numpy(), D.cpu().numpy())
            _assert_scores(got[i], ref, f"batched nQ={nQ} Nq={Nq} q={i}", lim)
            single = flash_maxsim_v2_multiquery(Qs[i], D).cpu().numpy()
            _assert_scores(got[i], single, "batched vs single")


class _RunConfig:
    """The one field of ColBERT's run config the reference's drop-in reads."""

    def __init__(self, total_visible_gpus):
        self.total_visible_gpus = total_visible_gpus


def test_plaid_packed_config_moves_host_tensors(cuda):
    """``config.total_visible_gpus > 0`` moves host Q, D_packed and D_lengths to the GPU
    before scoring, as the reference's drop-in does (``src/plaid_integration_benchmark.py:
    159-161``); with no GPU in the config (or no config) host tensors are refused."""
    import os

    import torch
    from tilemaxsim_amd import flashmaxsim_score_packed, flashmaxsim_score_packed_batched
    f = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "packed_zeros_d128.npz"),
                allow_pickle=False)
    Q, Dp, lens = (torch.from_numpy(f[k]) for k in ("Q", "D_packed", "lengths"))
    ref, lim = bar.with_bound(orc.maxsim_packed_zero_padded, f["Q"], f["D_packed"], f["lengths"])
    np.testing.assert_allclose(ref, f["scores"], rtol=1e-12)
    got = flashmaxsim_score_packed(Q[None], Dp, lens, _RunConfig(1))
    assert got.device.type == "cuda"
    _assert_scores(got.cpu().numpy(), f["scores"], "config, host tensors", lim)
    got_b = flashmaxsim_score_packed_batched(torch.stack([Q, Q.flip(0)]), Dp, lens, _RunConfig(8))
    _assert_scores(got_b[0].cpu().numpy(), f["scores"], "config, host tensors, batched", lim)
    _assert_scores(got_b[1].cpu().numpy(), got.cpu().numpy(), "a query's token order does not matter")
    got_m = flashmaxsim_score_packed(Q[None], Dp, lens, _RunConfig(1), padding="mask")
    offsets = np.concatenate([[0], np.cumsum(f["lengths"])]).astype(np.int64)
    _assert_scores(got_m.cpu().numpy(), *_oracle(orc.maxsim_varlen, f["Q"], f["D_packed"], offsets, f64=True,
                                                 what="config, host tensors, mask"))
    for config in (None, _RunConfig(0)):
        with pytest.raises(ValueError, match="GPU"):
            flashmaxsim_score_packed(Q[None], Dp, lens, config)
        with pytest.raises(ValueError, match="GPU"):
            flashmaxsim_score_packed_batched(Q[None], Dp, lens, config)
