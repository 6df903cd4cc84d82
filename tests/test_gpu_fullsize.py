"""Parity at the benchmark workloads' full sizes (C2-C5 with c2b/c3b/c5b, C2 in fp32, C3
in bf16, c6/c6b, top-k over C2's score matrix).

Every score of C2 (64 queries x 1M docs), C3 (32 queries x 2M varlen docs), C4 (16
queries x 200K docs at d = 256, 512 and 768) and C5 (32 queries x 5M PQ docs) is
compared with an independent fp32 restatement of the reference's materialise-then-reduce
oracle (``pytorch_maxsim_naive``, ``src/flash_maxsim_kernel.py:280-288``; for PQ the
decompress-then-score ``pytorch_pqsim_baseline``, ``src/flash_pqsim_kernel.py:283-313``),
run chunked on the same GPU with plain fp32 GEMMs (TF32 off): S = D_chunk @ Q^T, max over
each document's tokens, sum over query tokens. Bars on every document: |delta| <= 1e-3
relative + 1e-3 absolute (the north star's), and the fp32-accumulation bar of
``accum_bar.py`` with the restatement's own error added, on MaxSim(|Q|, |D|) from the
same restatement run on absolute values. Each query's top-100 must equal the
restatement's except for swaps among documents whose scores lie within the 1e-3
tolerance of each other (the north star's ranking criterion; the reference's consumer
is ``torch.topk``, ``src/cycle3_experiments.py:215``): every pick scores at least the
100th minus the tolerance, and every document that scores more than the tolerance above
the 100th is picked. Each test prints its largest errors. A seeded sample of documents,
always the first and the last (the largest offsets into multi-GB buffers), is also
checked against the float64 oracle, with the bar against it.
"""
import numpy as np
import pytest

import accum_bar as bar
from oracle import maxsim_oracle as orc
from oracle import residual_oracle as ro

pytestmark = pytest.mark.gpu

RTOL = bar.NORTH_STAR_RTOL
ATOL = bar.NORTH_STAR_ATOL


def _normal_fp16(torch, shape, seed, chunk=1 << 21):
    g = torch.Generator(device="cuda").manual_seed(seed)
    out = torch.empty(shape, dtype=torch.float16, device="cuda")
    flat = out.view(-1, shape[-1])
    for s in range(0, flat.shape[0], chunk):
        e = min(flat.shape[0], s + chunk)
        flat[s:e] = torch.nn.functional.normalize(torch.randn(e - s, shape[-1], device="cuda", generator=g),
                                                  dim=-1).half()
    return out


def _sample(n, k, seed):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, k)]))


def _release(torch):
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _fp32_no_tf32(torch):
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False


def _ref_fixed(torch, Qs, D, chunk_tokens=1 << 19, absolute=False):
    """fp32 MaxSim of every query in Qs (nQ, Nq, d) against D (B, Nd, d): (nQ, B);
    ``absolute`` scores |D| (each chunk taken absolute as it is read)."""
    _fp32_no_tf32(torch)
    nQ, Nq, d = Qs.shape
    B, Nd, _ = D.shape
    QT = Qs.reshape(nQ * Nq, d).float().t().contiguous()
    out = torch.empty(nQ, B, dtype=torch.float32, device="cuda")
    step = max(1, chunk_tokens // Nd)
    for b0 in range(0, B, step):
        b1 = min(B, b0 + step)
        Dc = D[b0:b1].reshape(-1, d).float()
        S = torch.mm(Dc.abs() if absolute else Dc, QT)  # ((b1-b0) Nd, nQ Nq)
        out[:, b0:b1] = S.view(b1 - b0, Nd, nQ, Nq).amax(dim=1).sum(dim=-1).t()
    return out


def _ref_varlen(torch, Qs, D_flat, offs, chunk_docs=2048, absolute=False):
    """fp32 MaxSim of every query in Qs against documents D_flat[offs[b]:offs[b+1]]
    (every document non-empty): each document's rows of S are gathered into a
    (docs, longest, queries) block, short documents repeating their last row, which
    leaves the max unchanged. ``absolute`` scores |D_flat|."""
    _fp32_no_tf32(torch)
    nQ, Nq, d = Qs.shape
    B = offs.numel() - 1
    QT = Qs.reshape(nQ * Nq, d).float().t().contiguous()
    offs_h = offs.cpu()
    lens = offs[1:] - offs[:-1]
    assert int(lens.min()) > 0
    L = int(lens.max())
    ar = torch.arange(L, device="cuda")
    out = torch.empty(nQ, B, dtype=torch.float32, device="cuda")
    for b0 in range(0, B, chunk_docs):
        b1 = min(B, b0 + chunk_docs)
        t0, t1 = int(offs_h[b0]), int(offs_h[b1])
        Dc = D_flat[t0:t1].float()
        S = torch.mm(Dc.abs() if absolute else Dc, QT)
        rows = (offs[b0:b1, None] - t0) + torch.minimum(ar[None, :], lens[b0:b1, None] - 1)
        m = S.index_select(0, rows.reshape(-1)).view(b1 - b0, L, nQ * Nq).amax(dim=1)
        out[:, b0:b1] = m.view(b1 - b0, nQ, Nq).sum(dim=-1).t()
    return out


def _ref_pq(torch, Qs, codebook, codes, chunk_docs=4096):
    """fp32 decompress-then-score: tokens rebuilt from the codebook in fp32, then MaxSim."""
    _fp32_no_tf32(torch)
    nQ, Nq, d = Qs.shape
    B, Nd, M = codes.shape
    cbf = codebook.float()
    QT = Qs.reshape(nQ * Nq, d).float().t().contiguous()
    msel = torch.arange(M, device="cuda")
    out = torch.empty(nQ, B, dtype=torch.float32, device="cuda")
    for b0 in range(0, B, chunk_docs):
        b1 = min(B, b0 + chunk_docs)
        Dc = cbf[msel, codes[b0:b1].long()]  # (nb, Nd, M, dsub)
        S = torch.mm(Dc.reshape(-1, d), QT)
        out[:, b0:b1] = S.view(b1 - b0, Nd, nQ, Nq).amax(dim=1).sum(dim=-1).t()
    return out


def _check_all(torch, got, ref, what, absref, d, nq):
    """Every score within RTOL/ATOL of the fp32 restatement and within the
    fp32-accumulation bar (``absref``: the restatement on absolute values); prints the
    largest errors."""
    err = (got - ref).abs()
    lim = RTOL * ref.abs() + ATOL
    acc = bar.rel(d, nq, restated=True) * absref
    rel = (err / ref.abs().clamp_min(1e-30)).max().item()
    print(f"{what}: {got.numel()} scores, max |delta| {err.max().item():.3e}, max relative {rel:.3e}, "
          f"max |delta| / accumulation bar {(err / acc).max().item():.3f}", flush=True)
    bad = int((err > lim).sum().item())
    assert bad == 0, f"{what}: {bad} scores outside the bar (worst |delta| {err.max().item():.3e})"
    bad = int((err > acc).sum().item())
    assert bad == 0, f"{what}: {bad} scores outside the fp32-accumulation bar"


def _check_top100(torch, got, ref, what, k=100):
    """Per query: the HIP top-k of our scores against torch.topk of the restatement's;
    identical except swaps among documents within the tolerance of each other."""
    from tilemaxsim_amd import topk
    gi = topk(got, k)[1]
    rv, ri = torch.topk(ref, k, dim=1)
    kth = rv[:, k - 1:k]
    tol = RTOL * kth.abs() + ATOL
    rg = torch.gather(ref, 1, gi)  # the restatement's scores of our picks, in our order
    assert bool((rg >= kth - tol).all()), f"{what}: a pick below the 100th score by more than the tolerance"
    assert bool((rg[:, 1:] <= rg[:, :-1] + tol).all()), f"{what}: order differs beyond the tolerance"
    clear = rv > kth + tol  # the restatement's picks that score clearly above its 100th
    picked = (ri[:, :, None] == gi[:, None, :]).any(dim=-1)
    assert bool((picked | ~clear).all()), f"{what}: a document clearly above the 100th score is not picked"
    same = int((gi == ri).sum().item())
    nset = sum(len(set(gi[q].tolist()) ^ set(ri[q].tolist())) for q in range(gi.shape[0]))
    print(f"{what}: top-{k} of {gi.shape[0]} queries, {same} of {gi.numel()} positions identical, "
          f"{nset // 2} set swaps (all within tolerance)", flush=True)


def test_c2_dense_and_batched_fullsize(cuda):
    """C2: 64 queries x 1M docs x Nd=180 x d=128 (46 GB); every query through the stream
    kernel (one HBM pass each, as the bench step) and all 64 through the batched kernel."""
    import torch
    from tilemaxsim_amd import flash_maxsim_batched_queries, flash_maxsim_v2_multiquery
    D = _normal_fp16(torch, (1_000_000, 180, 128), 11)
    Qs = _normal_fp16(torch, (64, 32, 128), 12)
    single = torch.stack([flash_maxsim_v2_multiquery(Qs[q], D) for q in range(64)])
    batched = flash_maxsim_batched_queries(Qs, D)
    ref = _ref_fixed(torch, Qs, D)
    absref = _ref_fixed(torch, Qs.abs(), D, absolute=True)
    _check_all(torch, single, ref, "C2 per-query stream kernel", absref, 128, 32)
    _check_all(torch, batched, ref, "C2 batched kernel", absref, 128, 32)
    _check_top100(torch, single, ref, "C2 per-query")
    _check_top100(torch, batched, ref, "C2 batched")
    idx = _sample(1_000_000, 60, 1)
    Dcpu = D[torch.from_numpy(idx).cuda()].cpu().numpy()
    for q in (0, 63):
        bar.assert_scores(single[q].cpu().numpy()[idx], *bar.with_bound(orc.maxsim_f64, Qs[q].cpu().numpy(), Dcpu),
                          f"C2 sample q={q}")
    del D, single, batched, ref, absref
    _release(torch)


def _normal_fp32(torch, shape, seed, chunk=1 << 21):
    g = torch.Generator(device="cuda").manual_seed(seed)
    out = torch.empty(shape, dtype=torch.float32, device="cuda")
    flat = out.view(-1, shape[-1])
    for s in range(0, flat.shape[0], chunk):
        e = min(flat.shape[0], s + chunk)
        flat[s:e] = torch.nn.functional.normalize(torch.randn(e - s, shape[-1], device="cuda", generator=g), dim=-1)
    return out


def test_c2_fp32_fullsize(cuda):
    """C2 in fp32 (1M docs x Nd=180 x d=128: 92 GB, `bench.py --config c2 --dtype fp32`):
    16 queries, each through the per-query kernel (fp32 documents read as whole lines,
    split into bf16 hi + lo terms, three MFMAs per product), every score against the
    fp32 restatement to the fp32 bar of test_gpu_fp32.py, (4 * 2^-16 + d * 2^-24) *
    MaxSim(|Q|, |D|), plus the restatement's own fp32-accumulation error."""
    import torch
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    D = _normal_fp32(torch, (1_000_000, 180, 128), 13)
    Qs = _normal_fp32(torch, (16, 32, 128), 14)
    got = torch.stack([flash_maxsim_v2_multiquery(Qs[q], D) for q in range(16)])
    ref = _ref_fixed(torch, Qs, D)
    absref = _ref_fixed(torch, Qs.abs(), D, absolute=True)
    err = (got - ref).abs()
    lim = (4 * 2.0 ** -16 + 128 * 2.0 ** -24 + bar.rel(128, 32)) * absref
    print(f"C2 fp32: {got.numel()} scores, max |delta| {err.max().item():.3e}, "
          f"max |delta| / bar {(err / lim).max().item():.3f}", flush=True)
    bad = int((err > lim).sum().item())
    assert bad == 0, f"C2 fp32: {bad} scores outside the fp32 bar"
    _check_top100(torch, got, ref, "C2 fp32 per-query")
    idx = _sample(1_000_000, 60, 3)
    Dcpu = D[torch.from_numpy(idx).cuda()].cpu().numpy()
    for q in (0, 15):
        Q = Qs[q].cpu().numpy()
        ref64 = orc.maxsim_f64(Q, Dcpu)
        abs64 = orc.maxsim_f64(np.abs(Q), np.abs(Dcpu))
        g = got[q].cpu().numpy()[idx].astype(np.float64)
        assert np.all(np.abs(g - ref64) <= (4 * 2.0 ** -16 + 128 * 2.0 ** -24) * abs64 + 1e-6), f"C2 fp32 sample q={q}"
    del D, got, ref, absref
    _release(torch)


def test_c3_varlen_fullsize(cuda):
    """C3: 32 queries x 2M docs, Nd ~ U[32, 300] (332M tokens, 85 GB), int64 offsets;
    every query through the varlen kernel and all 32 through the batched kernel (c3b)."""
    import torch
    from tilemaxsim_amd import flash_maxsim_multi_doc, flash_maxsim_multi_doc_batched
    rng = np.random.default_rng(77)
    lens = rng.integers(32, 301, size=2_000_000)
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    D = _normal_fp16(torch, (int(offs[-1]), 128), 21)
    Qs = _normal_fp16(torch, (32, 32, 128), 22)
    offs_t = torch.from_numpy(offs).cuda()
    single = torch.stack([flash_maxsim_multi_doc(Qs[q], D, offs_t, validate=False) for q in range(32)])
    batched = flash_maxsim_multi_doc_batched(Qs, D, offs_t, validate=False)
    ref = _ref_varlen(torch, Qs, D, offs_t)
    absref = _ref_varlen(torch, Qs.abs(), D, offs_t, absolute=True)
    _check_all(torch, single, ref, "C3 per-query varlen kernel", absref, 128, 32)
    _check_all(torch, batched, ref, "C3 batched kernel", absref, 128, 32)
    _check_top100(torch, single, ref, "C3 per-query")
    _check_top100(torch, batched, ref, "C3 batched")
    idx = _sample(2_000_000, 60, 2)
    rows = np.concatenate([np.arange(offs[b], offs[b + 1]) for b in idx])
    sub = D[torch.from_numpy(rows).cuda()].cpu().numpy()
    sub_offs = np.concatenate([[0], np.cumsum(lens[idx])]).astype(np.int64)
    for q in (0, 31):
        bar.assert_scores(single[q].cpu().numpy()[idx],
                          *bar.with_bound(orc.maxsim_varlen, Qs[q].cpu().numpy(), sub, sub_offs, f64=True),
                          f"C3 sample q={q}")
    del D, single, batched, ref, absref
    _release(torch)


def test_c3_bf16_fullsize(cuda):
    """C3's 332M-token corpus in bf16 (85 GB), 8 queries through the variable-length
    stream kernel (bf16 rows read as whole lines): every score against the fp32
    restatement, to the fp32-accumulation bar and the north star's 1e-3."""
    import torch
    from tilemaxsim_amd import flash_maxsim_multi_doc
    rng = np.random.default_rng(78)
    lens = rng.integers(32, 301, size=2_000_000)
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    D = _normal_fp16(torch, (int(offs[-1]), 128), 23).to(torch.bfloat16)
    _release(torch)
    Qs = _normal_fp16(torch, (8, 32, 128), 24).to(torch.bfloat16)
    offs_t = torch.from_numpy(offs).cuda()
    got = torch.stack([flash_maxsim_multi_doc(Qs[q], D, offs_t, validate=False) for q in range(8)])
    ref = _ref_varlen(torch, Qs, D, offs_t)
    absref = _ref_varlen(torch, Qs.abs(), D, offs_t, absolute=True)
    _check_all(torch, got, ref, "C3 bf16 per-query varlen stream kernel", absref, 128, 32)
    _check_top100(torch, got, ref, "C3 bf16 per-query")
    del D, got, ref, absref
    _release(torch)


@pytest.mark.parametrize("d", [256, 512, 768])
def test_c4_dtiled_fullsize(cuda, d):
    """C4: 16 queries x 200K docs x Nd=128 at d = 256, 512, 768 (13-39 GB), Q in LDS."""
    import torch
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    D = _normal_fp16(torch, (200_000, 128, d), 30 + d)
    Qs = _normal_fp16(torch, (16, 32, d), 31 + d)
    got = torch.stack([flash_maxsim_v2_multiquery(Qs[q], D) for q in range(16)])
    ref = _ref_fixed(torch, Qs, D)
    absref = _ref_fixed(torch, Qs.abs(), D, absolute=True)
    _check_all(torch, got, ref, f"C4 d={d}", absref, d, 32)
    _check_top100(torch, got, ref, f"C4 d={d}")
    idx = _sample(200_000, 40, 3)
    bar.assert_scores(got[0].cpu().numpy()[idx],
                      *bar.with_bound(orc.maxsim_f64, Qs[0].cpu().numpy(),
                                      D[torch.from_numpy(idx).cuda()].cpu().numpy()), f"C4 d={d} sample")
    del D, got, ref, absref
    _release(torch)


def test_c5_pq_fullsize(cuda):
    """C5: 32 queries x 5M docs x Nd=128 x M=16 uint8 codes (10.24 GB): every query
    through the MFMA kernel and all 32 through the batched kernel (c5b), against fp32
    decompress-then-score; the table-gather kernel on two queries."""
    import torch
    from tilemaxsim_amd import TileMaxSimPQ
    g = torch.Generator(device="cuda").manual_seed(41)
    codes = torch.randint(0, 256, (5_000_000, 128, 16), dtype=torch.uint8, device="cuda", generator=g)
    cb = torch.randn(16, 256, 8, device="cuda", generator=g).half()
    Qs = _normal_fp16(torch, (32, 32, 128), 42)
    pq = TileMaxSimPQ(cb)
    single = torch.stack([pq.score_batch(Qs[q], codes, validate=False) for q in range(32)])
    batched = pq.score_batch_queries(Qs, codes, validate=False)
    ref = _ref_pq(torch, Qs, cb, codes)
    absref = _ref_pq(torch, Qs.abs(), cb.abs(), codes)
    _check_all(torch, single, ref, "C5 per-query MFMA kernel", absref, 128, 32)
    _check_all(torch, batched, ref, "C5 batched kernel", absref, 128, 32)
    _check_top100(torch, single, ref, "C5 per-query")
    _check_top100(torch, batched, ref, "C5 batched")
    lut = torch.stack([pq.score_batch(Qs[q], codes, method="lut", validate=False) for q in (0, 31)])
    _check_all(torch, lut, ref[[0, 31]], "C5 table-gather kernel (queries 0 and 31)", absref[[0, 31]], 128, 32)
    idx = _sample(5_000_000, 60, 4)
    bar.assert_scores(single[0].cpu().numpy()[idx],
                      *bar.with_bound(orc.pq_decompress_score, Qs[0].cpu().numpy(), cb.cpu().numpy(),
                                      codes[torch.from_numpy(idx).cuda()].cpu().numpy(), f64=True), "C5 sample")
    del codes, single, batched, ref, absref
    _release(torch)


def test_c6_residual_fullsize(cuda):
    """c6: C3's corpus as a ColBERTv2 index (nbits=2, 262,144 centroids, 12 GB), one query
    through the fused kernel; c6b: 32 queries through the batched kernel. A seeded sample
    against the float64 codec oracle."""
    import torch
    from tilemaxsim_amd import flashmaxsim_score_residual, flashmaxsim_score_residual_batched
    rng = np.random.default_rng(77)
    lens = rng.integers(32, 301, size=2_000_000)
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(offs[-1])
    g = torch.Generator(device="cuda").manual_seed(51)
    codes = torch.randint(0, 1 << 18, (T,), dtype=torch.int32, device="cuda", generator=g)
    res = torch.randint(0, 256, (T, 32), dtype=torch.uint8, device="cuda", generator=g)
    cent = _normal_fp16(torch, (1 << 18, 128), 52)
    w = torch.tensor([-0.05, -0.012, 0.012, 0.05], dtype=torch.float16, device="cuda")
    Q = _normal_fp16(torch, (32, 128), 53)
    got = flashmaxsim_score_residual(Q, codes, res, cent, w, 2, torch.from_numpy(offs).cuda(), padding="mask",
                                     validate=False).cpu().numpy()
    idx = _sample(2_000_000, 40, 5)
    rows = torch.from_numpy(np.concatenate([np.arange(offs[b], offs[b + 1]) for b in idx])).cuda()
    sub_offs = np.concatenate([[0], np.cumsum(lens[idx])]).astype(np.int64)
    ref = ro.maxsim_residual(Q.cpu().numpy(), codes[rows].cpu().numpy(), res[rows].cpu().numpy(), cent.cpu().numpy(),
                             w.cpu().numpy(), 2, sub_offs)
    np.testing.assert_allclose(got[idx], ref, rtol=RTOL, atol=ATOL)
    # c6b: all 32 queries through the batched kernel, checked on the same sample
    Qs = _normal_fp16(torch, (32, 32, 128), 54)
    gotb = flashmaxsim_score_residual_batched(Qs, codes, res, cent, w, 2, torch.from_numpy(offs).cuda(),
                                              padding="mask", validate=False).cpu().numpy()
    sub = (codes[rows].cpu().numpy(), res[rows].cpu().numpy(), cent.cpu().numpy(), w.cpu().numpy())
    for q in (0, 17, 31):
        refq = ro.maxsim_residual(Qs[q].cpu().numpy(), *sub, 2, sub_offs)
        np.testing.assert_allclose(gotb[q][idx], refq, rtol=RTOL, atol=ATOL)
    del codes, res
    _release(torch)


def test_topk_over_c2_score_matrix(cuda):
    """The bench's top-100 over a (64, 1M) fp32 score matrix, bit for bit."""
    import torch
    from tilemaxsim_amd import topk
    g = torch.Generator(device="cuda").manual_seed(61)
    scores = torch.randn(64, 1_000_000, device="cuda", generator=g)
    v, i = topk(scores, 100)
    s = scores.cpu().numpy()
    v, i = v.cpu().numpy(), i.cpu().numpy()
    for row in range(64):
        ev, ei = orc.topk(s[row], 100)
        assert np.array_equal(i[row], ei) and np.array_equal(v[row], ev), row
