"""Parity at the benchmark workloads' full sizes (C2-C5 with c2b/c3b, c6/c6b, top-k over C2's score matrix).

Each test builds one configuration at its benchmark size on the GPU, scores it through
the public entry points, and checks a seeded sample of documents, always including the
first and the last (the largest offsets into multi-GB buffers), against the float64
oracle on copies of exactly those documents. Top-k is checked bit for bit on the whole
(64, 1M) score matrix. Tolerance: 1e-3 relative + 1e-3 absolute.
"""
import numpy as np
import pytest

from oracle import maxsim_oracle as orc
from oracle import residual_oracle as ro

pytestmark = pytest.mark.gpu

RTOL = ATOL = 1e-3


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


def test_c2_dense_and_batched_fullsize(cuda):
    """C2: 1M docs x Nd=180 x d=128 (46 GB); one query through the stream kernel and
    four through the batched-query kernel."""
    import torch
    from tilemaxsim_amd import flash_maxsim_batched_queries, flash_maxsim_v2_multiquery
    D = _normal_fp16(torch, (1_000_000, 180, 128), 11)
    Qs = _normal_fp16(torch, (4, 32, 128), 12)
    single = flash_maxsim_v2_multiquery(Qs[0], D)
    batched = flash_maxsim_batched_queries(Qs, D)
    idx = _sample(1_000_000, 60, 1)
    Dcpu = D[torch.from_numpy(idx).cuda()].cpu().numpy()
    Qcpu = Qs.cpu().numpy()
    for q in range(4):
        ref = orc.maxsim_f64(Qcpu[q], Dcpu)
        np.testing.assert_allclose(batched[q].cpu().numpy()[idx], ref, rtol=RTOL, atol=ATOL)
        if q == 0:
            np.testing.assert_allclose(single.cpu().numpy()[idx], ref, rtol=RTOL, atol=ATOL)
    del D, single, batched
    _release(torch)


def test_c3_varlen_fullsize(cuda):
    """C3: 2M docs, Nd ~ U[32, 300] (332M tokens, 85 GB), int64 offsets; one query through
    the varlen kernel and 32 through the batched kernel (c3b)."""
    import torch
    from tilemaxsim_amd import flash_maxsim_multi_doc, flash_maxsim_multi_doc_batched
    rng = np.random.default_rng(77)
    lens = rng.integers(32, 301, size=2_000_000)
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    D = _normal_fp16(torch, (int(offs[-1]), 128), 21)
    Q = _normal_fp16(torch, (32, 128), 22)
    got = flash_maxsim_multi_doc(Q, D, torch.from_numpy(offs).cuda()).cpu().numpy()
    idx = _sample(2_000_000, 60, 2)
    rows = np.concatenate([np.arange(offs[b], offs[b + 1]) for b in idx])
    sub = D[torch.from_numpy(rows).cuda()].cpu().numpy()
    sub_offs = np.concatenate([[0], np.cumsum(lens[idx])]).astype(np.int64)
    ref = orc.maxsim_varlen(Q.cpu().numpy(), sub, sub_offs, f64=True)
    np.testing.assert_allclose(got[idx], ref, rtol=RTOL, atol=ATOL)
    # c3b: 32 queries through the batched kernel, three of them checked on the sample
    Qs = _normal_fp16(torch, (32, 32, 128), 23)
    gotb = flash_maxsim_multi_doc_batched(Qs, D, torch.from_numpy(offs).cuda(), validate=False).cpu().numpy()
    for q in (0, 13, 31):
        refq = orc.maxsim_varlen(Qs[q].cpu().numpy(), sub, sub_offs, f64=True)
        np.testing.assert_allclose(gotb[q][idx], refq, rtol=RTOL, atol=ATOL)
    del D
    _release(torch)


def test_c4_dtiled_fullsize(cuda):
    """C4 at its largest width: 200K docs x Nd=128 x d=768 (39 GB), Q in LDS."""
    import torch
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    D = _normal_fp16(torch, (200_000, 128, 768), 31)
    Q = _normal_fp16(torch, (32, 768), 32)
    got = flash_maxsim_v2_multiquery(Q, D).cpu().numpy()
    idx = _sample(200_000, 40, 3)
    ref = orc.maxsim_f64(Q.cpu().numpy(), D[torch.from_numpy(idx).cuda()].cpu().numpy())
    np.testing.assert_allclose(got[idx], ref, rtol=RTOL, atol=ATOL)
    del D
    _release(torch)


def test_c5_pq_fullsize(cuda):
    """C5: 5M docs x Nd=128 x M=16 uint8 codes (10.24 GB), both PQ algorithms on a
    sample; the MFMA kernel on everything."""
    import torch
    from tilemaxsim_amd import TileMaxSimPQ
    g = torch.Generator(device="cuda").manual_seed(41)
    codes = torch.randint(0, 256, (5_000_000, 128, 16), dtype=torch.uint8, device="cuda", generator=g)
    cb = torch.randn(16, 256, 8, device="cuda", generator=g).half()
    Q = _normal_fp16(torch, (32, 128), 42)
    got = TileMaxSimPQ(cb).score_batch(Q, codes, validate=False).cpu().numpy()
    idx = _sample(5_000_000, 60, 4)
    ref = orc.pq_decompress_score(Q.cpu().numpy(), cb.cpu().numpy(), codes[torch.from_numpy(idx).cuda()].cpu().numpy(),
                                  f64=True)
    np.testing.assert_allclose(got[idx], ref, rtol=RTOL, atol=ATOL)
    del codes
    _release(torch)


def test_c6_residual_fullsize(cuda):
    """c6: C3's corpus as a ColBERTv2 index (nbits=2, 262,144 centroids, 12 GB), one query
    through the fused kernel; c6b: 32 queries through the batched kernel."""
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
