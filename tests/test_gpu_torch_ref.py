"""HIP entry points against plain PyTorch fp32 restatements of the reference's own
oracles, computed on the CPU:

* ``pytorch_maxsim_naive`` (``src/flash_maxsim_kernel.py:280-288``):
  ``einsum('qd,bnd->bqn', Q.float(), D.float()).max(-1).values.sum(-1)``;
* the masked scorer ``pytorch_maxsim_score`` (``src/e2e_retrieval_quality.py:105-110``):
  masked document tokens at -inf before the max;
* ``pytorch_pqsim_baseline`` (``src/flash_pqsim_kernel.py:283-313``): decompress the codes
  through the codebook to fp32, then the same MaxSim.

Bars: |score - reference| <= 1e-3 relative (+1e-3 absolute); for 16-bit inputs also the
fp32-accumulation bar of ``accum_bar.py`` with the fp32 restatement's own error added
(``restated=True``); and top-100 lists equal except for swaps among scores within the
1e-3 tolerance of the 100th. The float64 numpy oracle (``oracle/``) is the primary
checker; this file pins the same kernels to the reference's own arithmetic (fp32
products and sums in torch's order).
"""
import numpy as np
import pytest

import accum_bar as bar

pytestmark = pytest.mark.gpu

RTOL = bar.NORTH_STAR_RTOL
ATOL = bar.NORTH_STAR_ATOL


def _close(got, ref, lim=None, what=""):
    """The 1e-3 bar (torch's check), and the accumulation bar ``lim`` when given."""
    import torch
    torch.testing.assert_close(got, ref, rtol=RTOL, atol=ATOL)
    bar.assert_scores(got.numpy(), ref.numpy(), lim, what)


def _lim(fn, Q, X, *rest):
    """The accumulation bar against an fp32 restatement: ``fn`` on |Q| and |X|."""
    absref = fn(Q.abs(), X.abs(), *rest).double().numpy()
    return bar.bound(absref, Q.shape[-1], Q.shape[-2], restated=True)


def _naive(Q, D):
    import torch
    return torch.einsum("qd,bnd->bqn", Q.float(), D.float()).max(-1).values.sum(-1)


def _masked(Q, D, mask):
    import torch
    S = torch.einsum("qd,bnd->bqn", Q.float(), D.float())
    S = S.masked_fill(~mask[:, None, :], float("-inf"))
    return S.max(-1).values.sum(-1)


def _pq_baseline(Q, codebook, codes):
    import torch
    M = codebook.shape[0]
    D = torch.cat([codebook[m].float()[codes[:, :, m].long()] for m in range(M)], dim=-1)
    return _naive(Q, D)


def _check_topk(got, ref, k=100):
    import torch
    kth = torch.topk(ref, k).values[-1].item()
    gi = set(torch.topk(got, k).indices.tolist())
    ri = set(torch.topk(ref, k).indices.tolist())
    for d in gi ^ ri:
        assert abs(ref[d].item() - kth) <= RTOL * abs(kth) + ATOL, (d, ref[d].item(), kth)


def _normed(g, shape):
    import torch
    x = torch.randn(*shape, generator=g)
    return torch.nn.functional.normalize(x, dim=-1).half()


@pytest.mark.parametrize("nq,d,nd", [(32, 128, 180), (32, 256, 64), (20, 64, 33), (64, 128, 128), (32, 768, 40)])
def test_dense_vs_torch_naive(cuda, nq, d, nd):
    import torch
    from tilemaxsim_amd import flash_maxsim_v2_multiquery
    g = torch.Generator().manual_seed(nq * 1000 + d + nd)
    Q, D = _normed(g, (nq, d)), _normed(g, (600, nd, d))
    got = flash_maxsim_v2_multiquery(Q.cuda(), D.cuda()).cpu()
    ref = _naive(Q, D)
    _close(got, ref, _lim(_naive, Q, D), f"nq={nq} d={d} nd={nd}")
    _check_topk(got, ref)


def test_varlen_and_masked_vs_torch(cuda):
    import torch
    from tilemaxsim_amd import flash_maxsim_multi_doc, maxsim_score
    g = torch.Generator().manual_seed(5)
    B, Nmax, d = 400, 150, 128
    lens = torch.randint(1, Nmax + 1, (B,), generator=g)
    Q, D = _normed(g, (32, d)), _normed(g, (B, Nmax, d))
    mask = torch.arange(Nmax)[None, :] < lens[:, None]
    ref = _masked(Q, D, mask)
    lim = _lim(_masked, Q, D, mask)
    got = maxsim_score(Q.cuda(), D.cuda(), mask.cuda()).cpu()
    _close(got, ref, lim, "masked")
    flat = torch.cat([D[b, : lens[b]] for b in range(B)])
    offsets = torch.zeros(B + 1, dtype=torch.int64)
    offsets[1:] = torch.cumsum(lens, 0)
    got_v = flash_maxsim_multi_doc(Q.cuda(), flat.cuda(), offsets).cpu()
    _close(got_v, ref, lim, "varlen")
    _check_topk(got_v, ref)


@pytest.mark.parametrize("M,dsub", [(16, 8), (32, 4), (8, 16)])
def test_pq_vs_torch_baseline(cuda, M, dsub):
    import torch
    from tilemaxsim_amd import TileMaxSimPQ
    g = torch.Generator().manual_seed(M * 100 + dsub)
    K, B, Nd = 256, 500, 64
    C = torch.randn(M, K, dsub, generator=g).half()
    codes = torch.randint(0, K, (B, Nd, M), generator=g, dtype=torch.int64).to(torch.uint8)
    Q = _normed(g, (32, M * dsub))
    ref = _pq_baseline(Q, C, codes)
    lim = _lim(_pq_baseline, Q, C, codes)
    pq = TileMaxSimPQ(C.cuda())
    for method in ("auto", "lut"):
        got = pq.score_batch(Q.cuda(), codes.cuda(), method=method).cpu()
        _close(got, ref, lim, f"pq {method}")
    Qs = torch.stack([Q, _normed(g, (32, M * dsub))])
    got_b = pq.score_batch_queries(Qs.cuda(), codes.cuda()).cpu()
    _close(got_b[0], ref, lim, "pq batched q=0")
    _close(got_b[1], _pq_baseline(Qs[1], C, codes), _lim(_pq_baseline, Qs[1], C, codes), "pq batched q=1")
    _check_topk(got_b[0], ref)


def test_batched_queries_vs_torch_naive(cuda):
    import torch
    from tilemaxsim_amd import flash_maxsim_batched_queries
    g = torch.Generator().manual_seed(9)
    Qs, D = _normed(g, (6, 32, 128)), _normed(g, (700, 90, 128))
    got = flash_maxsim_batched_queries(Qs.cuda(), D.cuda()).cpu()
    for q in range(6):
        ref = _naive(Qs[q], D)
        _close(got[q], ref, _lim(_naive, Qs[q], D), f"batched q={q}")
        _check_topk(got[q], ref)


def test_fp32_dense_vs_torch_naive(cuda):
    """fp32 inputs, unnormalised as in the reference's precision experiment
    (``src/cycle6_rerun_scaling.py:96-106``)."""
    import torch
    from tilemaxsim_amd import flash_maxsim_multi_doc, flash_maxsim_v2_multiquery
    g = torch.Generator().manual_seed(77)
    Q, D = torch.randn(32, 128, generator=g), torch.randn(500, 70, 128, generator=g)
    ref = _naive(Q, D)
    got = flash_maxsim_v2_multiquery(Q.cuda(), D.cuda()).cpu()
    torch.testing.assert_close(got, ref, rtol=RTOL, atol=ATOL)
    _check_topk(got, ref)
    offsets = torch.arange(0, 501 * 70, 70, dtype=torch.int64)
    got_v = flash_maxsim_multi_doc(Q.cuda(), D.reshape(-1, 128).cuda(), offsets.cuda()).cpu()
    torch.testing.assert_close(got_v, ref, rtol=RTOL, atol=ATOL)
