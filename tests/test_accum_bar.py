"""The fp32-accumulation bar (``accum_bar.py``) separates fp32 accumulation from what a
lower-precision kernel would compute.

CPU: three restatements of the 16-bit MaxSim, each exact products from fp16 inputs --
accumulated in fp32 (what the reference's ``tl.dot`` does, ``src/flash_maxsim_v2.py:117``),
accumulated in fp16, and with every product rounded to bf16 before an exact sum. The
first stays inside the bar; the other two miss it for every document on "coherent"
inputs (every product rounds the same way) and for most documents on L2-normalised
Gaussian inputs, for dense documents and for PQ tokens decoded through a codebook.

GPU: every 16-bit kernel form scores the coherent inputs inside the bar.
"""
import numpy as np
import pytest
import torch

import accum_bar as bar
from oracle import maxsim_oracle as orc


def _coherent_q(rng, shape):
    """fp16 values m * 2^-f with m = 1 + (8n + 2) * 2^-10: rounding m to bf16 (7 fraction
    bits) drops 2 * 2^-10, a quarter of its unit in the last place, always downwards."""
    n = rng.integers(0, 128, shape)
    f = rng.integers(3, 6, shape)
    return ((1 + (8 * n + 2) / 1024.0) * 2.0 ** -f).astype(np.float16)


def _coherent_d(rng, shape):
    """Positive powers of two: a product with one keeps the other factor's significand."""
    return (2.0 ** -rng.integers(3, 7, shape)).astype(np.float16)


def _normal(rng, shape):
    x = rng.standard_normal(shape, dtype=np.float32)
    return (x / np.linalg.norm(x, axis=-1, keepdims=True)).astype(np.float16)


def _sims_fp32(Q, D):
    """Per (document, token, query token): products exact in fp32, summed in fp32 in
    order of the embedding dimension."""
    s = np.zeros((D.shape[0], D.shape[1], Q.shape[0]), np.float32)
    for k in range(Q.shape[1]):
        s = s + D[:, :, k].astype(np.float32)[:, :, None] * Q[:, k].astype(np.float32)[None, None, :]
    return s


def _sims_fp16_acc(Q, D):
    """The same products, each partial sum rounded to fp16."""
    s = np.zeros((D.shape[0], D.shape[1], Q.shape[0]), np.float16)
    for k in range(Q.shape[1]):
        p = D[:, :, k].astype(np.float32)[:, :, None] * Q[:, k].astype(np.float32)[None, None, :]
        s = (s.astype(np.float32) + p).astype(np.float16)
    return s


def _sims_bf16_products(Q, D):
    """Every product rounded to bf16, then summed exactly (float64)."""
    P = torch.from_numpy(D.astype(np.float32))[:, :, None, :] * torch.from_numpy(Q.astype(np.float32))[None, None]
    return P.to(torch.bfloat16).double().sum(-1).numpy()


def _scores(S):
    return np.asarray(S, np.float64).max(axis=1).sum(axis=-1)


def _ratios(Q, D, ref, lim):
    return {name: np.abs(_scores(fn(Q, D)) - ref) / lim
            for name, fn in (("fp32", _sims_fp32), ("fp16 accumulation", _sims_fp16_acc),
                             ("bf16 products", _sims_bf16_products))}


@pytest.mark.parametrize("inputs", ["coherent", "normal"])
def test_bar_separates_fp32_accumulation_from_lower_precision(inputs):
    rng = np.random.default_rng(3)
    if inputs == "coherent":
        Q, D = _coherent_q(rng, (32, 128)), _coherent_d(rng, (200, 64, 128))
    else:
        Q, D = _normal(rng, (32, 128)), _normal(rng, (200, 64, 128))
    ref, lim = bar.with_bound(orc.maxsim_f64, Q, D)
    r = _ratios(Q, D, ref, lim)
    assert r["fp32"].max() <= 1.0
    for name in ("fp16 accumulation", "bf16 products"):
        if inputs == "coherent":
            assert r[name].min() > 10.0, (name, r[name].min())
        else:
            assert np.mean(r[name] > 1.0) > 0.5, (name, np.mean(r[name] > 1.0))
            assert r[name].max() > 3.0, name


def test_bar_separates_pq_restatements():
    """PQ tokens decoded through a codebook of powers of two (M = 16, K = 256, dsub = 8)
    against coherent queries: the same separation for the decoded products."""
    rng = np.random.default_rng(9)
    C = _coherent_d(rng, (16, 256, 8))
    codes = rng.integers(0, 256, (150, 40, 16)).astype(np.uint8)
    Q = _coherent_q(rng, (32, 128))
    ref, lim = bar.with_bound(orc.pq_decompress_score, Q, C, codes, f64=True)
    D = orc.pq_decompress(C, codes, dtype=np.float32).astype(np.float16)
    np.testing.assert_allclose(orc.maxsim_f64(Q, D), ref, rtol=1e-15)
    r = _ratios(Q, D, ref, lim)
    assert r["fp32"].max() <= 1.0
    assert r["fp16 accumulation"].min() > 10.0 and r["bf16 products"].min() > 10.0


def test_bound_terms():
    """The bar's factor: (d + Nq) operations at 2^-23; a split query doubles the product
    terms and adds its split residual; an fp32 restatement adds its own (d + Nq)."""
    assert bar.rel(128, 32) == 160 * 2.0 ** -23
    assert bar.rel(128, 32, qsplit="fp16") == 288 * 2.0 ** -23 + 2.0 ** -21
    assert bar.rel(128, 32, qsplit="bf16") == 288 * 2.0 ** -23 + 2.0 ** -15
    assert bar.rel(128, 32, restated=True) == 2 * 160 * 2.0 ** -23
    lim = bar.bound(np.array([2.0, -np.inf, 0.0]), 128, 32)
    assert lim[0] == 2 * 160 * 2.0 ** -23 + 1e-30 and lim[1] == 1e-30 and lim[2] == 1e-30


@pytest.mark.gpu
def test_kernels_inside_the_bar_on_coherent_inputs(cuda):
    """Every 16-bit form on the coherent inputs: the one-pass stream kernel (d = 128), the
    small-batch kernel, the d-tiled kernel (d = 256), variable-length, masked, batched
    queries, the PLAID packed scorer and both PQ kernels and the batched PQ kernel."""
    import tilemaxsim_amd as tms
    from tilemaxsim_amd import _lib
    rng = np.random.default_rng(5)
    g = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    for d in (128, 256):
        Q, D = _coherent_q(rng, (32, d)), _coherent_d(rng, (300, 70, d))
        ref, lim = bar.with_bound(orc.maxsim_f64, Q, D)
        for limit in (0, 1 << 40):
            with _lib.rerank_limit(limit):
                bar.assert_scores(tms.flash_maxsim_v2_multiquery(g(Q), g(D)).cpu().numpy(), ref, lim,
                                  f"dense d={d} limit={limit}")
        lens = rng.integers(0, 71, 300)
        offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        flat = np.concatenate([D[b, : lens[b]] for b in range(300)])
        vref, vlim = bar.with_bound(orc.maxsim_varlen, Q, flat, offsets, f64=True)
        bar.assert_scores(tms.flash_maxsim_multi_doc(g(Q), g(flat), g(offsets)).cpu().numpy(), vref, vlim,
                          f"varlen d={d}")
        pref, plim = bar.with_bound(orc.maxsim_packed_zero_padded, Q, flat, lens)
        bar.assert_scores(tms.flashmaxsim_score_packed(g(Q), g(flat), g(lens)).cpu().numpy(), pref, plim,
                          f"packed d={d}")
        mask = rng.random((300, 70)) < 0.5
        mref, mlim = bar.with_bound(orc.maxsim_masked, Q, D, mask, f64=True)
        bar.assert_scores(tms.maxsim_score(g(Q), g(D), g(mask)).cpu().numpy(), mref, mlim, f"masked d={d}")
        Qs = np.stack([Q, _coherent_q(rng, (32, d)), _coherent_q(rng, (32, d))])
        got = tms.flash_maxsim_batched_queries(g(Qs), g(D)).cpu().numpy()
        for q in range(3):
            bar.assert_scores(got[q], *bar.with_bound(orc.maxsim_f64, Qs[q], D), f"batched d={d} q={q}")
    C = _coherent_d(rng, (16, 256, 8))
    codes = rng.integers(0, 256, (400, 50, 16)).astype(np.uint8)
    Qs = np.stack([_coherent_q(rng, (32, 128)) for _ in range(3)])
    pq = tms.TileMaxSimPQ(g(C))
    got_b = pq.score_batch_queries(g(Qs), g(codes)).cpu().numpy()
    for q in range(3):
        ref, lim = bar.with_bound(orc.pq_decompress_score, Qs[q], C, codes, f64=True)
        for method in ("mfma", "lut"):
            bar.assert_scores(pq.score_batch(g(Qs[q]), g(codes), method=method).cpu().numpy(), ref, lim,
                              f"pq {method} q={q}")
        bar.assert_scores(got_b[q], ref, lim, f"pq batched q={q}")
