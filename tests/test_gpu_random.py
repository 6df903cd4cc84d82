"""Seeded random sweep over shapes, dtypes and entry points against the float64 oracle.

Each case draws (from its own seed) the number of query tokens, documents, document
lengths (fixed, or ragged with empty documents), the embedding width (aligned widths
that take the register paths, widths that take the LDS path, and widths that are not
a multiple of 8), the dtype, whether the embeddings are L2-normalised, and the entry
point. The bars are those of the other parity tests: for fp16 / bf16 inputs scored
against the oracle on the same rounded values, 1e-3 relative (+1e-3 absolute) and the
fp32-accumulation bar of ``accum_bar.py``; for fp32 inputs (and for fp32 queries against
fp16 / bf16 documents, which are split, not rounded) the split-product bound of
``test_gpu_fp32.py``; -inf exactly where the oracle has it.

``TMS_RANDOM_SEEDS=N`` (default 160) widens the sweep: N seeds of the main case, 3N/8 of
the split-query case and 9N/40 of the PQ case.
"""
import os

import numpy as np
import pytest

import accum_bar as bar
from oracle import maxsim_oracle as orc

N_SEEDS = int(os.environ.get("TMS_RANDOM_SEEDS", "160"))

pytestmark = pytest.mark.gpu

WIDTHS = [32, 64, 96, 128, 128, 128, 40, 72, 100, 136, 192, 256, 320, 520]
ENTRY = ["dense", "masked", "varlen", "batched_dense", "batched_varlen", "packed_zeros"]


def _case(seed):
    rng = np.random.default_rng(seed)
    c = {
        "nq": int(rng.choice([1, 5, 16, 31, 32, 33, 64, 70])),
        "B": int(rng.integers(1, 300)),
        "nd": int(rng.choice([1, 7, 16, 33, 64, 128, 181])),
        "d": int(rng.choice(WIDTHS)),
        "dtype": str(rng.choice(["fp16", "bf16", "fp32"])),
        "norm": bool(rng.integers(0, 2)),
        "entry": ENTRY[seed % len(ENTRY)],
        "nQ": int(rng.integers(2, 6)),
    }
    return c, rng


def _round(x, dtype):
    """The values the kernel sees: fp32 numpy rounded to the input dtype, as fp32."""
    import torch
    t = torch.from_numpy(x)
    if dtype == "fp16":
        t = t.half()
    elif dtype == "bf16":
        t = t.bfloat16()
    return t, t.float().numpy()


def _check(got, ref, absref, dtype, d, what, nq=None):
    """fp32 embeddings: the split-product bar. 16-bit embeddings (and PQ, whose table
    path rounds fp32 products): 1e-3 relative and the fp32-accumulation bar for ``nq``
    query tokens."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    inf = np.isinf(ref)
    assert np.array_equal(np.isinf(got), inf), f"{what}: -inf pattern"
    assert np.all(got[inf] == ref[inf]), what
    fin = ~inf
    if dtype == "fp32":
        lim = (4 * 2.0 ** -16 + d * 2.0 ** -24) * np.asarray(absref, np.float64)[fin] + 1e-6
        assert np.all(np.abs(got[fin] - ref[fin]) <= lim), what
    else:
        bar.assert_scores(got, ref, bar.bound(absref, d, nq), what)


def _emb(rng, shape, norm):
    x = rng.standard_normal(shape, dtype=np.float32)
    if norm:
        x /= np.linalg.norm(x, axis=-1, keepdims=True) + 1e-12
    return x


@pytest.mark.parametrize("path", ["small_batch", "streaming"])
@pytest.mark.parametrize("seed", range(N_SEEDS))
def test_random_case(cuda, seed, path):
    """Each case with the small-batch kernel taking every call it can, and with it off."""
    from tilemaxsim_amd import _lib
    with _lib.rerank_limit(1 << 40 if path == "small_batch" else 0):
        _random_case(seed)


def _random_case(seed):
    import torch
    import tilemaxsim_amd as tms
    c, rng = _case(seed)
    nq, B, nd, d, dt, entry = c["nq"], c["B"], c["nd"], c["d"], c["dtype"], c["entry"]
    what = f"seed={seed} {c}"
    print(what, flush=True)
    dev = torch.device("cuda")
    Q_t, Q = _round(_emb(rng, (nq, d), c["norm"]), dt)
    if entry in ("dense", "batched_dense", "masked"):
        D_t, D = _round(_emb(rng, (B, nd, d), c["norm"]), dt)
        if entry == "dense":
            got = tms.flash_maxsim_v2_multiquery(Q_t.to(dev), D_t.to(dev)).cpu().numpy()
            _check(got, orc.maxsim_f64(Q, D), orc.maxsim_f64(np.abs(Q), np.abs(D)), dt, d, what, nq)
        elif entry == "masked":
            mask = rng.random((B, nd)) < 0.7
            mask[0] = False  # a fully masked document scores -inf
            got = tms.maxsim_score(Q_t.to(dev), D_t.to(dev), torch.from_numpy(mask).to(dev)).cpu().numpy()
            _check(got, orc.maxsim_masked(Q, D, mask, f64=True),
                   orc.maxsim_masked(np.abs(Q), np.abs(D), mask, f64=True), dt, d, what, nq)
        else:
            Qs_t, Qs = _round(_emb(rng, (c["nQ"], nq, d), c["norm"]), dt)
            got = tms.flash_maxsim_batched_queries(Qs_t.to(dev), D_t.to(dev)).cpu().numpy()
            for q in range(c["nQ"]):
                _check(got[q], orc.maxsim_f64(Qs[q], D), orc.maxsim_f64(np.abs(Qs[q]), np.abs(D)), dt, d,
                       f"{what} q={q}", nq)
        return
    lens = rng.integers(0, nd + 1, B)
    lens[rng.random(B) < 0.1] = 0
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(offsets[-1])
    Df_t, Df = _round(_emb(rng, (max(T, 1), d), c["norm"]), dt)
    off_t = torch.from_numpy(offsets).to(dev)
    if entry == "varlen":
        got = tms.flash_maxsim_multi_doc(Q_t.to(dev), Df_t.to(dev), off_t).cpu().numpy()
        _check(got, orc.maxsim_varlen(Q, Df, offsets, f64=True),
               orc.maxsim_varlen(np.abs(Q), np.abs(Df), offsets, f64=True), dt, d, what, nq)
    elif entry == "batched_varlen":
        Qs_t, Qs = _round(_emb(rng, (c["nQ"], nq, d), c["norm"]), dt)
        got = tms.flash_maxsim_multi_doc_batched(Qs_t.to(dev), Df_t.to(dev), off_t).cpu().numpy()
        for q in range(c["nQ"]):
            _check(got[q], orc.maxsim_varlen(Qs[q], Df, offsets, f64=True),
                   orc.maxsim_varlen(np.abs(Qs[q]), np.abs(Df), offsets, f64=True), dt, d, f"{what} q={q}", nq)
    else:  # PLAID packed, zero padding: scores the fp16 copies, as the reference does
        Qh = torch.from_numpy(Q).half()
        Dh = torch.from_numpy(Df).half()
        got = tms.flashmaxsim_score_packed(Q_t.to(dev), Df_t.to(dev), torch.from_numpy(lens).to(dev)).cpu().numpy()
        Qx, Dx = Qh.float().numpy(), Dh.float().numpy()[:T]
        ref = orc.maxsim_packed_zero_padded(Qx, Dx, lens)
        _check(got, ref, orc.maxsim_packed_zero_padded(np.abs(Qx), np.abs(Dx), lens), "fp16", d, what, nq)


@pytest.mark.parametrize("seed", range(N_SEEDS * 3 // 8))
def test_random_split_query_case(cuda, seed):
    """fp32 queries against fp16 / bf16 documents (never rounded: split into two terms of
    the documents' type), one and several queries, fixed-length and variable-length
    documents; the fp32 bar against the float64 oracle on the unrounded queries."""
    import torch
    import tilemaxsim_amd as tms
    rng = np.random.default_rng(50_000 + seed)
    nq = int(rng.choice([1, 5, 16, 32, 33, 64, 70]))
    B, nd = int(rng.integers(1, 200)), int(rng.choice([1, 7, 33, 64, 128]))
    d = int(rng.choice([32, 64, 96, 128, 40, 136, 256]))
    ddt = str(rng.choice(["fp16", "bf16"]))
    nQ = int(rng.integers(1, 7))
    norm = bool(rng.integers(0, 2))
    what = f"seed={seed} nq={nq} B={B} nd={nd} d={d} {ddt} nQ={nQ} norm={norm}"
    print(what, flush=True)
    dev = torch.device("cuda")
    Qs = _emb(rng, (nQ, nq, d), norm) * np.float32(rng.choice([1.0, 3e3, 1e-3]))
    if seed % 2 == 0:
        D_t, D = _round(_emb(rng, (B, nd, d), norm), ddt)
        got = tms.flash_maxsim_batched_queries(torch.from_numpy(Qs).to(dev), D_t.to(dev)).cpu().numpy()
        refs = [(orc.maxsim_f64(Qs[q], D), orc.maxsim_f64(np.abs(Qs[q]), np.abs(D))) for q in range(nQ)]
    else:
        lens = rng.integers(0, nd + 1, B)
        offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        Df_t, Df = _round(_emb(rng, (max(int(offsets[-1]), 1), d), norm), ddt)
        got = tms.flash_maxsim_multi_doc_batched(torch.from_numpy(Qs).to(dev), Df_t.to(dev),
                                                 torch.from_numpy(offsets).to(dev)).cpu().numpy()
        refs = [(orc.maxsim_varlen(Qs[q], Df, offsets, f64=True),
                 orc.maxsim_varlen(np.abs(Qs[q]), np.abs(Df), offsets, f64=True)) for q in range(nQ)]
    for q in range(nQ):
        _check(got[q], refs[q][0], refs[q][1], "fp32", d, f"{what} q={q}")


PQ_SHAPES = [  # (M, K, dsub)
    (16, 256, 8), (32, 256, 4), (8, 256, 16), (4, 256, 32), (64, 256, 2), (16, 100, 8), (16, 17, 8),
    (12, 256, 8), (6, 64, 5), (24, 256, 4), (16, 1, 8), (3, 256, 7),
]


@pytest.mark.parametrize("seed", range(N_SEEDS * 9 // 40))
def test_random_pq_case(cuda, seed):
    """PQ: shapes that take the MFMA kernel and shapes that take the table path, every
    codebook dtype, both methods where the shape allows, against decompress-then-score
    in float64 (``src/flash_pqsim_kernel.py:283-313``)."""
    import torch
    from tilemaxsim_amd import TileMaxSimPQ
    rng = np.random.default_rng(10_000 + seed)
    M, K, dsub = PQ_SHAPES[seed % len(PQ_SHAPES)]
    dt = str(rng.choice(["fp16", "bf16", "fp32"]))
    nq = int(rng.choice([1, 8, 32, 33, 64]))
    B, Nd = int(rng.integers(1, 200)), int(rng.choice([0, 1, 9, 64, 128]))
    C_t, C = _round(rng.standard_normal((M, K, dsub), dtype=np.float32), dt)
    Q_t, Q = _round(_emb(rng, (nq, M * dsub), True), dt)
    codes = rng.integers(0, K, (B, Nd, M)).astype(np.uint8)
    what = f"seed={seed} M={M} K={K} dsub={dsub} {dt} nq={nq} B={B} Nd={Nd}"
    print(what, flush=True)
    dev = torch.device("cuda")
    pq = TileMaxSimPQ(C_t.to(dev))
    ref = orc.pq_decompress_score(Q, C, codes, f64=True)
    absref = orc.pq_decompress_score(np.abs(Q), np.abs(C), codes, f64=True)
    for method in ("auto", "lut"):
        got = pq.score_batch(Q_t.to(dev), torch.from_numpy(codes).to(dev), method=method).cpu().numpy()
        # the table path rounds each fp32 product and table entry and sums M entries per
        # token: within the same (d + Nq) operations' bar as the MFMA path
        _check(got, ref, absref, "pq", M * dsub, f"{what} {method}", nq)
