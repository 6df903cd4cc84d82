"""GPU parity of the small-batch kernel (``rerank_maxsim_kernel``, ``csrc/tms_rerank.hip``).

Calls whose documents span few tiles split each document over 1, 2 or 4 waves of a
workgroup. Every case here runs the same inputs twice through the public entry points:
once with the small-batch kernel forced on (``tms_set_rerank_limit`` above the call's
tiles) and once forced off (limit 0: the streaming kernels). Both must give the same
bits (the kernels form the same per-tile MFMA sums, maxima are exact, and both sum
over query tokens in the same order), and both must match the float64 oracle within
1e-3 relative (+1e-3 absolute) and within the fp32-accumulation bar of ``accum_bar.py``,
with -inf and NaN exactly where the oracle has them.
"""
import numpy as np
import pytest

import accum_bar as bar
from oracle import maxsim_oracle as orc

pytestmark = pytest.mark.gpu

HUGE = 1 << 40


def _emb(rng, shape, norm=True):
    x = rng.standard_normal(shape, dtype=np.float32)
    if norm:
        x /= np.linalg.norm(x, axis=-1, keepdims=True) + 1e-12
    return x


def _rounded(x, dt):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x)).to(torch.float16 if dt == "fp16" else torch.bfloat16)
    return t, t.float().numpy()


def _both(fn):
    """fn() under the small-batch kernel and under the streaming kernels; same bits."""
    from tilemaxsim_amd import _lib
    with _lib.rerank_limit(HUGE):
        small = fn().cpu().numpy()
    with _lib.rerank_limit(0):
        stream = fn().cpu().numpy()
    assert small.dtype == np.float32 and small.shape == stream.shape
    assert np.array_equal(small.view(np.uint32), stream.view(np.uint32)), \
        f"paths differ: max |diff| {np.nanmax(np.abs(small.astype(np.float64) - stream))}"
    return small


def _check(got, ref, what, lim=None):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, what
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan), f"{what}: NaN pattern"
    keep = ~nan
    bar.assert_scores(got[keep], ref[keep], None if lim is None else np.broadcast_to(lim, ref.shape)[keep], what)


def _oracle(fn, Q, X, *rest, **kw):
    """(float64 oracle scores, their fp32-accumulation bar)."""
    return bar.with_bound(fn, Q, X, *rest, **kw)


# (nq, nd, d, B): nd sets the waves per document (1-3 tiles: 1 wave; 4-7: 2; >= 8: 4), B
# leaves the last workgroup partly empty; nq = 70 and 96 take a two-block launch and a
# one-block launch that adds onto it
FIXED = [
    (32, 16, 128, 1), (32, 16, 128, 6), (32, 33, 64, 7), (32, 64, 128, 5), (32, 100, 96, 3),
    (32, 128, 128, 1), (32, 128, 128, 1000), (32, 180, 128, 257), (1, 1, 32, 9), (33, 181, 128, 11),
    (64, 128, 128, 17), (70, 90, 64, 13), (96, 300, 32, 4), (5, 7, 96, 21), (32, 0, 128, 5),
]


@pytest.mark.parametrize("dt", ["fp16", "bf16"])
@pytest.mark.parametrize("nq,nd,d,B", FIXED)
def test_fixed(cuda, nq, nd, d, B, dt):
    import tilemaxsim_amd as tms
    rng = np.random.default_rng(nq * 1000 + nd * 7 + d + B)
    Qt, Q = _rounded(_emb(rng, (nq, d)), dt)
    Dt, D = _rounded(_emb(rng, (B, nd, d)), dt)
    Qg, Dg = Qt.cuda(), Dt.cuda()
    got = _both(lambda: tms.flash_maxsim_v2_multiquery(Qg, Dg))
    ref, lim = _oracle(orc.maxsim_f64, Q, D)
    _check(got, ref, f"fixed nq={nq} nd={nd} d={d} B={B} {dt}", lim)


@pytest.mark.parametrize("nq,nd,d,B,mdt,shift", [
    (32, 180, 128, 256, "bool", 0),   # word loads of the mask
    (32, 181, 128, 37, "bool", 0),    # nd % 4 != 0: byte loads
    (32, 128, 64, 50, "uint8", 1),    # a mask that starts 1 byte into its storage: byte loads
    (20, 64, 96, 9, "int32", 0),      # converted to bytes by the wrapper
    (64, 40, 32, 30, "int8", 0),
    (70, 16, 128, 5, "bool", 0),
])
def test_masked(cuda, nq, nd, d, B, mdt, shift):
    import torch
    import tilemaxsim_amd as tms
    rng = np.random.default_rng(nq + nd + d + B + shift)
    Qt, Q = _rounded(_emb(rng, (nq, d)), "fp16")
    Dt, D = _rounded(_emb(rng, (B, nd, d)), "fp16")
    mask = rng.random((B, nd)) < 0.6
    mask[0] = False                    # fully masked: -inf
    if B > 1:
        mask[1] = False
        mask[1, -1] = True             # only the last token counts
    if B > 2:
        mask[2] = True
    tdt = {"bool": torch.bool, "uint8": torch.uint8, "int32": torch.int32, "int8": torch.int8}[mdt]
    m = torch.from_numpy(mask).to(tdt)
    if shift:
        buf = torch.zeros(B * nd + shift, dtype=tdt)
        buf[shift:] = m.reshape(-1)
        mg = buf.cuda()[shift:].view(B, nd)
        assert mg.data_ptr() % 4 != 0
    else:
        mg = m.cuda()
    Qg, Dg = Qt.cuda(), Dt.cuda()
    got = _both(lambda: tms.maxsim_score(Qg, Dg, mg))
    ref, lim = _oracle(orc.maxsim_masked, Q, D, mask, f64=True)
    _check(got, ref, f"masked nq={nq} nd={nd} d={d} B={B} {mdt}", lim)


@pytest.mark.parametrize("nq,d,B,maxlen", [(32, 128, 300, 300), (32, 64, 41, 20), (70, 128, 23, 200),
                                           (16, 96, 100, 60), (32, 32, 5, 700)])
def test_varlen(cuda, nq, d, B, maxlen):
    import torch
    import tilemaxsim_amd as tms
    rng = np.random.default_rng(nq + d + B + maxlen)
    lens = rng.integers(0, maxlen + 1, B)
    lens[rng.random(B) < 0.15] = 0
    lens[-1] = 0
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(offsets[-1])
    Qt, Q = _rounded(_emb(rng, (nq, d)), "bf16")
    Dt, D = _rounded(_emb(rng, (max(T, 1), d)), "bf16")
    Qg, Dg, og = Qt.cuda(), Dt.cuda(), torch.from_numpy(offsets).cuda()
    got = _both(lambda: tms.flash_maxsim_multi_doc(Qg, Dg, og))
    ref, lim = _oracle(orc.maxsim_varlen, Q, D, offsets, f64=True)
    _check(got, ref, f"varlen nq={nq} d={d} B={B}", lim)
    # PLAID's zero-padding semantics: documents shorter than the longest score max(., 0)
    Ql = torch.from_numpy(Q).half()
    Dl = torch.from_numpy(D).half()
    lg = torch.from_numpy(lens).cuda()
    got = _both(lambda: tms.flashmaxsim_score_packed(Ql.cuda(), Dl.cuda(), lg))
    ref, lim = _oracle(orc.maxsim_packed_zero_padded, Ql.float().numpy(), Dl.float().numpy()[:T], lens)
    _check(got, ref, f"packed zeros nq={nq} d={d} B={B}", lim)


def test_varlen_invalid_offsets_score_nan(cuda):
    import torch
    import tilemaxsim_amd as tms
    rng = np.random.default_rng(5)
    Q = torch.from_numpy(_emb(rng, (32, 128))).half().cuda()
    D = torch.from_numpy(_emb(rng, (100, 128))).half().cuda()
    offs = [0, 30, 20, 60, 60, 101, 70, 100, 100]
    og = torch.tensor(offs, dtype=torch.int64).cuda()
    got = _both(lambda: tms.flash_maxsim_multi_doc(Q, D, og, validate=False))
    # documents 1 and 5 end before they start, 4 ends past T = 100; 3 and 7 are empty
    assert np.isnan(got[[1, 4, 5]]).all()
    assert np.isneginf(got[[3, 7]]).all()
    Qn, Dn = Q.float().cpu().numpy(), D.float().cpu().numpy()
    for b in (0, 2, 6):
        ref, lim = _oracle(orc.maxsim_f64, Qn, Dn[offs[b]:offs[b + 1]][None])
        _check(got[b:b + 1], ref, f"valid document {b} beside invalid ones", lim)


@pytest.mark.parametrize("nQ,nq", [(2, 32), (3, 32), (1, 96), (1, 40)])
def test_batched_entry_points_with_few_blocks(cuda, nQ, nq):
    """Two or three 32-token query blocks in all: the batched entry points take the
    small-batch kernel (two blocks per launch, a query split over launches adds up)."""
    import torch
    import tilemaxsim_amd as tms
    rng = np.random.default_rng(nQ * 100 + nq)
    Qt, Q = _rounded(_emb(rng, (nQ, nq, 128)), "fp16")
    Dt, D = _rounded(_emb(rng, (120, 150, 128)), "fp16")
    Qg, Dg = Qt.cuda(), Dt.cuda()
    got = _both(lambda: tms.flash_maxsim_batched_queries(Qg, Dg))
    refs = [_oracle(orc.maxsim_f64, Q[q], D) for q in range(nQ)]
    for q in range(nQ):
        _check(got[q], refs[q][0], f"dense batched q={q}", refs[q][1])
    offs = torch.arange(0, 121 * 150, 150, dtype=torch.int64).cuda()
    got = _both(lambda: tms.flash_maxsim_multi_doc_batched(Qg, Dg.view(-1, 128), offs))
    for q in range(nQ):
        _check(got[q], refs[q][0], f"varlen batched q={q}", refs[q][1])


def test_default_limit_takes_the_small_kernel_for_c1_and_not_for_large_calls(cuda):
    """At the default limit the C1 shape (1,000 documents x 128 tokens = 8,000 tiles) takes
    the small-batch kernel and a 1.3M-token call does not; either way the bits are those
    of both forced paths."""
    import torch
    import tilemaxsim_amd as tms
    from tilemaxsim_amd import _lib
    assert _lib.load().tms_set_rerank_limit(-1) == 16384
    g = torch.Generator(device="cuda").manual_seed(1)
    Q = torch.nn.functional.normalize(torch.randn(32, 128, device="cuda", generator=g), dim=-1).half()
    for B, nd in [(1000, 128), (8000, 160)]:
        D = torch.nn.functional.normalize(torch.randn(B, nd, 128, device="cuda", generator=g), dim=-1).half()
        default = tms.flash_maxsim_v2_multiquery(Q, D).cpu().numpy()
        forced = _both(lambda: tms.flash_maxsim_v2_multiquery(Q, D))
        assert np.array_equal(default.view(np.uint32), forced.view(np.uint32))
