"""GPU parity of the one-launch score + top-k path (``tms_maxsim_topk``: ``rerank_topk_kernel``
in ``csrc/tms_rerank.hip``), the reranking step of the reference's pipeline
(``src/cycle3_experiments.py:215``: score, then ``torch.topk``) for one query against at
most 1,024 documents.

Its scores, values and indices must be the bits of the two-call path
(``flash_maxsim_v2_multiquery`` then ``topk``): the same per-tile MFMA sums, the same
summation order over query tokens and the same selection code. The scores are also held
to the float64 oracle (1e-3 relative + 1e-3 absolute, and the fp32-accumulation bar of
``accum_bar.py``) and the selection to the oracle's top-k (value descending, ties by
lower index), bit for bit. Outputs start as sentinels (NaN values, index -1), so a
result the last workgroup failed to write cannot pass.
"""
import numpy as np
import pytest

import accum_bar as bar
from oracle import maxsim_oracle as orc

pytestmark = pytest.mark.gpu


def _emb(rng, shape):
    x = rng.standard_normal(shape, dtype=np.float32)
    return x / (np.linalg.norm(x, axis=-1, keepdims=True) + 1e-12)


def _rounded(x, dt):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x)).to(torch.float16 if dt == "fp16" else torch.bfloat16)
    return t, t.float().numpy()


def _fused_c(Qg, Dg, k, counter):
    """tms_maxsim_topk through the C ABI, outputs pre-filled with sentinels."""
    import torch
    from tilemaxsim_amd import _lib
    B, nd, d = Dg.shape
    dev = Dg.device
    scores = torch.full((B,), float("nan"), device=dev)
    vals = torch.full((k,), float("nan"), device=dev)
    idx = torch.full((k,), -1, dtype=torch.int64, device=dev)
    code = _lib.dtype_code(Dg.dtype)
    lib = _lib.load()
    rc = lib.tms_maxsim_topk(Qg.data_ptr(), Qg.shape[0], d, Dg.data_ptr(), B, nd, code, k, scores.data_ptr(),
                             vals.data_ptr(), idx.data_ptr(), counter.data_ptr(), _lib.stream_of(Dg))
    assert rc == 0, lib.tms_last_error().decode()
    return scores, vals, idx


def _same_bits(a, b, what):
    import torch
    assert a.shape == b.shape and a.dtype == b.dtype, what
    if a.dtype == torch.float32:
        a, b = a.view(torch.int32), b.view(torch.int32)
    assert torch.equal(a, b), f"{what}: first difference at {(a != b).nonzero()[:5].flatten().tolist()}"


def _against_two_calls(Qg, Dg, k, fused, Q=None, D=None, what=""):
    import torch
    from tilemaxsim_amd import flash_maxsim_v2_multiquery, topk
    s, v, i = fused
    torch.cuda.synchronize()
    ref_s = flash_maxsim_v2_multiquery(Qg, Dg)
    ref_v, ref_i = topk(ref_s, k)
    _same_bits(s, ref_s, f"{what} scores")
    _same_bits(v, ref_v, f"{what} values")
    _same_bits(i, ref_i, f"{what} indices")
    sn = s.cpu().numpy()
    ev, ei = orc.topk(sn, k)
    assert np.array_equal(i.cpu().numpy(), ei), f"{what}: indices against the oracle's top-k"
    assert np.array_equal(v.cpu().numpy().view(np.uint32), ev.astype(np.float32).view(np.uint32)), what
    if Q is not None:
        bar.assert_scores(sn, *bar.with_bound(orc.maxsim_f64, Q, D), what)


# (nq, nd, d, B, k): B sets the grid (one to 256 workgroups, the last one partly empty),
# nd the waves per document (1-3 tiles: 1 wave; 4-7: 2; >= 8: 4), and the call's waves
# the workgroup size (4 waves up to 1,024 waves, 8 up to 2,048, 16 above; 8 at most at
# d = 128 with two query blocks); nq one or two 32-token query blocks; k from 1 to B
# (the selection's every ordering form up to 1,024, at 256, 512 and 1,024 threads)
CASES = [
    (32, 180, 128, 256, 100), (32, 128, 128, 1000, 100), (32, 128, 128, 1024, 1024), (1, 1, 32, 1, 1),
    (1, 16, 32, 7, 7), (33, 181, 128, 11, 3), (64, 300, 96, 100, 10), (5, 7, 96, 21, 21),
    (32, 64, 64, 513, 257), (40, 33, 128, 999, 1), (32, 0, 128, 5, 3), (64, 16, 64, 1024, 300),
    (17, 100, 32, 300, 64), (32, 1, 128, 1024, 100),
    (32, 128, 128, 1000, 1000),  # 16-wave workgroups, bitonic ordering at 1,024 threads
    (64, 200, 128, 700, 300),    # two query blocks at d = 128: capped at 8 waves (350 workgroups)
    (17, 100, 96, 1024, 1024),   # 8-wave workgroups, bitonic ordering at 512 threads
]


@pytest.mark.parametrize("dt", ["fp16", "bf16"])
@pytest.mark.parametrize("nq,nd,d,B,k", CASES)
def test_fused_matches_two_calls_and_oracle(cuda, nq, nd, d, B, k, dt):
    import torch
    rng = np.random.default_rng(nq * 7919 + nd * 31 + d + B * 3 + k)
    Qt, Q = _rounded(_emb(rng, (nq, d)), dt)
    Dt, D = _rounded(_emb(rng, (B, nd, d)), dt)
    Qg, Dg = Qt.cuda(), Dt.cuda()
    from tilemaxsim_amd import _lib
    counter = torch.zeros(_lib.TMS_MAXSIM_TOPK_COUNTER_WORDS, dtype=torch.int32, device="cuda")
    fused = _fused_c(Qg, Dg, k, counter)
    _against_two_calls(Qg, Dg, k, fused, Q, D, f"nq={nq} nd={nd} d={d} B={B} k={k} {dt}")
    assert int(counter.abs().sum().item()) == 0, "the launch leaves every ticket counter at zero"


def test_tied_scores_rank_by_lower_index(cuda):
    """Duplicated documents score the same bits: ties go to the lower index, as in the
    two-call path."""
    import torch
    rng = np.random.default_rng(3)
    Qt, _ = _rounded(_emb(rng, (32, 128)), "fp16")
    base = _emb(rng, (8, 120, 128))
    D = base[rng.integers(0, 8, 700)]  # 700 documents, 8 distinct
    Dt, _ = _rounded(D, "fp16")
    Qg, Dg = Qt.cuda(), Dt.cuda()
    from tilemaxsim_amd import _lib
    counter = torch.zeros(_lib.TMS_MAXSIM_TOPK_COUNTER_WORDS, dtype=torch.int32, device="cuda")
    for k in (1, 50, 700):
        _against_two_calls(Qg, Dg, k, _fused_c(Qg, Dg, k, counter), what=f"ties k={k}")


def test_public_entry_point_repeated_calls(cuda, monkeypatch):
    """maxsim_topk takes the one launch for eager calls of at most 160K document tokens and
    reuses one counter per stream: a sequence of calls whose grids shrink and grow must
    each give the two-call results (a counter left non-zero would leave a call's top-k
    unwritten), and larger calls take the two kernels."""
    import importlib
    import torch
    import tilemaxsim_amd as tms
    topk_mod = importlib.import_module("tilemaxsim_amd.topk")
    taken = []
    real = topk_mod._one_launch

    def spy(*a):
        r = real(*a)
        taken.append(r is not None)
        return r
    monkeypatch.setattr(topk_mod, "_one_launch", spy)
    g = torch.Generator(device="cuda").manual_seed(9)
    Q = torch.nn.functional.normalize(torch.randn(32, 128, device="cuda", generator=g), dim=-1).half()
    # (B, nd, k, one launch?): 4-, 8- and 16-wave workgroups (256 x 180, 1,024 x 32 with
    # wpd 2, 1,000 x 128), and calls past 163,840 tokens (1,000 x 180, 1,024 x 300)
    seq = [(256, 180, 100, True), (7, 30, 5, True), (1000, 128, 100, True), (1000, 180, 100, False),
           (1024, 32, 1024, True), (512, 32, 512, True), (1, 16, 1, True), (1024, 300, 100, False),
           (300, 64, 100, True), (768, 180, 100, True), (64, 100, 64, True), (256, 180, 100, True)]
    for B, nd, k, one in seq:
        D = torch.nn.functional.normalize(torch.randn(B, nd, 128, device="cuda", generator=g), dim=-1).half()
        v, i = tms.maxsim_topk(Q, D, k)
        assert taken[-1] == one, (B, nd)
        s = tms.flash_maxsim_v2_multiquery(Q, D)
        rv, ri = tms.topk(s, k)
        _same_bits(v, rv, f"B={B} values")
        _same_bits(i, ri, f"B={B} indices")
    from tilemaxsim_amd import _lib
    scratch = [c for (dev, _), c in topk_mod._SCRATCH.items() if dev == 0]
    words = _lib.TMS_MAXSIM_TOPK_COUNTER_WORDS
    assert scratch and all(int(c[:words].abs().sum().item()) == 0 for c in scratch)  # the ticket counters


def test_public_entry_point_falls_back_outside_the_one_launch_shapes(cuda):
    """fp32, more than 64 query tokens, more than 1,024 documents, a query of another
    dtype: scored, then ranked, with the same results as the two calls."""
    import torch
    import tilemaxsim_amd as tms
    g = torch.Generator(device="cuda").manual_seed(4)

    def normed(*shape):
        return torch.nn.functional.normalize(torch.randn(*shape, device="cuda", generator=g), dim=-1)

    for Q, D, k in [(normed(32, 128), normed(100, 40, 128), 10),
                    (normed(70, 128).half(), normed(100, 40, 128).half(), 10),
                    (normed(32, 128).half(), normed(1500, 20, 128).half(), 100),
                    (normed(32, 128), normed(200, 40, 128).half(), 50)]:
        v, i = tms.maxsim_topk(Q, D, k)
        rv, ri = tms.topk(tms.flash_maxsim_v2_multiquery(Q, D), k)
        _same_bits(v, rv, "values")
        _same_bits(i, ri, "indices")


def test_threads_on_their_own_streams(cuda):
    """Four host threads, each on its own stream (default priority), call maxsim_topk 40
    times against their own candidates: each stream has its own counters and scratch
    scores, so every result is the two calls' result."""
    import threading
    import torch
    import tilemaxsim_amd as tms
    g = torch.Generator(device="cuda").manual_seed(21)

    def normed(*shape):
        return torch.nn.functional.normalize(torch.randn(*shape, device="cuda", generator=g), dim=-1).half()

    Q = normed(32, 128)
    work = [(normed(B, nd, 128), k) for B, nd, k in [(256, 180, 100), (1000, 128, 50), (64, 40, 64), (513, 96, 257)]]
    torch.cuda.synchronize()
    results = [None] * len(work)
    errors = []

    def run(t):
        try:
            D, k = work[t]
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                outs = [tms.maxsim_topk(Q, D, k) for _ in range(40)]
            s.synchronize()
            results[t] = outs
        except Exception as e:  # reported below, on the test's thread
            errors.append(e)

    threads = [threading.Thread(target=run, args=(t,)) for t in range(len(work))]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert not errors, errors
    for t, (D, k) in enumerate(work):
        rv, ri = tms.topk(tms.flash_maxsim_v2_multiquery(Q, D), k)
        for v, i in results[t]:
            _same_bits(v, rv, f"thread {t} values")
            _same_bits(i, ri, f"thread {t} indices")
