"""The entry points under HIP graph capture (torch.cuda.CUDAGraph): a serving loop can
capture scoring + top-k once and replay it for each new query.

Every kernel of the path is an ordinary launch on the current stream with no memset
and no host synchronisation, so capture records it as is. Each test replays the graph
several times, with new query values copied into the captured input and eager work and
synchronisations between the replays, and checks every replay against the eager call
on the same inputs, bit for bit (the same kernels run on the same bytes).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _normed(g, shape):
    import torch
    x = torch.randn(*shape, generator=g, device="cuda")
    return torch.nn.functional.normalize(x, dim=-1).half()


def _capture(fn):
    """Warm up on a side stream (as torch requires before capture), then capture fn()."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def _replay_and_check(g, out, Q_static, new_queries, eager):
    import torch
    for i, q in enumerate(new_queries):
        Q_static.copy_(q)
        g.replay()
        torch.cuda.synchronize()
        ref = eager(q)
        for got, exp in zip(out, ref):
            assert torch.equal(got, exp), f"replay {i}"
        _ = (q.float() * 2).sum().item()  # eager work and a host sync between replays


def test_graph_dense_score_and_topk(cuda):
    import torch
    from tilemaxsim_amd import flash_maxsim_v2_multiquery, topk
    g0 = torch.Generator(device="cuda").manual_seed(0)
    D = _normed(g0, (3000, 128, 128))
    Q = _normed(g0, (32, 128))

    def step(q):
        s = flash_maxsim_v2_multiquery(q, D)
        v, i = topk(s, 100)
        return s, v, i

    graph, out = _capture(lambda: step(Q))
    _replay_and_check(graph, out, Q, [_normed(g0, (32, 128)) for _ in range(4)], step)


def test_graph_one_launch_score_and_topk(cuda):
    """tms_maxsim_topk (score + top-k in one launch) captured through the C ABI: the graph
    holds its own ticket counter, zeroed by a fill kernel at the start of every replay;
    every replay matches scoring, then ranking, eagerly. (maxsim_topk itself takes the two
    kernels under capture, where one launch is no faster.)"""
    import torch
    from tilemaxsim_amd import _lib, flash_maxsim_v2_multiquery, topk
    g0 = torch.Generator(device="cuda").manual_seed(5)
    D = _normed(g0, (256, 180, 128))
    Q = _normed(g0, (32, 128))
    lib = _lib.load()

    def step(q):
        scores = torch.empty(256, device="cuda")
        vals = torch.empty(100, device="cuda")
        idx = torch.empty(100, dtype=torch.int64, device="cuda")
        counter = torch.zeros(_lib.TMS_MAXSIM_TOPK_COUNTER_WORDS, dtype=torch.int32, device="cuda")
        rc = lib.tms_maxsim_topk(q.data_ptr(), 32, 128, D.data_ptr(), 256, 180, _lib.TMS_DTYPE_F16, 100,
                                 scores.data_ptr(), vals.data_ptr(), idx.data_ptr(), counter.data_ptr(),
                                 _lib.stream_of(D))
        assert rc == 0, lib.tms_last_error().decode()
        return scores, vals, idx

    def eager(q):
        s = flash_maxsim_v2_multiquery(q, D)
        return (s, *topk(s, 100))

    graph, out = _capture(lambda: step(Q))
    _replay_and_check(graph, out, Q, [_normed(g0, (32, 128)) for _ in range(4)], eager)


def test_graph_varlen_and_batched(cuda):
    import torch
    from tilemaxsim_amd import flash_maxsim_multi_doc, flash_maxsim_multi_doc_batched, topk
    g0 = torch.Generator(device="cuda").manual_seed(1)
    rng = np.random.default_rng(1)
    lens = rng.integers(0, 200, 2000)
    offsets = torch.from_numpy(np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)).cuda()
    D = _normed(g0, (int(lens.sum()), 128))
    Qs = _normed(g0, (6, 32, 128))

    def step(qs):  # validate=False: the offsets check is a device-to-host copy, not capturable
        one = flash_maxsim_multi_doc(qs[0], D, offsets, validate=False)
        many = flash_maxsim_multi_doc_batched(qs, D, offsets, validate=False)
        v, i = topk(many, 50)
        return one, many, v, i

    graph, out = _capture(lambda: step(Qs))
    _replay_and_check(graph, out, Qs, [_normed(g0, (6, 32, 128)) for _ in range(3)], step)


def test_graph_pq(cuda):
    import torch
    from tilemaxsim_amd import TileMaxSimPQ, topk
    g0 = torch.Generator(device="cuda").manual_seed(2)
    C = torch.randn(16, 256, 8, generator=g0, device="cuda").half()
    codes = torch.randint(0, 256, (4000, 64, 16), dtype=torch.uint8, generator=g0, device="cuda")
    pq = TileMaxSimPQ(C)
    Q = _normed(g0, (32, 128))

    def step(q):  # validate=False: uint8 codes with K = 256 need no check
        a = pq.score_batch(q, codes, validate=False)
        b = pq.score_batch(q, codes, method="lut", validate=False)
        v, i = topk(a, 100)
        return a, b, v, i

    graph, out = _capture(lambda: step(Q))
    _replay_and_check(graph, out, Q, [_normed(g0, (32, 128)) for _ in range(3)], step)
