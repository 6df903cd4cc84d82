"""tms_topk_noalloc (the allocation-free top-k: intermediate keys in the library's fixed
device scratch array) against tms_topk with a caller workspace, through the C ABI.

Four calls in a row, each smaller than the one before, must each equal tms_topk bit
for bit: the scratch array keeps the previous call's keys, which must not leak into the
next result. The first fills the array to its documented limit (top-100 over (32, 5M)
scores: 32.0 MB of 32 MiB); every call takes at least one intermediate level, so every
call goes through the scratch array. A graph captured after one eager call replays
with the eager result.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _topk_ws(lib, torch, s, k):
    rows, n = s.shape
    ws_bytes = int(lib.tms_topk_workspace_size(rows, n, k))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=s.device)
    v = torch.empty(rows, k, dtype=torch.float32, device=s.device)
    i = torch.empty(rows, k, dtype=torch.int64, device=s.device)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.tms_topk(s.data_ptr(), rows, n, k, ws.data_ptr(), ws_bytes, v.data_ptr(), i.data_ptr(), st) == 0
    return v, i


def _topk_noalloc(lib, torch, s, k):
    rows, n = s.shape
    v = torch.empty(rows, k, dtype=torch.float32, device=s.device)
    i = torch.empty(rows, k, dtype=torch.int64, device=s.device)
    st = torch.cuda.current_stream().cuda_stream
    rc = lib.tms_topk_noalloc(s.data_ptr(), rows, n, k, v.data_ptr(), i.data_ptr(), st)
    assert rc == 0, lib.tms_last_error().decode()
    return v, i


def test_topk_noalloc_matches_workspace_entry(cuda):
    import torch
    from tilemaxsim_amd import _lib
    lib = _lib.load()
    g = torch.Generator(device="cuda").manual_seed(91)
    # (32, 5M): C5's top-100 shape at the array's limit; (64, 1M): C2's, 12.9 MB; then
    # smaller rows and another k, so stale keys of earlier calls sit past what each writes
    cases = [(32, 5_000_000, 100), (64, 1_000_000, 100), (5, 300_000, 37), (2, 50_000, 100)]
    need = [int(lib.tms_topk_workspace_size(r, n, k)) for r, n, k in cases]
    assert need[0] <= (32 << 20) < int(lib.tms_topk_workspace_size(34, 5_000_000, 100))
    assert all(a > b > 0 for a, b in zip(need, need[1:])), need
    for rows, n, k in cases:
        s = torch.randn(rows, n, device="cuda", generator=g)
        print(f"tms_topk_noalloc rows={rows} n={n} k={k}", flush=True)
        v0, i0 = _topk_ws(lib, torch, s, k)
        v1, i1 = _topk_noalloc(lib, torch, s, k)
        torch.cuda.synchronize()
        assert torch.equal(i0, i1)
        assert torch.equal(v0.view(torch.int32), v1.view(torch.int32))
        # and against the oracle on two rows
        from oracle import maxsim_oracle as orc
        sc = s.cpu().numpy()
        for r in (0, rows - 1):
            ev, ei = orc.topk(sc[r], k)
            assert np.array_equal(i1[r].cpu().numpy(), ei)


def test_topk_noalloc_rejects_oversized(cuda):
    from tilemaxsim_amd import _lib
    lib = _lib.load()
    need = int(lib.tms_topk_workspace_size(64, 50_000_000, 100))
    assert need > (32 << 20)
    # refused before any device work: no pointer is dereferenced
    rc = lib.tms_topk_noalloc(ctypes.c_void_p(16), 64, 50_000_000, 100, ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert rc == _lib.TMS_ERR_UNSUPPORTED
    assert b"scratch" in lib.tms_last_error()


def test_topk_noalloc_in_a_captured_graph(cuda):
    """One eager call (which loads the array and looks up its address on this device),
    then the call captured into a graph: every replay, with new scores and eager work and
    synchronisations between replays, equals tms_topk on the same scores."""
    import torch
    from tilemaxsim_amd import _lib
    lib = _lib.load()
    g = torch.Generator(device="cuda").manual_seed(17)
    rows, n, k = 8, 300_000, 100
    s = torch.randn(rows, n, device="cuda", generator=g)
    _topk_noalloc(lib, torch, s, k)  # the eager first call on this device
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        v, i = _topk_noalloc(lib, torch, s, k)
    for rep in range(4):
        s.copy_(torch.randn(rows, n, device="cuda", generator=g))
        graph.replay()
        torch.cuda.synchronize()
        ev, ei = _topk_ws(lib, torch, s, k)  # eager work between replays
        torch.cuda.synchronize()
        print(f"graph replay {rep}", flush=True)
        assert torch.equal(i, ei), rep
        assert torch.equal(v.view(torch.int32), ev.view(torch.int32)), rep
