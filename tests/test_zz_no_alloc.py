"""tms_topk_noalloc (the allocation-free top-k: intermediate keys in the library's fixed
device scratch array) against tms_topk with a caller workspace, through the C ABI.

Three calls in a row, each smaller than the one before, must each equal tms_topk bit
for bit: the scratch array keeps the previous call's keys, which must not leak into the
next result.
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
    # first call: C2's top-100 shape, (64, 1M) scores, 12.9 MB of scratch; second: smaller
    # rows and a different k, so stale keys of the first call sit past what it writes
    for rows, n, k in [(64, 1_000_000, 100), (5, 300_000, 37), (3, 4096, 100)]:
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
