"""The measurement probes of the C ABI (tms_read_probe, tms_lds_probe, tms_mfma_probe),
which bench.py runs to read the scoring kernels against what the part sustains: each
launch runs to completion, reports a positive time per wave where it reports one, and
leaves in its sink exactly what its loads and products imply. Not part of the scoring
path; no reference counterpart."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_read_probe_sink_is_the_xor_of_each_waves_chunks(cuda):
    """Wave w of the persistent grid reads chunks w, w + nwaves, ... (8 KiB each: lane l
    reads 16 bytes at l * 16 + j * 1024, j < 8) and writes the XOR of its words."""
    import torch
    from tilemaxsim_amd import _lib
    lib = _lib.load()
    chunk = 8192
    nwaves = _lib.TMS_READ_PROBE_SINK_WORDS // 64
    nchunks = 3 * nwaves + 5  # every wave reads three or four chunks
    g = torch.Generator(device="cuda").manual_seed(3)
    buf = torch.randint(0, 2 ** 31 - 1, (nchunks * chunk // 4,), dtype=torch.int32, device="cuda", generator=g)
    sink = torch.zeros(_lib.TMS_READ_PROBE_SINK_WORDS, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    assert lib.tms_read_probe(buf.data_ptr(), nchunks * chunk, sink.data_ptr(), sink.numel(), st) == 0
    torch.cuda.synchronize()
    x = buf.cpu().numpy().view(np.uint32).reshape(nchunks, 8, 64, 4)
    per_chunk = np.bitwise_xor.reduce(np.bitwise_xor.reduce(x, axis=3), axis=1)  # (nchunks, 64)
    padded = np.zeros((4 * nwaves, 64), np.uint32)
    padded[:nchunks] = per_chunk
    want = np.bitwise_xor.reduce(padded.reshape(4, nwaves, 64), axis=0).reshape(-1)
    assert np.array_equal(sink.cpu().numpy().view(np.uint32), want)


@pytest.mark.parametrize("pattern", range(12))
def test_lds_probe_patterns(cuda, pattern):
    """Patterns 0-7, 10 and 11 read each of a lane's 16 offsets 4,096 times and XOR them,
    so every sink word is 0; patterns 8 and 9 sum their MFMA accumulators, finite and the
    same bits on a second launch. Every wave reports a positive s_memtime count."""
    import torch
    from tilemaxsim_amd import _lib
    lib = _lib.load()
    nw = _lib.TMS_LDS_PROBE_WAVES
    st = torch.cuda.current_stream().cuda_stream
    runs = []
    for _ in range(2):
        cycles = torch.zeros(nw, dtype=torch.int64, device="cuda")
        sink = torch.full((nw * 64,), -1, dtype=torch.int32, device="cuda")
        assert lib.tms_lds_probe(pattern, cycles.data_ptr(), nw, sink.data_ptr(), sink.numel(), st) == 0
        torch.cuda.synchronize()
        assert (cycles > 0).all(), pattern
        runs.append(sink.cpu().numpy())
    if pattern < 8 or pattern >= 10:
        assert not runs[0].any(), pattern
    else:
        f = runs[0].view(np.float32)
        assert np.isfinite(f).all() and (f != 0).any(), pattern
        assert np.array_equal(runs[0], runs[1]), pattern


def test_mfma_probe_sums_its_products(cuda):
    """Each thread's sum is 8 accumulators x 20,000 repetitions of its four outputs of the
    16x16x32 product of its wave's operand fragments (A: lane (r, g) holds row r, k
    8g..8g+7; B: lane (c, g) holds column c, k 8g..8g+7; C: lane (c, g) holds rows
    4g..4g+3 of column c), to fp32 accumulation error."""
    import torch
    from tilemaxsim_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(5)
    ops = rng.uniform(-1, 1, (512, 8)).astype(np.float16)
    sink = torch.zeros(_lib.TMS_MFMA_PROBE_SINK_WORDS, dtype=torch.float32, device="cuda")
    flops = ctypes.c_int64(0)
    st = torch.cuda.current_stream().cuda_stream
    ops_g = torch.from_numpy(ops).cuda()
    assert lib.tms_mfma_probe(ops_g.data_ptr(), sink.data_ptr(), sink.numel(), ctypes.addressof(flops), st) == 0
    torch.cuda.synchronize()
    grid, iters = 512, 20_000
    assert flops.value == grid * 4 * iters * 8 * 16 * 16 * 32 * 2
    got = sink.cpu().numpy().reshape(grid, 256)
    assert np.array_equal(got, np.broadcast_to(got[0], got.shape))  # every workgroup reads the same operands
    a = ops[:256].astype(np.float64).reshape(4, 4, 16, 8)  # wave, g, r, 8 k values
    b = ops[256:].astype(np.float64).reshape(4, 4, 16, 8)  # wave, g, c, 8 k values
    for w in range(4):
        A = a[w].transpose(1, 0, 2).reshape(16, 32)  # [r][8g + e]
        B = b[w].transpose(1, 0, 2).reshape(16, 32).T  # [8g + e][c]
        C, Cabs = A @ B, np.abs(A) @ np.abs(B)
        for lane in range(64):
            c, g = lane % 16, lane // 16
            want = 8 * iters * C[4 * g:4 * g + 4, c].sum()
            tol = 8 * iters * Cabs[4 * g:4 * g + 4, c].sum() * 2e-3
            assert abs(got[0, 64 * w + lane] - want) <= tol, (w, lane, got[0, 64 * w + lane], want)
