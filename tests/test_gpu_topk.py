"""GPU top-k (tms_topk) against the oracle's top-k (value descending, ties by lower
index): bit-exact values and indices, which is the bar for index work.
``TMS_RANDOM_SEEDS=N`` (default 160) runs N/4 seeds of the random-row sweep."""
import os

import numpy as np
import pytest

from oracle import maxsim_oracle as orc

pytestmark = pytest.mark.gpu
N_ROW_SEEDS = int(os.environ.get("TMS_RANDOM_SEEDS", "160")) // 4


def _check_row(vals, idx, row, k):
    ev, ei = orc.topk(row, k)
    assert np.array_equal(idx, ei), (idx[:10], ei[:10])
    assert np.array_equal(vals.view(np.uint32), ev.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("n,k", [(1, 1), (100, 100), (4096, 100), (4097, 100), (50_000, 100), (1_000_000, 100),
                                 (1_000_000, 1024), (300_000, 7), (16_777_217, 100)])
def test_topk_matches_oracle(cuda, n, k):
    import torch
    from tilemaxsim_amd import topk
    rng = np.random.default_rng(n + k)
    x = rng.standard_normal(n).astype(np.float32)
    v, i = topk(torch.from_numpy(x).cuda(), k)
    assert v.shape == (k,) and i.dtype == torch.int64
    _check_row(v.cpu().numpy(), i.cpu().numpy(), x, k)


@pytest.mark.parametrize("dist", ["pq_scores", "clustered", "negative", "tiny_spread", "mixed_sign"])
def test_topk_concentrated_values(cuda, dist):
    """Rows whose keys share many leading bits (one query's MaxSim scores do): the
    selection skips the shared digits, which must not change the result. The last chunk
    of each row holds fewer than k keys in some rows, where nothing is skipped."""
    import torch
    from tilemaxsim_amd import topk
    rng = np.random.default_rng(11)
    n = 4096 * 7 + 37
    base = {"pq_scores": 83.0 + 2.0 * rng.standard_normal((3, n)),
            "clustered": 10.0 + 1e-3 * rng.random((3, n)),
            "negative": -50.0 - rng.random((3, n)),
            "tiny_spread": 1.0 + 1e-6 * rng.integers(0, 4, size=(3, n)),  # few distinct values: ties by index
            "mixed_sign": 1e-3 * rng.standard_normal((3, n))}[dist]
    rows = base.astype(np.float32)
    for k in (1, 100, 1024):
        v, i = topk(torch.from_numpy(rows).cuda(), k)
        v, i = v.cpu().numpy(), i.cpu().numpy()
        for r in range(3):
            _check_row(v[r], i[r], rows[r], k)


def test_topk_rows_ties_nan_inf(cuda):
    import torch
    from tilemaxsim_amd import topk
    rng = np.random.default_rng(7)
    rows = np.round(rng.standard_normal((5, 20000)) * 4).astype(np.float32)  # many exact ties
    rows[1, 17] = np.inf
    rows[1, 9000] = -np.inf
    rows[2, :] = -np.inf
    rows[3, 123] = np.nan
    rows[4, :] = 0.0
    v, i = topk(torch.from_numpy(rows).cuda(), 100)
    v, i = v.cpu().numpy(), i.cpu().numpy()
    for r in range(5):
        if r == 3:  # NaN ranks first, then the rest in order
            assert i[r, 0] == 123 and np.isnan(v[r, 0])
            rest = rows[r].copy()
            rest[123] = -np.inf
            ev, ei = orc.topk(rest, 99)
            assert np.array_equal(i[r, 1:], ei)
            continue
        _check_row(v[r], i[r], rows[r], 100)


def test_topk_signed_zeros_and_sign_bit_nan(cuda):
    """Keys are canonicalised: -0.0 ties with +0.0 by index, also at the k-th position,
    and a NaN with its sign bit set ranks above +inf like any NaN; the values keep the
    input's bits."""
    import torch
    from tilemaxsim_amd import topk
    rng = np.random.default_rng(5)
    n, k = 20000, 100
    rows = np.abs(rng.standard_normal((4, n))).astype(np.float32) + 1.0
    # row 0: 60 values above zero, then zeros of both signs straddle the k-th position
    rows[0, :] = -1.0 - np.abs(rng.standard_normal(n)).astype(np.float32)
    rows[0, rng.choice(n, 60, replace=False)] = 5.0
    zpos = rng.choice(np.flatnonzero(rows[0] < 0), 80, replace=False)
    rows[0, zpos] = np.where(np.arange(80) % 2 == 0, np.float32(-0.0), np.float32(0.0))
    # row 1: sign-bit NaN, +NaN and +inf
    neg_nan = np.array([0xFFC00000], dtype=np.uint32).view(np.float32)[0]
    rows[1, 777] = neg_nan
    rows[1, 10] = np.inf
    rows[1, 15000] = np.nan
    # row 2: the same across several chunks (the multi-level path), zeros at the boundary
    rows[2, :] = -3.0
    rows[2, rng.choice(n, 99, replace=False)] = 2.0
    rows[2, 4096 * 3 + 5] = -0.0
    rows[2, 4096 * 1 + 9] = 0.0
    rows[3, 4096 * 2] = -neg_nan  # +NaN with a payload-free bit pattern
    rows[3, 1] = neg_nan
    v, i = topk(torch.from_numpy(rows).cuda(), k)
    v, i = v.cpu().numpy(), i.cpu().numpy()
    for r in range(4):
        _check_row(v[r], i[r], rows[r], k)
    assert i[1, 0] == 777 and i[1, 1] == 15000 and i[1, 2] == 10
    assert v[1].view(np.uint32)[0] == 0xFFC00000  # the input's own NaN bits
    assert i[2, 99] == 4096 * 1 + 9  # +0.0 at index 4105 before -0.0 at 12293


def test_maxsim_topk_end_to_end(cuda):
    import torch
    from tilemaxsim_amd import maxsim_topk
    rng = np.random.default_rng(3)
    Qs = rng.standard_normal((4, 32, 128)).astype(np.float32)
    Qs /= np.linalg.norm(Qs, axis=-1, keepdims=True)
    D = rng.standard_normal((3000, 40, 128)).astype(np.float32)
    D /= np.linalg.norm(D, axis=-1, keepdims=True)
    Qs, D = Qs.astype(np.float16), D.astype(np.float16)
    v, i = maxsim_topk(torch.from_numpy(Qs).cuda(), torch.from_numpy(D).cuda(), 100)
    v1, i1 = maxsim_topk(torch.from_numpy(Qs[2]).cuda(), torch.from_numpy(D).cuda(), 100)
    assert v.shape == (4, 100) and v1.shape == (100,)
    for q in range(4):
        ref = orc.maxsim_f64(Qs[q], D)
        kth = np.sort(ref)[::-1][99]
        diff = set(i[q].cpu().numpy().tolist()) ^ set(orc.topk(ref, 100)[1].tolist())
        for d in diff:  # only swaps among scores within tolerance of the 100th
            assert abs(ref[d] - kth) <= 1e-3 * abs(kth) + 1e-3
    assert np.array_equal(i1.cpu().numpy(), i[2].cpu().numpy())


def test_topk_errors(cuda):
    import torch
    from tilemaxsim_amd import topk
    x = torch.zeros(10, device="cuda")
    with pytest.raises(ValueError):
        topk(x, 11)
    with pytest.raises(TypeError):
        topk(x.double(), 3)
    with pytest.raises(NotImplementedError):
        topk(torch.zeros(5000, device="cuda"), 2000)
    v, i = topk(x, 0)
    assert v.shape == (0,)


@pytest.mark.parametrize("seed", range(N_ROW_SEEDS))
def test_topk_random_rows(cuda, seed):
    """Seeded sweep: row count, row length (around the 4096-key chunk and the 1024-thread
    block), k (up to the row length and the 1024 maximum), and the value pattern (spread,
    concentrated, few distinct values, sprinkled NaN / +-inf / signed zeros)."""
    import torch
    from tilemaxsim_amd import topk
    rng = np.random.default_rng(70_000 + seed)
    rows_n = int(rng.choice([1, 2, 3, 8, 33]))
    n = int(rng.choice([1, 5, 100, 1023, 1024, 1025, 4095, 4096, 4097, 8192, 12289, 65536, 200_001]))
    k = int(min(n, rng.choice([1, 2, 31, 64, 100, 256, 257, 1000, 1024])))
    pattern = seed % 4
    if pattern == 0:
        x = rng.standard_normal((rows_n, n))
    elif pattern == 1:
        x = 40.0 + 1e-4 * rng.random((rows_n, n))
    elif pattern == 2:
        x = rng.integers(-3, 4, (rows_n, n)).astype(np.float64)
    else:
        x = rng.standard_normal((rows_n, n))
        m = rng.random((rows_n, n))
        x[m < 0.002] = np.nan
        x[(m >= 0.002) & (m < 0.004)] = np.inf
        x[(m >= 0.004) & (m < 0.006)] = -np.inf
        x[(m >= 0.006) & (m < 0.02)] = -0.0
        x[(m >= 0.02) & (m < 0.03)] = 0.0
    x = x.astype(np.float32)
    print(f"seed={seed} rows={rows_n} n={n} k={k} pattern={pattern}", flush=True)
    v, i = topk(torch.from_numpy(x).cuda(), k)
    v, i = v.cpu().numpy(), i.cpu().numpy()
    for r in range(rows_n):
        ev, ei = orc.topk(x[r], k)
        assert np.array_equal(i[r], ei), (seed, r)
        got_nan, exp_nan = np.isnan(v[r]), np.isnan(ev)
        assert np.array_equal(got_nan, exp_nan), (seed, r)
        assert np.array_equal(v[r][~got_nan].view(np.uint32), ev[~exp_nan].astype(np.float32).view(np.uint32)), (seed, r)


@pytest.mark.parametrize("n,k", [(n, k) for n in (1, 31, 64, 100, 128, 129, 200, 256, 257, 1000, 1024, 1025, 4096)
                                 for k in (1, 32, 33, 100, 128, 129, 200, 256, 257, 700, 1024) if k <= n])
def test_topk_short_rows_every_ordering_form(cuda, n, k):
    """Rows of at most 256 scores are ranked directly, all n keys, with 8, 4, 2 or 1 lanes
    per key (n <= 32, 64, 128, 256); rows of at most 1,024 scores (and last levels that
    small) run the radix passes over one 1,024-key chunk on four waves; longer
    single-chunk rows run 16 waves. The k selected keys are ordered by rank with 8, 4, 2
    or 1 lanes per key (k <= 32, 64, 128, 256 at four waves) or by a bitonic sort
    (k > 256). Every form against the oracle, bit for bit, on MaxSim-like values, a row
    with many ties, and a row with NaN (either sign bit), +-inf and +-0.0 sprinkled in."""
    import torch
    from tilemaxsim_amd import topk
    rng = np.random.default_rng(n * 7 + k)
    x = (10.0 + 0.5 * rng.standard_normal((3, n))).astype(np.float32)
    x[1] = np.round(x[1], 1)  # many ties, resolved by the lower index
    neg_nan = np.array([0xFFC00000], dtype=np.uint32).view(np.float32)[0]
    specials = np.array([np.nan, neg_nan, np.inf, -np.inf, 0.0, -0.0, -0.0, 0.0], dtype=np.float32)
    pos = rng.permutation(n)[:min(n, 2 * len(specials))]
    x[2, pos] = np.resize(specials, len(pos))
    v, i = topk(torch.from_numpy(x).cuda(), k)
    v, i = v.cpu().numpy(), i.cpu().numpy()
    for r in range(3):
        _check_row(v[r], i[r], x[r], k)


@pytest.mark.parametrize("k", [1, 2, 100, 127, 128, 129])
@pytest.mark.parametrize("spread", [False, True])
def test_topk_prefilter_every_candidate_count(cuda, k, spread):
    """Chunks that pass k keys on (k <= 128) first drop the keys below a bound taken from
    each wave's j-th largest thread maximum (j = ceil(k / 4)) and select among the rest,
    gathered in LDS, when at most 1,024 remain (1 to 4 per thread); with more, the chunk
    keeps its registers. A chunk's element e * 256 + t sits in thread t (wave t // 64),
    slot e. Here the first j threads of every wave hold h high keys each, all other keys
    low, so the candidates number 4j * h (all high keys tie when spread is False: the
    bound then falls on them and the index decides) -- h = 1, 3, 6, 10 give 1, 2, 3 and 4
    candidates per thread at k = 100, and h = 11 and 16 overflow the buffer. Every form
    against the oracle, bit for bit, at the first level and at the level the chunks'
    survivors feed."""
    import torch
    from tilemaxsim_amd import topk
    rng = np.random.default_rng(500 + k + (1000 if spread else 0))
    j = -(-k // 4)
    hs = (1, 3, 6, 10, 11, 16)
    n = 4096 * len(hs) * 2 + 777  # two chunks per h, and a ragged last chunk
    rows = []
    for r in range(2):
        x = rng.random(n).astype(np.float32)  # low keys in [0, 1)
        for c in range(n // 4096):
            h = hs[c % len(hs)]
            blk = np.zeros((16, 256), dtype=np.float32)
            lanes = (np.arange(256) % 64) < j
            hi = 11.0 + (rng.random((h, 256)) * 0.5 if spread else 0.0)
            blk[:h, lanes] = np.broadcast_to(hi, (h, 256))[:, lanes]
            sel = np.zeros((16, 256), dtype=bool)
            sel[:h, lanes] = True
            chunk = x[c * 4096:(c + 1) * 4096].reshape(16, 256)
            chunk[sel] = blk[sel]
        rows.append(x)
    x = np.stack(rows)
    print(f"k={k} spread={spread} n={n}", flush=True)
    v, i = topk(torch.from_numpy(x).cuda(), k)
    v, i = v.cpu().numpy(), i.cpu().numpy()
    for r in range(x.shape[0]):
        _check_row(v[r], i[r], x[r], k)
