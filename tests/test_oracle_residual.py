"""Pins for oracle/residual_oracle.py (the ColBERTv2 residual codec restated, colbert-ai
0.2.22) against facts that do not come from its own formulas: hand-derived bytes of the
bit layout, the codec's table-driven decoder as an independent second route, numpy's
packbits/searchsorted, closed forms of the decompression, brute-force MaxSim, and
planted mistakes that each check must reject."""
import numpy as np
import pytest

from oracle import maxsim_oracle as mo
from oracle import residual_oracle as ro


def _one(nbits, d, dim, bucket):
    b = np.zeros((1, d), dtype=np.uint8)
    b[0, dim] = bucket
    return ro.pack_buckets(b, nbits)[0]


# Expected bytes follow from the format alone: per dimension, bits 0..nbits-1 of the
# bucket (least significant first) enter one bit stream, dimension after dimension,
# and the stream fills each byte from its most significant bit.
@pytest.mark.parametrize("nbits,d,dim,bucket,expect", [
    (1, 8, 0, 1, [0x80]),
    (1, 8, 7, 1, [0x01]),
    (1, 16, 9, 1, [0x00, 0x40]),
    (2, 8, 0, 1, [0x80, 0x00]),        # bit0 of dim 0 is stream bit 0
    (2, 8, 0, 2, [0x40, 0x00]),        # bit1 of dim 0 is stream bit 1
    (2, 8, 1, 3, [0x30, 0x00]),
    (2, 8, 3, 1, [0x02, 0x00]),
    (2, 8, 4, 2, [0x00, 0x40]),
    (4, 8, 0, 1, [0x80, 0, 0, 0]),
    (4, 8, 0, 8, [0x10, 0, 0, 0]),     # bit3 of dim 0 is stream bit 3
    (4, 8, 1, 1, [0x08, 0, 0, 0]),
    (4, 8, 7, 15, [0, 0, 0, 0x0F]),
])
def test_bit_layout_known_answers(nbits, d, dim, bucket, expect):
    packed = _one(nbits, d, dim, bucket)
    assert packed.tolist() == expect
    back = ro.unpack_buckets(packed[None], nbits, d)[0]
    assert back[dim] == bucket and back.sum() == bucket


@pytest.mark.parametrize("nbits", [1, 2, 4])
def test_direct_unpack_matches_the_codecs_table_route(nbits):
    rng = np.random.default_rng(nbits)
    d = 128
    b = rng.integers(0, 1 << nbits, size=(300, d)).astype(np.uint8)
    packed = ro.pack_buckets(b, nbits)
    assert packed.shape == (300, d * nbits // 8)
    assert np.array_equal(ro.unpack_buckets(packed, nbits, d), b)
    assert np.array_equal(ro.unpack_buckets_via_tables(packed, nbits, d), b)
    # every byte value decodes identically both ways
    allbytes = np.arange(256, dtype=np.uint8)[:, None]
    kpb = 8 // nbits
    assert np.array_equal(ro.unpack_buckets(allbytes, nbits, kpb), ro.unpack_buckets_via_tables(allbytes, nbits, kpb))


def test_codec_tables_known_entries():
    rev, lookup = ro.colbert_tables(2)
    assert rev[0b01_00_00_00] == 0b10_00_00_00 and rev[0b00_00_00_10] == 0b00_00_00_01
    assert rev[0b11_01_10_00] == 0b11_10_01_00
    assert lookup.shape == (256, 4) and lookup[0b00_01_10_11].tolist() == [0, 1, 2, 3]
    rev1, lookup1 = ro.colbert_tables(1)
    assert np.array_equal(rev1, np.arange(256)) and lookup1[0x80].tolist() == [1, 0, 0, 0, 0, 0, 0, 0]


def test_bucketize_boundaries_and_codes_brute_force():
    cut = np.array([-0.5, 0.0, 0.5], dtype=np.float32)
    C = np.zeros((3, 8), dtype=np.float16)
    C[0, 0], C[1, 1], C[2, 2] = 1.0, 1.0, 1.0
    E = np.zeros((4, 8), dtype=np.float16)
    E[0, 0] = 1.0            # residual 0 everywhere
    E[1, 1], E[1, 3] = 1.0, 0.5   # residual 0.5 exactly on the top cutoff
    E[2, 2], E[2, 4] = 1.0, 0.75
    E[3, 1], E[3, 5] = 0.9, -0.5
    codes, res = ro.compress(E, C, cut, 2)
    assert codes.tolist() == [0, 1, 2, 1]
    b = ro.unpack_buckets(res, 2, 8)
    # torch.bucketize(right=False): a value equal to a cutoff stays in the lower bucket
    assert b[0].tolist() == [1] * 8
    assert b[1, 3] == 2 and b[2, 4] == 3 and b[3, 5] == 0 and b[3, 1] == 1  # 0.9 - 1.0 = -0.1
    rng = np.random.default_rng(5)
    E = rng.standard_normal((40, 16)).astype(np.float16)
    C = rng.standard_normal((7, 16)).astype(np.float16)
    codes, res = ro.compress(E, C, cut, 2)
    for t in range(40):
        dots = [sum(float(E[t, j]) * float(C[c, j]) for j in range(16)) for c in range(7)]
        assert codes[t] == int(np.argmax(dots))
        r = [float(np.float16(float(E[t, j]) - float(C[codes[t], j]))) for j in range(16)]
        assert ro.unpack_buckets(res[t:t + 1], 2, 16)[0].tolist() == [sum(c < x for c in cut) for x in r]


def test_decompress_closed_forms():
    d = 16
    C = np.zeros((2, d), dtype=np.float16)
    C[0, 0], C[0, 1] = 3.0, 4.0     # norm 5
    zero_w = np.zeros(4, dtype=np.float16)
    res = ro.pack_buckets(np.zeros((1, d), dtype=np.uint8), 2)
    out = ro.decompress(np.array([0], np.int32), res, C, zero_w, 2)[0]
    assert out[0] == np.float16(0.6) and out[1] == np.float16(0.8) and not out[2:].any()
    # a zero centroid plus one weight in every dimension: all entries 1/sqrt(d) = 0.25
    w = np.array([0.1, 0.3, 0.2, -0.4], dtype=np.float16)
    res = ro.pack_buckets(np.full((1, d), 2, dtype=np.uint8), 2)
    out = ro.decompress(np.array([1], np.int32), res, C, w, 2)[0]
    assert np.all(out == np.float16(0.25))
    # the weight is added in half precision before normalising
    C2 = np.full((1, d), 1.0, dtype=np.float16)
    res = ro.pack_buckets(np.full((1, d), 3, dtype=np.uint8), 2)
    v = ro.decompress_unnormalised(np.array([0], np.int32), res, C2, w, 2)[0]
    assert np.all(v == np.float16(1.0) + np.float16(-0.4))


def test_round_trip_recovers_the_embedding():
    rng = np.random.default_rng(8)
    d, T = 128, 500
    C = rng.standard_normal((64, d)).astype(np.float32)
    C /= np.linalg.norm(C, axis=1, keepdims=True)
    E = C[rng.integers(0, 64, T)] + 0.05 * rng.standard_normal((T, d))
    E = (E / np.linalg.norm(E, axis=1, keepdims=True)).astype(np.float16)
    C = C.astype(np.float16)
    r = E.astype(np.float32) - C[ro.compress(E, C, np.zeros(15, np.float32), 4)[0]].astype(np.float32)
    qs = np.quantile(r, np.arange(1, 16) / 16)
    ws = np.quantile(r, np.arange(16) / 16 + 1 / 32)
    codes, res = ro.compress(E, C, qs.astype(np.float32), 4)
    D = ro.decompress(codes, res, C, ws.astype(np.float16), 4).astype(np.float32)
    cos = (D * E.astype(np.float32)).sum(1) / np.linalg.norm(E.astype(np.float32), axis=1)
    assert cos.min() > 0.98
    assert np.allclose(np.linalg.norm(D, axis=1), 1.0, atol=2e-3)


def _brute_scores(Q, D, rows, pad_len):
    out = []
    for se in rows:
        if se is None:
            out.append(np.nan)
            continue
        s, e = se
        total = 0.0
        for q in Q.astype(np.float64):
            vals = [float(np.dot(q, D[t].astype(np.float64))) for t in range(s, e)]
            if pad_len and e - s < pad_len:
                vals.append(0.0)
            total += max(vals) if vals else -np.inf
        out.append(total)
    return np.array(out)


@pytest.mark.parametrize("pad_len", [0, 9])
def test_maxsim_residual_brute_force(pad_len):
    rng = np.random.default_rng(21 + pad_len)
    d, nbits = 32, 2
    C = rng.standard_normal((10, d)).astype(np.float16)
    lens = np.array([3, 0, 9, 1, 5])
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(offsets[-1])
    codes = rng.integers(0, 10, T).astype(np.int32)
    res = ro.pack_buckets(rng.integers(0, 4, (T, d)).astype(np.uint8), nbits)
    w = np.array([-0.3, -0.1, 0.1, 0.3], dtype=np.float16)
    Q = rng.standard_normal((4, d)).astype(np.float16)
    D = ro.decompress(codes, res, C, w, nbits)
    pids = np.array([4, 2, 2, 0, 1, 7, -1, 3])
    got = ro.maxsim_residual(Q, codes, res, C, w, nbits, offsets, pids, pad_len)
    rows = [(int(offsets[p]), int(offsets[p + 1])) if 0 <= p < 5 else None for p in pids]
    exp = _brute_scores(Q, D, rows, pad_len)
    if pad_len:
        exp[[i for i, p in enumerate(pids) if p == 1]] = 0.0
    np.testing.assert_allclose(got, exp, rtol=1e-12)
    assert np.isnan(got[5]) and np.isnan(got[6])
    # all documents, no pids: the plain varlen oracle on the decompressed tokens
    np.testing.assert_allclose(ro.maxsim_residual(Q, codes, res, C, w, nbits, offsets),
                               mo.maxsim_varlen(Q, D, offsets, f64=True), rtol=1e-12)


# ---------------------------------------------------------------- planted mistakes
def test_planted_bit_order_mistakes_are_caught():
    b = np.zeros((1, 8), dtype=np.uint8)
    b[0, 0] = 1
    msb_first_per_dim = np.packbits(((b[..., None] >> np.arange(1, -1, -1)) & 1).reshape(1, 16), axis=-1)
    little_bytes = np.packbits(((b[..., None] >> np.arange(2)) & 1).reshape(1, 16), axis=-1, bitorder="little")
    assert msb_first_per_dim[0].tolist() != [0x80, 0x00]  # the known answer for (2, 8, 0, 1)
    assert little_bytes[0].tolist() != [0x80, 0x00]
    assert ro.pack_buckets(b, 2)[0].tolist() == [0x80, 0x00]


def test_planted_bucketize_right_is_caught():
    cut = np.array([-0.5, 0.0, 0.5], dtype=np.float32)
    x = np.array([0.5], dtype=np.float32)
    assert np.searchsorted(cut, x, side="right")[0] == 3  # right=True would put it above
    C = np.zeros((1, 8), dtype=np.float16)
    E = np.zeros((1, 8), dtype=np.float16)
    E[0, 3] = 0.5
    assert ro.unpack_buckets(ro.compress(E, C, cut, 2)[1], 2, 8)[0, 3] == 2


def test_planted_missing_normalisation_is_caught():
    C = np.zeros((1, 16), dtype=np.float16)
    C[0, 0], C[0, 1] = 3.0, 4.0
    res = ro.pack_buckets(np.zeros((1, 16), dtype=np.uint8), 2)
    raw = ro.decompress_unnormalised(np.array([0], np.int32), res, C, np.zeros(4, np.float16), 2)[0]
    assert raw[0] != np.float16(0.6)  # skipping the normalisation fails the closed form


def _kernel_index(rng, T, d, nbits, ncent):
    C = rng.standard_normal((ncent, d)).astype(np.float32)
    C /= np.linalg.norm(C, axis=1, keepdims=True)
    codes = rng.integers(0, ncent, T).astype(np.int32)
    buckets = rng.integers(0, 1 << nbits, (T, d)).astype(np.uint8)
    w = np.sort(rng.normal(0, 0.05, 1 << nbits)).astype(np.float16)
    return C.astype(np.float16), codes, ro.pack_buckets(buckets, nbits), w


def test_kernel_envelope_closed_forms():
    """One token v = (3, 4, 0, ...) (zero bucket weights): |v| = 5 exactly, so both norms
    are 5 and inv = fp32(1/5). The fused form scores <q, v> * inv; the batched form rounds
    x = fp16(v * inv) first: fp16(0.6000000089) = 0.60009765625, fp16(0.8000000119) =
    0.7998046875."""
    d, nbits = 32, 2
    C = np.zeros((1, d), np.float16)
    C[0, 0], C[0, 1] = 3, 4
    w = np.zeros(4, np.float16)
    codes = np.zeros(1, np.int32)
    res = ro.pack_buckets(np.zeros((1, d), np.uint8), nbits)
    Q = np.zeros((2, d), np.float16)
    Q[0, 0], Q[0, 1] = 0.5, 0.25
    Q[1, 1] = -1.0
    offs = np.array([0, 1], np.int64)
    n_lo, n_hi = ro.norm_candidates(ro.decompress_unnormalised(codes, res, C, w, nbits))
    assert n_lo.tolist() == [5.0] and n_hi.tolist() == [5.0]
    inv = float(np.float32(1) / np.float32(5))
    lo, hi, a = ro.maxsim_residual_kernel_envelope(Q, codes, res, C, w, nbits, offs, form="fused")
    assert lo[0] == hi[0] == 2.5 * inv + (-4.0) * inv
    assert a[0] == 2.5 * inv + 4.0 * inv
    lo, hi, a = ro.maxsim_residual_kernel_envelope(Q, codes, res, C, w, nbits, offs, form="batched")
    x0, x1 = 0.60009765625, 0.7998046875
    assert np.float16(3 * np.float32(inv)) == x0 and np.float16(4 * np.float32(inv)) == x1
    assert lo[0] == hi[0] == (0.5 * x0 + 0.25 * x1) + (-x1)


def test_norm_candidates_cover_every_fp32_summation_order():
    """The norms a kernel forms from fp32 sums of the squares in any order (here: 24
    random orders per token, sequential fp32 sums, fp32 square root, fp16 rounding) are
    always one of the two candidates; where the two differ they are adjacent fp16
    values, and some tokens of a random index do fall on a boundary."""
    rng = np.random.default_rng(41)
    C, codes, res, w = _kernel_index(rng, 6000, 64, 2, 50)
    V = ro.decompress_unnormalised(codes, res, C, w, 2)
    n_lo, n_hi = ro.norm_candidates(V)
    sq = V.astype(np.float32) ** 2
    for _ in range(24):
        perm = rng.permutation(V.shape[1])
        n2 = np.zeros(V.shape[0], np.float32)
        for k in perm:
            n2 = (n2 + sq[:, k]).astype(np.float32)
        n = np.sqrt(n2).astype(np.float16).astype(np.float64)
        assert np.all((n == n_lo) | (n == n_hi))
    two = n_lo != n_hi
    assert 0 < two.sum() < 0.05 * len(two)
    assert np.all(np.nextafter(n_lo[two].astype(np.float16), np.float16(np.inf)).astype(np.float64) == n_hi[two])


@pytest.mark.parametrize("form", ["fused", "batched"])
def test_kernel_envelope_holds_simulated_kernels(form):
    """A float32 simulation of each kernel (norm from an fp32 sum of squares in a random
    order, fp32 dot products, the fused form's fp32 multiply by inv, the batched form's
    fp16 rounding of x) over a random index with ragged and empty documents lies within
    the envelope widened by the fp32-accumulation bar. The codec's decompress-then-score
    differs from the fused form by more than that bar somewhere (the fused kernel never
    rounds v / n to fp16), so its envelope is not the codec's oracle under another name;
    the batched form rounds x as the codec does (by a multiply where the codec divides)."""
    import accum_bar as bar
    rng = np.random.default_rng(7 if form == "fused" else 8)
    d, nbits, nq = 64, 2, 20
    lens = rng.integers(0, 12, 300)
    lens[::17] = 0
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    C, codes, res, w = _kernel_index(rng, int(offs[-1]), d, nbits, 40)
    Q = rng.standard_normal((nq, d)).astype(np.float32)
    Q = (Q / np.linalg.norm(Q, axis=1, keepdims=True)).astype(np.float16)
    lo, hi, absref = ro.maxsim_residual_kernel_envelope(Q, codes, res, C, w, nbits, offs, form=form)
    V = ro.decompress_unnormalised(codes, res, C, w, nbits).astype(np.float32)
    perm = rng.permutation(d)
    n2 = np.zeros(V.shape[0], np.float32)
    for k in perm:
        n2 = (n2 + V[:, k] * V[:, k]).astype(np.float32)
    n = np.maximum(np.sqrt(n2).astype(np.float16).astype(np.float32), np.float32(5.9604645e-8))
    inv = (np.float32(1) / n).astype(np.float32)
    Qf = Q.astype(np.float32)
    if form == "fused":
        P = (V @ Qf.T).astype(np.float32) * inv[:, None]
    else:
        X = (V * inv[:, None]).astype(np.float16).astype(np.float32)
        P = (X @ Qf.T).astype(np.float32)
    sim = np.array([P[s:e].max(axis=0).sum(dtype=np.float32) if e > s else -np.inf
                    for s, e in zip(offs[:-1], offs[1:])])
    b = bar.bound(absref, d, nq)
    fin = np.isfinite(lo)
    assert np.array_equal(np.isinf(sim), ~fin)
    assert np.all(sim[fin] >= lo[fin] - b[fin]) and np.all(sim[fin] <= hi[fin] + b[fin])
    if form == "fused":
        codec = ro.maxsim_residual(Q, codes, res, C, w, nbits, offs)
        assert np.any(np.abs(codec[fin] - sim[fin]) > b[fin])
