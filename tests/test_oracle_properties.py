"""Property-based pins for the oracle (hypothesis draws the shapes, lengths, seeds and
value patterns; every check compares against a route that does not share the oracle's
code: pure-Python loops, sorting, or a mathematical identity).

* dense MaxSim == float64 brute force; invariant under permuting and duplicating
  document tokens, zero-padding d, and positive scaling of Q;
* variable-length MaxSim == the per-document slices (empty documents -inf);
* PQ table gather == decompress-then-score;
* top-k == a stable sort on (NaN first, value descending, index ascending), with -0.0
  and +0.0 tied;
* residual bucket packing round-trips, and the codec's table route decodes alike.
"""
import math

import numpy as np
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from oracle import maxsim_oracle as orc
from oracle import residual_oracle as ro

SETTINGS = settings(max_examples=150, deadline=None, suppress_health_check=[HealthCheck.too_slow])


def _brute(Q, D):
    """sum_i max_j <Q_i, D_b,j> with Python floats, one document at a time."""
    out = []
    for doc in D:
        s = 0.0
        for q in Q:
            s += max(math.fsum(float(a) * float(b) for a, b in zip(q, t)) for t in doc)
        out.append(s)
    return np.array(out)


@SETTINGS
@given(nq=st.integers(1, 5), nd=st.integers(1, 6), d=st.integers(1, 9), b=st.integers(1, 4),
       seed=st.integers(0, 2**31 - 1))
def test_dense_is_brute_force(nq, nd, d, b, seed):
    rng = np.random.default_rng(seed)
    Q = rng.standard_normal((nq, d)).astype(np.float16)
    D = rng.standard_normal((b, nd, d)).astype(np.float16)
    np.testing.assert_allclose(orc.maxsim_f64(Q, D), _brute(Q, D), rtol=1e-12, atol=1e-12)


@SETTINGS
@given(nq=st.integers(1, 6), nd=st.integers(1, 12), d=st.integers(1, 16), b=st.integers(1, 5),
       pad=st.integers(1, 7), scale=st.floats(0.125, 8.0), seed=st.integers(0, 2**31 - 1))
def test_dense_invariants(nq, nd, d, b, pad, scale, seed):
    rng = np.random.default_rng(seed)
    Q = rng.standard_normal((nq, d))
    D = rng.standard_normal((b, nd, d))
    ref = orc.maxsim_f64(Q, D)
    perm = rng.permutation(nd)
    np.testing.assert_allclose(orc.maxsim_f64(Q, D[:, perm]), ref, rtol=1e-12, atol=1e-12)
    dup = np.concatenate([D, D[:, : max(1, nd // 2)]], axis=1)
    np.testing.assert_allclose(orc.maxsim_f64(Q, dup), ref, rtol=1e-12, atol=1e-12)
    Qp = np.concatenate([Q, np.zeros((nq, pad))], axis=1)
    Dp = np.concatenate([D, rng.standard_normal((b, nd, pad))], axis=2)  # padded query dims meet anything
    np.testing.assert_allclose(orc.maxsim_f64(Qp, Dp), ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(orc.maxsim_f64(Q * scale, D), ref * scale, rtol=1e-12, atol=1e-12)


@SETTINGS
@given(lens=st.lists(st.integers(0, 7), min_size=1, max_size=8), nq=st.integers(1, 4), d=st.integers(1, 8),
       seed=st.integers(0, 2**31 - 1))
def test_varlen_is_per_document_slices(lens, nq, d, seed):
    rng = np.random.default_rng(seed)
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    Q = rng.standard_normal((nq, d)).astype(np.float16)
    flat = rng.standard_normal((int(offs[-1]), d)).astype(np.float16)
    got = orc.maxsim_varlen(Q, flat, offs, f64=True)
    for i, n in enumerate(lens):
        if n == 0:
            assert got[i] == -np.inf
        else:
            ref = _brute(Q, flat[None, offs[i]:offs[i + 1]])[0]
            assert abs(got[i] - ref) <= 1e-12 * max(1.0, abs(ref))


@SETTINGS
@given(m=st.integers(1, 4), k=st.integers(1, 9), dsub=st.integers(1, 4), nd=st.integers(1, 5), b=st.integers(1, 4),
       nq=st.integers(1, 4), seed=st.integers(0, 2**31 - 1))
def test_pq_table_gather_equals_decompress_then_score(m, k, dsub, nd, b, nq, seed):
    rng = np.random.default_rng(seed)
    C = rng.standard_normal((m, k, dsub)).astype(np.float16)
    Q = rng.standard_normal((nq, m * dsub)).astype(np.float16)
    codes = rng.integers(0, k, (b, nd, m))
    gather = orc.pq_score_lut(orc.pq_build_lut(Q, C), codes).astype(np.float64)
    dec = orc.pq_decompress_score(Q, C, codes, f64=True)
    np.testing.assert_allclose(gather, dec, rtol=1e-5, atol=1e-5)
    # the decompressed vectors are the codebook rows themselves
    Dap = orc.pq_decompress(C, codes)
    for j in range(m):
        np.testing.assert_array_equal(Dap[..., j * dsub:(j + 1) * dsub], C[j][codes[..., j]].astype(np.float32))


_values = st.one_of(st.sampled_from([0.0, -0.0, 1.0, -1.0, 2.5, math.inf, -math.inf, math.nan]),
                    st.floats(-4.0, 4.0, width=32))


@SETTINGS
@given(vals=st.lists(_values, min_size=1, max_size=60), data=st.data())
def test_topk_is_a_stable_sort(vals, data):
    s = np.array(vals, dtype=np.float32)
    k = data.draw(st.integers(1, len(vals)))
    got_v, got_i = orc.topk(s, k)

    def key(i):
        v = float(s[i])
        return (0 if math.isnan(v) else 1, 0.0 if math.isnan(v) else -(v + 0.0), i)  # -0.0 + 0.0 is +0.0

    order = sorted(range(len(vals)), key=key)[:k]
    assert got_i.tolist() == order
    assert np.array_equal(got_v.view(np.uint32), s[order].view(np.uint32))


@SETTINGS
@given(nbits=st.sampled_from([1, 2, 4]), groups=st.integers(1, 6), t=st.integers(1, 5), seed=st.integers(0, 2**31 - 1))
def test_residual_packing_round_trips(nbits, groups, t, seed):
    rng = np.random.default_rng(seed)
    d = 8 * groups
    b = rng.integers(0, 1 << nbits, (t, d)).astype(np.uint8)
    packed = ro.pack_buckets(b, nbits)
    assert packed.shape == (t, d * nbits // 8)
    assert np.array_equal(ro.unpack_buckets(packed, nbits, d), b)
    assert np.array_equal(ro.unpack_buckets_via_tables(packed, nbits, d), b)
    # bit j of dimension i's bucket is bit (i * nbits + j) of the row, most significant first
    bits = np.unpackbits(packed, axis=1)
    for i in range(d):
        for j in range(nbits):
            assert np.array_equal(bits[:, i * nbits + j], (b[:, i] >> j) & 1)
