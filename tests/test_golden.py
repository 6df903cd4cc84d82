"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every fixture (and the C restatement agrees).
GPU: every HIP entry point reproduces the fixture scores to 1e-3 relative (+1e-3 absolute)
and, for the dense, variable-length, masked, packed and PQ fixtures, to the
fp32-accumulation bar of ``accum_bar.py`` (on MaxSim(|Q|, |D|) of the fixture's inputs).
"""
import os

import numpy as np
import pytest

import accum_bar as bar
from oracle import c_oracle
from oracle import maxsim_oracle as orc
from oracle import residual_oracle as ro

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def test_fixtures_reproduce_on_cpu():
    f = _load("dense_d128.npz")
    np.testing.assert_allclose(orc.maxsim_f64(f["Q"], f["D"]), f["scores"], rtol=1e-12)
    np.testing.assert_allclose(c_oracle.maxsim_dense(f["Q"], f["D"]), f["scores"], rtol=1e-12)
    f = _load("dense_d256.npz")
    np.testing.assert_allclose(orc.maxsim_f64(f["Q"], f["D"]), f["scores"], rtol=1e-12)
    f = _load("varlen_d64.npz")
    got = orc.maxsim_varlen(f["Q"], f["D_flat"], f["offsets"], f64=True)
    np.testing.assert_allclose(got, f["scores"], rtol=1e-12)
    np.testing.assert_allclose(c_oracle.maxsim_varlen(f["Q"], f["D_flat"], f["offsets"]), f["scores"], rtol=1e-12)
    f = _load("masked_d128.npz")
    np.testing.assert_allclose(orc.maxsim_masked(f["Q"], f["D"], f["mask"], f64=True), f["scores"], rtol=1e-12)
    f = _load("pq_m16_k256.npz")
    np.testing.assert_allclose(orc.pq_decompress_score(f["Q"], f["codebook"], f["codes"], f64=True), f["scores"],
                               rtol=1e-12)
    np.testing.assert_allclose(orc.pq_build_lut(f["Q"], f["codebook"])[:2], f["lut_q01"], rtol=1e-5, atol=1e-6)
    f = _load("packed_zeros_d128.npz")
    np.testing.assert_allclose(orc.maxsim_packed_zero_padded(f["Q"], f["D_packed"], f["lengths"]), f["scores"],
                               rtol=1e-12)
    f = _load("residual_d128_nb2.npz")
    args = (f["codes"], f["residuals"], f["centroids"], f["bucket_weights"], 2)
    assert np.array_equal(ro.decompress(*args), f["decompressed"])
    pad = int((f["offsets"][1:] - f["offsets"][:-1])[f["pids"]].max())
    for name, p in (("scores_zeros", pad), ("scores_mask", 0)):
        got = ro.maxsim_residual(f["Q"], *args, f["offsets"], f["pids"], p)
        assert np.array_equal(np.isinf(got), np.isinf(f[name]))
        fin = ~np.isinf(got)
        np.testing.assert_allclose(got[fin], f[name][fin], rtol=1e-12)


def _close(got, ref, lim=None, what=""):
    bar.assert_scores(got, ref, lim, what)


def _lim(fn, Q, X, *rest, **kw):
    """The fp32-accumulation bar for a fixture's scores, from its inputs."""
    return bar.with_bound(fn, Q, X, *rest, **kw)[1]


@pytest.mark.gpu
def test_fixtures_on_gpu(cuda):
    import torch
    import tilemaxsim_amd as tms
    g = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    for name in ("dense_d128.npz", "dense_d256.npz"):
        f = _load(name)
        _close(tms.flash_maxsim_v2_multiquery(g(f["Q"]), g(f["D"])).cpu().numpy(), f["scores"],
               _lim(orc.maxsim_f64, f["Q"], f["D"]), name)
    f = _load("varlen_d64.npz")
    _close(tms.flash_maxsim_multi_doc(g(f["Q"]), g(f["D_flat"]), g(f["offsets"])).cpu().numpy(), f["scores"],
           _lim(orc.maxsim_varlen, f["Q"], f["D_flat"], f["offsets"], f64=True), "varlen_d64")
    f = _load("masked_d128.npz")
    _close(tms.maxsim_score(g(f["Q"]), g(f["D"]), g(f["mask"])).cpu().numpy(), f["scores"],
           _lim(orc.maxsim_masked, f["Q"], f["D"], f["mask"], f64=True), "masked_d128")
    f = _load("pq_m16_k256.npz")
    pq = tms.TileMaxSimPQ(g(f["codebook"]))
    lim = _lim(orc.pq_decompress_score, f["Q"], f["codebook"], f["codes"], f64=True)
    for method in ("mfma", "lut"):
        _close(pq.score_batch(g(f["Q"]), g(f["codes"]), method=method).cpu().numpy(), f["scores"], lim,
               f"pq {method}")
    lut = pq.build_distance_table(g(f["Q"])).cpu().numpy()
    np.testing.assert_allclose(lut[:2], f["lut_q01"], rtol=1e-5, atol=1e-5)
    f = _load("packed_zeros_d128.npz")
    got = tms.flashmaxsim_score_packed(g(f["Q"]), g(f["D_packed"]), torch.from_numpy(f["lengths"]))
    _close(got.cpu().numpy(), f["scores"],
           _lim(orc.maxsim_packed_zero_padded, f["Q"], f["D_packed"], f["lengths"]), "packed_zeros_d128")
    f = _load("residual_d128_nb2.npz")
    idx = (g(f["codes"]), g(f["residuals"]), g(f["centroids"]), g(f["bucket_weights"]), 2)
    dec = tms.decompress_residual(*idx).cpu().numpy()
    ulps = np.abs(dec.view(np.int16).astype(np.int32) - f["decompressed"].view(np.int16).astype(np.int32))
    assert ulps.max() <= 1
    for name, padding in (("scores_zeros", "zeros"), ("scores_mask", "mask")):
        got = tms.flashmaxsim_score_residual(g(f["Q"]), *idx, g(f["offsets"]), g(f["pids"]), padding=padding)
        _close(got.cpu().numpy(), f[name])
