"""Write the golden fixtures under tests/golden/ (seeded inputs + float64 expected scores).

The reference holds no vectors for this path, so the expected values come from the
float64 oracle (oracle/maxsim_oracle.py, oracle/residual_oracle.py), which
tests/test_oracle.py and tests/test_oracle_residual.py pin against brute force, closed
forms, invariants, hand-derived bit layouts and the C restatement. The fixtures freeze
those values so both the oracle and the GPU kernels are checked against the same
bytes on every machine.

Run from the repo root: ``python tests/golden/make_golden.py``.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import maxsim_oracle as orc  # noqa: E402
from oracle import residual_oracle as ro  # noqa: E402


def _h(rng, shape, normalize=False):
    x = rng.standard_normal(shape, dtype=np.float32)
    if normalize:
        x /= np.linalg.norm(x, axis=-1, keepdims=True) + 1e-12
    return x.astype(np.float16)


def main():
    rng = np.random.default_rng(20260101)
    # dense: Nq=32, d=128 (the d <= 128 kernel), 6 docs x 37 tokens (ragged last tile)
    Q = _h(rng, (32, 128), normalize=True)
    D = _h(rng, (6, 37, 128), normalize=True)
    np.savez_compressed(os.path.join(HERE, "dense_d128.npz"), Q=Q, D=D, scores=orc.maxsim_f64(Q, D))
    # dense d-tiled: Nq=33 (two query blocks), d=256, unnormalised as the reference's tests
    Q = _h(rng, (33, 256))
    D = _h(rng, (4, 21, 256))
    np.savez_compressed(os.path.join(HERE, "dense_d256.npz"), Q=Q, D=D, scores=orc.maxsim_f64(Q, D))
    # varlen with empty documents
    lens = np.array([5, 0, 40, 1, 17, 0, 33])
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    Q = _h(rng, (32, 64), normalize=True)
    Dflat = _h(rng, (int(offsets[-1]), 64), normalize=True)
    np.savez_compressed(os.path.join(HERE, "varlen_d64.npz"), Q=Q, D_flat=Dflat, offsets=offsets,
                        scores=orc.maxsim_varlen(Q, Dflat, offsets, f64=True))
    # masked, with a fully masked document
    Q = _h(rng, (16, 128), normalize=True)
    D = _h(rng, (5, 24, 128), normalize=True)
    mask = rng.random((5, 24)) < 0.5
    mask[2] = False
    np.savez_compressed(os.path.join(HERE, "masked_d128.npz"), Q=Q, D=D, mask=mask,
                        scores=orc.maxsim_masked(Q, D, mask, f64=True))
    # PQ: M=16, K=256, dsub=8 (the reference self-test layout), randn codebook
    C = _h(rng, (16, 256, 8))
    Q = _h(rng, (32, 128), normalize=True)
    codes = rng.integers(0, 256, size=(4, 50, 16)).astype(np.uint8)
    lut = np.einsum("qmj,mkj->qmk", Q[:2].astype(np.float64).reshape(2, 16, 8), C.astype(np.float64))
    np.savez_compressed(os.path.join(HERE, "pq_m16_k256.npz"), Q=Q, codebook=C, codes=codes,
                        lut_q01=lut, scores=orc.pq_decompress_score(Q, C, codes, f64=True))
    # PLAID packed documents with the reference drop-in's zero padding (an empty document)
    lens = np.array([12, 3, 0, 29, 7])
    Q = _h(rng, (32, 128), normalize=True)
    Dp = _h(rng, (int(lens.sum()), 128), normalize=True)
    Dp[: lens[0]] *= -1  # negative similarities make the zero padding visible
    np.savez_compressed(os.path.join(HERE, "packed_zeros_d128.npz"), Q=Q, D_packed=Dp, lengths=lens,
                        scores=orc.maxsim_packed_zero_padded(Q, Dp, lens))
    # ColBERTv2 residual-compressed index (nbits=2): decompressed tokens and scores of
    # candidate documents, both padding semantics
    lens = np.array([9, 0, 21, 4, 16])
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(offsets[-1])
    cent = _h(rng, (32, 128), normalize=True)
    codes = rng.integers(0, 32, size=T).astype(np.int32)
    residuals = ro.pack_buckets(rng.integers(0, 4, size=(T, 128)).astype(np.uint8), 2)
    weights = np.array([-0.05, -0.012, 0.012, 0.05], dtype=np.float16)
    pids = np.array([4, 2, 0, 1, 2], dtype=np.int64)
    Q = _h(rng, (32, 128), normalize=True)
    np.savez_compressed(os.path.join(HERE, "residual_d128_nb2.npz"), Q=Q, codes=codes, residuals=residuals,
                        centroids=cent, bucket_weights=weights, offsets=offsets, pids=pids,
                        decompressed=ro.decompress(codes, residuals, cent, weights, 2),
                        scores_zeros=ro.maxsim_residual(Q, codes, residuals, cent, weights, 2, offsets, pids,
                                                        int(lens[pids].max())),
                        scores_mask=ro.maxsim_residual(Q, codes, residuals, cent, weights, 2, offsets, pids, 0))
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
