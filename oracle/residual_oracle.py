"""CPU oracle for residual-compressed (ColBERTv2) documents -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module; the product path never calls it.

Where the format comes from. The reference does not store compressed documents itself.
Its PLAID drop-in (``src/plaid_integration_benchmark.py:154-183``, patched into ColBERT
at ``:328-333``) receives documents that ColBERT's search has already decompressed from
its residual-compressed index. ColBERT is a third-party dependency absent from the
reference checkout: the package ``colbert-ai``, pinned at **0.2.22**
(``src/plaid_integration_benchmark.py:23``). Its codec is ``ResidualCodec`` in
``colbert/indexing/codecs/residual.py`` of that package. The package is not installed
here and its source is not in ``/root/reference``, so the citations below name the
package's functions, not line numbers. This module restates the codec's published
algorithm (Santhanam et al., "ColBERTv2", NAACL 2022, section 3):

index build (:func:`compress`)
  * ``code[t] = argmax_c <centroid[c], emb[t]>`` (``ResidualCodec.compress_into_codes``);
  * ``r = fp16(emb[t] - centroid[code[t]])`` (``ResidualCodec.compress``: the batch is
    half and ``lookup_centroids`` returns half rows);
  * ``bucket[j] = #{i : cutoffs[i] < r[j]}`` (``ResidualCodec.binarize``:
    ``torch.bucketize`` with its default ``right=False``), with ``2**nbits - 1``
    cutoffs;
  * bits ``0 .. nbits-1`` of every dimension's bucket, least significant bit first
    (``binarize``: ``(bucket >> arange(nbits)) & 1``), dimensions in order, packed eight
    to a byte with the first bit in the most significant position (``binarize`` calls
    ``numpy.packbits`` on the CPU and the package's ``packbits`` extension on the GPU,
    which packs the same way). A token's residual row is ``d * nbits / 8`` bytes
    (:func:`pack_buckets`).

decompression, GPU path of the codec (:func:`decompress`; ``ResidualCodec.decompress``
with ``use_gpu``, whose per-element work is the package's ``decompress_residuals``
CUDA extension, ``colbert/indexing/codecs/decompress_residuals.cu``)
  * ``v = fp16(centroid[code] + bucket_weights[bucket])``: a half add per element; the
    bucket comes from ``decompression_lookup_table[reversed_bit_map[byte]]`` (the two
    tables built in ``ResidualCodec.__init__``, restated in :func:`colbert_tables`);
  * ``n = fp16(sqrt(sum_j v_j**2))``, accumulated in fp32;
  * ``out = fp16(v / n)``: ``torch.nn.functional.normalize(v, p=2, dim=-1)`` applied to a
    half tensor.

One case differs on purpose: a token whose decoded vector is all zeros. ``normalize``
clamps the norm at ``eps = 1e-12``, which is 0 once the clamp is done in half
precision, so the codec's 0 / 0 gives NaN in every dimension. This oracle clamps the
norm at 1e-12 in fp32 and the HIP kernels at fp16's smallest subnormal (the two clamps
agree for every nonzero fp16 vector, whose half norm is at least that subnormal); both
return the zero vector, whose dot product with any query token is 0. Real indexes do
not hold such tokens: it takes a centroid that the residual weights cancel exactly in
every dimension.

The codec's own decoder does not extract bits directly. It maps each residual byte
through a bit-reversal table and then through the ``itertools.product`` table of bucket
tuples. :func:`colbert_tables` and :func:`unpack_buckets_via_tables` restate that
route, so the tests can check the direct bit extraction of :func:`unpack_buckets`
against it.

:func:`maxsim_residual` scores a query against documents of such tokens. Document
``b`` is index rows ``[offsets[p], offsets[p+1])`` with ``p = pids[b]``. It follows the
PLAID drop-in's semantics (``maxsim_oracle.maxsim_packed_zero_padded`` for
``pad_len > 0``, plain varlen MaxSim otherwise).

:func:`maxsim_residual_kernel_envelope` restates, with the same semantics, the
arithmetic of this build's two residual MaxSim kernels, which do not round ``v / n`` to
fp16 the way the codec's decompression does (the single-query kernel scales
``<q, v>`` by ``1 / n``; the batched kernel rounds ``fp16(v * (1 / n))``), as an
interval that holds both fp16 norms a kernel's fp32 sum of squares can round to
(:func:`norm_candidates`). It is pinned in ``tests/test_oracle_residual.py`` by closed
forms (a (3, 4, 0, ...) token in both forms), by fp32 simulations of both kernels with
the squares summed in random orders (each inside the envelope and its accumulation
bar; 24 orders over 6,000 tokens always land on one of the two norms, and a zero-width
envelope is caught), and by the fused form differing from the codec's scores by more
than that bar.
"""
from __future__ import annotations

import itertools

import numpy as np

from . import maxsim_oracle as _mo


def pack_buckets(buckets: np.ndarray, nbits: int) -> np.ndarray:
    """(T, d) bucket indices < 2**nbits -> (T, d*nbits/8) uint8 residual rows."""
    b = np.asarray(buckets, dtype=np.uint8)
    T, d = b.shape
    assert (d * nbits) % 8 == 0, (d, nbits)
    bits = (b[..., None] >> np.arange(nbits, dtype=np.uint8)) & 1  # (T, d, nbits), LSB first
    return np.packbits(bits.reshape(T, d * nbits), axis=-1)


def unpack_buckets(residuals: np.ndarray, nbits: int, d: int) -> np.ndarray:
    """(T, d*nbits/8) uint8 -> (T, d) bucket indices (inverse of :func:`pack_buckets`)."""
    r = np.asarray(residuals, dtype=np.uint8)
    T = r.shape[0]
    bits = np.unpackbits(r, axis=-1).reshape(T, d, nbits).astype(np.uint8)
    return (bits << np.arange(nbits, dtype=np.uint8)).sum(axis=-1).astype(np.uint8)


def colbert_tables(nbits: int):
    """The codec's two decode tables, restated from their published construction:
    ``reversed_bit_map[byte]`` reverses the bit order inside every ``nbits`` group of
    the byte (groups stay in place); ``lookup[z]`` is the ``z``-th tuple of
    ``itertools.product(range(2**nbits), repeat=8 // nbits)``."""
    mask = (1 << nbits) - 1
    rev = np.zeros(256, dtype=np.uint8)
    for byte in range(256):
        z = 0
        for hi in range(8, 0, -nbits):  # groups from the most significant end
            x = (byte >> (hi - nbits)) & mask
            y = 0
            for k in range(nbits):
                y |= ((x >> k) & 1) << (nbits - 1 - k)
            z = (z << nbits) | y
        rev[byte] = z
    lookup = np.array(list(itertools.product(range(1 << nbits), repeat=8 // nbits)), dtype=np.uint8)
    return rev, lookup


def unpack_buckets_via_tables(residuals: np.ndarray, nbits: int, d: int) -> np.ndarray:
    """Bucket indices by the codec's table route: byte -> reversed_bit_map -> lookup."""
    rev, lookup = colbert_tables(nbits)
    r = np.asarray(residuals, dtype=np.uint8)
    return lookup[rev[r].astype(np.int64)].reshape(r.shape[0], d)


def compress(embs: np.ndarray, centroids: np.ndarray, bucket_cutoffs: np.ndarray, nbits: int):
    """Index build: fp16 (T, d) embeddings -> (int32 codes (T,), uint8 residuals)."""
    E = np.asarray(embs, dtype=np.float16)
    C = np.asarray(centroids, dtype=np.float16)
    codes = np.argmax(E.astype(np.float32) @ C.astype(np.float32).T, axis=1).astype(np.int32)
    r = (E.astype(np.float32) - C[codes].astype(np.float32)).astype(np.float16)
    cut = np.asarray(bucket_cutoffs, dtype=np.float32)
    assert cut.shape == ((1 << nbits) - 1,), cut.shape
    buckets = np.searchsorted(cut, r.astype(np.float32), side="left").astype(np.uint8)
    return codes, pack_buckets(buckets, nbits)


def decompress_unnormalised(codes, residuals, centroids, bucket_weights, nbits: int) -> np.ndarray:
    """``fp16(centroid[code] + bucket_weights[bucket])`` per dimension, (T, d) fp16."""
    C = np.asarray(centroids, dtype=np.float16)
    d = C.shape[1]
    w = np.asarray(bucket_weights, dtype=np.float16)
    assert w.shape == (1 << nbits,), w.shape
    b = unpack_buckets(residuals, nbits, d)
    c = C[np.asarray(codes, dtype=np.int64)]
    return (c.astype(np.float32) + w[b].astype(np.float32)).astype(np.float16)


def decompress(codes, residuals, centroids, bucket_weights, nbits: int) -> np.ndarray:
    """The codec's GPU decompression: (T, d) fp16 unit vectors."""
    v = decompress_unnormalised(codes, residuals, centroids, bucket_weights, nbits).astype(np.float32)
    n = np.sqrt((v * v).sum(axis=1, dtype=np.float32), dtype=np.float32).astype(np.float16).astype(np.float32)
    n = np.maximum(n, np.float32(1e-12))
    return (v / n[:, None]).astype(np.float16)


def doc_rows(offsets: np.ndarray, pids) -> list:
    """(start, end) index rows of every scored document, or None for an invalid one."""
    offsets = np.asarray(offsets, dtype=np.int64)
    ndocs = offsets.shape[0] - 1
    ids = range(ndocs) if pids is None else np.asarray(pids, dtype=np.int64)
    out = []
    for p in ids:
        p = int(p)
        if p < 0 or p >= ndocs or offsets[p] < 0 or offsets[p + 1] < offsets[p]:
            out.append(None)
        else:
            out.append((int(offsets[p]), int(offsets[p + 1])))
    return out


def maxsim_residual(Q, codes, residuals, centroids, bucket_weights, nbits: int, offsets, pids=None,
                    pad_len: int = 0) -> np.ndarray:
    """float64 MaxSim of Q (Nq, d) against the decompressed documents.

    ``pad_len > 0``: a document shorter than ``pad_len`` also sees zero vectors (each
    query token's max is at least 0; an empty document scores 0), as the PLAID drop-in
    computes after padding. ``pad_len == 0``: varlen semantics (empty -> -inf).
    Invalid documents (pid or offsets out of range) score NaN."""
    D = decompress(codes, residuals, centroids, bucket_weights, nbits)
    Qd = np.asarray(Q, dtype=np.float64)
    rows = doc_rows(offsets, pids)
    out = np.empty(len(rows), dtype=np.float64)
    for i, se in enumerate(rows):
        if se is None or se[1] > D.shape[0]:
            out[i] = np.nan
            continue
        s, e = se
        if e == s:
            out[i] = 0.0 if (pad_len > 0 and Qd.shape[0] > 0) else (-np.inf if Qd.shape[0] > 0 else 0.0)
            continue
        m = (D[s:e].astype(np.float64) @ Qd.T).max(axis=0)
        if pad_len > 0 and e - s < pad_len:
            m = np.maximum(m, 0.0)
        out[i] = m.sum()
    return out


def norm_candidates(V: np.ndarray):
    """The fp16 norms a kernel can form from fp16 rows ``V`` (T, d): ``fp16(sqrt(n2))``
    with ``n2`` an fp32 sum of the squares in any order and the square root rounded to
    fp32, so ``sqrt(n2)`` lies within ``(d + 8) * 2^-24`` (relative) of the exact norm.
    Returns float64 arrays ``(n_lo, n_hi)`` of fp16 values, equal wherever that interval
    holds no fp16 rounding boundary, each clamped at the smallest positive fp16."""
    v = np.asarray(V, dtype=np.float64)
    s = np.sqrt((v * v).sum(axis=1))
    eps = (v.shape[1] + 8) * 2.0 ** -24
    tiny = float(np.float16(5.9604645e-8))
    lo = np.maximum((s * (1.0 - eps)).astype(np.float16).astype(np.float64), tiny)
    hi = np.maximum((s * (1.0 + eps)).astype(np.float16).astype(np.float64), tiny)
    return lo, hi


def maxsim_residual_kernel_envelope(Q, codes, residuals, centroids, bucket_weights, nbits: int, offsets,
                                    pids=None, pad_len: int = 0, form: str = "fused"):
    """float64 scores in the arithmetic of this build's residual MaxSim kernels, as
    ``(lo, hi, absref)`` per scored document (semantics of :func:`maxsim_residual`).

    Both kernels form ``v = fp16(centroid + weight)`` and ``inv = fp32(1 / n)`` with
    ``n`` one of :func:`norm_candidates`' values. ``form="fused"`` (the single-query
    kernel) scores ``<q, v> * inv``; ``form="batched"`` scores ``<q, x>`` with
    ``x = fp16(fp32(v) * inv)``. Neither rounds ``v / n`` to fp16 the way the codec's
    decompression does. Where a token's fp16 norm can fall either way, ``lo`` / ``hi``
    take each product's smaller / larger value over the two norms, so an exact-arithmetic
    kernel score lies in [lo, hi]. ``absref`` is the same MaxSim over absolute values
    (the fp32-accumulation bar's reference)."""
    V = decompress_unnormalised(codes, residuals, centroids, bucket_weights, nbits)
    Qd = np.asarray(Q, dtype=np.float64)
    n_lo, n_hi = norm_candidates(V)
    Vd = V.astype(np.float64)
    prods, aprods = [], []
    for n in (n_lo, n_hi):
        inv = (np.float32(1.0) / n.astype(np.float32)).astype(np.float64)
        if form == "fused":
            prods.append((Vd @ Qd.T) * inv[:, None])
            aprods.append((np.abs(Vd) @ np.abs(Qd).T) * inv[:, None])
        elif form == "batched":
            X = (V.astype(np.float32) * inv.astype(np.float32)[:, None]).astype(np.float16).astype(np.float64)
            prods.append(X @ Qd.T)
            aprods.append(np.abs(X) @ np.abs(Qd).T)
        else:
            raise ValueError(f"form must be 'fused' or 'batched', got {form!r}")
    pmin, pmax = np.minimum(prods[0], prods[1]), np.maximum(prods[0], prods[1])
    amax = np.maximum(aprods[0], aprods[1])
    rows = doc_rows(offsets, pids)
    out = np.empty((3, len(rows)), dtype=np.float64)
    for i, se in enumerate(rows):
        if se is None or se[1] > V.shape[0]:
            out[:, i] = np.nan
            continue
        s, e = se
        if e == s:
            out[:, i] = 0.0 if (pad_len > 0 and Qd.shape[0] > 0) else (-np.inf if Qd.shape[0] > 0 else 0.0)
            continue
        ms = [pmin[s:e].max(axis=0), pmax[s:e].max(axis=0), amax[s:e].max(axis=0)]
        if pad_len > 0 and e - s < pad_len:
            ms[0], ms[1] = np.maximum(ms[0], 0.0), np.maximum(ms[1], 0.0)
        out[:, i] = [m.sum() for m in ms]
    return out[0], out[1], out[2]


def maxsim_residual_f32(Q, codes, residuals, centroids, bucket_weights, nbits: int, offsets, pids=None,
                        pad_len: int = 0, chunk: int = 4096) -> np.ndarray:
    """The reference pipeline's CPU cost model for the ``cpu_baseline``: decompress the
    documents, then fp32 varlen MaxSim (``maxsim_oracle.maxsim_varlen``). ``pids`` must
    be None (all documents) and ``pad_len`` 0."""
    assert pids is None and pad_len == 0
    D = decompress(codes, residuals, centroids, bucket_weights, nbits)
    return _mo.maxsim_varlen(Q, D, offsets)
