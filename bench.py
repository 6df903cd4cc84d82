"""Benchmark of the fused MaxSim scoring path on one MI355X.

Default workload (C2, the configuration the headline metric is quoted on):
64 queries x 1,000,000 documents, Nq = 32, Nd = 180, d = 128, fp16 L2-normalised
Gaussian embeddings (~46 GB resident in HBM). One step scores every query against
every document with ``flash_maxsim_v2_multiquery`` (one HBM pass over the corpus per
query, as the reference's V2-MQ kernel) and takes the top-100 per query.

Other workloads (``--config``): c1 (CPU-sized plumbing check), rerank (the reference's
end-to-end reranking call: 1 query x 256 candidates x 180 tokens), c2b (C2 with all 64
queries through the batched-query kernel), c3 (2M variable-length documents), c3b (c3
through the batched-query kernel), c4
(d-tiled, ``--d 256|512|768``), c5 (PQ/ADC, 5M documents of uint8 codes), c5b (c5
through the batched-query kernel), c6 (C3's
corpus as a ColBERTv2 residual-compressed index, fused decode + MaxSim per query), c6b
(the same index, all queries through the batched residual kernel), prec (the
reference's precision experiment: 1 query x 10K raw-Gaussian documents, Nd = 128,
d = 128), copy (counter calibration), readprobe (a read-only streaming kernel over a
C2-sized 46 GB buffer: the read rate any streaming kernel reaches on this part), topk
(top-100 of each row of C2's (64, 1M) score matrix, plus other row shapes).
``--dtype fp16|bf16|fp32`` sets the embedding dtype of c1, rerank, c2, c4 and prec.

Prints ONE JSON line on stdout. ``value`` is (query, document) pairs scored per second
over the whole step; ``roofline`` is the dominant kernel's algorithmic bandwidth from
HIP events around each of its launches; ``cpu_baseline`` times the reference's PyTorch
scoring path (restated in ``oracle/torch_ref.py``, fp32 on the CPU with
``torch.set_num_threads(os.cpu_count())``) on this host, streaming 500-document chunks of
a prefix of the corpus larger than the host's last-level cache (20,000 documents for the
dense and variable-length configs, 100,000 for PQ) and extrapolated linearly to docs/s
(``extrapolated``, ``prefix_docs``), with the numpy restatement beside it.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

HBM_PEAK_GBS = 8000.0
METRIC = "docs scored/sec + achieved HBM GB/s (% of peak), N_q=32 d=128 fp16"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None,
                   help="timed steps (default 5; 200 for the microsecond-scale c1 and rerank)")
    p.add_argument("--warmup", type=int, default=None, help="untimed steps first (default 1; 20 for c1 and rerank)")
    p.add_argument("--config", default="c2",
                   choices=["c1", "rerank", "c2", "c2b", "c3", "c3b", "c4", "c5", "c5b", "c6", "c6b", "prec", "copy",
                            "readprobe", "ldsprobe", "mfmaprobe", "topk"])
    p.add_argument("--d", type=int, default=512, help="embedding width for --config c4")
    p.add_argument("--dtype", default="fp16", choices=["fp16", "bf16", "fp32"],
                   help="embedding dtype for --config c1, rerank, c2, c2b, c4 and prec")
    p.add_argument("--qdtype", default=None, choices=["fp32"],
                   help="--config c2b: fp32 queries against the --dtype documents (split, never rounded)")
    p.add_argument("--ncent", type=int, default=1 << 18,
                   help="--config c6 / c6b: centroids in the index (2^18, ColBERT's choice for ~332M tokens)")
    p.add_argument("--lds-pattern", type=int, default=None, choices=range(12),
                   help="--config ldsprobe: time this pattern alone (default: pattern 1 timed, all ten reported)")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline time budget")
    p.add_argument("--no-cpu-baseline", action="store_true")
    return p.parse_args()


# ----------------------------------------------------------------------------- data
def normalized_fp16(torch, shape, gen, chunk_rows=1 << 21, dtype=None, normalize=True):
    """Gaussian -> L2-normalise each token in fp32 -> fp16 (or ``dtype``), generated in
    chunks on the GPU. ``normalize=False`` keeps the raw Gaussian values."""
    out = torch.empty(shape, dtype=dtype or torch.float16, device="cuda")
    flat = out.view(-1, shape[-1])
    for s in range(0, flat.shape[0], chunk_rows):
        e = min(flat.shape[0], s + chunk_rows)
        x = torch.randn(e - s, shape[-1], device="cuda", generator=gen)
        flat[s:e] = torch.nn.functional.normalize(x, dim=-1) if normalize else x
    return out


DTYPES = {"fp16": ("float16", 2), "bf16": ("bfloat16", 2), "fp32": ("float32", 4)}


def topk_rows(scores, k):
    """Per-query top-k of the (queries, docs) score matrix with the HIP top-k kernel."""
    from tilemaxsim_amd import topk
    return topk(scores, k)


class KernelTimer:
    """HIP events around each launch of the dominant kernel, on the stream it runs on. The
    event pairs are created before the timed steps (``prepare``), so a step pays only for
    recording them."""

    def __init__(self, torch):
        self.torch = torch
        self.pairs = []
        self.pool = []
        self.enabled = False

    def prepare(self, n):
        ev = lambda: self.torch.cuda.Event(enable_timing=True)
        self.pool = [(ev(), ev()) for _ in range(n)]
        self.pool.reverse()

    def __call__(self, fn):
        if not self.enabled:
            return fn()
        if self.pool:
            s, e = self.pool.pop()
        else:
            s, e = self.torch.cuda.Event(enable_timing=True), self.torch.cuda.Event(enable_timing=True)
        s.record()
        r = fn()
        e.record()
        self.pairs.append((s, e))
        return r

    def avg_ms(self):
        ts = [s.elapsed_time(e) for s, e in self.pairs]
        return float(np.mean(ts)), float(np.median(ts)), len(ts)


# ----------------------------------------------------------------------------- workloads
class Dense:
    kernel = "dense_maxsim_kernel"

    def __init__(self, torch, n_queries, B, Nd, d, Nq=32, name="c2", topk=100, dtype="fp16", normalize=True):
        self.torch, self.nQ, self.B, self.Nd, self.d, self.Nq, self.k = torch, n_queries, B, Nd, d, Nq, topk
        self.name, self.dtype, self.normalize = name, dtype, normalize
        tname, self.esize = DTYPES[dtype]
        # fixed-length fp16 / bf16 documents with d in {32, 64, 96, 128} run the streaming
        # kernel, or the small-batch kernel when the call spans few tiles
        self.kernel = "dense_maxsim_kernel"
        if d <= 128 and d % 32 == 0 and dtype != "fp32":
            from tilemaxsim_amd import _lib
            small = B * ((Nd + 15) // 16) <= _lib.load().tms_set_rerank_limit(-1) and (Nq + 31) // 32 <= 3
            self.kernel = "rerank_maxsim_kernel" if small else "stream_maxsim_kernel"
        gen = torch.Generator(device="cuda").manual_seed(1234)
        log(f"[bench] generating {B} docs x {Nd} x {d} {dtype} ({B * Nd * d * self.esize / 1e9:.2f} GB)")
        tdt = getattr(torch, tname)
        self.D = normalized_fp16(torch, (B, Nd, d), gen, dtype=tdt, normalize=normalize)
        self.Q = normalized_fp16(torch, (n_queries, Nq, d), gen, dtype=tdt, normalize=normalize)
        self.scores = torch.empty(n_queries, B, dtype=torch.float32, device="cuda")

    def step(self, timer):
        from tilemaxsim_amd import flash_maxsim_v2_multiquery
        if self.nQ == 1:  # one query (c1, rerank, prec): rank its scores where they are
            s = timer(lambda: flash_maxsim_v2_multiquery(self.Q[0], self.D))
            return topk_rows(s.unsqueeze(0), min(self.k, self.B))
        for i in range(self.nQ):
            s = timer(lambda: flash_maxsim_v2_multiquery(self.Q[i], self.D))
            self.scores[i].copy_(s)
        return topk_rows(self.scores, min(self.k, self.B))

    def bytes_per_launch(self):
        return (self.Nq * self.d + self.B * self.Nd * self.d) * self.esize + self.B * 4

    def pairs_per_step(self):
        return self.nQ * self.B

    def batched_line(self, torch, steps=3):
        """C2 only, after the timed steps: the same step (every query against every
        document, then the top-k) with all queries in one flash_maxsim_batched_queries
        call per step; HIP events around each call and around each whole step."""
        if self.name != "c2" or self.dtype == "fp32":  # fp32 runs batched as --config c2b --dtype fp32
            return None
        from tilemaxsim_amd import flash_maxsim_batched_queries
        calls, whole = [], []
        for i in range(steps + 1):
            e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
            e[0].record()
            s = flash_maxsim_batched_queries(self.Q, self.D)
            e[1].record()
            self.scores.copy_(s)
            topk_rows(self.scores, min(self.k, self.B))
            e[2].record()
            if i > 0:  # the first step warms up
                calls.append(e)
        torch.cuda.synchronize()
        call_ms = float(np.mean([a.elapsed_time(b) for a, b, _ in calls]))
        step_ms = float(np.mean([a.elapsed_time(c) for a, _, c in calls]))
        tf = 2 * self.nQ * self.Nq * self.B * self.Nd * self.d / (call_ms * 1e-3) / 1e12
        line = {"value": round(self.pairs_per_step() / (step_ms * 1e-3), 1), "unit": "docs/s", "ms_per_step": round(step_ms, 3),
                "steps": steps, "kernel": "batched_tile_kernel", "launch_ms_mean": round(call_ms, 4),
                "achieved_tflops": round(tf, 1), "peak_tflops": 2500.0, "frac": round(tf / 2500.0, 4),
                "note": "flash_maxsim_batched_queries: 32 queries share each HBM pass (see --config c2b)"}
        line.update(gemm_ceiling(torch, tf))
        return line

    def graph_line(self, torch, replays=200):
        """C1 and rerank only, after the timed steps: the same step (score, then top-k) captured once
        in a HIP graph (torch.cuda.CUDAGraph) and replayed, as a serving loop would for
        each new query; HIP events around the replays. The eager step pays the Python
        and launch cost of every call; a replay pays one graph launch."""
        if self.name not in ("c1", "rerank"):
            return None
        ident = lambda f: f()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.step(ident)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step(ident)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(replays):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 / replays
        ms = e0.elapsed_time(e1) / replays
        return {"ms_per_step": round(ms, 4), "wall_ms_per_step": round(wall_ms, 4), "replays": replays,
                "value": round(self.pairs_per_step() / (ms * 1e-3), 1), "unit": "docs/s",
                "note": "the step captured once in a HIP graph and replayed"}

    def one_launch_line(self, torch, steps=200, warmup=20):
        """C1 and rerank only, after the timed steps: the same step through maxsim_topk, which
        scores and ranks in one launch (tms_maxsim_topk) when the call has at most
        ONE_LAUNCH_MAX_TOKENS document tokens (rerank: 46K; C1: 128K); wall clock around
        eager steps, as for the timed steps, and a check that the results are those of the
        timed step."""
        if self.name not in ("c1", "rerank") or self.nQ != 1 or self.dtype == "fp32":
            return None
        from tilemaxsim_amd import maxsim_topk
        from tilemaxsim_amd.topk import ONE_LAUNCH_MAX_TOKENS, _one_launch_workgroups
        if self.B * self.Nd > ONE_LAUNCH_MAX_TOKENS:
            return None
        wg = _one_launch_workgroups(self.B, self.Nd, self.d, self.Nq)
        k = min(self.k, self.B)
        q = self.Q[0]
        v, i = maxsim_topk(q, self.D, k)
        rv, ri = self.step(lambda f: f())
        same = bool(torch.equal(i, ri[0]) and torch.equal(v.view(torch.int32), rv[0].view(torch.int32)))
        for _ in range(warmup):
            maxsim_topk(q, self.D, k)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            maxsim_topk(q, self.D, k)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        return {"ms_per_step": round(ms, 4), "steps": steps, "value": round(self.pairs_per_step() / (ms * 1e-3), 1),
                "unit": "docs/s", "kernel": "rerank_topk_kernel", "workgroups": wg, "same_results": same,
                "note": "maxsim_topk: scores and top-k in one launch (eager)"}

    def config(self):
        values = "L2-normalised Gaussian" if self.normalize else "unnormalised Gaussian"
        cfg = {"workload": f"{self.name}: {self.nQ} queries x {self.B:,} docs, Nq={self.Nq}, Nd={self.Nd}, d={self.d}, "
                           f"{self.dtype} {values}, top-{self.k} per query",
               "queries": self.nQ, "docs": self.B, "Nq": self.Nq, "Nd": self.Nd, "d": self.d, "top_k": self.k,
               "dtype": self.dtype, "kernel": "flash_maxsim_v2_multiquery (one HBM pass per query)"}
        if self.name == "prec":
            cfg["reference_shape"] = ("the reference's precision experiment: src/cycle6_rerun_scaling.py:96-115, "
                                      "src/run_all_experiments.py:287-347")
        return cfg

    def cpu_baseline(self, seconds):
        from oracle import maxsim_oracle as orc
        from oracle import torch_ref as tr
        n = min(self.B, CPU_PREFIX_DOCS)
        Qt, Dt = self.Q[0].cpu(), self.D[:n].cpu()
        nbytes = Dt.numel() * Dt.element_size()
        # torch: the reference's own formulation; each chunk is cast .float() in the timed calls
        base = _time_cpu_prefix(lambda b0, b1: tr.maxsim_naive(Qt, Dt[b0:b1], chunk=500), n, self.B, seconds,
                                "query 0, torch fp32 einsum -> max -> sum (pytorch_maxsim_naive)", nbytes)
        if self.dtype == "bf16":  # numpy has no bfloat16: cast once, outside the timed calls
            Dt = Dt.float()
        Q, D = self.Q[0].float().cpu().numpy() if self.dtype == "bf16" else Qt.numpy(), Dt.numpy()
        base["numpy_port"] = _time_cpu_prefix(lambda b0, b1: orc.maxsim_naive(Q, D[b0:b1], chunk=500), n, self.B,
                                              seconds / 2, "query 0, numpy fp32 materialise-then-reduce",
                                              D.nbytes, torch_threads=False)
        return base


def gemm_ceiling(torch, achieved_tflops):
    """The practical fp16 MFMA ceiling on this part, measured in the same process: a large
    square fp16 GEMM through torch (hipBLASLt), which runs at the same power-limited clock
    as any MFMA-bound kernel."""
    n = 8192
    a = torch.randn(n, n, device="cuda").half()
    b = torch.randn(n, n, device="cuda").half()
    for _ in range(3):
        torch.mm(a, b)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(20):
        torch.mm(a, b)
    e1.record()
    torch.cuda.synchronize()
    gemm_tf = 2 * n ** 3 / (e0.elapsed_time(e1) / 20 * 1e-3) / 1e12
    return {"gemm_fp16_8192_tflops": round(gemm_tf, 1), "frac_of_gemm": round(achieved_tflops / gemm_tf, 4)}


class DenseBatched(Dense):
    """C2 data, all queries scored by the batched-query entry point: each workgroup's
    eight waves hold 32 query blocks and share one HBM pass over the documents, which
    moves the path from the HBM roof to the MFMA roof."""
    MFMA_PEAK_TFLOPS = 2500.0
    MFMA_PEAK_TFLOPS_F32 = 157.3

    def __init__(self, *args, qdtype=None, **kw):
        super().__init__(*args, **kw)
        self.kernel = "batched_tile_kernel"  # fixed-length documents at implicit offsets
        self.qdtype = qdtype
        if qdtype == "fp32":  # fp32 queries against 16-bit documents: two MFMAs per product
            gen = self.torch.Generator(device="cuda").manual_seed(99)
            self.Q = normalized_fp16(self.torch, tuple(self.Q.shape), gen, dtype=self.torch.float32)

    def step(self, timer):
        from tilemaxsim_amd import flash_maxsim_batched_queries
        s = timer(lambda: flash_maxsim_batched_queries(self.Q, self.D))
        self.scores.copy_(s)
        return topk_rows(self.scores, min(self.k, self.B))

    def flops_per_launch(self):
        return 2 * self.nQ * self.Nq * self.B * self.Nd * self.d

    def bytes_per_launch(self):  # algorithmic: every query against one read of the corpus
        return (self.nQ * self.Nq * self.d + self.B * self.Nd * self.d) * self.esize + self.nQ * self.B * 4

    launch_desc = "one flash_maxsim_batched_queries call (one kernel per 32 query blocks)"

    def extra_roofline(self, launch_ms):
        tf = self.flops_per_launch() / (launch_ms * 1e-3) / 1e12
        if self.dtype != "fp32" and self.qdtype == "fp32":  # two 16-bit MFMAs per product (q_lo, q_hi)
            out = gemm_ceiling(self.torch, tf)
            out.update({"mfma_executed_tflops": round(2 * tf, 1),
                        "mfma_executed_frac": round(2 * tf / self.MFMA_PEAK_TFLOPS, 4)})
            return out
        if self.dtype != "fp32":
            return gemm_ceiling(self.torch, tf)
        # fp32: priced against the fp32 dense MFMA peak; the kernel runs each product as
        # three bf16 MFMAs (hi*hi + hi*lo + lo*hi), whose rate is given against bf16's peak
        return {"peak": self.MFMA_PEAK_TFLOPS_F32, "frac": round(tf / self.MFMA_PEAK_TFLOPS_F32, 4),
                "peak_note": "fp32 dense MFMA peak; products run as three bf16 MFMAs",
                "bf16_mfma_executed_tflops": round(3 * tf, 1),
                "bf16_mfma_executed_frac": round(3 * tf / self.MFMA_PEAK_TFLOPS, 4)}

    def config(self):
        c = super().config()
        c["workload"] += " (batched-query kernel)"
        c["kernel"] = "flash_maxsim_batched_queries (32 query blocks per HBM pass)"
        if self.qdtype:
            c["workload"] += f", {self.qdtype} queries"
            c["query_dtype"] = self.qdtype
            c["kernel"] = "flash_maxsim_batched_queries (16 split query blocks per HBM pass)"
        return c


class Varlen(Dense):
    def __init__(self, torch, n_queries, B, lo, hi, d, Nq=32, topk=100):
        self.torch, self.nQ, self.B, self.d, self.Nq, self.k = torch, n_queries, B, d, Nq, topk
        self.name = "c3"
        rng = np.random.default_rng(77)
        lens = rng.integers(lo, hi + 1, size=B)
        offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        self.T = int(offs[-1])
        self.lo, self.hi = lo, hi
        # 16-bit documents with d in {32, 64, 96, 128} stream through the variable-length
        # instantiation of the streaming kernel (queries held in registers); subclasses
        # that run other kernels name them as class attributes
        if self.kernel == "dense_maxsim_kernel" and d <= 128 and d % 32 == 0:
            self.kernel = "stream_maxsim_kernel"
        gen = torch.Generator(device="cuda").manual_seed(4321)
        log(f"[bench] generating {B} varlen docs, {self.T} tokens x {d} fp16 ({self.T * d * 2 / 1e9:.2f} GB)")
        self.D = normalized_fp16(torch, (self.T, d), gen)
        self.offsets = torch.from_numpy(offs).cuda()
        self.Q = normalized_fp16(torch, (n_queries, Nq, d), gen)
        self.scores = torch.empty(n_queries, B, dtype=torch.float32, device="cuda")
        from tilemaxsim_amd import flash_maxsim_multi_doc
        flash_maxsim_multi_doc(self.Q[0], self.D, self.offsets, validate=True)  # offsets checked once, at load

    def step(self, timer):
        from tilemaxsim_amd import flash_maxsim_multi_doc
        for i in range(self.nQ):
            s = timer(lambda: flash_maxsim_multi_doc(self.Q[i], self.D, self.offsets, validate=False))
            self.scores[i].copy_(s)
        return topk_rows(self.scores, self.k)

    def bytes_per_launch(self):
        return self.Nq * self.d * 2 + self.T * self.d * 2 + (self.B + 1) * 8 + self.B * 4

    def config(self):
        return {"workload": f"c3: {self.nQ} queries x {self.B:,} variable-length docs (Nd~U[{self.lo},{self.hi}], "
                            f"{self.T:,} tokens), Nq={self.Nq}, d={self.d}, fp16, top-{self.k} per query",
                "queries": self.nQ, "docs": self.B, "tokens": self.T, "Nq": self.Nq, "d": self.d, "top_k": self.k,
                "kernel": "flash_maxsim_multi_doc (offsets, no padding)"}

    def cpu_baseline(self, seconds):
        from oracle import maxsim_oracle as orc
        from oracle import torch_ref as tr
        n = min(self.B, CPU_PREFIX_DOCS)
        offs_t = self.offsets[: n + 1].cpu()
        Qt, Dt = self.Q[0].cpu(), self.D[: int(offs_t[-1])].cpu()
        nbytes = Dt.numel() * Dt.element_size()
        base = _time_cpu_prefix(lambda b0, b1: tr.maxsim_varlen_masked(Qt, Dt, offs_t[b0:b1 + 1] , chunk=500), n,
                                self.B, seconds, "query 0, torch fp32: 500-doc chunks padded to their longest, "
                                "einsum -> masked_fill(-inf) -> max -> sum (pytorch_maxsim_score)", nbytes)
        offs = offs_t.numpy()
        Q, Dflat = Qt.numpy(), Dt.numpy()
        base["numpy_port"] = _time_cpu_prefix(lambda b0, b1: orc.maxsim_varlen(Q, Dflat, offs[b0:b1 + 1]), n,
                                              self.B, seconds / 2,
                                              "query 0, numpy fp32 per-token sims + segmented max", Dflat.nbytes,
                                              torch_threads=False)
        return base


class VarlenBatched(Varlen):
    """C3's corpus and queries, all queries scored by one batched call
    (flash_maxsim_multi_doc_batched): each tile is loaded once per workgroup and scored
    from LDS by 32 query blocks, which moves the path to the MFMA roof."""
    kernel = "batched_tile_kernel"
    MFMA_PEAK_TFLOPS = 2500.0
    launch_desc = "one flash_maxsim_multi_doc_batched call (one kernel per 32 query blocks)"

    def __init__(self, *args, **kw):
        super().__init__(*args, **kw)
        self.name = "c3b"

    def step(self, timer):
        from tilemaxsim_amd import flash_maxsim_multi_doc_batched
        s = timer(lambda: flash_maxsim_multi_doc_batched(self.Q, self.D, self.offsets, validate=False))
        self.scores.copy_(s)
        return topk_rows(self.scores, self.k)

    def flops_per_launch(self):
        return 2 * self.nQ * self.Nq * self.T * self.d

    def bytes_per_launch(self):
        return self.nQ * self.Nq * self.d * 2 + self.T * self.d * 2 + (self.B + 1) * 8 + self.nQ * self.B * 4

    def extra_roofline(self, launch_ms):
        return gemm_ceiling(self.torch, self.flops_per_launch() / (launch_ms * 1e-3) / 1e12)

    def config(self):
        c = super().config()
        c["workload"] = c["workload"].replace("c3:", "c3b:", 1) + " (batched-query kernel)"
        c["kernel"] = "flash_maxsim_multi_doc_batched (tiles shared through LDS by 32 query blocks)"
        return c


class Residual(Varlen):
    """C3's corpus shape stored as a ColBERTv2 residual-compressed index (colbert-ai 0.2.22
    codec, nbits=2): int32 centroid ids + 32-byte residual rows per token, 2^18 fp16
    centroids (ColBERT's choice, 2^floor(log2(16 sqrt(#tokens))), for ~332M tokens).
    Each query is scored by the fused decode + MaxSim kernel (flashmaxsim_score_residual,
    plain MaxSim semantics): the decompressed tokens never exist in memory."""
    kernel = "residual_maxsim_kernel"
    unfused_key = "unfused_decompress_then_score_ms"

    def __init__(self, torch, n_queries, B, lo, hi, d=128, nbits=2, ncent=1 << 18, Nq=32, topk=100):
        self.torch, self.nQ, self.B, self.d, self.Nq, self.k = torch, n_queries, B, d, Nq, topk
        self.nbits, self.ncent = nbits, ncent
        self.name = "c6"
        rng = np.random.default_rng(77)
        lens = rng.integers(lo, hi + 1, size=B)
        offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        self.T = int(offs[-1])
        self.lo, self.hi = lo, hi
        self.rb = d * nbits // 8
        gen = torch.Generator(device="cuda").manual_seed(4321)
        log(f"[bench] generating a residual index: {B} varlen docs, {self.T} tokens, {ncent} centroids, "
            f"nbits={nbits} ({self.T * (4 + self.rb) / 1e9:.2f} GB)")
        self.codes = torch.randint(0, ncent, (self.T,), dtype=torch.int32, device="cuda", generator=gen)
        self.res = torch.randint(0, 256, (self.T, self.rb), dtype=torch.uint8, device="cuda", generator=gen)
        self.centroids = normalized_fp16(torch, (ncent, d), gen)
        # bucket weights at the quantiles of a small residual spread, as the codec fits them
        self.weights = torch.tensor(np.sort(np.random.default_rng(5).normal(0, 0.04, 1 << nbits)),
                                    dtype=torch.float16, device="cuda")
        self.offsets = torch.from_numpy(offs).cuda()
        self.Q = normalized_fp16(torch, (n_queries, Nq, d), gen)
        self.scores = torch.empty(n_queries, B, dtype=torch.float32, device="cuda")
        self._score(0, validate=True)  # offsets checked once, at load

    def _score(self, i, validate=False):
        from tilemaxsim_amd import flashmaxsim_score_residual
        return flashmaxsim_score_residual(self.Q[i], self.codes, self.res, self.centroids, self.weights, self.nbits,
                                          self.offsets, padding="mask", validate=validate)

    def step(self, timer):
        for i in range(self.nQ):
            s = timer(lambda: self._score(i))
            self.scores[i].copy_(s)
        return topk_rows(self.scores, self.k)

    def bytes_per_launch(self):  # the compressed index streamed once, plus the centroid table once
        return (self.Nq * self.d * 2 + self.T * (4 + self.rb) + (self.B + 1) * 8 + self.B * 4
                + self.ncent * self.d * 2)

    def unfused_ms(self):
        """The unfused flow for comparison (outside the timed steps): decompress the whole
        index into fp16 tokens in HBM, then varlen MaxSim over them, for one query."""
        from tilemaxsim_amd import decompress_residual, flash_maxsim_multi_doc
        torch = self.torch
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        D = decompress_residual(self.codes, self.res, self.centroids, self.weights, self.nbits)
        flash_maxsim_multi_doc(self.Q[0], D, self.offsets, validate=False)
        e1.record()
        torch.cuda.synchronize()
        del D
        return e0.elapsed_time(e1)

    def config(self):
        return {"workload": f"c6: residual-compressed c3 corpus, {self.nQ} queries x {self.B:,} docs "
                            f"(Nd~U[{self.lo},{self.hi}], {self.T:,} tokens), nbits={self.nbits}, "
                            f"{self.ncent:,} centroids, Nq={self.Nq}, d={self.d}, top-{self.k} per query",
                "queries": self.nQ, "docs": self.B, "tokens": self.T, "Nq": self.Nq, "d": self.d,
                "nbits": self.nbits, "centroids": self.ncent, "top_k": self.k,
                "kernel": "flashmaxsim_score_residual (decode in registers + MFMA)",
                "roofline_bytes": "compressed index bytes (codes + residuals + offsets) + centroid table per launch"}

    def cpu_baseline(self, seconds):
        from oracle import residual_oracle as ro
        n = min(self.B, CPU_PREFIX_DOCS)
        offs = self.offsets[: n + 1].cpu().numpy()
        t = int(offs[-1])
        Q = self.Q[0].cpu().numpy()
        codes, res = self.codes[:t].cpu().numpy(), self.res[:t].cpu().numpy()
        C, w = self.centroids.cpu().numpy(), self.weights.cpu().numpy()

        def score(b0, b1):
            t0, t1 = int(offs[b0]), int(offs[b1])
            return ro.maxsim_residual_f32(Q, codes[t0:t1], res[t0:t1], C, w, self.nbits, offs[b0:b1 + 1] - t0)

        return _time_cpu_prefix(score, n, self.B, seconds, "query 0, numpy decompress (restated codec) then fp32 "
                                "varlen MaxSim", codes.nbytes + res.nbytes, torch_threads=False)


class ResidualBatched(Residual):
    """c6's index and queries, all queries scored by one batched call
    (flashmaxsim_score_residual_batched): each 16-token tile is decoded once per pass and
    shared through LDS by 32 query blocks, which moves the path to the MFMA roof."""
    kernel = "residual_batched_kernel"
    MFMA_PEAK_TFLOPS = 2500.0
    launch_desc = "one flashmaxsim_score_residual_batched call (one kernel per 32 query blocks)"
    unfused_key = "per_query_fused_all_queries_ms"

    def __init__(self, *args, **kw):
        super().__init__(*args, **kw)
        self.name = "c6b"

    def step(self, timer):
        from tilemaxsim_amd import flashmaxsim_score_residual_batched
        s = timer(lambda: flashmaxsim_score_residual_batched(self.Q, self.codes, self.res, self.centroids,
                                                             self.weights, self.nbits, self.offsets, padding="mask",
                                                             validate=False))
        self.scores.copy_(s)
        return topk_rows(self.scores, self.k)

    def flops_per_launch(self):
        return 2 * self.nQ * self.Nq * self.T * self.d

    def bytes_per_launch(self):  # the compressed index and the centroid table once for all queries
        return (self.nQ * self.Nq * self.d * 2 + self.T * (4 + self.rb) + (self.B + 1) * 8
                + self.nQ * self.B * 4 + self.ncent * self.d * 2)

    def extra_roofline(self, launch_ms):
        return gemm_ceiling(self.torch, self.flops_per_launch() / (launch_ms * 1e-3) / 1e12)

    def unfused_ms(self):
        """The per-query fused kernel over the same index, for comparison (outside the
        timed steps): one flashmaxsim_score_residual call per query, all queries."""
        torch = self.torch
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(self.nQ):
            self._score(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    def config(self):
        c = super().config()
        c["workload"] = c["workload"].replace("c6:", "c6b:", 1) + " (batched-query kernel)"
        c["kernel"] = "flashmaxsim_score_residual_batched (tile decoded once into LDS, shared by 32 query blocks)"
        return c


class PQ:
    kernel = "pq_mfma_score_kernel"

    def __init__(self, torch, n_queries, B, Nd, M=16, K=256, dsub=8, Nq=32, topk=100):
        self.torch, self.nQ, self.B, self.Nd, self.M, self.K, self.dsub, self.Nq, self.k = (
            torch, n_queries, B, Nd, M, K, dsub, Nq, topk)
        gen = torch.Generator(device="cuda").manual_seed(99)
        log(f"[bench] generating {B} docs x {Nd} x {M} uint8 codes ({B * Nd * M / 1e9:.2f} GB)")
        self.codes = torch.randint(0, K, (B, Nd, M), dtype=torch.uint8, device="cuda", generator=gen)
        self.codebook = torch.randn(M, K, dsub, device="cuda", generator=gen).half()
        self.Q = normalized_fp16(torch, (n_queries, Nq, M * dsub), gen)
        self.scores = torch.empty(n_queries, B, dtype=torch.float32, device="cuda")
        from tilemaxsim_amd import TileMaxSimPQ
        self.pq = TileMaxSimPQ(self.codebook)

    def step(self, timer):
        for i in range(self.nQ):
            s = timer(lambda: self.pq.score_batch(self.Q[i], self.codes, validate=False))
            self.scores[i].copy_(s)
        return topk_rows(self.scores, self.k)

    def bytes_per_launch(self):
        return self.B * self.Nd * self.M  # code bytes: the north-star roofline for PQ

    def extra_roofline(self, launch_ms):
        """Beside the code-bytes roofline: the reference's own PQ IO formula
        (src/benchmark.py:226: table + codes + output), the LDS rate of this kernel's
        codebook gather (16 B per code per token) against the LDS peak for
        ds_read_b128 (256 B/clk/CU x 256 CUs at 2.4 GHz = 157.3 TB/s: a conflict-free
        wave-instruction of 1 KiB takes 4 LDS cycles, tms_lds_probe pattern 0) and
        against the PQ gather pattern's own ceiling at that clock (12 LDS cycles per
        wave-instruction, pattern 1: 52.4 TB/s), and the MFMA rate of scoring the decoded
        tokens beside an fp16 GEMM measured in the same process."""
        ref_bytes = self.Nq * self.M * self.K * 4 + self.B * self.Nd * self.M + self.B * self.Nq * 4
        lds_bytes = self.B * self.Nd * self.M * 16
        lds_tbs = lds_bytes / (launch_ms * 1e-3) / 1e12
        # the decoded tokens are scored on MFMA: 2 Nq d flops per token, as dense MaxSim
        flops = 2 * self.Nq * self.M * self.dsub * self.B * self.Nd
        mfma_tf = flops / (launch_ms * 1e-3) / 1e12
        out = {"bytes_reference_formula": ref_bytes,
               "gbs_reference_formula": round(ref_bytes / (launch_ms * 1e-3) / 1e9, 1),
               "lds_gather_bytes_per_launch": lds_bytes, "lds_gather_tbs": round(lds_tbs, 2),
               "lds_peak_tbs": 157.3, "lds_frac": round(lds_tbs / 157.3, 4),
               "lds_pq_pattern_ceiling_tbs": 52.4, "lds_frac_of_pattern_ceiling": round(lds_tbs / 52.4, 4),
               "mfma_flops_per_launch": flops, "mfma_tflops": round(mfma_tf, 1)}
        out.update(gemm_ceiling(self.torch, mfma_tf))
        out.update(self.table_gather_line())
        return out

    def table_gather_line(self, calls=2):
        """The reference's algorithm on the same data, after the timed steps: build the
        (Nq, M, K) fp32 distance table and gather from it (TileMaxSimPQ.score_batch with
        method="lut"), HIP events around each call."""
        torch = self.torch
        f = lambda: self.pq.score_batch(self.Q[0], self.codes, method="lut", validate=False)
        f()
        ts = []
        for _ in range(calls):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            f()
            e1.record()
            ts.append((e0, e1))
        torch.cuda.synchronize()
        ms = float(np.mean([a.elapsed_time(b) for a, b in ts]))
        code_bytes = self.B * self.Nd * self.M
        return {"table_gather_ms": round(ms, 3), "table_gather_docs_per_s": round(self.B / (ms * 1e-3), 1),
                "table_gather_code_gbs": round(code_bytes / (ms * 1e-3) / 1e9, 1),
                "table_gather_note": "the reference's algorithm (fp32 distance table in LDS, gathered per code) on "
                                     "the same query and codes, one call per query"}

    def pairs_per_step(self):
        return self.nQ * self.B

    def config(self):
        return {"workload": f"c5: PQ/ADC, {self.nQ} queries x {self.B:,} docs x Nd={self.Nd}, M={self.M}, K={self.K}, "
                            f"dsub={self.dsub}, uint8 codes, fp16 codebook, top-{self.k} per query",
                "queries": self.nQ, "docs": self.B, "Nq": self.Nq, "Nd": self.Nd, "M": self.M, "K": self.K,
                "dsub": self.dsub, "top_k": self.k,
                "kernel": "TileMaxSimPQ.score_batch (codebook gather in LDS + MFMA)",
                "roofline_bytes": "code bytes B*Nd*M per launch"}

    def cpu_baseline(self, seconds):
        from oracle import maxsim_oracle as orc
        from oracle import torch_ref as tr
        n = min(self.B, 5 * CPU_PREFIX_DOCS)  # 205 MB of codes; each chunk decodes to 33 MB of fp32
        Qt, Ct, codes_t = self.Q[0].cpu(), self.codebook.cpu(), self.codes[:n].cpu()
        nbytes = codes_t.numel()
        base = _time_cpu_prefix(lambda b0, b1: tr.pq_decompress_score(Qt, Ct, codes_t[b0:b1], chunk=500), n, self.B,
                                seconds, "query 0, torch fp32 decompress per subspace then einsum -> max -> sum "
                                "(pytorch_pqsim_baseline)", nbytes)
        Q, C, codes = Qt.numpy(), Ct.numpy(), codes_t.numpy()
        base["numpy_port"] = _time_cpu_prefix(lambda b0, b1: orc.pq_decompress_score(Q, C, codes[b0:b1], chunk=500),
                                              n, self.B, seconds / 2, "query 0, numpy decompress-then-score",
                                              nbytes, torch_threads=False)
        return base


class PQBatched(PQ):
    """c5's codes and queries, all queries scored by one batched call
    (TileMaxSimPQ.score_batch_queries): each tile of codes is decoded once per pass
    through the codebook in LDS and shared by 32 query blocks, so the decode is paid once
    for all the queries and the call is MFMA-bound."""
    kernel = "batched_tile_kernel"
    MFMA_PEAK_TFLOPS = 2500.0
    launch_desc = "one TileMaxSimPQ.score_batch_queries call (one kernel per 32 query blocks)"

    def step(self, timer):
        s = timer(lambda: self.pq.score_batch_queries(self.Q, self.codes, validate=False))
        self.scores.copy_(s)
        return topk_rows(self.scores, self.k)

    def flops_per_launch(self):
        return 2 * self.nQ * self.Nq * self.M * self.dsub * self.B * self.Nd

    def bytes_per_launch(self):  # the codes once for all queries
        return self.nQ * self.Nq * self.M * self.dsub * 2 + self.B * self.Nd * self.M + self.nQ * self.B * 4

    def extra_roofline(self, launch_ms):
        """The north-star view per query: code bytes scored per second for each query
        (nQ passes' worth of codes in one call) against the 8 TB/s HBM peak, and the MFMA
        rate beside an fp16 GEMM measured in the same process."""
        per_query_gbs = self.nQ * self.B * self.Nd * self.M / (launch_ms * 1e-3) / 1e9
        out = {"code_bytes_per_query_gbs": round(per_query_gbs, 1),
               "code_bytes_per_query_frac_of_hbm": round(per_query_gbs / HBM_PEAK_GBS, 4)}
        out.update(gemm_ceiling(self.torch, self.flops_per_launch() / (launch_ms * 1e-3) / 1e12))
        return out

    def config(self):
        c = super().config()
        c["workload"] = c["workload"].replace("c5:", "c5b:", 1) + " (batched-query kernel)"
        c["kernel"] = "TileMaxSimPQ.score_batch_queries (tiles decoded once into LDS, shared by 32 query blocks)"
        return c


class Copy:
    """Plain device-to-device copy of a known size (torch's copy kernel): the reference
    point that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes."""
    kernel = "copy"

    def __init__(self, torch, nbytes=4 << 30):
        self.torch, self.n = torch, nbytes
        self.src = torch.ones(nbytes // 2, dtype=torch.float16, device="cuda")
        self.dst = torch.empty_like(self.src)

    def step(self, timer):
        timer(lambda: self.dst.copy_(self.src))

    def bytes_per_launch(self):
        return 2 * self.n  # read + write

    def pairs_per_step(self):
        return 0

    def config(self):
        return {"workload": f"copy: {self.n} bytes device to device (rocprof counter calibration)"}

    def cpu_baseline(self, seconds):
        return None


class TopK:
    """Top-100 of every row of C2's score matrix (64 queries x 1M documents, MaxSim-like
    scores 10 + 0.5 N(0, 1), fp32) with tms_topk: the step the reference takes with
    torch.topk after scoring (src/cycle3_experiments.py:215). HIP events time each whole
    call (every level of the tournament); the extra rows time other row shapes the same
    way, each checked against torch.topk on the GPU."""
    kernel = "topk_level_kernel"
    dtype = "fp32"
    SHAPES = [(32, 5_000_000, 100), (1, 1000, 100), (1, 256, 100), (1, 128, 100)]

    def __init__(self, torch, rows=64, n=1_000_000, k=100):
        self.torch, self.rows, self.n, self.k = torch, rows, n, k
        self.gen = torch.Generator(device="cuda").manual_seed(7)
        self.scores = 10 + 0.5 * torch.randn(rows, n, device="cuda", generator=self.gen)

    def step(self, timer):
        from tilemaxsim_amd import topk
        return timer(lambda: topk(self.scores, self.k))

    def bytes_per_launch(self):
        return self.rows * self.n * 4

    def pairs_per_step(self):
        return self.rows * self.n

    def config(self):
        return {"workload": f"topk: top-{self.k} of each row of a ({self.rows}, {self.n:,}) fp32 score matrix "
                            "(C2's scores, MaxSim-like values)", "rows": self.rows, "n": self.n, "k": self.k}

    def cpu_baseline(self, seconds):
        return None

    def extra_roofline(self, k_mean):
        from tilemaxsim_amd import topk
        torch = self.torch
        v, i = topk(self.scores, self.k)
        ref = torch.topk(self.scores, self.k)
        out = {"matches_torch_topk": bool(torch.equal(v, ref.values) and torch.equal(i, ref.indices)), "rows": []}
        for rows, n, k in self.SHAPES:
            s = 10 + 0.5 * torch.randn(rows, n, device="cuda", generator=self.gen)
            reps = 200 if rows * n < 1_000_000 else 10
            for _ in range(5):
                v, i = topk(s, k)
            ev = []
            for _ in range(reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                v, i = topk(s, k)
                e1.record()
                ev.append((e0, e1))
            torch.cuda.synchronize()
            ms = sorted(a.elapsed_time(b) for a, b in ev)
            ref = torch.topk(s, k)
            out["rows"].append({"rows": rows, "n": n, "k": k, "ms_p50": round(ms[len(ms) // 2], 4),
                                "gbs": round(rows * n * 4 / (ms[len(ms) // 2] * 1e-3) / 1e9, 1),
                                "matches_torch_topk": bool(torch.equal(v, ref.values) and torch.equal(i, ref.indices))})
            del s
        return out


class ReadProbe:
    """A read-only streaming kernel (tms_read_probe: 8 KiB per wave-iteration, persistent
    XCD-grouped grid) over a C2-sized 46.08 GB buffer: the rate at which this part
    delivers a document stream to any kernel, against which the scoring kernels'
    fractions of the 8 TB/s spec are read."""
    kernel = "read_probe_kernel"

    def __init__(self, torch, nbytes=46_080_000_000):
        from tilemaxsim_amd import _lib
        self.torch, self.n, self.lib = torch, nbytes, _lib.load()
        self.buf = torch.ones(nbytes, dtype=torch.uint8, device="cuda")
        self.sink = torch.empty(_lib.TMS_READ_PROBE_SINK_WORDS, dtype=torch.int32, device="cuda")
        self.check = _lib.check

    def step(self, timer):
        stream = self.torch.cuda.current_stream().cuda_stream
        timer(lambda: self.check(self.lib.tms_read_probe(self.buf.data_ptr(), self.n, self.sink.data_ptr(),
                                                         self.sink.numel(), stream)))

    def bytes_per_launch(self):
        return self.n

    def pairs_per_step(self):
        return 0

    def config(self):
        return {"workload": f"readprobe: {self.n} bytes read once per launch (C2's corpus size), no writes "
                            "beyond one word per thread"}

    def cpu_baseline(self, seconds):
        return None


class LdsProbe:
    """LDS gather probe (tms_lds_probe): the cost of a ds_read_b128 wave-instruction when
    lane l hits bank group l % 16 (pattern 0), when the 16 lanes of an MFMA lane group
    read random rows of one codebook subspace as the PQ kernel's gathers do (pattern 1,
    the timed one), when they all hit one bank group (pattern 2), and when each bank
    group gets four lanes of every 16 (pattern 3); patterns 4 to 7 repeat them at the PQ
    kernel's occupancy and footprint (two 8-wave workgroups per CU, 64 KiB each), patterns
    8 and 9 repeat 5 and 4 with the PQ kernel's matrix work beside the gathers (two MFMAs
    per gathered fragment, random fp16 data), and patterns 10 and 11 tell the part's pass
    rule (four passes of the 16 lanes that share lane bit 5 and the parity of lane bits
    2-4) from passes of 16 consecutive lanes. ``--lds-pattern`` times one pattern alone
    (for counter runs). LDS bytes, not HBM bytes."""
    kernel = "lds_probe_kernel"
    _P = {0: "conflict-free (lane l -> bank group l % 16, random rows)",
          1: "PQ codebook gather (one subspace per 16-lane group, random codes)",
          2: "one bank group per 16-lane group, random rows",
          3: "lane l -> bank group (l / 4) % 16: balanced over the wave, 4-way in every pass"}
    PATTERNS = {**{p: f"{w}; one 16-wave workgroup per CU, 128 KiB" for p, w in _P.items()},
                **{p + 4: f"{w}; two 8-wave workgroups per CU, 64 KiB each (the PQ kernel's shape)"
                   for p, w in _P.items()},
                8: f"{_P[1]}; the PQ kernel's shape, two MFMAs per gathered fragment",
                9: f"{_P[0]}; the PQ kernel's shape, two MFMAs per gathered fragment",
                10: "lane l -> bank group l % 8 + 8 * bit 4 of l: conflict-free by the pass rule, 2-way in passes "
                    "of 16 consecutive lanes; one 16-wave workgroup per CU, 128 KiB",
                11: "lane l -> bank group l % 8 + 8 * parity of bits 2-4 of l: 2-way by the pass rule, "
                    "conflict-free in passes of 16 consecutive lanes; one 16-wave workgroup per CU, 128 KiB"}

    def __init__(self, torch, pattern=None):
        self.pattern = pattern
        from tilemaxsim_amd import _lib
        self.torch, self.lib, self.check = torch, _lib.load(), _lib.check
        self.nw = _lib.TMS_LDS_PROBE_WAVES
        self.cycles = torch.empty(self.nw, dtype=torch.int64, device="cuda")
        self.sink = torch.empty(self.nw * 64, dtype=torch.int32, device="cuda")
        self.instr_per_wave = 4096 * 16

    def run(self, pattern):
        stream = self.torch.cuda.current_stream().cuda_stream
        self.check(self.lib.tms_lds_probe(pattern, self.cycles.data_ptr(), self.nw, self.sink.data_ptr(),
                                          self.sink.numel(), stream))

    def step(self, timer):
        timer(lambda: self.run(1 if self.pattern is None else self.pattern))

    def bytes_per_launch(self):
        return self.nw * self.instr_per_wave * 1024  # LDS bytes read by all waves

    def pairs_per_step(self):
        return 0

    def config(self):
        return {"workload": "ldsprobe: 4,096 waves x 65,536 ds_read_b128 per wave, 16 waves per CU (one "
                            "workgroup over 128 KiB, or two over 64 KiB each), six lane -> address patterns, "
                            "and two of them with MFMAs beside the gathers",
                "pattern": self.pattern}

    def cpu_baseline(self, seconds):
        return None

    def extra_roofline(self, k_mean):
        torch = self.torch
        out = {}
        for p, what in self.PATTERNS.items():
            if self.pattern is not None and p != self.pattern:
                continue
            self.run(p)
            ms = []
            for _ in range(5):
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                self.run(p)
                e.record()
                e.synchronize()
                ms.append(s.elapsed_time(e))
            cyc = float(self.cycles.double().mean().item())
            per_instr = cyc / (16 * self.instr_per_wave)  # 16 waves share one CU's LDS
            out[str(p)] = {"pattern": what, "ms": round(float(np.mean(ms)), 4),
                           "s_memtime_cycles_per_wave_instr": round(per_instr, 3),
                           "bytes_per_cycle_per_cu": round(1024 / per_instr, 1)}
        return {"bound": "lds", "peak": None, "frac": None, "unit": "GB/s (LDS reads, all CUs)", "patterns": out}


class MfmaProbe:
    """MFMA probe (tms_mfma_probe): v_mfma_f32_16x16x32_f16 and nothing else, 2 waves per
    SIMD, on random fp16 operands: the sustained MFMA rate of this part at the clock it
    holds under that load, the practical ceiling of the shared-tile kernels."""
    kernel = "mfma_probe_kernel"
    MFMA_PEAK_TFLOPS = 2500.0
    launch_desc = "one tms_mfma_probe launch"

    def __init__(self, torch):
        import ctypes
        from tilemaxsim_amd import _lib
        self.torch, self.lib, self.check = torch, _lib.load(), _lib.check
        gen = torch.Generator(device="cuda").manual_seed(5)
        self.ops = (torch.rand(512 * 8, device="cuda", generator=gen) * 2 - 1).half()
        self.sink = torch.empty(_lib.TMS_MFMA_PROBE_SINK_WORDS, dtype=torch.float32, device="cuda")
        self._flops = ctypes.c_int64(0)
        self.run()

    def run(self):
        import ctypes
        stream = self.torch.cuda.current_stream().cuda_stream
        self.check(self.lib.tms_mfma_probe(self.ops.data_ptr(), self.sink.data_ptr(), self.sink.numel(),
                                           ctypes.addressof(self._flops), stream))

    def step(self, timer):
        timer(self.run)

    def flops_per_launch(self):
        return self._flops.value

    def bytes_per_launch(self):
        return 0

    def pairs_per_step(self):
        return 0

    def config(self):
        return {"workload": "mfmaprobe: 512 workgroups x 4 waves, 20,000 x 8 v_mfma_f32_16x16x32_f16 per wave on "
                            "random fp16 operands held in registers"}

    def cpu_baseline(self, seconds):
        return None


def _cpu_model():
    """The host CPU's model name (Linux /proc/cpuinfo), else the architecture."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


CPU_PREFIX_DOCS = 20_000  # documents in a dense CPU-baseline prefix (0.9 GB at C2: far above any host LLC)


def _time_cpu_prefix(score_chunk, n_docs, total_docs, seconds, sample, prefix_bytes, torch_threads=True,
                     chunk=500):
    """Times ``score_chunk(b0, b1)`` over consecutive ``chunk``-document slices of a prefix
    of ``n_docs`` documents, cycling through the prefix until ``seconds`` have passed, on
    every host core. Each slice is scored once per pass and the prefix is larger than the
    host's last-level cache, so every pass reads its documents from DRAM, as a full pass
    over the corpus would; documents are independent, so the rate extrapolates linearly
    to the full corpus (``extrapolated`` unless the prefix is the corpus)."""
    import torch
    threads = os.cpu_count() or 1
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    from threadpoolctl import threadpool_limits
    try:
        with threadpool_limits(limits=threads):
            score_chunk(0, min(chunk, n_docs))  # warm-up
            docs, passes, b0 = 0, 0, 0
            t0 = time.perf_counter()
            while True:
                b1 = min(n_docs, b0 + chunk)
                score_chunk(b0, b1)
                docs += b1 - b0
                b0 = b1
                if b0 >= n_docs:
                    b0, passes = 0, passes + 1
                el = time.perf_counter() - t0
                if el >= seconds and (passes >= 1 or el >= 4 * seconds):
                    break
        used = torch.get_num_threads()
    finally:
        torch.set_num_threads(prev)
    out = {"value": docs / el, "unit": "docs/s (1 query)", "cores": used if torch_threads else threads,
           "kind": "port", "extrapolated": n_docs < total_docs, "prefix_docs": n_docs,
           "prefix_bytes": int(prefix_bytes), "corpus_docs": total_docs,
           "os_cpu_count": os.cpu_count(), "cpu_model": _cpu_model(),
           "sample": f"{sample}: {docs:,} documents ({passes} full passes over a {n_docs:,}-document prefix of "
                     f"{prefix_bytes / 1e6:.0f} MB, {chunk} at a time) in {el:.1f} s"}
    if torch_threads:
        out.update({"impl": f"torch {torch.__version__} (CPU, fp32)", "torch_num_threads": used})
    return out


def _time_torch_cpu(fn, docs_per_call, seconds, sample):
    """Times a torch CPU function on every host core (torch.set_num_threads(os.cpu_count()))."""
    import torch
    threads = os.cpu_count() or 1
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        fn()  # warm-up
        n = 0
        t0 = time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
        used = torch.get_num_threads()
    finally:
        torch.set_num_threads(prev)
    return {"value": docs_per_call * n / el, "unit": "docs/s (1 query)", "cores": used, "kind": "port",
            "impl": f"torch {torch.__version__} (CPU, fp32)", "torch_num_threads": used,
            "os_cpu_count": os.cpu_count(), "cpu_model": _cpu_model(),
            "sample": f"{sample} {n}x in {el:.1f} s"}


def _time_cpu(fn, docs_per_call, seconds, sample):
    """Times a numpy function with its BLAS on every host core."""
    from threadpoolctl import threadpool_limits
    threads = os.cpu_count() or 1
    with threadpool_limits(limits=threads):
        fn()  # warm-up
        n = 0
        t0 = time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
    return {"value": docs_per_call * n / el, "unit": "docs/s (1 query)", "cores": threads, "kind": "port",
            "sample": f"{sample} {n}x in {el:.1f} s; host {_cpu_model()}, os.cpu_count()={os.cpu_count()}, "
                      f"{threads} threads"}


def _traffic(kernel, config):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if present."""
    path = os.path.join(HERE, "profiles", f"{kernel}_{config}_traffic.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        t = json.load(f)
    return t.get("bytes_per_launch"), os.path.relpath(path, HERE)


def main():
    args = parse()
    tiny = args.config in ("c1", "rerank")  # steps of tens of microseconds: more of them
    if args.steps is None:
        args.steps = 200 if tiny else 5
    if args.warmup is None:
        args.warmup = 20 if tiny else 1
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (got --gpus {args.gpus}); documents shard across GPUs "
              "with no communication besides a top-k merge, which is not part of this build", file=sys.stderr)
        sys.exit(2)
    if args.qdtype and args.config != "c2b":
        print("bench.py: --qdtype applies to --config c2b", file=sys.stderr)
        sys.exit(2)
    if args.dtype != "fp16" and args.config not in ("c1", "rerank", "c2", "c2b", "c4", "prec"):
        print(f"bench.py: --dtype applies to --config c1, rerank, c2, c2b, c4 and prec (got {args.config})",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    import tilemaxsim_amd  # noqa: F401  (fails loudly if libtilemaxsim.so is missing)

    if args.config == "c1":
        wl = Dense(torch, 1, 1000, 128, 128, name="c1", dtype=args.dtype)
    elif args.config == "rerank":
        # the reference's end-to-end reranking call: one query against a chunk of 256
        # candidates zero-padded to 180 tokens (src/e2e_retrieval_quality.py:267-291)
        wl = Dense(torch, 1, 256, 180, 128, name="rerank", dtype=args.dtype)
    elif args.config == "c2":
        wl = Dense(torch, 64, 1_000_000, 180, 128, name="c2", dtype=args.dtype)
    elif args.config == "prec":
        # the reference's precision experiment: 1 query, B = 10K, Nd = 128, d = 128, raw randn
        wl = Dense(torch, 1, 10_000, 128, 128, name="prec", dtype=args.dtype, normalize=False)
    elif args.config == "c2b":
        wl = DenseBatched(torch, 64, 1_000_000, 180, 128, name="c2b", dtype=args.dtype, qdtype=args.qdtype)
    elif args.config == "c3":
        wl = Varlen(torch, 32, 2_000_000, 32, 300, 128)
    elif args.config == "c3b":
        wl = VarlenBatched(torch, 32, 2_000_000, 32, 300, 128)
    elif args.config == "c4":
        wl = Dense(torch, 16, 200_000, 128, args.d, name=f"c4_d{args.d}", dtype=args.dtype)
    elif args.config == "c5":
        wl = PQ(torch, 32, 5_000_000, 128)
    elif args.config == "c5b":
        wl = PQBatched(torch, 32, 5_000_000, 128)
    elif args.config == "c6":
        wl = Residual(torch, 32, 2_000_000, 32, 300, ncent=args.ncent)
    elif args.config == "c6b":
        wl = ResidualBatched(torch, 32, 2_000_000, 32, 300, ncent=args.ncent)
    elif args.config == "readprobe":
        wl = ReadProbe(torch)
    elif args.config == "topk":
        wl = TopK(torch)
    elif args.config == "ldsprobe":
        wl = LdsProbe(torch, args.lds_pattern)
    elif args.config == "mfmaprobe":
        wl = MfmaProbe(torch)
    else:
        wl = Copy(torch)
    torch.cuda.synchronize()

    timer = KernelTimer(torch)
    log(f"[bench] warmup {args.warmup} step(s)")
    for _ in range(args.warmup):
        wl.step(timer)
    torch.cuda.synchronize()
    timer.prepare(args.steps * getattr(wl, "nQ", 1))
    timer.enabled = True
    log(f"[bench] timing {args.steps} step(s)")
    t0 = time.perf_counter()
    for i in range(args.steps):
        wl.step(timer)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = elapsed * 1e3 / args.steps
    k_mean, k_p50, k_n = timer.avg_ms()
    log(f"[bench] {ms_step:.2f} ms/step, kernel mean {k_mean:.4f} ms over {k_n} launches")

    nbytes = wl.bytes_per_launch()
    achieved = nbytes / (k_mean * 1e-3) / 1e9
    tconf = args.config if args.config != "c4" else f"c4_d{args.d}"
    if args.qdtype:  # another kernel instantiation and pass count: its own traffic file
        tconf += f"_q{args.qdtype}"
    traffic, traffic_src = _traffic(wl.kernel, tconf if args.dtype == "fp16" else f"{tconf}_{args.dtype}")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": wl.kernel, "bytes_per_launch": nbytes, "launch_ms_mean": round(k_mean, 5),
                "launch_ms_p50": round(k_p50, 5), "launches": k_n}
    if traffic_src:
        roofline["traffic_source"] = traffic_src
    if hasattr(wl, "flops_per_launch"):  # MFMA-bound path: price the call against dense fp16 MFMA
        tf = wl.flops_per_launch() / (k_mean * 1e-3) / 1e12
        roofline.update({"bound": "mfma", "achieved": round(tf, 1), "peak": wl.MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / wl.MFMA_PEAK_TFLOPS, 4), "flops_per_launch": wl.flops_per_launch(),
                         "launch": wl.launch_desc})

    # GPU-side extra lines first: the CPU baseline's threads can keep the host busy for a
    # while after it returns, which slows a loop of short launches
    batched = wl.batched_line(torch) if hasattr(wl, "batched_line") else None
    graph = wl.graph_line(torch) if hasattr(wl, "graph_line") else None
    one_launch = wl.one_launch_line(torch) if hasattr(wl, "one_launch_line") else None

    cpu = None
    if not args.no_cpu_baseline:
        log(f"[bench] CPU baseline on {os.cpu_count()} threads, ~{1.5 * args.cpu_seconds:.0f} s")
        cpu = wl.cpu_baseline(args.cpu_seconds)
    if hasattr(wl, "extra_roofline"):
        roofline.update(wl.extra_roofline(k_mean))
    if hasattr(wl, "unfused_ms"):  # after the timed steps (c6: needs a decompressed copy of the corpus)
        roofline[wl.unfused_key] = round(wl.unfused_ms(), 3)

    pairs = wl.pairs_per_step()
    out = {
        "metric": METRIC, "value": round(pairs / (ms_step * 1e-3), 1), "unit": "docs/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": getattr(wl, "dtype", "fp16"),
        "data": "synthetic (seeded; no dataset)", "config": wl.config(),
        "hbm_gbs": round(achieved, 1) if roofline["bound"] == "hbm" else None,
        "hbm_pct_of_peak": round(100 * achieved / HBM_PEAK_GBS, 2) if roofline["bound"] == "hbm" else None,
        "roofline": roofline, "cpu_baseline": cpu,
    }
    if batched:  # c2: the same workload through the batched-query path
        out["batched_queries"] = batched
    if graph:  # c1, rerank: the same step replayed from a HIP graph
        out["graph_replay"] = graph
    if one_launch:  # rerank: the same step scored and ranked in one launch
        out["one_launch"] = one_launch
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
