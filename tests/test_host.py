"""CPU tests of the host layer: the C ABI library loads and exports every declared
symbol, argument errors surface before any HIP call (Python and C side), and the
package has no CPU fallback."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "tilemaxsim.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tms_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from tilemaxsim_amd import _lib
    lib = _lib.load()
    declared = _declared_symbols()
    assert "tms_maxsim_dense" in declared and "tms_pq_score" in declared
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, f"declared in include/tilemaxsim.h but not exported: {missing}"
    bound = set(_lib.SIGNATURES) | {"tms_last_error"}
    assert set(declared) == bound, "ctypes signatures out of sync with the header"
    assert lib.tms_version() >= 100


def _prototypes():
    """name -> (return type, [parameter types]) of every prototype in the header, each
    type reduced to what ctypes passes: 'ptr' for any pointer, else the C type name."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"^\s*#.*$", "", text, flags=re.M)  # preprocessor lines
    protos = {}
    for ret, name, params in re.findall(r"([A-Za-z_][\w\s\*]*?)\s*\b(tms_\w+)\s*\(([^)]*)\)\s*;", text):
        def kind(decl):
            decl = " ".join(decl.split())
            if "*" in decl:
                return "ptr"
            words = [w for w in decl.split() if w != "const"]
            return words[0] if len(words) == 1 else " ".join(words[:-1])
        plist = [p for p in (x.strip() for x in params.split(",")) if p and p != "void"]
        protos[name] = (kind(ret), [kind(p) for p in plist])
    return protos


def test_ctypes_signatures_match_header_prototypes():
    """Arity and integer widths of every ctypes binding equal the header's prototype:
    pointers as c_void_p, int64_t as c_int64, int as c_int, and the return type."""
    from tilemaxsim_amd import _lib
    ctype_of = {"ptr": ctypes.c_void_p, "int64_t": ctypes.c_int64, "int": ctypes.c_int}
    protos = _prototypes()
    assert set(protos) == set(_lib.SIGNATURES) | {"tms_last_error"}
    assert protos["tms_last_error"] == ("ptr", [])
    for name, argtypes in _lib.SIGNATURES.items():
        ret, params = protos[name]
        want = [ctype_of[p] for p in params]
        assert argtypes == want, f"{name}: ctypes {argtypes} != header {params}"
        assert _lib.RESTYPES.get(name, ctypes.c_int) == ctype_of[ret], f"{name}: return type {ret}"
    lib = _lib.load()
    for name, argtypes in _lib.SIGNATURES.items():
        fn = getattr(lib, name)
        assert fn.argtypes == argtypes and fn.restype == _lib.RESTYPES.get(name, ctypes.c_int), name


def test_rerank_limit_sets_and_restores():
    from tilemaxsim_amd import _lib
    lib = _lib.load()
    default = lib.tms_set_rerank_limit(-1)
    assert default == 16384
    with _lib.rerank_limit(0) as prev:
        assert prev == default and lib.tms_set_rerank_limit(-1) == 0
        with _lib.rerank_limit(1 << 40):
            assert lib.tms_set_rerank_limit(-1) == 1 << 40
        assert lib.tms_set_rerank_limit(-1) == 0
    assert lib.tms_set_rerank_limit(-1) == default


def test_library_is_built_for_gfx950():
    from tilemaxsim_amd import _lib
    blob = open(_lib.LIB_PATH, "rb").read()
    assert b"gfx950" in blob


def _c_call(name, *args):
    from tilemaxsim_amd import _lib
    lib = _lib.load()
    rc = getattr(lib, name)(*args)
    return rc, lib.tms_last_error().decode()


def test_c_abi_rejects_bad_arguments_without_touching_the_gpu():
    from tilemaxsim_amd import _lib
    # negative sizes
    rc, msg = _c_call("tms_maxsim_dense", None, -1, 128, None, 10, 5, 0, None, None)
    assert rc == 1 and "negative" in msg
    # unknown dtype
    rc, msg = _c_call("tms_maxsim_dense", None, 32, 128, None, 10, 5, 7, None, None)
    assert rc == 2 and "dtype" in msg
    # NULL output with work to do
    rc, msg = _c_call("tms_maxsim_dense", 16, 32, 128, 16, 10, 5, 0, None, None)
    assert rc == 1 and "out" in msg
    # fp32 (TMS_DTYPE_F32 = 2) passes the dense dtype check and stops at the same NULL output
    rc, msg = _c_call("tms_maxsim_dense", 16, 32, 128, 16, 10, 5, 2, None, None)
    assert rc == 1 and "out" in msg
    # the MFMA PQ scorer takes 16-bit codebooks only: fp32 is refused before any HIP call
    rc, msg = _c_call("tms_pq_score", 16, 32, 16, 16, 256, 8, 2, 16, 10, 5, 16, None)
    assert rc == 2 and "dtype" in msg
    rc, msg = _c_call("tms_pq_score_batched", 16, 2, 32, 16, 16, 256, 8, 2, 16, 10, 5, 16, None)
    assert rc == 2 and "dtype" in msg
    # the LDS probe checks its pattern and buffers before launching
    rc, msg = _c_call("tms_lds_probe", 12, 16, 4096, 16, 4096 * 64, None)
    assert rc == 1 and "pattern" in msg
    rc, msg = _c_call("tms_lds_probe", -1, 16, 4096, 16, 4096 * 64, None)
    assert rc == 1 and "pattern" in msg
    rc, msg = _c_call("tms_lds_probe", 1, 16, 100, 16, 4096 * 64, None)
    assert rc == 1 and "cycles" in msg
    # empty batch: nothing to do, success, no HIP call
    rc, _ = _c_call("tms_maxsim_dense", None, 32, 128, None, 0, 5, 0, None, None)
    assert rc == 0
    # d beyond the supported width
    rc, msg = _c_call("tms_maxsim_dense", 16, 32, 70000, 16, 10, 5, 0, 16, None)
    assert rc == 2 and "65536" in msg
    # varlen without offsets
    rc, msg = _c_call("tms_maxsim_varlen", 16, 32, 128, 16, 100, None, 10, 0, 16, None)
    assert rc == 1 and "offsets" in msg
    # masked without a mask
    rc, msg = _c_call("tms_maxsim_masked", 16, 32, 128, 16, None, 10, 5, 0, 16, None)
    assert rc == 1 and "mask" in msg
    # tms_maxsim_varlen_batched(Qs, nQ, nq, d, D_flat, T, offsets, B, pad_len, dtype, out, stream)
    rc, msg = _c_call("tms_maxsim_varlen_batched", 16, 4, 32, 128, 16, 100, None, 10, 0, 0, 16, None)
    assert rc == 1 and "offsets" in msg and "varlen_batched" in msg
    rc, msg = _c_call("tms_maxsim_varlen_batched", 16, 4, 32, 128, 16, 100, 16, 10, -1, 0, 16, None)
    assert rc == 1 and "pad_len" in msg
    rc, _ = _c_call("tms_maxsim_varlen_batched", 16, 0, 32, 128, 16, 100, 16, 10, 0, 0, None, None)
    assert rc == 0  # no queries
    # PQ: unsupported MFMA shape; fp32 queries with int32 codes (no MFMA form); dtype flags
    rc, msg = _c_call("tms_pq_score", 16, 32, 16, 16, 256, 3, 0, 16, 10, 5, 16, None)
    assert rc == 2 and "tms_pq_score_lut" in msg
    q32_i32 = _lib.TMS_DTYPE_F16 | _lib.TMS_QUERY_F32 | _lib.TMS_CODES_I32
    rc, msg = _c_call("tms_pq_score", 16, 32, 16, 16, 256, 8, q32_i32, 16, 10, 5, 16, None)
    assert rc == 2 and "uint8" in msg
    rc, msg = _c_call("tms_pq_score", 16, 32, 16, 16, 256, 8, 2 | _lib.TMS_CODES_I16, 16, 10, 5, 16, None)
    assert rc == 2 and "dtype 2" in msg  # fp32 codebooks take the table path, whatever the code width
    # tms_pq_score_lut_ex(lut, nq, M, K, codes, code_bytes, B, nd, out, stream)
    rc, msg = _c_call("tms_pq_score_lut_ex", 16, 32, 16, 256, 16, 3, 10, 5, 16, None)
    assert rc == 1 and "code_bytes" in msg
    rc, msg = _c_call("tms_pq_score_lut_ex", 16, 32, 1 << 16, 1 << 16, 16, 4, 10, 5, 16, None)
    assert rc == 2 and "2^31" in msg
    # tms_pq_score_batched(Qs, nQ, nq, codebook, M, K, dsub, dtype, codes, B, nd, out, stream)
    rc, msg = _c_call("tms_pq_score_batched", 16, -2, 32, 16, 16, 256, 8, 0, 16, 10, 5, 16, None)
    assert rc == 1 and "negative" in msg
    rc, msg = _c_call("tms_pq_score_batched", 16, 3, 32, 16, 16, 256, 3, 0, 16, 10, 5, 16, None)
    assert rc == 2 and "tms_pq_score_lut" in msg
    rc, _ = _c_call("tms_pq_score_batched", 16, 0, 32, 16, 16, 256, 8, 0, 16, 10, 5, None, None)
    assert rc == 0  # no queries


def test_topk_workspace_sizes():
    from tilemaxsim_amd import _lib
    lib = _lib.load()
    assert lib.tms_topk_workspace_size(1, 4096, 100) == 0          # one chunk: no workspace
    assert lib.tms_topk_workspace_size(1, 4097, 100) == 2 * 100 * 8  # 2 chunks x k keys
    # 1M: 245 chunks -> 24500 keys -> 6 chunks -> 600 keys; ping-pong buffers, 3 rows
    assert lib.tms_topk_workspace_size(3, 1_000_000, 100) == (24500 + 600) * 3 * 8
    assert lib.tms_topk_workspace_size(1, 10, 11) == 0 and lib.tms_topk_workspace_size(1, 10**6, 2000) == 0
    rc, msg = _c_call("tms_topk", 16, 1, 10, 11, None, 0, 16, 16, None)
    assert rc == 1 and "exceeds" in msg
    rc, msg = _c_call("tms_topk", 16, 1, 10**6, 100, None, 0, 16, 16, None)
    assert rc == 1 and "workspace" in msg


def test_maxsim_topk_c_abi_rejects_bad_arguments():
    # tms_maxsim_topk(Q, nq, d, D, B, nd, dtype, k, scores, out_values, out_indices, counter, stream)
    ok = (16, 32, 128, 16, 10, 5, 0, 3, 16, 16, 16, 16, None)

    def call(**kw):
        names = ["Q", "nq", "d", "D", "B", "nd", "dtype", "k", "scores", "vals", "idx", "counter", "stream"]
        args = dict(zip(names, ok))
        args.update(kw)
        return _c_call("tms_maxsim_topk", *[args[n] for n in names])

    rc, msg = call(nq=-1)
    assert rc == 1 and "negative" in msg
    rc, msg = call(k=11)
    assert rc == 1 and "exceeds" in msg
    rc, msg = call(dtype=2)  # fp32: score, then tms_topk
    assert rc == 2 and "fp16 / bf16" in msg and "tms_topk" in msg
    for bad in (dict(nq=65), dict(d=48), dict(d=160), dict(B=1025, k=3), dict(k=0), dict(B=0, k=0), dict(nq=0)):
        rc, msg = call(**bad)
        assert rc == 2 and "tms_topk" in msg, bad
    rc, msg = call(counter=None)
    assert rc == 1 and "NULL" in msg
    rc, msg = call(Q=24)
    assert rc == 2 and "aligned" in msg
    rc, msg = call(D=40)
    assert rc == 2 and "aligned" in msg


def test_header_constants_match_the_python_mirror():
    """Every #define of include/tilemaxsim.h that _lib.py mirrors has the same value."""
    import re
    from tilemaxsim_amd import _lib
    text = open(os.path.join(REPO, "include", "tilemaxsim.h")).read()
    defines = dict(re.findall(r"^#define (TMS_\w+) (\S+)", text, re.M))
    mirrored = [n for n in defines if hasattr(_lib, n)]
    assert "TMS_MAXSIM_TOPK_COUNTER_WORDS" in mirrored and len(mirrored) >= 3
    for n in mirrored:
        assert int(eval(defines[n].replace("LL", ""))) == getattr(_lib, n), n


def test_one_launch_workgroups_mirror_the_launch():
    """The workgroup count bench.py reports for tms_maxsim_topk is the launch's own: 1, 2
    or 4 waves per document (while B x waves < 2,048 and at most one wave per 16-token
    tile), then 4, 8 or 16 waves a workgroup (the fewest that keep the launch within 256
    workgroups; at most 8 at d = 128 with two query blocks)."""
    from tilemaxsim_amd.topk import ONE_LAUNCH_MAX_TOKENS, _one_launch_workgroups
    assert ONE_LAUNCH_MAX_TOKENS == 163840
    # (B, nd) -> workgroups: 256 x 180 = 12 tiles -> 4 waves each, 1,024 waves, 4 a group;
    # 1,000 x 128 -> 4,000 waves, 16 a group; 1,024 documents stop at 2 waves (2,048
    # waves, 8 a group); 16 x 32 = 2 tiles -> 2 waves; 16-token documents -> 1 wave
    for (B, nd), wg in {(256, 180): 256, (1000, 128): 250, (64, 100): 64, (1024, 300): 256, (16, 32): 8,
                        (1, 1): 1, (7, 16): 2, (5, 0): 2, (300, 64): 150, (512, 32): 256}.items():
        assert _one_launch_workgroups(B, nd) == wg, (B, nd)
        assert _one_launch_workgroups(B, nd) <= 256
    assert _one_launch_workgroups(1000, 128, d=128, nq=64) == 500  # 8 waves a group there


def test_residual_c_abi_rejects_bad_arguments():
    # tms_residual_decompress(codes, residuals, T, centroids, ncent, d, weights, nbits, out, stream)
    rc, msg = _c_call("tms_residual_decompress", 16, 16, 10, 16, 4, 128, 16, 3, 16, None)
    assert rc == 2 and "nbits" in msg
    rc, msg = _c_call("tms_residual_decompress", 16, 16, 10, 16, 4, 256, 16, 2, 16, None)
    assert rc == 2 and "d=256" in msg
    rc, msg = _c_call("tms_residual_decompress", 16, 16, 10, 16, 0, 128, 16, 2, 16, None)
    assert rc == 1 and "centroids" in msg
    rc, msg = _c_call("tms_residual_decompress", 16, 16, 10, 16, 4, 128, None, 2, 16, None)
    assert rc == 1 and "NULL" in msg
    rc, msg = _c_call("tms_residual_decompress", 16, 16, 10, 24, 4, 128, 16, 2, 16, None)
    assert rc == 1 and "aligned" in msg
    rc, _ = _c_call("tms_residual_decompress", None, None, 0, 16, 4, 128, 16, 2, None, None)
    assert rc == 0  # nothing to decompress, no HIP call
    # tms_maxsim_residual(Q, nq, d, centroids, ncent, weights, nbits, codes, residuals, T,
    #                     offsets, ndocs, pids, B, pad_len, out, stream)
    rc, msg = _c_call("tms_maxsim_residual", 16, 32, 128, 16, 4, 16, 2, 16, 16, 10, 16, 3, None, 5, 0, 16, None)
    assert rc == 1 and "ndocs" in msg
    rc, msg = _c_call("tms_maxsim_residual", 16, 32, 128, 16, 4, 16, 2, 16, 16, 10, None, 3, None, 3, 0, 16, None)
    assert rc == 1 and "offsets" in msg
    rc, msg = _c_call("tms_maxsim_residual", 16, 32, 128, 16, 4, 16, 2, 16, 16, 10, 16, 3, None, 3, -1, 16, None)
    assert rc == 1 and "negative" in msg
    rc, _ = _c_call("tms_maxsim_residual", 16, 32, 128, 16, 4, 16, 2, 16, 16, 10, 16, 3, None, 0, 0, None, None)
    assert rc == 0  # no documents to score
    # tms_maxsim_residual_batched(Qs, nQ, nq, d, centroids, ncent, weights, nbits, codes, residuals, T,
    #                             offsets, ndocs, pids, B, pad_len, out, stream)
    rc, msg = _c_call("tms_maxsim_residual_batched", 16, -1, 32, 128, 16, 4, 16, 2, 16, 16, 10, 16, 3, None, 3, 0, 16,
                      None)
    assert rc == 1 and "negative" in msg and "batched" in msg
    rc, msg = _c_call("tms_maxsim_residual_batched", 16, 4, 32, 128, 16, 4, 16, 3, 16, 16, 10, 16, 3, None, 3, 0, 16,
                      None)
    assert rc == 2 and "nbits" in msg
    rc, msg = _c_call("tms_maxsim_residual_batched", 16, 4, 32, 128, 16, 4, 16, 2, 16, 16, 10, 16, 3, None, 5, 0, 16,
                      None)
    assert rc == 1 and "ndocs" in msg
    rc, msg = _c_call("tms_maxsim_residual_batched", 16, 4, 32, 128, 16, 4, 16, 2, 16, 16, 10, None, 3, None, 3, 0,
                      16, None)
    assert rc == 1 and "offsets" in msg
    rc, msg = _c_call("tms_maxsim_residual_batched", 24, 4, 32, 128, 16, 4, 16, 2, 16, 16, 10, 16, 3, None, 3, 0, 16,
                      None)
    assert rc == 1 and "aligned" in msg
    rc, _ = _c_call("tms_maxsim_residual_batched", 16, 0, 32, 128, 16, 4, 16, 2, 16, 16, 10, 16, 3, None, 3, 0, None,
                    None)
    assert rc == 0  # no queries: nothing to do, no HIP call


def test_python_errors_before_device_checks():
    from tilemaxsim_amd import (TileMaxSimPQ, flash_maxsim_multi_doc, flash_maxsim_single,
                                flash_maxsim_v2_multiquery, maxsim_score)
    Q = torch.zeros(32, 128, dtype=torch.float16)
    D = torch.zeros(4, 10, 128, dtype=torch.float16)
    with pytest.raises(TypeError):
        flash_maxsim_v2_multiquery(np.zeros((32, 128)), D)
    with pytest.raises(ValueError):
        flash_maxsim_v2_multiquery(Q, D[0])
    with pytest.raises(AssertionError):
        flash_maxsim_v2_multiquery(Q[:, :64], D)
    with pytest.raises(TypeError):
        flash_maxsim_v2_multiquery(Q, D.double())
    with pytest.raises(ValueError, match="GPU"):
        flash_maxsim_v2_multiquery(Q, D.float())  # float32 documents are taken (on the GPU)
    with pytest.raises(ValueError, match="contiguous"):
        flash_maxsim_v2_multiquery(Q, D.transpose(0, 1))
    with pytest.raises(ValueError, match="GPU"):
        flash_maxsim_v2_multiquery(Q, D)  # CPU tensors: no CPU path
    with pytest.raises(ValueError):
        flash_maxsim_single(Q, D)
    with pytest.raises(TypeError):
        flash_maxsim_multi_doc(Q, D[0], torch.tensor([0.0, 10.0]))
    with pytest.raises(ValueError):
        flash_maxsim_multi_doc(Q, D[0], torch.zeros(2, 2, dtype=torch.int64))
    with pytest.raises(ValueError):
        maxsim_score(Q, D, torch.ones(4, 9, dtype=torch.bool))
    from tilemaxsim_amd import flash_maxsim_multi_doc_batched, flashmaxsim_score_packed_batched
    with pytest.raises(ValueError, match="nQ, Nq, d"):
        flash_maxsim_multi_doc_batched(Q, D[0], torch.tensor([0, 10]))
    with pytest.raises(TypeError):
        flash_maxsim_multi_doc_batched(Q[None], D[0], torch.tensor([0.0, 10.0]))
    with pytest.raises(ValueError, match="GPU"):
        flash_maxsim_multi_doc_batched(Q[None], D[0], torch.tensor([0, 10]))
    with pytest.raises(ValueError, match="padding"):
        flashmaxsim_score_packed_batched(Q[None], D[0], torch.tensor([10]), padding="none")
    with pytest.raises(ValueError):
        TileMaxSimPQ(torch.zeros(16, 256, dtype=torch.float16))
    with pytest.raises(TypeError):
        TileMaxSimPQ(torch.zeros(16, 256, 8, dtype=torch.float64))
    with pytest.raises(ValueError, match="GPU"):
        TileMaxSimPQ(torch.zeros(16, 256, 8))
    with pytest.raises(ValueError, match="GPU"):
        TileMaxSimPQ(torch.zeros(16, 256, 8, dtype=torch.float16))


def test_residual_python_errors_before_device_checks():
    from tilemaxsim_amd import decompress_residual, flashmaxsim_score_residual
    codes = torch.zeros(10, dtype=torch.int32)
    res = torch.zeros(10, 32, dtype=torch.uint8)
    cent = torch.zeros(4, 128, dtype=torch.float16)
    w = torch.zeros(4, dtype=torch.float16)
    with pytest.raises(NotImplementedError, match="nbits"):
        decompress_residual(codes, res, cent, w, 3)
    with pytest.raises(ValueError, match="residual rows"):
        decompress_residual(codes, res[:, :16], cent, w, 2)
    with pytest.raises(ValueError, match="disagree"):
        decompress_residual(codes[:9], res, cent, w, 2)
    with pytest.raises(TypeError, match="uint8"):
        decompress_residual(codes, res.to(torch.int16), cent, w, 2)
    with pytest.raises(TypeError, match="int32 or int64"):
        decompress_residual(codes.float(), res, cent, w, 2)
    with pytest.raises(ValueError, match="2\\*\\*nbits"):
        decompress_residual(codes, res, cent, w[:3], 2)
    with pytest.raises(ValueError, match="GPU"):
        decompress_residual(codes, res, cent, w, 2)  # CPU tensors: no CPU path
    offs = torch.tensor([0, 4, 10])
    with pytest.raises(ValueError, match="padding"):
        flashmaxsim_score_residual(torch.zeros(32, 128), codes, res, cent, w, 2, offs, padding="none")
    with pytest.raises(ValueError, match="GPU"):
        flashmaxsim_score_residual(torch.zeros(32, 128), codes, res, cent, w, 2, offs)
    from tilemaxsim_amd import flashmaxsim_score_residual_batched
    with pytest.raises(ValueError, match="padding"):
        flashmaxsim_score_residual_batched(torch.zeros(2, 32, 128), codes, res, cent, w, 2, offs, padding="pad")
    with pytest.raises(NotImplementedError, match="nbits"):
        flashmaxsim_score_residual_batched(torch.zeros(2, 32, 128), codes, res, cent, w, 3, offs)
    with pytest.raises(ValueError, match="GPU"):
        flashmaxsim_score_residual_batched(torch.zeros(2, 32, 128), codes, res, cent, w, 2, offs)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from tilemaxsim_amd import _lib
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(ImportError, match="no CPU fallback"):
        _lib.load()


def test_product_never_imports_the_oracle():
    pkg = os.path.join(REPO, "tilemaxsim_amd")
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                text = open(os.path.join(root, f)).read()
                assert not re.search(r"^\s*(import|from)\s+oracle\b", text, flags=re.M), f
                assert "maxsim_oracle" not in text and "c_oracle" not in text, f


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus N > 1 exits with status 2 and says why, before
    importing torch or touching a device."""
    import subprocess
    import sys
    res = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 2, (res.returncode, res.stderr)
    assert "one GPU" in res.stderr and res.stdout == ""
    # --dtype only applies to the dense fixed-length configs
    res = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--config", "c5", "--dtype", "fp32"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2 and "--dtype" in res.stderr, (res.returncode, res.stderr)


def test_c_consumer_links_and_gets_error_statuses(tmp_path):
    """tests/c_abi_consumer.c, built with gcc against include/tilemaxsim.h and
    libtilemaxsim.so, calls entry points with invalid arguments from C and checks the
    status codes and tms_last_error(); no call reaches the GPU."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    lib_dir = os.path.join(REPO, "tilemaxsim_amd")
    exe = str(tmp_path / "c_abi_consumer")
    build = subprocess.run([gcc, "-std=c11", "-Wall", "-Werror", "-I", os.path.join(REPO, "include"),
                            os.path.join(REPO, "tests", "c_abi_consumer.c"), "-L", lib_dir, "-ltilemaxsim",
                            f"-Wl,-rpath,{lib_dir}", "-o", exe], capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, (run.returncode, run.stdout, run.stderr)
    assert run.stdout.startswith("ok ")


def test_plaid_config_without_gpus_keeps_host_tensors_and_refuses_them():
    """``config.total_visible_gpus == 0`` (or no config) leaves host tensors where they
    are, and the GPU check refuses them before any HIP call, as without a config."""
    from tilemaxsim_amd import flashmaxsim_score_packed, flashmaxsim_score_packed_batched
    from tilemaxsim_amd.plaid import _to_configured_gpu

    class Config:
        total_visible_gpus = 0

    Q, D, lens = torch.zeros(1, 32, 128), torch.zeros(10, 128), torch.tensor([4, 6])
    assert all(a is b for a, b in zip(_to_configured_gpu(Config(), Q, D, lens), (Q, D, lens)))
    assert all(a is b for a, b in zip(_to_configured_gpu(None, Q, D, lens), (Q, D, lens)))
    for config in (None, Config()):
        with pytest.raises(ValueError, match="GPU"):
            flashmaxsim_score_packed(Q, D, lens, config)
        with pytest.raises(ValueError, match="GPU"):
            flashmaxsim_score_packed_batched(Q, D, lens, config)
