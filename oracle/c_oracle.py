"""ctypes binding + build recipe for ``oracle/maxsim_oracle.c`` -- TEST INFRASTRUCTURE ONLY.

``build()`` compiles the C restatement with gcc into ``oracle/_build/libmaxsim_oracle.so``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "maxsim_oracle.c")
LIB = os.path.join(HERE, "_build", "libmaxsim_oracle.so")

_lib = None


def build() -> str:
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    cmd = ["gcc", "-O2", "-std=c11", "-shared", "-fPIC", SRC, "-o", LIB, "-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed:\n{res.stdout}\n{res.stderr}")
    return LIB


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB) or os.path.getmtime(LIB) < os.path.getmtime(SRC):
            build()
        _lib = ctypes.CDLL(LIB)
    return _lib


def _f(x):
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def maxsim_dense(Q, D):
    Q, D = _f(Q), _f(D)
    B, nd, d = D.shape
    out = np.empty(B, np.float64)
    load().orc_maxsim_dense(_p(Q), ctypes.c_int64(Q.shape[0]), ctypes.c_int64(d), _p(D), ctypes.c_int64(B),
                            ctypes.c_int64(nd), _p(out))
    return out


def maxsim_masked(Q, D, mask):
    Q, D = _f(Q), _f(D)
    m = np.ascontiguousarray(np.asarray(mask, dtype=bool).astype(np.uint8))
    B, nd, d = D.shape
    out = np.empty(B, np.float64)
    load().orc_maxsim_masked(_p(Q), ctypes.c_int64(Q.shape[0]), ctypes.c_int64(d), _p(D), _p(m), ctypes.c_int64(B),
                             ctypes.c_int64(nd), _p(out))
    return out


def maxsim_varlen(Q, Dflat, offsets):
    Q, Dflat = _f(Q), _f(Dflat)
    offs = np.ascontiguousarray(np.asarray(offsets, dtype=np.int64))
    B = offs.shape[0] - 1
    out = np.empty(B, np.float64)
    load().orc_maxsim_varlen(_p(Q), ctypes.c_int64(Q.shape[0]), ctypes.c_int64(Q.shape[1]), _p(Dflat), _p(offs),
                             ctypes.c_int64(B), _p(out))
    return out


def pq_build_lut(Q, C):
    Q, C = _f(Q), _f(C)
    M, K, dsub = C.shape
    out = np.empty((Q.shape[0], M, K), np.float64)
    load().orc_pq_build_lut(_p(Q), ctypes.c_int64(Q.shape[0]), _p(C), ctypes.c_int64(M), ctypes.c_int64(K),
                            ctypes.c_int64(dsub), _p(out))
    return out


def pq_score(Q, C, codes):
    Q, C = _f(Q), _f(C)
    c = np.ascontiguousarray(np.asarray(codes, dtype=np.uint8))
    M, K, dsub = C.shape
    B, nd, _ = c.shape
    out = np.empty(B, np.float64)
    load().orc_pq_score(_p(Q), ctypes.c_int64(Q.shape[0]), _p(C), ctypes.c_int64(M), ctypes.c_int64(K),
                        ctypes.c_int64(dsub), _p(c), ctypes.c_int64(B), ctypes.c_int64(nd), _p(out))
    return out
