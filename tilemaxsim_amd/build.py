"""Build ``libtilemaxsim.so`` (gfx950 HIP kernels + C ABI) in-tree with hipcc.

Usage: ``python -m tilemaxsim_amd.build`` (or ``build()`` from ``__graft_entry__``).
Each ``csrc/*.hip`` file is compiled to an object in ``csrc/_build/`` in parallel,
then linked into ``tilemaxsim_amd/libtilemaxsim.so``.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(CSRC, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libtilemaxsim.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed-FP32 VALU forms stay disabled for all device code on this part.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Embeddings are finite: max/min need no NaN canonicalisation (halves the VALU max work).
    "-fno-honor-nans",
    "-I", os.path.join(REPO_DIR, "include"),
    "-I", CSRC,
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build tilemaxsim_amd)")


def _compile(src: str, obj: str) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{res.stdout}\n{res.stderr}")


def build(verbose: bool = True) -> str:
    """Compile every kernel source for gfx950 and link the shared library. Returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    objs = [os.path.join(BUILD_DIR, os.path.basename(s)[:-4] + ".o") for s in srcs]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(lambda so: _compile(*so), zip(srcs, objs)))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} source(s)", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
