"""A C program scores through the header on the GPU (``tests/c_abi_scoring.c``): it
owns every device buffer, calls tms_maxsim_dense, tms_topk, tms_maxsim_topk,
tms_maxsim_varlen and tms_pq_score on the default stream, and checks each result
against a float64 restatement of its own, to the fp32-accumulation bar (and the top-k,
and the one-launch path's bits, exactly)."""
import os
import shutil
import subprocess

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def test_c_program_scores_through_the_header(cuda, tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    lib_dir = os.path.join(REPO, "tilemaxsim_amd")
    exe = str(tmp_path / "c_abi_scoring")
    build = subprocess.run([gcc, "-std=c11", "-O2", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
                            "-I", os.path.join(REPO, "include"), "-I", os.path.join(ROCM, "include"),
                            os.path.join(REPO, "tests", "c_abi_scoring.c"), "-L", lib_dir, "-ltilemaxsim",
                            "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-lm", f"-Wl,-rpath,{lib_dir}",
                            f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}", "-o", exe], capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(run.stdout, run.stderr, flush=True)
    assert run.returncode == 0, (run.returncode, run.stdout, run.stderr)
    assert run.stdout.strip().endswith("ok")
