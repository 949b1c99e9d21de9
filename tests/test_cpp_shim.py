"""The C++ shim include/clove/gemm.h used the way the reference's C++ callers
use its API: tests/cpp/test_gemm_shim.cpp runs the six GEMM cases of the
reference's test program (tests/test_gemm.cu:99-243) with the reference's own
comparison rule, plus INT8, INT4 (both modes), batched, SwiGLU and the INT4
MLP calls, against the oracle.  Built by __graft_entry__.build() (tests/cpp/Makefile).
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_gemm_shim")


def test_shim_program_built_and_linked():
    # the C++ spelling of the API compiles against the headers and links
    # against the library (no GPU needed)
    assert os.path.isfile(BIN), "run __graft_entry__.build() first"
    out = subprocess.run(["ldd", BIN], capture_output=True, text=True, check=True).stdout
    assert "libclove_gemm.so" in out and "not found" not in out


@pytest.mark.gpu
def test_shim_cases_on_gpu():
    print("running", BIN, flush=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all cases passed" in r.stdout
