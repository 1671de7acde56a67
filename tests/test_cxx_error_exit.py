"""The C++ entry points (include/kernels.h) keep the reference's error
convention, CUDA_CHECK_LAST (FINAL_CLEAN_CODE/include/common.h:20-30): a
failing call prints "HIP error at <file>:<line> — <message>" to stderr and
exits with EXIT_FAILURE.  The cases use arguments the library rejects on the
host, so no GPU is needed (tests/cxx/error_exit.cpp)."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cxx", "error_exit")

CASES = ["layernorm_forward", "layernorm_backward", "bias_gelu_forward", "residual_add",
         "embedding_backward", "layernorm_forward_save_null"]


@pytest.fixture(scope="module")
def exe():
    if not os.path.exists(EXE):
        subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cxx"), "error_exit"],
                       check=True, capture_output=True)
    return EXE


@pytest.mark.parametrize("case", CASES)
def test_failing_call_prints_and_exits(exe, case):
    r = subprocess.run([exe, case], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1, (r.returncode, r.stdout, r.stderr)  # EXIT_FAILURE
    assert "returned normally" not in r.stdout
    line = r.stderr.strip().splitlines()[-1]
    assert re.fullmatch(r"HIP error at \S+:\d+ — mi_\w+: .+", line), line
