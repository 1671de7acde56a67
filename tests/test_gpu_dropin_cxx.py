"""Runs tests/cxx/dropin_test: a C++ program written against include/kernels.h
(the reference's own kernel signatures, default per-thread stream,
exit-on-error) that replays the reference's test scenarios
(FINAL_CLEAN_CODE/tests/test_layernorm.cu, test_fusion_benchmark.cu's fused
vs unfused pairs, NEW_code/tests/test_embedding.cu) and checks the results
against the CPU oracle.  The program is built by __graft_entry__.build()."""
import os
import subprocess

import pytest

from gpu_util import note

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cxx", "dropin_test")


def test_cxx_dropin_program(dev):
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} is not built: run __graft_entry__.build() first")
    note("cxx dropin_test")
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=90)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASSED (0 failures)" in r.stdout
