"""Runs tests/cxx/threads_test: two host threads call the reducing entry
points of include/kernels.h (layernorm_backward_residual on [8192, 768],
gelu_backward_with_bias_backward on [8192, 3072]) on their own data at the
same time, each on its per-thread default stream, as callers of the
reference's `--default-stream per-thread` build may
(FINAL_CLEAN_CODE/Makefile:33).  Every iteration's dgamma, dbeta and dbias,
and the final grad_residual and grad_in, must equal bit for bit what one
thread alone gets: the library gives each calling thread its own workspace
slot for the per-thread stream.  The program is built by
__graft_entry__.build()."""
import os
import subprocess

import pytest

from gpu_util import note

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cxx", "threads_test")


def test_two_threads_on_per_thread_streams_match_one_thread(dev):
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} is not built: run __graft_entry__.build() first")
    note("cxx threads_test: 2 threads x 40 iterations")
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=100)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "threads_test: OK" in r.stdout
