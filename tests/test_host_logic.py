"""Host logic that needs no GPU, compiled with g++ under AddressSanitizer and
UBSan (tests/cxx/host_checks.cpp): the unsigned trip count of the row-band and
LayerNorm-backward row loops (csrc/mi_index.hpp) at row counts near INT_MAX,
and the workspace pool (csrc/workspace_pool.hpp) under concurrent growth and
with per-thread slots (the per-thread default stream's keying)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "cme213-final-project_amd", "csrc")
SRC = os.path.join(ROOT, "tests", "cxx", "host_checks.cpp")
INT_MAX = 2**31 - 1


@pytest.fixture(scope="module")
def exe(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    out = str(tmp_path_factory.mktemp("host") / "host_checks")
    subprocess.run([gxx, "-std=c++17", "-O1", "-g", "-pthread", "-fsanitize=address,undefined",
                    "-fno-sanitize-recover=undefined", "-I", CSRC, SRC, "-o", out], check=True)
    return out


def test_trip_count_near_int_max(exe):
    # (first, rows, step): the row-band kernel (first = workgroup, step = 256
    # workgroups) and the LayerNorm backward (first = workgroup * groups,
    # step = 256 workgroups * 8 groups) at row counts within one step of
    # INT_MAX, where rows - first + step - 1 no longer fits an int.
    cases = [(0, INT_MAX - 1, 256), (255, INT_MAX - 1, 256), (2047, INT_MAX - 1, 2048),
             (5, INT_MAX, 2048), (2040, INT_MAX, 2048), (0, INT_MAX, 1), (17, 16, 256),
             (16, 16, 256), (0, 1, 2048), (3, 8192, 2048), (1, INT_MAX - 1, 256),
             (100, INT_MAX - 1, 2048), (0, INT_MAX - 1, 2048)]
    args = [str(v) for c in cases for v in c]
    got = [int(x) for x in subprocess.run([exe, "trips", *args], capture_output=True, text=True,
                                          check=True).stdout.split()]
    want = [-(-(n - f) // s) if f < n else 0 for f, n, s in cases]
    assert got == want
    # the cases that matter are those the 32-bit form overflows on
    assert sum(n - f + s - 1 > INT_MAX for f, n, s in cases) >= 5


def test_workspace_pool_never_frees_a_handed_out_buffer(exe):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0")
    r = subprocess.run([exe, "pool"], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "pool ok" in r.stdout


def test_workspace_pool_per_thread_slots(exe):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0")
    r = subprocess.run([exe, "slots"], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "slots ok: 8 slots" in r.stdout
