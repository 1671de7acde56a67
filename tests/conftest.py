"""pytest configuration: the `gpu` marker and import paths.

Tests marked `gpu` need an AMD GPU and the built HIP library; everything else
runs on the CPU (oracle pinning, host logic, ABI export checks).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "cme213-final-project_amd"), os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and libcme213_amd.so")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


# Column sums of the BASELINE configs whose achieved relative error the
# session summary prints: (label, substring of the pytest node id).
COLSUM_CONFIGS = [
    ("config 0 LN [4096,768]", "test_layernorm_forward_backward[4096-768-20260]"),
    ("headline LN [8192,768]", "test_layernorm_forward_backward[8192-768-20261]"),
    ("config 1 GELU [8192,3072]", "test_bias_gelu_forward_backward[8192-3072-20261]"),
    ("config 3 block x2 [8192,768]", "test_block_sequence_chain[8192-768-3072-2-False]"),
    ("config 3 block x12 [1024,768]", "test_block_sequence_chain[1024-768-3072-12-True]"),
    ("config 4 LN [4096,1600]", "test_layernorm_forward_backward[4096-1600-20264]"),
    ("config 4 GELU [4096,6400]", "test_bias_gelu_forward_backward[4096-6400-20264]"),
    ("config 4 block x1 [4096,1600]", "test_block_sequence_chain[4096-1600-6400-1-False]"),
    ("config 4 block x48 [128,1600]", "test_block_sequence_chain[128-1600-6400-48-True]"),
    ("config 4 wide LN [32768,4096]", "test_wide_sweep_config4"),
]


def pytest_terminal_summary(terminalreporter):
    """One line per BASELINE config: the largest |gpu - ref| / |ref| of its
    column sums (dgamma, dbeta, dbias) over the columns that do not cancel
    (|ref| >= ||terms||_2), each asserted <= 1e-4 by tol.colsum_relative."""
    import tol
    if not tol.COLSUM_LOG:
        return
    lines = []
    for label, key in COLSUM_CONFIGS:
        recs = [r for r in tol.COLSUM_LOG if key in r[0]]
        if not recs:
            continue
        worst = max(r[2] for r in recs)
        kept = sum(r[3] for r in recs)
        cols = sum(r[4] for r in recs)
        lines.append(f"  {label}: max rel err {worst:.2e} over {kept} of {cols} columns "
                     f"({len(recs)} sums)")
    if lines:
        terminalreporter.write_line("column sums, non-cancelling columns (|ref| >= ||t||_2), "
                                    "bound 1e-4 relative:")
        for ln in lines:
            terminalreporter.write_line(ln)
