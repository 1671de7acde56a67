"""CPU checks of bench.py's contract: the algorithmic byte counts behind
`value` and `roofline.achieved`, against per-operation figures worked out
by hand from each benchmark config's interface tensors (read once, written
once, accumulated outputs twice; MB = 1e6 B, two decimals), and the one-GPU
rule (no GPU is touched)."""
import os
import subprocess
import sys

import pytest

from cme213_amd import workloads as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def mb(b):
    return round(b / 1e6, 2)


def test_headline_bytes_match_the_stated_figures():
    b = W.headline_bytes()
    assert {k: mb(v) for k, v in b.items()} == {"ln_fwd": 50.40, "ln_bwd": 75.57,
                                                "gelu_fwd": 201.34, "gelu_bwd": 302.01}
    assert sum(b.values()) == 629_328_896
    # 70% of 8 TB/s, the north-star bar, is 112.4 us per step
    assert round(sum(b.values()) / (0.7 * 8e12) * 1e6, 1) == 112.4


def test_config_bytes_match_the_stated_figures():
    # config 0: LN fwd + bwd at [4096, 768]
    assert (mb(W.ln_fwd_bytes(4096, 768)), mb(W.ln_bwd_bytes(4096, 768))) == (25.20, 37.79)
    assert mb(W.ln_fwd_bytes(4096, 768) + W.ln_bwd_bytes(4096, 768)) == 63.00
    # config 1: bias+GELU fwd + bwd at [8192, 3072]
    assert (mb(W.gelu_fwd_bytes(8192, 3072)), mb(W.gelu_bwd_bytes(8192, 3072))) == (201.34, 302.01)
    # config 3, one layer: residual+LN twice and bias+GELU forward; GELU backward and the
    # residual LN backward twice
    R, C, F = 8192, 768, 3072
    fwd = 2 * W.res_ln_fwd_bytes(R, C) + W.gelu_fwd_bytes(R, F)
    bwd = W.gelu_bwd_bytes(R, F) + 2 * W.ln_bwd_residual_bytes(R, C)
    assert (mb(fwd), mb(bwd)) == (402.81, 503.49)
    assert round(12 * (fwd + bwd) / 1e9, 3) == 10.876
    # the wide sweep of config 4: LN fwd 1.074 GB, bwd 1.611 GB at [32768, 4096]
    assert (round(W.ln_fwd_bytes(32768, 4096) / 1e9, 3),
            round(W.ln_bwd_bytes(32768, 4096) / 1e9, 3)) == (1.074, 1.611)


def test_more_than_one_gpu_is_refused_before_any_gpu_call():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2, (r.returncode, r.stdout, r.stderr)
    assert r.stdout == ""  # no JSON line
    assert "one GPU" in r.stderr


def test_config_block_records_a_failed_config_and_keeps_the_others(monkeypatch):
    # bench.config_suite runs each config's own bench.py command; a stand-in
    # for subprocess.run fails one of them and answers the others, so no GPU
    # is touched: the failure is recorded, the other configs are reported.
    import json
    import types

    sys.path.insert(0, ROOT)
    import bench

    def fake_run(cmd, capture_output, text, timeout):
        name = cmd[cmd.index("--workload") + 1]
        if name == "block12":
            return types.SimpleNamespace(returncode=1, stdout="", stderr="boom")
        line = {"ms_per_step": 0.02, "config": {"bytes_per_step": 100_000_000}}
        return types.SimpleNamespace(returncode=0, stdout=json.dumps(line) + "\n", stderr="")

    monkeypatch.setattr(subprocess, "run", fake_run)
    out = bench.config_suite(400.0)
    assert set(out) == {k for k, *_ in bench.CONFIG_SUITE}
    assert "error" in out["config3_block12"] and "boom" in out["config3_block12"]["error"]
    ok = out["config0_ln"]
    assert ok["us_per_step"] == 20.0 and ok["gbs"] == 5000.0 and ok["pct_of_peak"] == 62.5
    assert ok["meets_target"] is False  # 20 us against 11.3 us
    assert out["config2_embedding"]["meets_target"] is None  # BASELINE.md states no target
