"""bench.py's contract without a GPU: the refusal of more than one GPU, the
roofline arithmetic of the dominant kernel, the per-variant arithmetic type,
the committed HBM-traffic lookup and the per-iteration flop and byte counts
(closed forms pinned to the figures of the metric's own table)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from flashgmm_amd.configs import CONFIGS  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_iteration_flops_and_bytes_match_the_metric_table():
    # F = 12 N K d and B = 4 (2Nd + 2N + 6K(2d+1)): C2 25.77 GFLOP / 69.2 MB,
    # C5 824.6 GFLOP / 1085 MB
    assert CONFIGS[2].flops_per_iter() == pytest.approx(25.77e9, rel=1e-3)
    assert CONFIGS[2].bytes_per_iter() == pytest.approx(69.2e6, rel=2e-3)
    assert CONFIGS[5].flops_per_iter() == pytest.approx(824.6e9, rel=1e-3)
    assert CONFIGS[5].bytes_per_iter() == pytest.approx(1085e6, rel=2e-3)


def test_sparse_roofline_prices_algorithmic_flops_at_the_fp32_peak():
    cfg = CONFIGS[2]
    t1 = 80e-6
    r = bench.dominant_roofline(cfg, "sparse", {"pass1": {"ms_avg": t1 * 1e3},
                                                "pass2": {"ms_avg": 1.0}})
    flops = 4.0 * cfg.N * cfg.K * cfg.d
    assert r["kernel"].startswith("pass1") and r["flops_per_launch"] == flops
    assert r["peak"] == pytest.approx(157.3)
    assert r["achieved"] == pytest.approx(flops / t1 / 1e12)
    assert r["frac"] == pytest.approx(flops / t1 / 157.3e12)
    issued = r["issued_bf16_mfma"]
    assert issued["flops_per_launch"] == 3 * flops
    assert issued["frac"] == pytest.approx(3 * flops / t1 / 2.5e15)


def test_dense_roofline_takes_the_slower_pass():
    cfg = CONFIGS[3]
    r = bench.dominant_roofline(cfg, "mfma", {"pass1": {"ms_avg": 0.1}, "pass2": {"ms_avg": 0.3}})
    flops = 8.0 * cfg.N * cfg.K * cfg.d
    assert r["kernel"].startswith("pass2") and r["flops_per_launch"] == flops
    assert r["frac"] == pytest.approx(flops / 0.3e-3 / 157.3e12)
    assert r["frac_at_kernel_precision"] == pytest.approx(flops / 0.3e-3 / bench.pass2_peak())
    r = bench.dominant_roofline(cfg, "mfma", {"pass1": {"ms_avg": 0.4}, "pass2": {"ms_avg": 0.3}})
    assert r["kernel"].startswith("pass1") and r["peak"] == pytest.approx(78.6)


def test_arithmetic_type_names_the_variant():
    assert "bf16x3" in bench.arithmetic_type("sparse")
    assert "f32 matrix-core" in bench.arithmetic_type("x32")
    assert "f32 matrix-core Pass-1" in bench.arithmetic_type("mixed")
    assert bench.arithmetic_type("mfma").startswith("f64 matrix cores")
    assert bench.arithmetic_type("valu") == "f64 (vector ALU)"


def test_traffic_comes_from_the_committed_profile():
    t = bench.measured_traffic(2, "sparse", "pass1 (log-normalizer sweep, ...)")
    assert t is not None and t > 32 * 2**20   # X (32 MiB) is read at least once
    assert bench.measured_traffic(2, "mixed", "pass1 (...)") is None
    assert bench.measured_traffic(4, "sparse", "pass1 (...)") is None
