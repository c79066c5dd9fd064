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


def test_sparse_roofline_is_bf16_utilisation():
    """The sparse Pass 1 issues 3 bf16 products per fp32-class product over
    the padded Kp x 2dpb contraction; its fraction is that work against the
    bf16 peak, so it can never exceed 1 for a kernel that really issues it.
    The metric's fp32 framing is kept as a rate and a ratio."""
    cfg = CONFIGS[2]
    t1 = 80e-6
    r = bench.dominant_roofline(cfg, "sparse", {"pass1": {"ms_avg": t1 * 1e3},
                                                "pass2": {"ms_avg": 1.0}})
    issued = 3 * 2 * cfg.N * 256 * 2 * 128
    assert r["kernel"].startswith("pass1") and r["flops_per_launch"] == issued
    assert r["peak"] == pytest.approx(2500.0)
    assert r["frac"] == pytest.approx(issued / t1 / 2.5e15)
    nkd = cfg.N * cfg.K * cfg.d
    assert r["fp32_class_tflops"] == pytest.approx(4 * nkd / t1 / 1e12)
    assert r["t_fp32_roofline_over_t"] == pytest.approx(4 * nkd / 157.3e12 / t1)
    # padding: K = 1000 -> Kp = 1024, d = 100 -> dp = 112 -> dpb = 128
    c = bench.CONFIGS[4].__class__(**{**cfg.__dict__, "K": 1000, "d": 100})
    assert bench.pass_work(c, "sparse", 1)[0] == 3 * 2 * cfg.N * 1024 * 2 * 128


def test_dense_roofline_takes_the_slower_pass():
    cfg = CONFIGS[3]
    r = bench.dominant_roofline(cfg, "mfma", {"pass1": {"ms_avg": 0.1}, "pass2": {"ms_avg": 0.3}})
    N, Kp, dp = cfg.N, 128, 64
    f32, f64 = 2 * N * Kp * dp, 2 * N * Kp * 2 * dp + 2 * N * Kp * dp
    peak = (f32 + f64) / (f32 / 157.3e12 + f64 / 78.6e12)
    assert r["kernel"].startswith("pass2") and r["flops_per_launch"] == f32 + f64
    assert r["peak"] == pytest.approx(peak / 1e12)
    assert r["frac"] == pytest.approx((f32 + f64) / 0.3e-3 / peak)
    r = bench.dominant_roofline(cfg, "mfma", {"pass1": {"ms_avg": 0.4}, "pass2": {"ms_avg": 0.3}})
    assert r["kernel"].startswith("pass1") and r["peak"] == pytest.approx(78.6)
    assert r["flops_per_launch"] == 2 * N * Kp * 2 * dp


def test_work_model_fraction_is_at_most_one_for_feasible_times():
    """The work model prices executed work at the peaks: any measured time
    at or above t_model gives a fraction <= 1."""
    for cid, v, counts in ((2, "sparse", {"entries": 120000, "flagged": 3}), (1, "mfma", {}),
                           (3, "mixed", {}), (1, "valu", {})):
        cfg = CONFIGS[cid]
        m = bench.work_model(cfg, v, 1.0, counts)
        t_model_ms = m["t_model_us"] / 1e3
        assert bench.work_model(cfg, v, t_model_ms, counts)["frac"] == pytest.approx(1.0)
        assert bench.work_model(cfg, v, 2 * t_model_ms, counts)["frac"] == pytest.approx(0.5)
    m = bench.work_model(CONFIGS[2], "sparse", 0.15, {"entries": 120000, "flagged": 0})
    assert m["bf16_sweep_us"] == pytest.approx(3 * 2 * 65536 * 256 * 256 / 2.5e15 * 1e6)
    assert m["hbm_bytes"] == CONFIGS[2].bytes_per_iter() + 24 * 120000


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
    assert bench.measured_traffic(2, "sparse", "pass9 (...)") is None
