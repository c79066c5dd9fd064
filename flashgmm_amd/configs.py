"""Benchmark configurations and the seeded synthetic-mixture generator.

The five configurations are the diagonal-covariance GMM EM workloads the
benchmark and the parity tests run (N points, K components, d dimensions,
fp32).  Every consumer (GPU path, fp64 oracle, CPU baseline) draws its inputs
from :func:`make_problem`, so all of them see bit-identical fp32 arrays.

Generator (numpy PCG64, ``default_rng(1000 + config_id)``, drawn in fp64 and
cast to fp32 at the end):

1. true means ``mu*_k ~ U[lo, hi]^d``;
2. per-dimension standard deviations ``sigma*_kj`` (uniform, or log-uniform);
3. mixture weights: equal, or ``Dirichlet(alpha)``;
4. labels ``z = rng.choice(K, N_mix, p=w)``;
5. ``X = mu*_z + sigma*_z * standard_normal``;
6. optional uniform outliers (1 % of N in ``[-20, 20]^d``), appended;
7. one ``rng.permutation`` of the rows.

Initial parameters follow the EM driver's convention: ``mu0`` = K distinct
random data points (``rng.choice(N, K, replace=False)``), ``var0 = 1``,
``log_pi0 = -log K``.
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np


@dataclasses.dataclass(frozen=True)
class Config:
    cid: int
    N: int
    K: int
    d: int
    mean_lo: float
    mean_hi: float
    std_kind: str          # "uniform" or "loguniform"
    std_lo: float
    std_hi: float
    dirichlet_alpha: float | None   # None = equal weights
    outlier_frac: float
    iters: int
    note: str

    @property
    def name(self) -> str:
        return f"C{self.cid}"

    def flops_per_iter(self) -> float:
        """Algorithmic flops of one fused EM iteration: three dense
        N x K x d contractions at 4 flops per (n, k, j) each."""
        return 12.0 * self.N * self.K * self.d

    def bytes_per_iter(self) -> float:
        """Algorithmic HBM bytes of one fused EM iteration: X read by both
        passes, the log-normalizer written and read back, and the O(Kd)
        parameters / statistics moved six times."""
        N, K, d = self.N, self.K, self.d
        return 4.0 * (2 * N * d + 2 * N + 6 * K * (2 * d + 1))


CONFIGS = {
    1: Config(1, 4096, 8, 32, -5.0, 5.0, "uniform", 0.5, 1.5, None, 0.0, 20,
              "small CPU-runnable case"),
    2: Config(2, 65536, 256, 128, -5.0, 5.0, "uniform", 0.5, 1.5, 1.0, 0.0, 20,
              "headline shape"),
    3: Config(3, 262144, 128, 64, -3.0, 3.0, "uniform", 0.5, 2.0, None, 0.0, 20,
              "overlapping clusters"),
    4: Config(4, 65536, 1024, 64, -5.0, 5.0, "uniform", 0.5, 1.5, 0.5, 0.0, 20,
              "K >> d"),
    5: Config(5, 1048576, 512, 128, -5.0, 5.0, "loguniform", 0.25, 4.0, 1.0, 0.01, 10,
              "large N with 1% outliers"),
}


def make_problem(cid: int, N: int | None = None):
    """Return ``(X, mu0, var0, log_pi0)`` as C-contiguous fp32 numpy arrays.

    ``N`` overrides the configuration's point count (same generator, same
    seed), used for reduced-size parity cases of the large configurations.
    """
    cfg = CONFIGS[cid]
    n = cfg.N if N is None else int(N)
    K, d = cfg.K, cfg.d
    rng = np.random.default_rng(1000 + cid)
    mu_true = rng.uniform(cfg.mean_lo, cfg.mean_hi, size=(K, d))
    if cfg.std_kind == "loguniform":
        sd = np.exp(rng.uniform(math.log(cfg.std_lo), math.log(cfg.std_hi), size=(K, d)))
    else:
        sd = rng.uniform(cfg.std_lo, cfg.std_hi, size=(K, d))
    if cfg.dirichlet_alpha is None:
        w = np.full(K, 1.0 / K)
    else:
        w = rng.dirichlet(np.full(K, cfg.dirichlet_alpha))
    n_out = int(n * cfg.outlier_frac)
    n_mix = n - n_out
    z = rng.choice(K, size=n_mix, p=w)
    X = mu_true[z] + sd[z] * rng.standard_normal((n_mix, d))
    if n_out:
        X = np.concatenate([X, rng.uniform(-20.0, 20.0, size=(n_out, d))], axis=0)
    X = np.ascontiguousarray(X[rng.permutation(n)], dtype=np.float32)
    idx = rng.choice(n, size=K, replace=False)
    mu0 = np.ascontiguousarray(X[idx])
    var0 = np.ones((K, d), dtype=np.float32)
    log_pi0 = np.full(K, -math.log(K), dtype=np.float32)
    return X, mu0, var0, log_pi0


def make_shape(N: int, K: int, d: int, overlap: bool = False, seed: int = 7):
    """A seeded problem of any shape, for measurements beyond the five
    configurations (same conventions as :func:`make_problem`: C2's mean and
    standard-deviation ranges, equal weights, initial means = K data points,
    unit variances).  ``overlap``: all K true means within 0.02 of one centre
    (per coordinate), so every component lies inside every point's exact
    window -- the sparse variant's worst case, where each point's list
    overflows and the dense fp64 pass takes it."""
    rng = np.random.default_rng(seed)
    if overlap:
        mu_true = rng.uniform(-5.0, 5.0, size=(1, d)) + 0.02 * rng.standard_normal((K, d))
    else:
        mu_true = rng.uniform(-5.0, 5.0, size=(K, d))
    sd = rng.uniform(0.5, 1.5, size=(K, d))
    z = rng.integers(0, K, size=N)
    X = np.ascontiguousarray(mu_true[z] + sd[z] * rng.standard_normal((N, d)), dtype=np.float32)
    idx = rng.choice(N, size=K, replace=False)
    mu0 = np.ascontiguousarray(X[idx])
    var0 = np.ones((K, d), dtype=np.float32)
    log_pi0 = np.full(K, -math.log(K), dtype=np.float32)
    return X, mu0, var0, log_pi0
