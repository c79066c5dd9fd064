"""Writes the golden fixtures in tests/golden/*.npz.

The reference repository stores no golden vectors for this path, so the
expected values come from an independent implementation of the same
mathematics: scikit-learn's diagonal-covariance GaussianMixture (fp64).
Inputs are fp32 arrays exactly as the HIP path receives them.

Per case the file holds
  inputs   X[N,d], mu[K,d], var[K,d], log_pi[K]                (float32)
  ln       GaussianMixture.score_samples(X)                     (float64)
  gamma    GaussianMixture.predict_proba(X)                     (float64)
  n_k      sklearn _estimate_gaussian_parameters nk - 10*eps   (float64)
  s_k      n_k * means                                          (float64)
  sq_k     gamma^T X^2                                          (float64)
  new_mu, new_var, new_log_pi   M-step with the native clamps applied to
           sklearn's means / covariances (reg_covar = 0)       (float64)

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
from sklearn.mixture import GaussianMixture
from sklearn.mixture._gaussian_mixture import _estimate_gaussian_parameters

HERE = os.path.dirname(os.path.abspath(__file__))


def sk_model(mu, var, log_pi):
    K, d = mu.shape
    gm = GaussianMixture(n_components=K, covariance_type="diag")
    gm.weights_ = np.exp(log_pi.astype(np.float64))
    gm.means_ = mu.astype(np.float64)
    gm.covariances_ = var.astype(np.float64)
    gm.precisions_cholesky_ = 1.0 / np.sqrt(gm.covariances_)
    gm.precisions_ = 1.0 / gm.covariances_
    gm.converged_ = True
    gm.n_iter_ = 0
    return gm


def case(name, X, mu, var, log_pi):
    X, mu, var, log_pi = (np.ascontiguousarray(a, np.float32) for a in (X, mu, var, log_pi))
    gm = sk_model(mu, var, log_pi)
    X64 = X.astype(np.float64)
    ln = gm.score_samples(X64)
    gamma = gm.predict_proba(X64)
    nk, means, covs = _estimate_gaussian_parameters(X64, gamma, 0.0, "diag")
    nk = nk - 10 * np.finfo(np.float64).eps   # sklearn adds 10*eps to nk
    s_k = nk[:, None] * means
    sq_k = gamma.T @ (X64 * X64)
    N = X.shape[0]
    # native clamps (flash_gmm_cuda.cu:310-320) on top of sklearn's estimates
    safe = nk > 1e-8
    new_mu = np.where(safe[:, None], means, s_k / 1e-8)
    new_var = np.maximum(np.where(safe[:, None], covs, sq_k / 1e-8 - new_mu ** 2), 1e-6)
    new_log_pi = np.log(np.maximum(nk / N, 1e-8))
    np.savez(os.path.join(HERE, f"{name}.npz"), X=X, mu=mu, var=var, log_pi=log_pi, ln=ln,
             gamma=gamma, n_k=nk, s_k=s_k, sq_k=sq_k, new_mu=new_mu, new_var=new_var,
             new_log_pi=new_log_pi)
    print(f"{name}: N={N} K={mu.shape[0]} d={mu.shape[1]}  ln[0]={ln[0]:.6f}")


def main():
    rng = np.random.default_rng(7)
    # 1. single component: ln is the diagonal-Gaussian log-pdf plus log pi
    X = rng.normal(1.0, 2.0, (64, 3))
    case("k1_d3", X, np.array([[0.5, -1.0, 2.0]]), np.array([[1.5, 0.25, 4.0]]), np.array([0.0]))
    # 2. small well-separated mixture
    mu = rng.uniform(-5, 5, (4, 8))
    z = rng.integers(0, 4, 200)
    X = mu[z] + rng.normal(0, 1, (200, 8)) * rng.uniform(0.5, 1.5, (4, 8))[z]
    case("k4_d8", X, mu + rng.normal(0, 0.3, mu.shape), rng.uniform(0.5, 2.0, (4, 8)),
         np.log(rng.dirichlet(np.ones(4))))
    # 3. the small benchmark configuration's shape, first 512 points
    import sys
    sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
    from flashgmm_amd.configs import make_problem
    Xc, muc, varc, lpc = make_problem(1)
    case("c1_head512", Xc[:512], muc, varc, lpc)
    # 4. overlapping components with unequal, non-normalised weights
    mu = rng.normal(0, 0.5, (6, 5))
    X = rng.normal(0, 1, (300, 5))
    case("overlap_k6_d5", X, mu, rng.uniform(0.3, 3.0, (6, 5)), rng.normal(-2.0, 0.5, 6))
    # 5. a component nobody belongs to (n_k underflows -> clamps) and a tiny variance
    mu = np.array([[0.0, 0.0], [1e3, 1e3], [0.5, 0.5]])
    X = rng.normal(0, 1, (128, 2))
    case("empty_component", X, mu, np.array([[1.0, 1.0], [1.0, 1.0], [1e-3, 1e-3]]),
         np.log(np.array([0.5, 0.25, 0.25])))
    # 6. ragged sizes: d not a multiple of 4, K not a multiple of 16
    mu = rng.uniform(-3, 3, (17, 33))
    z = rng.integers(0, 17, 333)
    X = mu[z] + rng.normal(0, 1, (333, 33))
    case("ragged_k17_d33", X, mu + rng.normal(0, 0.2, mu.shape), rng.uniform(0.5, 1.5, (17, 33)),
         np.full(17, -np.log(17)))


if __name__ == "__main__":
    main()
