"""EM drivers with the reference's Python API (``flash_gmm/native_wrapper.py``).

``NativeStandardGMM`` and ``NativeFlashGMM`` keep the reference's
constructors, initialisation, loop, early-stop rule and ``history`` records
(``native_wrapper.py:47-148``): ``log_likelihood`` of iteration ``it`` is the
mean log-normalizer under the parameters entering that iteration.
``NativeFlashGMM.fit_device`` runs the same iterations with ``tol = 0``
entirely on the device (one host synchronisation at the end);
``predict_proba`` / ``predict`` follow ``FlashGMM``'s
(``flash_gmm/flash_gmm.py:185-193``) on the gamma-returning flash E-step.
"""
from __future__ import annotations

import time

import torch

from . import flash_gmm_native as _C


def _init_params(K: int, d: int, seed: int, X: torch.Tensor):
    """native_wrapper.py:115-121: K random points, variance = mean of the
    per-dimension data variances, uniform weights."""
    N = X.shape[0]
    gen = torch.Generator(device=X.device).manual_seed(seed)
    idx = torch.randperm(N, generator=gen, device=X.device)[:K]
    mu = X[idx].clone()
    var = torch.ones(K, d, device=X.device) * X.var(dim=0, keepdim=True).mean()
    log_pi = torch.full((K,), -torch.log(torch.tensor(float(K))), device=X.device)
    return mu, var, log_pi


class NativeStandardGMM:
    """Standard EM on the HIP kernels: the E-step materialises the N x K
    log-density matrix and gamma, the M-step reads gamma back
    (``native_wrapper.py:47-96``)."""

    def __init__(self, K: int, d: int, max_iter: int = 100, tol: float = 1e-4, seed: int = 42):
        self.K = K
        self.d = d
        self.max_iter = max_iter
        self.tol = tol
        self.seed = seed
        self.mu = None
        self.var = None
        self.log_pi = None

    def _init_params(self, X: torch.Tensor):
        self.mu, self.var, self.log_pi = _init_params(self.K, self.d, self.seed, X)

    def fit(self, X: torch.Tensor, verbose: bool = False):
        self._init_params(X)
        prev_ll = -float("inf")
        history = []
        for it in range(self.max_iter):
            t0 = time.time()
            gamma, log_norm = _C.standard_e_step(X, self.mu, self.var, self.log_pi)
            avg_ll = log_norm.mean().item()
            self.mu, self.var, self.log_pi = _C.standard_m_step(X, gamma)
            elapsed = time.time() - t0
            history.append({"iter": it, "log_likelihood": avg_ll, "time_ms": elapsed * 1000})
            if verbose and (it % 10 == 0 or it < 5):
                print(f"  iter {it:3d}: LL={avg_ll:.4f}  time={elapsed*1000:.1f}ms")
            if abs(avg_ll - prev_ll) < self.tol:
                if verbose:
                    print(f"  Converged at iter {it}")
                break
            prev_ll = avg_ll
        return history

    def predict_proba(self, X: torch.Tensor) -> torch.Tensor:
        return _C.standard_e_step(X, self.mu, self.var, self.log_pi)[0]

    def predict(self, X: torch.Tensor) -> torch.Tensor:
        return self.predict_proba(X).argmax(dim=1)


class NativeFlashGMM:
    """Flash-GMM EM on the HIP kernels (no N x K array is materialised)."""

    def __init__(self, K: int, d: int, BN: int = 64, BK: int = 8,
                 max_iter: int = 100, tol: float = 1e-4, seed: int = 42):
        self.K = K
        self.d = d
        self.BN = BN
        self.BK = BK
        self.max_iter = max_iter
        self.tol = tol
        self.seed = seed
        self.mu = None
        self.var = None
        self.log_pi = None

    def _init_params(self, X: torch.Tensor):
        self.mu, self.var, self.log_pi = _init_params(self.K, self.d, self.seed, X)

    def fit(self, X: torch.Tensor, verbose: bool = False):
        self._init_params(X)
        prev_ll = -float("inf")
        history = []
        for it in range(self.max_iter):
            t0 = time.time()
            self.mu, self.var, self.log_pi, log_norm = _C.flash_em_fused(
                X, self.mu, self.var, self.log_pi, self.BN, self.BK)
            avg_ll = log_norm.mean().item()
            elapsed = time.time() - t0
            history.append({"iter": it, "log_likelihood": avg_ll, "time_ms": elapsed * 1000})
            if verbose and (it % 10 == 0 or it < 5):
                print(f"  iter {it:3d}: LL={avg_ll:.4f}  time={elapsed*1000:.1f}ms")
            if abs(avg_ll - prev_ll) < self.tol:
                if verbose:
                    print(f"  Converged at iter {it}")
                break
            prev_ll = avg_ll
        return history

    def fit_device(self, X: torch.Tensor, n_iter: int | None = None, init=None):
        """``n_iter`` (default ``max_iter``) iterations with tol = 0, all on the
        device.  ``init=(mu, var, log_pi)`` warm-starts instead of the
        reference initialisation.  Returns the same ``history`` records; each
        ``time_ms`` is the loop's wall time divided evenly."""
        n_iter = self.max_iter if n_iter is None else int(n_iter)
        if init is None:
            self._init_params(X)
        else:
            self.mu, self.var, self.log_pi = (t.to(X.device, torch.float32) for t in init)
        if X.is_cuda:
            torch.cuda.synchronize(X.device)
        t0 = time.time()
        self.mu, self.var, self.log_pi, traj = _C.em_fit(X, self.mu, self.var, self.log_pi,
                                                         n_iter)
        lls = traj.cpu().tolist()
        per = (time.time() - t0) * 1000 / n_iter
        return [{"iter": i, "log_likelihood": ll, "time_ms": per} for i, ll in enumerate(lls)]

    def predict_proba(self, X: torch.Tensor) -> torch.Tensor:
        """gamma [N, K] under the current parameters (flash E-step)."""
        return _C.flash_e_step(X, self.mu, self.var, self.log_pi, BK=self.BK)[0]

    def predict(self, X: torch.Tensor) -> torch.Tensor:
        return self.predict_proba(X).argmax(dim=1)
