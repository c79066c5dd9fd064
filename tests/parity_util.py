"""Helpers shared by the GPU parity tests: cached problems and oracle runs,
the parity checks with the tolerances the suite states, host->device copies."""
import functools

import numpy as np

from flashgmm_amd.configs import make_problem
from oracle import oracle as O


def ulp32(x):
    return np.spacing(np.abs(np.asarray(x, np.float64)).astype(np.float32)).astype(np.float64)


def check_params(got, ref64, label):
    """mu, var: |gpu - ref| <= max(1e-5, 2 ulp_fp32(ref)); pi = exp(log_pi):
    |gpu - ref| <= 1e-5.  NaN must match NaN (empty components of the
    standard M-step)."""
    g_mu, g_var, g_lp = (np.asarray(a, np.float64) for a in got)
    r_mu, r_var, r_lp = (np.asarray(a, np.float64) for a in ref64)
    for name, g, r in (("mu", g_mu, r_mu), ("var", g_var, r_var)):
        assert np.array_equal(np.isnan(g), np.isnan(r)), f"{label}: {name} NaN pattern differs"
        ok = ~np.isnan(r)
        err = np.where(ok, np.abs(g - r), 0.0)
        tol = np.maximum(1e-5, 2 * ulp32(np.where(ok, r, 0.0)))
        ratio = err / tol
        i = int(ratio.argmax())
        assert ratio.flat[i] <= 1.0, (f"{label}: {name} err {err.flat[i]:.3e} > tol "
                                      f"{tol.flat[i]:.3e} at {np.unravel_index(i, err.shape)} "
                                      f"(value {r.flat[i]:.6g}; max err {err.max():.3e})")
    epi = np.abs(np.exp(g_lp) - np.exp(r_lp)).max()
    assert epi <= 1e-5, f"{label}: pi max err {epi:.3e}"


def check_ln(got, ref, label, tol=1e-5):
    e = np.max(np.abs(np.asarray(got, np.float64) - ref) / np.abs(ref))
    assert e <= tol, f"{label}: log_normalizer max rel err {e:.3e}"


def check_gamma(got, ref, label, tol=1e-6):
    """Responsibilities: absolute error <= tol (they lie in [0, 1])."""
    g = np.asarray(got, np.float64)
    assert g.shape == ref.shape, f"{label}: gamma shape {g.shape} != {ref.shape}"
    e = np.abs(g - ref)
    i = int(e.argmax())
    assert e.flat[i] <= tol, (f"{label}: gamma err {e.flat[i]:.3e} at "
                              f"{np.unravel_index(i, e.shape)} (value {ref.flat[i]:.6g})")


@functools.lru_cache(maxsize=None)
def problem(cid, N):
    return make_problem(cid, N)


@functools.lru_cache(maxsize=None)
def oracle_iter(cid, N):
    X, mu, var, lp = problem(cid, N)
    _, _, _, ln, (n_k, s_k, sq_k) = O.c_em_fused(X, mu, var, lp, with_stats=True)
    m64, v64, l64 = O.c_m_step_update(n_k, s_k, sq_k, X.shape[0])
    return m64, v64, l64, ln, n_k, s_k, sq_k


def to_dev(cuda, *arrs):
    import torch
    return [torch.from_numpy(np.ascontiguousarray(a)).to(cuda) for a in arrs]
