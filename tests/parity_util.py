"""Helpers shared by the GPU parity tests: cached problems and oracle runs,
the parity checks with the tolerances the suite states, host->device copies."""
import functools

import numpy as np

from flashgmm_amd.configs import make_problem
from oracle import oracle as O


def ulp32(x):
    return np.spacing(np.abs(np.asarray(x, np.float64)).astype(np.float32)).astype(np.float64)


def param_tol(ref):
    """Per-entry bar for mu and var: 1e-5 absolute below 256; one fp32 ulp of
    the value from 256 up.  Below 256 a correctly rounded fp32 output lies
    within half an ulp (<= 7.6e-6) of the truth, so 1e-5 is attainable and is
    the bar.  From 256 up half an ulp is >= 1.53e-5: no fp32 output can meet
    1e-5 there, and one ulp admits the correctly rounded value and its
    neighbour (rounding of the output plus at most half an ulp of error in
    the computation before it)."""
    r = np.abs(np.asarray(ref, np.float64))
    return np.where(r < 256.0, 1e-5, np.maximum(1e-5, ulp32(r)))


def check_params(got, ref64, label):
    """mu, var: |gpu - ref| <= param_tol(ref); pi = exp(log_pi):
    |gpu - ref| <= 1e-5.  NaN must match NaN (empty components of the
    standard M-step).  Prints and returns the largest errors seen."""
    g_mu, g_var, g_lp = (np.asarray(a, np.float64) for a in got)
    r_mu, r_var, r_lp = (np.asarray(a, np.float64) for a in ref64)
    seen = {}
    for name, g, r in (("mu", g_mu, r_mu), ("var", g_var, r_var)):
        assert np.array_equal(np.isnan(g), np.isnan(r)), f"{label}: {name} NaN pattern differs"
        ok = ~np.isnan(r)
        err = np.where(ok, np.abs(g - r), 0.0)
        tol = param_tol(np.where(ok, r, 0.0))
        ratio = err / tol
        i = int(ratio.argmax())
        seen[name] = float(err.max())
        assert ratio.flat[i] <= 1.0, (f"{label}: {name} err {err.flat[i]:.3e} > tol "
                                      f"{tol.flat[i]:.3e} at {np.unravel_index(i, err.shape)} "
                                      f"(value {r.flat[i]:.6g}; max err {err.max():.3e})")
    epi = float(np.abs(np.exp(g_lp) - np.exp(r_lp)).max()) if g_lp.size else 0.0
    seen["pi"] = epi
    assert epi <= 1e-5, f"{label}: pi max err {epi:.3e}"
    print(f"[parity] {label}: max |err| mu {seen['mu']:.2e} var {seen['var']:.2e} "
          f"pi {seen['pi']:.2e}", flush=True)
    return seen


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
