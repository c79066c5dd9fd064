"""CPU oracle for the fused diagonal-GMM EM iteration -- TEST INFRASTRUCTURE.

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import it.
The HIP library under ``flashgmm_amd/`` does not import, link or call it.

It exposes three restatements of the reference algorithm:

* ``np_*``  -- numpy, fp64, tiled exactly like the reference's PyTorch oracle
  (``flash_gmm/flash_gmm.py:76-145``, ``flash_gmm/flash_e_step.py:144-219``)
  with the native path's M-step clamps (``flash_gmm/csrc/flash_gmm_cuda.cu:310-320``).
  Small and medium sizes.
* ``c_*``   -- the C restatement in ``fgmm_oracle.c`` (fp64, OpenMP), used at
  full benchmark sizes; ``c32_*`` follows the reference C++ path's fp32
  arithmetic order (``flash_gmm/csrc/flash_gmm_cpu.cpp``).
* ``ref_module()`` -- the reference's own CPU extension compiled from its
  sources into ``oracle/_ref`` (``make -C oracle ref``), when present.

Pinning (each check lives in ``tests/test_oracle.py``):

* ``np_log_normalizer`` / ``c_log_normalizer``: sklearn ``score_samples``
  golden vectors, the K=1 closed form (scipy ``norm.logpdf``), the
  identical-components identity, a pure-Python ``math.fsum`` brute force, the
  reference's compiled CPU path (``oracle/_ref``).
* ``np_accumulate_stats`` / ``c_accumulate_stats``: sklearn ``predict_proba``
  golden responsibilities, ``sum_k n_k = N``, the K=1 closed form (sums of X
  and X**2), additivity over point chunks, brute force.
* ``np_m_step_update`` / ``c_m_step_update``: sklearn
  ``_estimate_gaussian_parameters(reg_covar=0)`` golden vectors, the clamp
  special cases (n=0, var<1e-6), the reference's compiled fused path.
* ``np_standard_m_step`` / ``c_standard_m_step``: the same sklearn vectors;
  the reference's compiled ``standard_m_step``.
* ``c_fit``: EM monotonicity of the log-likelihood trajectory and the
  reference's compiled fused iteration chained over 20 steps.
"""
from __future__ import annotations

import ctypes
import glob
import importlib.util
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LOG_2PI = math.log(2.0 * math.pi)   # flash_gmm/csrc/flash_gmm_cuda.cu:21

# ---------------------------------------------------------------------------
# numpy restatement (fp64)
# ---------------------------------------------------------------------------


def np_precompute(var, log_pi):
    """inv_var and log_coeff (flash_gmm/csrc/flash_gmm_cuda.cu:40-57)."""
    v = np.asarray(var, dtype=np.float64)
    d = v.shape[1]
    iv = 1.0 / v
    lc = np.asarray(log_pi, np.float64) - 0.5 * (d * LOG_2PI + np.log(v).sum(1))
    return iv, lc


def np_loglik(X, mu, var, log_pi):
    """L_nk = log pi_k + log N(x_n | mu_k, diag var_k), shape (N, K), fp64
    (flash_gmm/standard_gmm.py:103-106)."""
    X = np.asarray(X, np.float64)
    mu = np.asarray(mu, np.float64)
    iv, lc = np_precompute(var, log_pi)
    out = np.empty((X.shape[0], mu.shape[0]))
    for k in range(mu.shape[0]):
        diff = X - mu[k]
        out[:, k] = lc[k] - 0.5 * (diff * diff * iv[k]).sum(1)
    return out


def np_log_normalizer(X, mu, var, log_pi, BK=8, chunk=16384):
    """Pass 1: online log-sum-exp over component tiles of BK
    (flash_gmm/flash_e_step.py:144-177, flash_gmm/flash_gmm.py:76-105)."""
    X = np.asarray(X, np.float64)
    mu = np.asarray(mu, np.float64)
    iv, lc = np_precompute(var, log_pi)
    N, K = X.shape[0], mu.shape[0]
    out = np.empty(N)
    for a in range(0, N, chunk):
        x = X[a:a + chunk]
        run_max = np.full(x.shape[0], -np.inf)
        run_sum = np.zeros(x.shape[0])
        for t in range(0, K, BK):
            sl = slice(t, min(t + BK, K))
            diff = x[:, None, :] - mu[None, sl, :]
            L = lc[None, sl] - 0.5 * (diff * diff * iv[None, sl, :]).sum(2)
            new_max = np.maximum(run_max, L.max(1))
            run_sum = run_sum * np.exp(run_max - new_max) + np.exp(L - new_max[:, None]).sum(1)
            run_max = new_max
        out[a:a + chunk] = run_max + np.log(run_sum)
    return out


def np_accumulate_stats(X, mu, var, log_pi, ln, BK=8, chunk=16384):
    """Pass 2: gamma = exp(L - ln) recomputed per tile; n_k, s_k = gamma^T X,
    sq_k = gamma^T X^2 (flash_gmm/flash_e_step.py:179-219)."""
    X = np.asarray(X, np.float64)
    mu = np.asarray(mu, np.float64)
    ln = np.asarray(ln, np.float64)
    iv, lc = np_precompute(var, log_pi)
    N, d = X.shape
    K = mu.shape[0]
    n_k, s_k, sq_k = np.zeros(K), np.zeros((K, d)), np.zeros((K, d))
    for a in range(0, N, chunk):
        x = X[a:a + chunk]
        for t in range(0, K, BK):
            sl = slice(t, min(t + BK, K))
            diff = x[:, None, :] - mu[None, sl, :]
            L = lc[None, sl] - 0.5 * (diff * diff * iv[None, sl, :]).sum(2)
            g = np.exp(L - ln[a:a + chunk, None])
            n_k[sl] += g.sum(0)
            s_k[sl] += g.T @ x
            sq_k[sl] += g.T @ (x * x)
    return n_k, s_k, sq_k


def np_m_step_update(n_k, s_k, sq_k, N):
    """M-step with the native clamps (flash_gmm/csrc/flash_gmm_cuda.cu:310-320)."""
    n_k = np.asarray(n_k, np.float64)
    inv = 1.0 / np.maximum(n_k, 1e-8)
    mu = np.asarray(s_k, np.float64) * inv[:, None]
    var = np.maximum(np.asarray(sq_k, np.float64) * inv[:, None] - mu * mu, 1e-6)
    log_pi = np.log(np.maximum(n_k / N, 1e-8))
    return mu, var, log_pi


def np_em_fused(X, mu, var, log_pi, BK=8):
    """One fused iteration (flash_gmm/csrc/flash_gmm_cuda.cu:402-504)."""
    ln = np_log_normalizer(X, mu, var, log_pi, BK)
    n_k, s_k, sq_k = np_accumulate_stats(X, mu, var, log_pi, ln, BK)
    m, v, lp = np_m_step_update(n_k, s_k, sq_k, X.shape[0])
    return m, v, lp, ln


def np_standard_e_step(X, mu, var, log_pi):
    """Standard E-step: materialise L, row log-sum-exp, gamma
    (flash_gmm/csrc/flash_gmm_cpu.cpp:51-100)."""
    L = np_loglik(X, mu, var, log_pi)
    mx = L.max(1, keepdims=True)
    ln = mx[:, 0] + np.log(np.exp(L - mx).sum(1))
    return np.exp(L - ln[:, None]), ln


def np_standard_m_step(X, gamma):
    """Standard M-step: no n_k clamp, var = gamma^T X^2/n - mu^2 clamped at
    1e-6, log(n/N) (flash_gmm/csrc/flash_gmm_cpu.cpp:292-311)."""
    X = np.asarray(X, np.float64)
    g = np.asarray(gamma, np.float64)
    n_k = g.sum(0)
    mu = (g.T @ X) / n_k[:, None]
    var = np.maximum((g.T @ (X * X)) / n_k[:, None] - mu * mu, 1e-6)
    return mu, var, np.log(n_k / X.shape[0])


# ---------------------------------------------------------------------------
# C restatement (fp64 + reference-order fp32), OpenMP
# ---------------------------------------------------------------------------

_LIB = None
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_L, _I = ctypes.c_long, ctypes.c_int


def lib_path():
    return os.path.join(HERE, "libfgmm_oracle.so")


def clib():
    """Load ``libfgmm_oracle.so`` (built by ``make -C oracle``)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = lib_path()
    if not os.path.exists(path):
        raise RuntimeError(f"oracle library missing: {path} (run `make -C oracle`)")
    lib = ctypes.CDLL(path)
    sig = {
        "orc_num_threads": ([], _I),
        "orc_log_normalizer": ([_f32p, _f32p, _f32p, _f32p, _L, _I, _I, _I, _f64p], None),
        "orc_accumulate_stats": ([_f32p, _f32p, _f32p, _f32p, _f64p, _L, _I, _I, _f64p, _f64p, _f64p], None),
        "orc_m_step_update": ([_f64p, _f64p, _f64p, _L, _I, _I, _f64p, _f64p, _f64p], None),
        "orc_em_fused": ([_f32p, _f32p, _f32p, _f32p, _L, _I, _I, _I, _f32p, _f32p, _f32p, _f64p,
                          _f64p, _f64p, _f64p], None),
        "orc_fit": ([_f32p, _f32p, _f32p, _f32p, _L, _I, _I, _I, _f64p, _f32p, _f32p, _f32p], None),
        "orc_standard_e_step": ([_f32p, _f32p, _f32p, _f32p, _L, _I, _I, _f64p, _f64p], None),
        "orc_flash_e_step": ([_f32p, _f32p, _f32p, _f32p, _L, _I, _I, _I, _f64p, _f64p], None),
        "orc_standard_m_step": ([_f32p, _f64p, _L, _I, _I, _f64p, _f64p, _f64p], None),
        "orc32_em_fused": ([_f32p, _f32p, _f32p, _f32p, _L, _I, _I, _I, _f32p, _f32p, _f32p, _f32p], None),
        "orc32_standard_e_step": ([_f32p, _f32p, _f32p, _f32p, _L, _I, _I, _f32p, _f32p], None),
        "orc32_standard_m_step": ([_f32p, _f32p, _L, _I, _I, _f32p, _f32p, _f32p], None),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _LIB = lib
    return lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def c_log_normalizer(X, mu, var, log_pi, BK=8):
    X, mu, var, log_pi = map(_f32, (X, mu, var, log_pi))
    N, d = X.shape
    out = np.empty(N)
    clib().orc_log_normalizer(X, mu, var, log_pi, N, mu.shape[0], d, BK, out)
    return out


def c_accumulate_stats(X, mu, var, log_pi, ln):
    X, mu, var, log_pi = map(_f32, (X, mu, var, log_pi))
    N, d = X.shape
    K = mu.shape[0]
    n_k, s_k, sq_k = np.empty(K), np.empty((K, d)), np.empty((K, d))
    clib().orc_accumulate_stats(X, mu, var, log_pi, np.ascontiguousarray(ln, np.float64),
                                N, K, d, n_k, s_k, sq_k)
    return n_k, s_k, sq_k


def c_m_step_update(n_k, s_k, sq_k, N):
    n_k = np.ascontiguousarray(n_k, np.float64)
    s_k = np.ascontiguousarray(s_k, np.float64)
    sq_k = np.ascontiguousarray(sq_k, np.float64)
    K, d = s_k.shape
    mu, var, lp = np.empty((K, d)), np.empty((K, d)), np.empty(K)
    clib().orc_m_step_update(n_k, s_k, sq_k, int(N), K, d, mu, var, lp)
    return mu, var, lp


def c_em_fused(X, mu, var, log_pi, BK=8, with_stats=False):
    """One fused iteration in fp64; new parameters rounded to fp32 like the
    API's outputs, ln kept in fp64."""
    X, mu, var, log_pi = map(_f32, (X, mu, var, log_pi))
    N, d = X.shape
    K = mu.shape[0]
    nm, nv, nl = np.empty((K, d), np.float32), np.empty((K, d), np.float32), np.empty(K, np.float32)
    ln = np.empty(N)
    n_k, s_k, sq_k = np.empty(K), np.empty((K, d)), np.empty((K, d))
    clib().orc_em_fused(X, mu, var, log_pi, N, K, d, BK, nm, nv, nl, ln, n_k, s_k, sq_k)
    if with_stats:
        return nm, nv, nl, ln, (n_k, s_k, sq_k)
    return nm, nv, nl, ln


def c_fit(X, mu0, var0, log_pi0, iters):
    """EM driver with tol=0: returns (trajectory[iters] of mean ln, mu, var,
    log_pi) with fp32 parameters between iterations."""
    X, mu0, var0, log_pi0 = map(_f32, (X, mu0, var0, log_pi0))
    N, d = X.shape
    K = mu0.shape[0]
    traj = np.empty(iters)
    mu, var, lp = np.empty((K, d), np.float32), np.empty((K, d), np.float32), np.empty(K, np.float32)
    clib().orc_fit(X, mu0, var0, log_pi0, N, K, d, iters, traj, mu, var, lp)
    return traj, mu, var, lp


def c_standard_e_step(X, mu, var, log_pi):
    X, mu, var, log_pi = map(_f32, (X, mu, var, log_pi))
    N, d = X.shape
    K = mu.shape[0]
    g, ln = np.empty((N, K)), np.empty(N)
    clib().orc_standard_e_step(X, mu, var, log_pi, N, K, d, g, ln)
    return g, ln


def c_flash_e_step(X, mu, var, log_pi, BK=4):
    X, mu, var, log_pi = map(_f32, (X, mu, var, log_pi))
    N, d = X.shape
    K = mu.shape[0]
    g, ln = np.empty((N, K)), np.empty(N)
    clib().orc_flash_e_step(X, mu, var, log_pi, N, K, d, BK, g, ln)
    return g, ln


def c_standard_m_step(X, gamma):
    X = _f32(X)
    g = np.ascontiguousarray(gamma, np.float64)
    N, d = X.shape
    K = g.shape[1]
    mu, var, lp = np.empty((K, d)), np.empty((K, d)), np.empty(K)
    clib().orc_standard_m_step(X, g, N, K, d, mu, var, lp)
    return mu, var, lp


def c32_em_fused(X, mu, var, log_pi, BK=8):
    """Reference-order fp32 fused iteration (flash_gmm_cpu.cpp:177-287)."""
    X, mu, var, log_pi = map(_f32, (X, mu, var, log_pi))
    N, d = X.shape
    K = mu.shape[0]
    nm, nv, nl = np.empty((K, d), np.float32), np.empty((K, d), np.float32), np.empty(K, np.float32)
    ln = np.empty(N, np.float32)
    clib().orc32_em_fused(X, mu, var, log_pi, N, K, d, BK, nm, nv, nl, ln)
    return nm, nv, nl, ln


def c32_standard_e_step(X, mu, var, log_pi):
    """Reference-order fp32 standard E-step (flash_gmm_cpu.cpp:51-100);
    returns (gamma [N, K], log_normalizer [N])."""
    X, mu, var, log_pi = map(_f32, (X, mu, var, log_pi))
    N, d = X.shape
    K = mu.shape[0]
    g, ln = np.empty((N, K), np.float32), np.empty(N, np.float32)
    clib().orc32_standard_e_step(X, mu, var, log_pi, N, K, d, g, ln)
    return g, ln


def c32_standard_m_step(X, gamma):
    """fp32 standard M-step (flash_gmm_cpu.cpp:292-311); returns (mu, var, log_pi)."""
    X, gamma = _f32(X), _f32(gamma)
    N, d = X.shape
    K = gamma.shape[1]
    m, v, lp = np.empty((K, d), np.float32), np.empty((K, d), np.float32), np.empty(K, np.float32)
    clib().orc32_standard_m_step(X, gamma, N, K, d, m, v, lp)
    return m, v, lp


def c32_standard_em(X, mu, var, log_pi):
    """Reference-order fp32 standard E-step + M-step
    (flash_gmm_cpu.cpp:51-100 then :292-311)."""
    g, ln = c32_standard_e_step(X, mu, var, log_pi)
    return (*c32_standard_m_step(X, g), ln)


def c_num_threads():
    return clib().orc_num_threads()


# ---------------------------------------------------------------------------
# the reference's own CPU extension, compiled into oracle/_ref
# ---------------------------------------------------------------------------

def ref_module():
    """Import ``flash_gmm_ref_cpu`` from ``oracle/_ref`` or return None.

    Built by ``make -C oracle ref`` from the reference's
    ``flash_gmm/csrc/binding.cpp`` and ``flash_gmm_cpu.cpp`` (CPU only); the
    prebuilt module travels with the tree, the sources do not."""
    cands = sorted(glob.glob(os.path.join(HERE, "_ref", "flash_gmm_ref_cpu*.so")))
    if not cands:
        return None
    import torch  # noqa: F401  (libtorch must be loaded first)
    if "flash_gmm_ref_cpu" in sys.modules:
        return sys.modules["flash_gmm_ref_cpu"]
    spec = importlib.util.spec_from_file_location("flash_gmm_ref_cpu", cands[0])
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    sys.modules["flash_gmm_ref_cpu"] = mod
    return mod
