"""The drop-in module on CPU tensors: the host path (libflashgmm_cpu.so, C++/OpenMP).

The reference routes CPU tensors to its OpenMP code
(flash_gmm/csrc/binding.cpp:48,59,75,91).  Here the same calls run this
package's host library.  It is held to the GPU path's parity bar against the
fp64 oracle:
  * ln: relative 1e-5;
  * mu, var: 1e-5 absolute below 256, one fp32 ulp from 256 up;
  * pi: 1e-5;
  * gamma: 1e-6 absolute;
  * the 20-iteration LL trajectory: relative 1e-4.
Results must not depend on the thread count.
"""
import os

import numpy as np
import pytest
import torch

from flashgmm_amd import flash_gmm_native as C
from flashgmm_amd.configs import make_problem
from oracle import oracle as O
from parity_util import check_gamma, check_ln, check_params, oracle_iter

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def host(*arrs):
    return [torch.from_numpy(np.ascontiguousarray(a)) for a in arrs]


@pytest.mark.parametrize("cid,N", [(1, None), (2, 4096), (3, 8192), (4, 4096), (5, 4096)])
def test_em_fused_on_cpu_tensors(cid, N):
    X, mu, var, lp = make_problem(cid, N)
    m64, v64, l64, ln, *_ = oracle_iter(cid, N)
    out = C.flash_em_fused(*host(X, mu, var, lp))
    assert all(o.device.type == "cpu" and o.dtype == torch.float32 for o in out)
    check_params([o.numpy() for o in out[:3]], (m64, v64, l64), f"cpu C{cid}")
    check_ln(out[3].numpy(), ln, f"cpu C{cid}")


def test_results_do_not_depend_on_thread_count():
    X, mu, var, lp = make_problem(2, 3000)
    t = host(X, mu, var, lp)
    saved = torch.get_num_threads()
    try:
        torch.set_num_threads(1)
        a = C.flash_em_fused(*t)
        g1 = C.standard_m_step(t[0], C.standard_e_step(*t)[0])
        torch.set_num_threads(max(2, saved))
        b = C.flash_em_fused(*t)
        g2 = C.standard_m_step(t[0], C.standard_e_step(*t)[0])
    finally:
        torch.set_num_threads(saved)
    for x, y in zip(a + g1, b + g2):
        assert torch.equal(x, y)


def test_stage_entry_points_on_cpu():
    X, mu, var, lp = make_problem(4, 4096)
    _, _, _, ln64, *_ = oracle_iter(4, 4096)
    t = host(X, mu, var, lp)
    ln = C.flash_log_normalizer(*t)
    check_ln(ln.numpy(), ln64, "cpu pass1")
    n_k, s_k, sq_k = C.flash_accumulate_stats(*t, ln)
    r = O.c_accumulate_stats(X, mu, var, lp, ln.numpy().astype(np.float64))
    for g, ref in zip((n_k, s_k, sq_k), r):
        g = g.numpy().astype(np.float64)
        scale = np.abs(ref).reshape(ref.shape[0], -1).max(axis=1) + 1e-30
        err = np.abs(g - ref).reshape(ref.shape[0], -1).max(axis=1) / scale
        assert err.max() <= 1e-6, err.max()
    mu2, var2, lp2 = C.m_step_update(n_k, s_k, sq_k, X.shape[0])
    ref = O.c_m_step_update(n_k.numpy(), s_k.numpy(), sq_k.numpy(), X.shape[0])
    for g, r_ in zip((mu2, var2, lp2), ref):
        e = np.abs(g.numpy().astype(np.float64) - r_)
        assert np.all(e <= np.maximum(np.spacing(np.abs(r_).astype(np.float32)), 1e-12))


@pytest.mark.parametrize("fn", ["standard_e_step", "flash_e_step"])
def test_e_steps_on_cpu(fn):
    X, mu, var, lp = make_problem(2, 2048)
    g_ref, ln_ref = O.c_standard_e_step(X, mu, var, lp)
    gamma, ln = getattr(C, fn)(*host(X, mu, var, lp))
    assert gamma.shape == (2048, mu.shape[0])
    check_gamma(gamma.numpy(), g_ref, f"cpu {fn}")
    check_ln(ln.numpy(), ln_ref, f"cpu {fn}")


def test_standard_m_step_on_cpu_keeps_reference_arithmetic():
    """No clamp on n_k: an empty component gives NaN mean and variance and
    log_pi = -inf, as the reference's standard M-step does."""
    with np.load(os.path.join(GOLDEN, "empty_component.npz"), allow_pickle=False) as z:
        g = {k: z[k] for k in z.files}
    X = g["X"]
    gam, _ = O.c_standard_e_step(X, g["mu"], g["var"], g["log_pi"])
    gam = gam.astype(np.float32)
    gam[:, 0] = 0.0                      # component 0 receives nothing
    mu, var, lp = C.standard_m_step(*host(X, gam))
    r = O.c_standard_m_step(X, gam)
    assert np.isnan(mu.numpy()[0]).all() and np.isnan(var.numpy()[0]).all()
    assert np.isneginf(lp.numpy()[0])
    check_params((mu.numpy(), var.numpy(), lp.numpy()), r, "cpu standard m-step")


@pytest.mark.parametrize("name", ["k1_d3", "k4_d8", "c1_head512", "overlap_k6_d5",
                                  "empty_component", "ragged_k17_d33"])
def test_golden_vectors_on_cpu(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        g = {k: z[k] for k in z.files}
    out = C.flash_em_fused(*host(g["X"], g["mu"], g["var"], g["log_pi"]))
    check_ln(out[3].numpy(), g["ln"], f"cpu {name}")
    check_params([o.numpy() for o in out[:3]], (g["new_mu"], g["new_var"], g["new_log_pi"]),
                 f"cpu {name}")


def test_em_fit_and_wrappers_on_cpu():
    """The iteration loop on the host follows the fp64 oracle's trajectory at
    C1 full size (tests/golden/trajectories.json); NativeFlashGMM.fit and
    fit_device accept CPU tensors and record the same history."""
    import json
    from flashgmm_amd.native_wrapper import NativeFlashGMM, NativeStandardGMM
    ref = json.load(open(os.path.join(GOLDEN, "trajectories.json")))["C1"]
    X, mu, var, lp = make_problem(1)
    t = host(X, mu, var, lp)
    _, _, _, traj = C.em_fit(*t, ref["iters"])
    assert traj.dtype == torch.float64 and traj.device.type == "cpu"
    e = np.abs(traj.numpy() - np.array(ref["ll"])) / np.abs(ref["ll"])
    assert e.max() <= 1e-4, e.max()
    h1 = NativeFlashGMM(K=8, d=32, max_iter=8, tol=0.0).fit(t[0])
    h2 = NativeFlashGMM(K=8, d=32, max_iter=8, tol=0.0).fit_device(t[0])
    for a, b in zip(h1, h2):
        # fit averages the fp32 log-normalizer (as the reference), fit_device in fp64
        assert abs(a["log_likelihood"] - b["log_likelihood"]) <= 1e-6 * abs(b["log_likelihood"])
    hs = NativeStandardGMM(K=8, d=32, max_iter=8, tol=0.0).fit(t[0])
    assert hs[-1]["log_likelihood"] >= hs[0]["log_likelihood"]
    gmm = NativeFlashGMM(K=8, d=32, max_iter=3)
    gmm.fit(t[0])
    assert gmm.predict(t[0]).shape == (X.shape[0],)


def test_cpu_errors_match_the_reference_checks():
    X, mu, var, lp = host(*make_problem(1, 64))
    with pytest.raises(RuntimeError, match="X must be float32"):
        C.flash_em_fused(X.double(), mu, var, lp)
    with pytest.raises(RuntimeError, match="X must be float32"):
        C.standard_m_step(X.double(), torch.zeros(64, 8))
    with pytest.raises(RuntimeError, match="X must be 2D"):
        C.standard_e_step(X.reshape(-1), mu, var, lp)
    with pytest.raises(RuntimeError, match="var must be"):
        C.flash_em_fused(X, mu, var[:, :3], lp)
    with pytest.raises(RuntimeError, match="mu must be float32"):
        C.flash_em_fused(X, mu.double(), var, lp)


def test_top_level_module_is_the_drop_in():
    import flash_gmm_native as _C
    assert _C is C
    for name in ("flash_em_fused", "standard_e_step", "flash_e_step", "standard_m_step",
                 "flash_log_normalizer", "flash_accumulate_stats", "m_step_update"):
        assert callable(getattr(_C, name))


def test_host_library_exports_its_header():
    import ctypes
    import re
    from flashgmm_amd import _lib
    text = open(os.path.join(os.path.dirname(GOLDEN), "..", "include", "flashgmm_cpu.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = sorted(set(re.findall(r"\b(fgmm_cpu_\w+)\s*\(", text)))
    assert names == sorted(_lib.CPU_SIGNATURES)
    raw = ctypes.CDLL(_lib.CPU_LIB_PATH)
    for n in names:
        assert hasattr(raw, n)
