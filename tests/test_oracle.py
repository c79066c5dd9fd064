"""Pins the CPU oracle (oracle/) before it is trusted as the GPU checker.

Every oracle function is checked against at least one of: the sklearn golden
vectors (tests/golden/), a closed form, a brute-force fp64 sum, an invariant,
or the reference's own CPU extension compiled from its sources (oracle/_ref).
The mutation tests plant plausible mistakes in a copy of the oracle and show
that these checks reject them.
"""
import glob
import math
import os

import numpy as np
import pytest
from scipy.stats import norm

from oracle import oracle as O

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), 1e-300)))


def absd(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def golden_ln_ok(fn, g, tol=1e-10):
    return rel(fn(g["X"], g["mu"], g["var"], g["log_pi"]), g["ln"]) <= tol


# ---------------------------------------------------------------------------
# golden vectors (sklearn)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_log_normalizer_vs_sklearn(path):
    g = load(path)
    assert rel(O.np_log_normalizer(g["X"], g["mu"], g["var"], g["log_pi"]), g["ln"]) < 1e-12
    assert rel(O.c_log_normalizer(g["X"], g["mu"], g["var"], g["log_pi"]), g["ln"]) < 1e-12
    # tile size does not change the result (online log-sum-exp)
    for bk in (1, 3, 8, 64):
        assert rel(O.c_log_normalizer(g["X"], g["mu"], g["var"], g["log_pi"], BK=bk), g["ln"]) < 1e-12


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_responsibilities_and_stats_vs_sklearn(path):
    g = load(path)
    X, mu, var, lp = g["X"], g["mu"], g["var"], g["log_pi"]
    gam, ln = O.np_standard_e_step(X, mu, var, lp)
    assert absd(gam, g["gamma"]) < 1e-12
    gam_c, ln_c = O.c_standard_e_step(X, mu, var, lp)
    assert absd(gam_c, g["gamma"]) < 1e-12 and rel(ln_c, g["ln"]) < 1e-12
    gf, lf = O.c_flash_e_step(X, mu, var, lp, BK=3)
    assert absd(gf, g["gamma"]) < 1e-12 and rel(lf, g["ln"]) < 1e-12
    for n_k, s_k, sq_k in (O.np_accumulate_stats(X, mu, var, lp, g["ln"]),
                           O.c_accumulate_stats(X, mu, var, lp, g["ln"])):
        scale = max(1.0, float(np.abs(g["sq_k"]).max()))
        assert absd(n_k, g["n_k"]) < 1e-9
        assert absd(s_k, g["s_k"]) < 1e-9 * scale
        assert absd(sq_k, g["sq_k"]) < 1e-9 * scale


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_m_step_vs_sklearn(path):
    g = load(path)
    N = g["X"].shape[0]
    for mu, var, lp in (O.np_m_step_update(g["n_k"], g["s_k"], g["sq_k"], N),
                        O.c_m_step_update(g["n_k"], g["s_k"], g["sq_k"], N)):
        assert absd(mu, g["new_mu"]) < 1e-9
        assert absd(var, g["new_var"]) < 1e-9
        assert absd(lp, g["new_log_pi"]) < 1e-9
    m, v, lp = O.np_em_fused(g["X"], g["mu"], g["var"], g["log_pi"])[:3]
    assert absd(m, g["new_mu"]) < 1e-9 and absd(v, g["new_var"]) < 1e-9
    assert absd(lp, g["new_log_pi"]) < 1e-9


def test_standard_m_step_vs_sklearn():
    g = load([p for p in GOLDEN if "k4_d8" in p][0])
    for mu, var, lp in (O.np_standard_m_step(g["X"], g["gamma"]),
                        O.c_standard_m_step(g["X"], g["gamma"])):
        assert absd(mu, g["new_mu"]) < 1e-9 and absd(var, g["new_var"]) < 1e-9
        assert absd(lp, g["new_log_pi"]) < 1e-9


# ---------------------------------------------------------------------------
# closed forms, brute force, invariants
# ---------------------------------------------------------------------------
def test_single_component_closed_form():
    rng = np.random.default_rng(0)
    X = rng.normal(0, 3, (100, 5)).astype(np.float32)
    mu = rng.normal(0, 1, (1, 5)).astype(np.float32)
    var = rng.uniform(0.2, 4.0, (1, 5)).astype(np.float32)
    lp = np.array([-0.7], np.float32)
    want = float(lp[0]) + norm.logpdf(X.astype(np.float64), mu.astype(np.float64),
                                      np.sqrt(var.astype(np.float64))).sum(1)
    assert rel(O.c_log_normalizer(X, mu, var, lp), want) < 1e-13
    # with log_pi = 0 every point has gamma = 1: stats are plain sums
    n_k, s_k, sq_k = O.c_accumulate_stats(X, mu, var, np.zeros(1, np.float32),
                                          O.c_log_normalizer(X, mu, var, np.zeros(1, np.float32)))
    X64 = X.astype(np.float64)
    assert abs(n_k[0] - 100) < 1e-10
    assert absd(s_k[0], X64.sum(0)) < 1e-10 and absd(sq_k[0], (X64 ** 2).sum(0)) < 1e-9


def test_identical_components_identity():
    rng = np.random.default_rng(1)
    X = rng.normal(0, 1, (50, 4)).astype(np.float32)
    mu1 = rng.normal(0, 1, (1, 4)).astype(np.float32)
    var1 = rng.uniform(0.5, 2, (1, 4)).astype(np.float32)
    lp = np.log(np.array([0.1, 0.2, 0.3, 0.4])).astype(np.float32)
    ln = O.c_log_normalizer(X, np.repeat(mu1, 4, 0), np.repeat(var1, 4, 0), lp)
    single = O.c_log_normalizer(X, mu1, var1, np.zeros(1, np.float32))
    lse = math.log(sum(math.exp(float(v)) for v in lp))
    assert rel(ln, single + lse) < 1e-13


def _brute(X, mu, var, lp):
    N, d = X.shape
    K = mu.shape[0]
    ln = []
    L = [[0.0] * K for _ in range(N)]
    for n in range(N):
        for k in range(K):
            terms = [math.log(2 * math.pi)] * d
            terms += [math.log(float(var[k, j])) for j in range(d)]
            terms += [(float(X[n, j]) - float(mu[k, j])) ** 2 / float(var[k, j]) for j in range(d)]
            L[n][k] = float(lp[k]) - 0.5 * math.fsum(terms)
        m = max(L[n])
        ln.append(m + math.log(math.fsum(math.exp(v - m) for v in L[n])))
    n_k = [math.fsum(math.exp(L[n][k] - ln[n]) for n in range(N)) for k in range(K)]
    s_k = [[math.fsum(math.exp(L[n][k] - ln[n]) * float(X[n, j]) for n in range(N))
            for j in range(d)] for k in range(K)]
    return np.array(ln), np.array(n_k), np.array(s_k)


def test_brute_force_tiny():
    rng = np.random.default_rng(2)
    X = rng.normal(0, 2, (7, 3)).astype(np.float32)
    mu = rng.normal(0, 2, (4, 3)).astype(np.float32)
    var = rng.uniform(0.3, 3, (4, 3)).astype(np.float32)
    lp = rng.normal(-1.4, 0.3, 4).astype(np.float32)
    ln, n_k, s_k = _brute(X, mu, var, lp)
    assert rel(O.np_log_normalizer(X, mu, var, lp, BK=3), ln) < 1e-13
    assert rel(O.c_log_normalizer(X, mu, var, lp, BK=3), ln) < 1e-13
    nk2, sk2, _ = O.c_accumulate_stats(X, mu, var, lp, ln)
    assert absd(nk2, n_k) < 1e-12 and absd(sk2, s_k) < 1e-12


def test_invariants():
    from flashgmm_amd.configs import make_problem
    X, mu, var, lp = make_problem(1)
    ln = O.c_log_normalizer(X, mu, var, lp)
    n_k, s_k, sq_k = O.c_accumulate_stats(X, mu, var, lp, ln)
    assert abs(n_k.sum() - X.shape[0]) < 1e-8 * X.shape[0]
    # permutation-equivariant in points, invariant in components
    p = np.random.default_rng(3).permutation(X.shape[0])
    q = np.random.default_rng(4).permutation(mu.shape[0])
    assert rel(O.c_log_normalizer(X[p], mu, var, lp), ln[p]) < 1e-13
    assert rel(O.c_log_normalizer(X, mu[q], var[q], lp[q]), ln) < 1e-13
    n2, s2, _ = O.c_accumulate_stats(X, mu[q], var[q], lp[q], ln)
    assert absd(n2, n_k[q]) < 1e-9 and absd(s2, s_k[q]) < 1e-8
    # statistics are additive over point chunks
    h = X.shape[0] // 3
    a = O.c_accumulate_stats(X[:h], mu, var, lp, ln[:h])
    b = O.c_accumulate_stats(X[h:], mu, var, lp, ln[h:])
    assert absd(a[0] + b[0], n_k) < 1e-9 and absd(a[2] + b[2], sq_k) < 1e-7


def test_m_step_clamps():
    n_k = np.array([0.0, 5.0])
    s_k = np.array([[0.0, 0.0], [5.0, 10.0]])
    sq_k = np.array([[0.0, 0.0], [5.0 + 1e-9, 20.0]])   # second comp: var -> 0 -> 1e-6
    mu, var, lp = O.c_m_step_update(n_k, s_k, sq_k, 10)
    assert np.all(mu[0] == 0.0) and np.all(var[0] == 1e-6) and lp[0] == math.log(1e-8)
    assert np.allclose(mu[1], [1.0, 2.0]) and var[1, 0] == 1e-6 and var[1, 1] == pytest.approx(0.0 + 1e-6, abs=1e-12)
    assert lp[1] == pytest.approx(math.log(0.5))


def test_fit_monotone_and_consistent():
    from flashgmm_amd.configs import make_problem
    X, mu, var, lp = make_problem(1)
    traj, m, v, l = O.c_fit(X, mu, var, lp, 20)
    assert np.all(np.diff(traj) >= -1e-9 * np.abs(traj[1:]))   # EM never decreases the LL
    # chaining the single-iteration oracle gives the same trajectory
    p = (mu, var, lp)
    for it in range(3):
        nm, nv, nl, ln = O.c_em_fused(X, *p)
        assert abs(ln.mean() - traj[it]) <= 1e-12 * abs(traj[it])
        p = (nm, nv, nl)


# ---------------------------------------------------------------------------
# the reference's own CPU path (compiled from its sources into oracle/_ref)
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def ref():
    mod = O.ref_module()
    if mod is None:
        pytest.skip("oracle/_ref not built (make -C oracle ref needs the reference sources)")
    return mod


def test_fp32_restatement_matches_reference_bitwise(ref):
    import torch
    from flashgmm_amd.configs import make_problem
    torch.set_num_threads(O.c_num_threads())
    X, mu, var, lp = make_problem(1)
    t = [torch.from_numpy(a) for a in (X, mu, var, lp)]
    for bk in (4, 8):
        r = [o.numpy() for o in ref.flash_em_fused(*t, 64, bk)]
        c = O.c32_em_fused(X, mu, var, lp, BK=bk)
        for a, b in zip(r, c):
            assert np.array_equal(a, b)
    # the standard E-step: responsibilities and log-normalizer bit for bit
    g_ref, ln_ref = (o.numpy() for o in ref.standard_e_step(*t))
    g_c32, ln_c32 = O.c32_standard_e_step(X, mu, var, lp)
    assert np.array_equal(g_ref, g_c32)
    assert np.array_equal(ln_ref, ln_c32)
    # the standard M-step runs ATen GEMMs in the reference (the BLAS's
    # summation order), so from the same gamma it is not reproducible bit for
    # bit; both fp32 versions sit within fp32 summation error of the fp64
    # M-step of that gamma (measured at C1: BLAS mu 1.2e-6, var 1.1e-5; the
    # restatement's sequential sums over 4096 points mu 8.3e-6, var 6.4e-5)
    m_ref, v_ref, l_ref = (o.numpy() for o in ref.standard_m_step(t[0], torch.from_numpy(g_ref)))
    m_c, v_c, l_c = O.c32_standard_m_step(X, g_ref)
    m64, v64, l64 = O.c_standard_m_step(X, g_ref)
    for name, a, b, r, tol in (("mu", m_ref, m_c, m64, 2e-5), ("var", v_ref, v_c, v64, 1.5e-4),
                               ("log_pi", l_ref, l_c, l64, 5e-6)):
        for who, v in (("reference", a), ("restatement", b)):
            e = np.abs(v.astype(np.float64) - r).max()
            assert e <= tol, f"{who} standard M-step {name}: {e:.2e} from fp64"


def test_fp64_oracle_vs_reference(ref):
    """The fp64 restatement and the reference's fp32 code agree to fp32
    accuracy on the small configuration (they are the same algorithm)."""
    import torch
    from flashgmm_amd.configs import make_problem
    X, mu, var, lp = make_problem(1)
    t = [torch.from_numpy(a) for a in (X, mu, var, lp)]
    r_mu, r_var, r_lp, r_ln = (o.numpy().astype(np.float64) for o in ref.flash_em_fused(*t, 64, 8))
    c_mu, c_var, c_lp, c_ln = O.c_em_fused(X, mu, var, lp)
    assert rel(c_ln, r_ln) < 2e-6
    assert absd(c_mu, r_mu) < 1e-4 and absd(c_var, r_var) < 1e-4 and absd(c_lp, r_lp) < 1e-5
    g, ln = ref.standard_e_step(*t)
    gc, lnc = O.c_standard_e_step(X, mu, var, lp)
    assert absd(g.numpy(), gc) < 1e-4 and rel(lnc, ln.numpy()) < 2e-6
    gf, lnf = ref.flash_e_step(*t, 4)
    assert absd(gf.numpy(), gc) < 1e-4
    m, v, l = (o.numpy() for o in ref.standard_m_step(t[0], torch.from_numpy(gc.astype(np.float32))))
    mc, vc, lc = O.c_standard_m_step(X, gc)
    assert absd(m, mc) < 1e-4 and absd(v, vc) < 1e-3 and absd(l, lc) < 1e-5


def test_fit_vs_reference_trajectory(ref):
    import torch
    from flashgmm_amd.configs import make_problem
    X, mu, var, lp = make_problem(1)
    traj, *_ = O.c_fit(X, mu, var, lp, 20)
    p = [torch.from_numpy(a) for a in (mu, var, lp)]
    Xt = torch.from_numpy(X)
    for it in range(20):
        m, v, l, ln = ref.flash_em_fused(Xt, *p, 64, 8)
        assert abs(float(ln.double().mean()) - traj[it]) <= 1e-4 * abs(traj[it])
        p = [m, v, l]


# ---------------------------------------------------------------------------
# planted mistakes: each mutant of the oracle must fail a check above
# ---------------------------------------------------------------------------
def _mutant_no_logdet(X, mu, var, lp):
    iv, lc = O.np_precompute(var, lp)
    lc = lc + 0.5 * np.log(np.asarray(var, np.float64)).sum(1)      # dropped log-det
    X = np.asarray(X, np.float64)
    L = np.stack([lc[k] - 0.5 * (((X - mu[k]) ** 2) * iv[k]).sum(1) for k in range(len(lc))], 1)
    m = L.max(1, keepdims=True)
    return m[:, 0] + np.log(np.exp(L - m).sum(1))


def _mutant_var_not_inverse(X, mu, var, lp):
    iv, lc = O.np_precompute(var, lp)
    X = np.asarray(X, np.float64)
    v = np.asarray(var, np.float64)                                   # var used as inv_var
    L = np.stack([lc[k] - 0.5 * (((X - mu[k]) ** 2) * v[k]).sum(1) for k in range(len(lc))], 1)
    m = L.max(1, keepdims=True)
    return m[:, 0] + np.log(np.exp(L - m).sum(1))


def _mutant_sign(X, mu, var, lp):
    iv, lc = O.np_precompute(var, lp)
    X = np.asarray(X, np.float64)
    L = np.stack([lc[k] + 0.5 * (((X - mu[k]) ** 2) * iv[k]).sum(1) for k in range(len(lc))], 1)
    m = L.max(1, keepdims=True)
    return m[:, 0] + np.log(np.exp(L - m).sum(1))


def _mutant_max_not_lse(X, mu, var, lp):
    return O.np_loglik(X, mu, var, lp).max(1)                          # hard max, no sum


@pytest.mark.parametrize("mutant", [_mutant_no_logdet, _mutant_var_not_inverse, _mutant_sign,
                                    _mutant_max_not_lse])
def test_mutants_rejected(mutant):
    caught = [not golden_ln_ok(mutant, load(p), tol=1e-6) for p in GOLDEN]
    assert any(caught), f"{mutant.__name__} passed every golden check"


def test_mutant_m_step_rejected():
    g = load([p for p in GOLDEN if "k4_d8" in p][0])
    N = g["X"].shape[0]
    mu = g["s_k"] / g["n_k"][:, None]
    var_centered_wrong = g["sq_k"] / g["n_k"][:, None] + mu * mu          # sign flip on mu^2
    assert absd(var_centered_wrong, g["new_var"]) > 1e-3
    lp_unclamped_wrong = np.log(g["n_k"])                                  # forgot / N
    assert absd(lp_unclamped_wrong, g["new_log_pi"]) > 1e-3
    _ = N
