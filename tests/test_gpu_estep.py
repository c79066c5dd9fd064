"""GPU parity of the gamma-returning E-steps (flash_e_step, standard_e_step)
and the standard M-step, through the C ABI, against the fp64 oracle.

Tolerances:
  * gamma: absolute error <= 1e-6 (gamma lies in [0, 1]);
  * log_normalizer: relative error <= 1e-5;
  * standard M-step mu, var: |gpu - fp64| <= 1e-5 below 256, one fp32 ulp from 256 up
    (parity_util.param_tol),
    pi = exp(log_pi): <= 1e-5 -- from the same fp32 gamma the device gets;
  * NativeStandardGMM mean log-likelihood trajectory: relative <= 1e-4.
"""
import functools

import numpy as np
import pytest

from oracle import oracle as O
from parity_util import check_gamma, check_ln, check_params, problem, to_dev

pytestmark = pytest.mark.gpu

CASES = [(1, None), (2, 16384), (3, 16384), (4, 8192), (5, 16384)]
IDS = [f"C{c}" + (f"_N{n}" if n else "") for c, n in CASES]


def variants_for(K, d):
    return ["valu"] + (["mfma"] if d <= 128 else [])


@functools.lru_cache(maxsize=None)
def oracle_gamma(cid, N):
    X, mu, var, lp = problem(cid, N)
    return O.c_standard_e_step(X, mu, var, lp)


def random_problem(N, K, d, seed=11):
    rng = np.random.default_rng(seed)
    X = (rng.uniform(-4, 4, (K, d))[rng.integers(0, K, N)] + rng.normal(0, 1, (N, d)))
    X = X.astype(np.float32)
    mu = (X[rng.choice(N, K, replace=N < K)] + rng.normal(0, 0.1, (K, d))).astype(np.float32)
    var = rng.uniform(0.5, 2.0, (K, d)).astype(np.float32)
    lp = np.log(rng.dirichlet(np.ones(K))).astype(np.float32)
    return X, mu, var, lp


@pytest.mark.parametrize("cid,N", CASES, ids=IDS)
def test_e_steps_match_oracle(cuda, cid, N):
    from flashgmm_amd import flash_gmm_native as C
    X, mu, var, lp = problem(cid, N)
    g_ref, ln_ref = oracle_gamma(cid, N)
    t = to_dev(cuda, X, mu, var, lp)
    for variant in variants_for(*mu.shape):
        for fn in ("flash_e_step", "standard_e_step"):
            label = f"{fn} C{cid} N={X.shape[0]} {variant}"
            print(f"[case] {label}", flush=True)
            g, ln = getattr(C, fn)(*t, variant=variant)
            assert g.shape == (X.shape[0], mu.shape[0]) and ln.shape == (X.shape[0],)
            check_ln(ln.cpu().numpy(), ln_ref, label)
            check_gamma(g.cpu().numpy(), g_ref, label)


E_EDGE = {
    "N1": (1, 3, 5), "K1": (300, 1, 7), "d1": (257, 4, 1), "d33_K17": (1000, 17, 33),
    "d256": (300, 5, 256), "d130_K20": (100, 20, 130), "K33_N1025": (1025, 33, 64),
    "K70_d16": (513, 70, 16),
}


@pytest.mark.parametrize("name", sorted(E_EDGE))
def test_e_steps_edge_shapes(cuda, name):
    from flashgmm_amd import flash_gmm_native as C
    N, K, d = E_EDGE[name]
    X, mu, var, lp = random_problem(N, K, d)
    g_ref, ln_ref = O.c_standard_e_step(X, mu, var, lp)
    t = to_dev(cuda, X, mu, var, lp)
    for variant in variants_for(K, d):
        for fn in ("flash_e_step", "standard_e_step"):
            label = f"{fn} {name} {variant}"
            print(f"[case] {label}", flush=True)
            g, ln = getattr(C, fn)(*t, variant=variant)
            check_ln(ln.cpu().numpy(), ln_ref, label)
            check_gamma(g.cpu().numpy(), g_ref, label)


def _std_m_ref(X, g32):
    return O.c_standard_m_step(X, g32.astype(np.float64))


@pytest.mark.parametrize("cid,N", CASES, ids=IDS)
def test_standard_m_step_matches_oracle(cuda, cid, N):
    from flashgmm_amd import flash_gmm_native as C
    X, *_ = problem(cid, N)
    g32 = oracle_gamma(cid, N)[0].astype(np.float32)
    ref = _std_m_ref(X, g32)
    Xd, gd = to_dev(cuda, X, g32)
    print(f"[case] standard_m_step C{cid} N={X.shape[0]}", flush=True)
    out = [o.cpu().numpy() for o in C.standard_m_step(Xd, gd)]
    check_params(out, ref, f"standard_m_step C{cid}")


@pytest.mark.parametrize("name", sorted(E_EDGE))
def test_standard_m_step_edge_shapes(cuda, name):
    from flashgmm_amd import flash_gmm_native as C
    N, K, d = E_EDGE[name]
    X, mu, var, lp = random_problem(N, K, d)
    g32 = O.c_standard_e_step(X, mu, var, lp)[0].astype(np.float32)
    print(f"[case] standard_m_step {name}", flush=True)
    out = [o.cpu().numpy() for o in C.standard_m_step(*to_dev(cuda, X, g32))]
    check_params(out, _std_m_ref(X, g32), f"standard_m_step {name}")


def test_standard_m_step_empty_component_and_unaligned(cuda):
    """A component with no responsibility gets NaN mean/variance and
    log_pi = -inf (no clamp, as the reference's ATen M-step); gamma and X at
    4-byte offsets and K not a multiple of 4 take the scalar load path."""
    import torch
    from flashgmm_amd import flash_gmm_native as C
    X, mu, var, lp = random_problem(2000, 7, 40, seed=5)
    g32 = O.c_standard_e_step(X, mu, var, lp)[0].astype(np.float32)
    g32[:, 3] = 0.0
    ref = _std_m_ref(X, g32)
    assert np.isnan(ref[0][3]).all() and ref[2][3] == -np.inf
    bx = torch.zeros(X.size + 1, dtype=torch.float32, device=cuda)
    bx[1:] = torch.from_numpy(X.ravel()).to(cuda)
    bg = torch.zeros(g32.size + 1, dtype=torch.float32, device=cuda)
    bg[1:] = torch.from_numpy(g32.ravel()).to(cuda)
    Xu, gu = bx[1:].view(X.shape), bg[1:].view(g32.shape)
    assert Xu.data_ptr() % 16 != 0 and gu.data_ptr() % 16 != 0
    print("[case] standard_m_step empty component, unaligned", flush=True)
    mu2, var2, lp2 = (o.cpu().numpy() for o in C.standard_m_step(Xu, gu))
    assert np.isnan(mu2[3]).all() and np.isnan(var2[3]).all() and lp2[3] == -np.inf
    keep = [k for k in range(7) if k != 3]
    check_params((mu2[keep], var2[keep], lp2[keep]),
                 (ref[0][keep], ref[1][keep], ref[2][keep]), "empty component")


def test_native_standard_gmm_trajectory(cuda):
    """NativeStandardGMM.fit against the same loop on the fp64 oracle (gamma
    and parameters rounded to fp32 between steps, as the device keeps them),
    from the wrapper's own initialisation; and against NativeFlashGMM."""
    import torch
    from flashgmm_amd.native_wrapper import NativeFlashGMM, NativeStandardGMM, _init_params
    X, *_ = problem(1, None)
    Xd = torch.from_numpy(X).to(cuda)
    print("[case] NativeStandardGMM C1 10 iterations", flush=True)
    h = NativeStandardGMM(K=8, d=32, max_iter=10, tol=0.0).fit(Xd)
    assert [r["iter"] for r in h] == list(range(10))
    mu, var, lp = (t.cpu().numpy() for t in _init_params(8, 32, 42, Xd))
    traj = []
    for _ in range(10):
        g, ln = O.c_standard_e_step(X, mu, var, lp)
        traj.append(ln.mean())
        mu, var, lp = (a.astype(np.float32) for a in _std_m_ref(X, g.astype(np.float32)))
    got = np.array([r["log_likelihood"] for r in h])
    e = np.abs(got - np.array(traj)) / np.abs(np.array(traj))
    assert e.max() <= 1e-4, f"standard trajectory rel err {e.max():.3e}"
    hf = NativeFlashGMM(K=8, d=32, max_iter=10, tol=0.0).fit(Xd)
    for a, b in zip(h, hf):
        assert abs(a["log_likelihood"] - b["log_likelihood"]) <= 1e-5 * abs(b["log_likelihood"])
    # early stop follows the reference rule |dLL| < tol
    h3 = NativeStandardGMM(K=8, d=32, max_iter=100, tol=1e-4).fit(Xd)
    assert len(h3) < 100 and abs(h3[-1]["log_likelihood"] - h3[-2]["log_likelihood"]) < 1e-4


def test_predict_proba_and_predict(cuda):
    import torch
    from flashgmm_amd.native_wrapper import NativeFlashGMM, NativeStandardGMM
    X, *_ = problem(1, None)
    Xd = torch.from_numpy(X).to(cuda)
    for cls in (NativeFlashGMM, NativeStandardGMM):
        print(f"[case] {cls.__name__}.predict_proba", flush=True)
        gmm = cls(K=8, d=32, max_iter=5, tol=0.0)
        gmm.fit(Xd)
        g_ref, _ = O.c_standard_e_step(X, *(t.cpu().numpy() for t in (gmm.mu, gmm.var,
                                                                       gmm.log_pi)))
        check_gamma(gmm.predict_proba(Xd).cpu().numpy(), g_ref, f"{cls.__name__} proba")
        top2 = np.sort(g_ref, axis=1)[:, -2:]
        sure = (top2[:, 1] - top2[:, 0]) > 1e-4
        pred = gmm.predict(Xd).cpu().numpy()
        assert np.array_equal(pred[sure], g_ref.argmax(1)[sure])


def test_flash_e_step_large_full_size_properties(cuda):
    """C2 at full size: rows of gamma sum to 1 and the standard and flash
    E-steps agree; gamma fed to standard_m_step reproduces one fused
    iteration (the fused path's clamps are inactive here)."""
    import torch
    from flashgmm_amd import flash_gmm_native as C
    X, mu, var, lp = problem(2, None)
    t = to_dev(cuda, X, mu, var, lp)
    print("[case] C2 full-size E-step properties", flush=True)
    gf, lnf = C.flash_e_step(*t)
    gs, lns = C.standard_e_step(*t)
    assert (gf.double().sum(1) - 1).abs().max().item() <= 1e-5
    assert (gf - gs).abs().max().item() <= 1e-6
    assert ((lnf.double() - lns.double()).abs() / lns.double().abs()).max().item() <= 1e-6
    fused = C.flash_em_fused(*t)
    std = C.standard_m_step(t[0], gf)
    for a, b in zip(fused[:3], std):
        assert (a.double() - b.double()).abs().max().item() <= 2e-5
    del gs
    torch.cuda.synchronize()
