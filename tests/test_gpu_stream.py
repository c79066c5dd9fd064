"""Streaming EM iteration (X fed in chunks from host or device memory)
against the fp64 oracle and against the resident fused iteration.

Tolerances: mu, var |gpu - fp64| <= 1e-5 (one fp32 ulp from 256 up); pi <= 1e-5; the
log-normalizer is per point, so it must equal the resident Pass 1 bit for
bit; the mean log-likelihood matches the oracle to 1e-10 relative.
"""
import numpy as np
import pytest

from parity_util import check_params, oracle_iter, problem, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cls,where,chunk", [
    ("StreamingFlashGMM", "host", 20000),
    ("StreamingFlashGMMAsync", "host", 20000),
    ("StreamingFlashGMMAsync", "pinned", 16384),
    ("StreamingFlashGMM", "device", 8192),
    ("StreamingFlashGMMAsync", "host", 1 << 20),        # one chunk
])
def test_streamed_iteration_matches_oracle(cuda, cls, where, chunk):
    import torch
    from flashgmm_amd import flash_gmm_native as C
    from flashgmm_amd import streaming
    X, mu, var, lp = problem(2, None)
    m64, v64, l64, ln64, *_ = oracle_iter(2, None)
    p = to_dev(cuda, mu, var, lp)
    Xt = torch.from_numpy(X)
    if where == "pinned":
        Xt = Xt.pin_memory()
    elif where == "device":
        Xt = Xt.to(cuda)
    print(f"[case] {cls} X on {where} chunk={chunk}", flush=True)
    gmm = getattr(streaming, cls)(chunk_size=chunk)
    new_mu, new_var, new_lp, ln = gmm.em_step(Xt, *p)
    check_params([t.cpu().numpy() for t in (new_mu, new_var, new_lp)], (m64, v64, l64),
                 f"{cls} {where}")
    ln_res = C.flash_log_normalizer(torch.from_numpy(X).to(cuda), *p)
    assert torch.equal(ln, ln_res)
    ll = gmm.ll_mean.item()
    assert abs(ll - ln64.mean()) <= 1e-10 * abs(ln64.mean())


def test_streamed_ragged_small_and_x32_request(cuda):
    """Chunk sizes that leave a short last chunk, d not a multiple of 4,
    and an x32 request (the streaming path runs the fp64 matrix cores)."""
    import torch
    from flashgmm_amd import streaming
    from oracle import oracle as O
    rng = np.random.default_rng(5)
    N, K, d = 3001, 17, 33
    X = (rng.uniform(-3, 3, (K, d))[rng.integers(0, K, N)] + rng.normal(0, 1, (N, d))).astype(np.float32)
    mu = X[rng.choice(N, K, replace=False)].copy()
    var = rng.uniform(0.5, 2.0, (K, d)).astype(np.float32)
    lp = np.log(rng.dirichlet(np.ones(K))).astype(np.float32)
    ref = O.c_em_fused(X, mu, var, lp)
    p = to_dev(cuda, mu, var, lp)
    for chunk, variant in ((700, None), (64, "valu"), (1000, "x32"), (333, "mixed"),
                           (500, "sparse")):
        print(f"[case] ragged stream chunk={chunk} variant={variant}", flush=True)
        out = streaming.StreamingFlashGMMAsync(chunk_size=chunk, variant=variant).em_step(
            torch.from_numpy(X), *p)
        check_params([t.cpu().numpy() for t in out[:3]], ref[:3], f"ragged {chunk} {variant}")
        e = np.abs(out[3].cpu().numpy() - ref[3]) / np.abs(ref[3])
        assert e.max() <= 1e-5
