"""Writes tests/golden/full_size/iter1_C<c>.npz: the fp64 oracle's one-iteration
output of a benchmark configuration at FULL size.

Contents:
  * new_mu, new_var, new_log_pi: float64;
  * the first iteration's log-normalizer, summarised:
    - ln_idx, ln_val: 8192 seeded sample rows and their values (float64);
    - ln_sum, ln_min, ln_max: over all N.

The GPU test (tests/test_gpu_parity.py::test_full_size_one_iteration) holds
the device's one fused iteration at that size to the parity bar, without
re-running the CPU oracle there. At C5 (N = 1048576) that run takes about a
minute on 8 cores.

Run from the repository root:  python tests/golden/make_full_iteration.py [cid ...]
(default: 5)
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from flashgmm_amd.configs import CONFIGS, make_problem  # noqa: E402
from oracle import oracle as O  # noqa: E402

SAMPLE = 8192


def main(cids):
    for cid in cids:
        cfg = CONFIGS[cid]
        t0 = time.time()
        X, mu, var, lp = make_problem(cid)
        _, _, _, ln, (n_k, s_k, sq_k) = O.c_em_fused(X, mu, var, lp, with_stats=True)
        m64, v64, l64 = O.c_m_step_update(n_k, s_k, sq_k, X.shape[0])
        idx = np.sort(np.random.default_rng(77).choice(cfg.N, SAMPLE, replace=False))
        path = os.path.join(HERE, "full_size", f"iter1_C{cid}.npz")
        np.savez_compressed(path, N=cfg.N, K=cfg.K, d=cfg.d,
                            new_mu=np.asarray(m64, np.float64),
                            new_var=np.asarray(v64, np.float64),
                            new_log_pi=np.asarray(l64, np.float64),
                            ln_idx=idx.astype(np.int64), ln_val=np.asarray(ln, np.float64)[idx],
                            ln_sum=float(np.sum(ln, dtype=np.float64)),
                            ln_min=float(np.min(ln)), ln_max=float(np.max(ln)))
        print(f"C{cid}: {path} ({os.path.getsize(path) / 1024:.0f} KiB) in "
              f"{time.time() - t0:.0f}s", flush=True)


if __name__ == "__main__":
    main([int(a) for a in sys.argv[1:]] or [5])
