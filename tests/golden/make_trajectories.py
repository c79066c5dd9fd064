"""Writes tests/golden/trajectories.json: the fp64 oracle's mean
log-likelihood trajectory for every benchmark configuration at FULL size
(20 iterations; 10 for C5), plus the first iteration's log-normalizer
summary statistics.  The GPU test compares the device EM loop against these
numbers without re-running the (minutes-long) CPU oracle.

Run from the repository root:  python tests/golden/make_trajectories.py [cid ...]
"""
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from flashgmm_amd.configs import CONFIGS, make_problem  # noqa: E402
from oracle import oracle as O  # noqa: E402


def main(cids):
    path = os.path.join(HERE, "trajectories.json")
    out = json.load(open(path)) if os.path.exists(path) else {}
    for cid in cids:
        cfg = CONFIGS[cid]
        t0 = time.time()
        X, mu, var, lp = make_problem(cid)
        traj, m, v, l = O.c_fit(X, mu, var, lp, cfg.iters)
        out[f"C{cid}"] = {"N": cfg.N, "K": cfg.K, "d": cfg.d, "iters": cfg.iters,
                          "ll": [float(x) for x in traj],
                          "final_mu_sum": float(m.astype("float64").sum()),
                          "final_var_sum": float(v.astype("float64").sum())}
        json.dump(out, open(path, "w"), indent=1)
        print(f"C{cid}: {cfg.iters} iterations in {time.time() - t0:.0f}s", flush=True)


if __name__ == "__main__":
    main([int(a) for a in sys.argv[1:]] or sorted(CONFIGS))
