"""Benchmark: fused Flash-GMM EM iterations per second on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 2] [--config 2] [--all]
                    [--variant auto|valu|mfma|x32|mixed|sparse] [--no-cpu-baseline]

A step is one fused EM iteration (precompute -> Pass 1 -> Pass 2 ->
reduction/M-step) over the configuration's full synthetic data set, which is
resident in HBM before timing starts.  The timed region runs ``steps``
iterations back to back on the device (parameters fed forward on the device,
no host synchronisation inside), bracketed by ``torch.cuda.synchronize()``.
Each pass's launch durations are measured live with HIP events on the launch
stream (``fgmm_profile_*``); the dominant kernel's give the roofline figure.

Default workload: configuration 2 (N=65536, K=256, d=128, fp32), the metric's
headline shape.  ``--all`` adds one JSON line per configuration after the
headline line.  The CPU baseline is the reference's own C++/OpenMP standard
E+M (``flash_gmm_cpu.cpp`` standard_e_step + standard_m_step) compiled into
``oracle/_ref``, timed on a bounded sample of the same workload on rank 0;
if that build is absent, this repository's fp32 restatement of it
(``oracle/fgmm_oracle.c``) is timed instead and labelled "port".
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

from flashgmm_amd.configs import CONFIGS, make_problem  # noqa: E402

HBM_PEAK = 8.0e12        # B/s, MI355X
FP32_PEAK = 157.3e12     # FLOP/s, MI355X dense fp32 (vector = matrix)
FP64_PEAK = 78.6e12      # FLOP/s, MI355X dense fp64 (vector = matrix)
BF16_PEAK = 2.5e15       # FLOP/s, MI355X dense bf16 matrix cores


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    ap.add_argument("--all", action="store_true", help="also report every configuration")
    ap.add_argument("--variant", default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="target CPU time for the baseline sample")
    ap.add_argument("--stream-chunk", type=int, default=0,
                    help="instead of the resident benchmark, time the streaming iteration "
                         "(X in pinned host memory, chunks of this many rows copied while "
                         "the previous chunk computes) on --config")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="before timing, run one plain device-to-device copy of this "
                         "many MiB (a known-size kernel to calibrate HBM byte counters)")
    return ap.parse_args()


def copy_probe(mib: int) -> None:
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def pass2_peak() -> float:
    # Pass 2's 8 flops per (n,k,j) run at different precisions: the distance
    # recompute (4) and sum gamma*x^2 (2) on fp64 matrix cores, sum gamma*x (2)
    # on fp32 matrix cores.  The binding peak is the time-weighted mix.
    return 8.0 / (6.0 / FP64_PEAK + 2.0 / FP32_PEAK)


FP32_SWEEP = ("x32", "mixed")   # Pass 1 on fp32 matrix cores
BF16_SWEEP = ("sparse",)        # Pass 1 on bf16 matrix cores, operands split hi + lo


def arithmetic_type(variant: str) -> str:
    """What the variant computes in (inputs and outputs are fp32 throughout)."""
    if variant in BF16_SWEEP:
        return ("f64 (pairs near each point's maximum, statistics, reduction) + "
                "bf16x3 matrix-core bound sweep with fp32 accumulation")
    if variant == "x32":
        return "f32 matrix-core sweeps with error bounds + f64 window pairs and reduction"
    if variant in ("mfma", "mixed"):
        return ("f64 matrix cores (distance, sum gamma x^2, reduction) + f32 (gamma, sum gamma x)"
                + (" + f32 matrix-core Pass-1 bound sweep" if variant == "mixed" else ""))
    return "f64 (vector ALU)"


def dominant_roofline(cfg, variant, kernels):
    """Roofline of the kernel that takes the most time per iteration.

    Pass 1 is a dense sweep over all (n, k): 4 flops per (n, k, j) (the
    x^2 and x contractions), on fp32 matrix cores for x32 and mixed, on fp64
    matrix cores (fp64 VALU for valu) for mfma/valu, and for sparse on bf16
    matrix cores with each operand split into bf16 hi + lo, three products
    (lo*hi, hi*lo, hi*hi) per algorithmic product.  The metric prices the
    algorithmic 4NKd against the fp32 matrix-core peak; for the bf16 sweep
    the issued matrix-core work (3 x 4NKd) against the bf16 peak is reported
    beside it.  The dense Pass 2 recomputes the distance and accumulates
    gamma^T [X, X^2]: 8 flops per (n, k, j) at its fp64/fp32 instruction mix.
    The sparse variant's Pass 2 touches only the listed pairs and is not
    dominant."""
    nkd = float(cfg.N) * cfg.K * cfg.d
    t1 = kernels["pass1"]["ms_avg"] / 1e3
    t2 = kernels["pass2"]["ms_avg"] / 1e3
    if variant == "sparse" or t1 >= t2:
        if variant in BF16_SWEEP:
            peak, unit = FP32_PEAK, "bf16 matrix cores, split operands"
        elif variant in FP32_SWEEP:
            peak, unit = FP32_PEAK, "fp32 matrix cores"
        else:
            peak, unit = FP64_PEAK, "fp64"
        flops, t = 4.0 * nkd, t1
        out = {"kernel": f"pass1 (log-normalizer sweep, {unit})", "peak": peak / 1e12}
        if variant in BF16_SWEEP and t > 0:
            issued = 3.0 * flops
            out["issued_bf16_mfma"] = {"flops_per_launch": issued,
                                       "achieved": issued / t / 1e12, "peak": BF16_PEAK / 1e12,
                                       "unit": "TFLOP/s", "frac": issued / t / BF16_PEAK}
    else:
        flops, t = 8.0 * nkd, t2
        peak = FP32_PEAK
        out = {"kernel": "pass2 (gamma recompute + sufficient statistics)",
               "peak": peak / 1e12,
               "peak_at_kernel_precision": pass2_peak() / 1e12}
    achieved = flops / t if t > 0 else 0.0
    out.update({"bound": "mfma", "achieved": achieved / 1e12, "unit": "TFLOP/s",
                "frac": achieved / peak, "flops_per_launch": flops})
    if "peak_at_kernel_precision" in out:
        out["frac_at_kernel_precision"] = achieved / pass2_peak()
    return out


def run_gpu(cid, steps, warmup, variant):
    import torch
    from flashgmm_amd import _lib
    from flashgmm_amd import flash_gmm_native as C

    cfg = CONFIGS[cid]
    dev = torch.device("cuda:0")
    X, mu0, var0, lp0 = make_problem(cid)
    Xd = torch.from_numpy(X).to(dev)
    mu = torch.from_numpy(mu0).to(dev)
    var = torch.from_numpy(var0).to(dev)
    lp = torch.from_numpy(lp0).to(dev)
    lib = _lib.load()
    vname = C.resolve_variant(cfg.N, cfg.K, cfg.d, variant)

    # warmup (also builds the workspace)
    if warmup > 0:
        C.em_fit(Xd, mu, var, lp, warmup, variant=variant)
    torch.cuda.synchronize()
    _lib.check(lib.fgmm_profile_enable(1))
    ms = (ctypes.c_double * 4)()
    cnt = (ctypes.c_long * 4)()
    _lib.check(lib.fgmm_profile_read(ms, cnt))  # reset
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    mu_o, var_o, lp_o, traj = C.em_fit(Xd, mu, var, lp, steps, variant=variant)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _lib.check(lib.fgmm_profile_read(ms, cnt))
    _lib.check(lib.fgmm_profile_enable(0))
    # the same loop without events, for the headline number
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    C.em_fit(Xd, mu, var, lp, steps, variant=variant)
    torch.cuda.synchronize()
    elapsed_clean = time.perf_counter() - t0
    ll = traj.cpu().numpy()
    kern = {name: {"ms_avg": ms[i] / max(cnt[i], 1), "launches": int(cnt[i])}
            for i, name in enumerate(["precompute", "pass1", "pass2", "reduce_mstep"])}
    return {"elapsed": min(elapsed, elapsed_clean), "elapsed_profiled": elapsed,
            "kernels": kern, "ll_first": float(ll[0]), "ll_last": float(ll[-1]),
            "variant": vname}


def run_stream(cid, steps, warmup, chunk, variant):
    """Streaming iterations: X stays in pinned host memory, every iteration
    copies it to the device once, chunk by chunk, overlapped with compute."""
    import torch
    from flashgmm_amd import streaming

    cfg = CONFIGS[cid]
    dev = torch.device("cuda:0")
    X, mu0, var0, lp0 = make_problem(cid)
    Xh = torch.from_numpy(X).pin_memory()
    p = [torch.from_numpy(a).to(dev) for a in (mu0, var0, lp0)]
    gmm = streaming.StreamingFlashGMMAsync(chunk_size=chunk, variant=variant)
    for _ in range(warmup):
        p = list(gmm.em_step(Xh, *p)[:3])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    lls = []
    for _ in range(steps):
        out = gmm.em_step(Xh, *p)
        p = list(out[:3])
        lls.append(gmm.ll_mean)
    torch.cuda.synchronize()
    sec = time.perf_counter() - t0
    return {
        "metric": "EM iters/s, X streamed from pinned host memory (N=%d,K=%d,d=%d fp32)"
                  % (cfg.N, cfg.K, cfg.d),
        "value": steps / sec, "unit": "iter/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": 1000 * sec / steps, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f64", "data": "synthetic",
        "config": {"workload": f"C{cid} streamed: diag-cov GMM EM N={cfg.N} K={cfg.K} d={cfg.d} fp32",
                   "N": cfg.N, "K": cfg.K,
                   "d": cfg.d, "chunk_rows": chunk},
        "host_to_device_GBps": cfg.N * cfg.d * 4 / (sec / steps) / 1e9,
        "ll_last": float(lls[-1].item()),
    }


def cpu_baseline(cid, budget_s):
    """Times the reference's standard E+M on the host (bounded sample)."""
    import torch
    from oracle import oracle as O

    cfg = CONFIGS[cid]
    cores = len(os.sched_getaffinity(0))
    X, mu, var, lp = make_problem(cid)
    ref = O.ref_module()
    if ref is not None:
        torch.set_num_threads(cores)
        Xt, mut, vt, lpt = (torch.from_numpy(a) for a in (X, mu, var, lp))

        def one():
            g, _ = ref.standard_e_step(Xt, mut, vt, lpt)
            ref.standard_m_step(Xt, g)
        kind = "reference"
    else:
        def one():
            O.c32_standard_em(X, mu, var, lp)
        kind = "port"
    one()  # warm-up iteration
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s or len(times) >= cfg.iters:
            break
    per = float(np.mean(times))
    return {"value": 1.0 / per, "unit": "EM iters/s", "cores": cores, "kind": kind,
            "sample": f"{len(times)} standard E+M iteration(s) of C{cid} at full size "
                      f"(N={cfg.N}, K={cfg.K}, d={cfg.d}) after 1 warm-up, "
                      f"{per*1000:.1f} ms each"}


def measured_traffic(cid, variant, kernel):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 counter runs (profiles/hbm_traffic.json), or None when that
    workload, variant and kernel were not profiled."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        rec = json.load(open(path)).get(f"C{cid}")
    except (OSError, ValueError):
        return None
    if not rec or rec.get("variant") != variant:
        return None
    r = rec.get(kernel.split(" ")[0])
    return None if r is None else r["read_bytes"] + r["write_bytes"]


def line_for(cid, args, with_cpu):
    cfg = CONFIGS[cid]
    r = run_gpu(cid, args.steps, args.warmup, args.variant)
    sec = r["elapsed"]
    its = args.steps / sec
    F_total = cfg.flops_per_iter()
    roof_t = max(F_total / FP32_PEAK, cfg.bytes_per_iter() / HBM_PEAK)
    roof = dominant_roofline(cfg, r["variant"], r["kernels"])
    roof["traffic"] = measured_traffic(cid, r["variant"], roof["kernel"])
    roof["traffic_unit"] = "HBM bytes/launch (rocprofv3 FETCH_SIZE x2 + WRITE_SIZE, profiles/)"
    out = {
        "metric": "EM iters/s (N=65536,K=256,d=128 fp32) + % of HBM / fp32-MFMA roofline",
        "value": its,
        "unit": "EM iters/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sec * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": arithmetic_type(r["variant"]),
        "data": "synthetic (seeded mixture generator, flashgmm_amd/configs.py)",
        "config": {"workload": f"C{cid}: diag-cov GMM EM N={cfg.N} K={cfg.K} d={cfg.d} fp32",
                   "N": cfg.N, "K": cfg.K, "d": cfg.d, "kernel_variant": r["variant"]},
        "roofline": roof,
        "iteration_roofline_frac": roof_t / (sec / args.steps),
        "kernels_ms": {k: v["ms_avg"] for k, v in r["kernels"].items()},
        "ll_first": r["ll_first"],
        "ll_last": r["ll_last"],
    }
    if with_cpu:
        out["cpu_baseline"] = cpu_baseline(cid, args.cpu_seconds)
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "the multi-GPU layout is described in DESIGN.md", file=sys.stderr)
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))
    if args.copy_probe_mib > 0:
        copy_probe(args.copy_probe_mib)
    if args.stream_chunk > 0:
        if rank == 0:
            print(json.dumps(run_stream(args.config, args.steps, args.warmup, args.stream_chunk,
                                        args.variant)), flush=True)
        return
    head = line_for(args.config, args, with_cpu=(rank == 0 and not args.no_cpu_baseline))
    if rank == 0:
        print(json.dumps(head), flush=True)
    if args.all:
        for cid in sorted(CONFIGS):
            if cid == args.config:
                continue
            o = line_for(cid, args, with_cpu=False)
            if rank == 0:
                print(json.dumps(o), flush=True)


if __name__ == "__main__":
    main()
