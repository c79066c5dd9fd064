"""Benchmark: fused Flash-GMM EM iterations per second on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 2] [--config 2]
                    [--configs 1,2,3,4,5] [--variant auto|valu|mfma|x32|mixed|sparse]
                    [--no-cpu-baseline] [--cpu-seconds S]

A step is one fused EM iteration (precompute -> Pass 1 -> Pass 2 ->
reduction/M-step) over the configuration's full synthetic data set, which is
resident in HBM before timing starts.  The timed region runs ``steps``
iterations back to back on the device (parameters fed forward on the device,
no host synchronisation inside), bracketed by ``torch.cuda.synchronize()``.

Each configuration runs twice after the warm-up:
  * a clean run: its wall time is ``value`` / ``ms_per_step``;
  * a profiled run: HIP events on the launch stream around every pass
    (``fgmm_profile_*``) give the per-pass durations and the dominant
    kernel's roofline; its own wall time is reported beside the event sums,
    which it contains.

ONE JSON line is printed.  Its top level describes the headline
configuration (default C2: N=65536, K=256, d=128, fp32, the metric's shape);
``configs`` holds the same figures for every configuration in --configs
(default all five; C5 runs its own 10-iteration step count).

Roofline figures are utilisation of the units that execute the work:
  * ``roofline``: the dominant kernel's issued work against its unit's peak.
    For the sparse variant's Pass 1 that is the bf16 matrix-core sweep,
    3 x 4NKd products (operands split hi + lo), against 2.5 PFLOP/s.
  * ``work_model``: the iteration's executed work -- the issued matrix-core
    flops at their precisions, the fp64 work on the listed pairs, the
    algorithmic HBM bytes -- priced at the peaks, over the measured time.
The metric's own framing (4NKd fp32-class products per Pass 1 against the
157.3 TFLOP/s fp32 matrix-core peak) is kept as a rate,
``fp32_class_tflops``, and as ``t_fp32_roofline_over_t`` (how many times
faster than an fp32 matrix-core kernel at peak could run the same products):
a ratio, not a utilisation.

The CPU baseline is the reference's own C++/OpenMP standard E+M
(``flash_gmm_cpu.cpp`` standard_e_step + standard_m_step) compiled into
``oracle/_ref``, timed on all host cores on a bounded sample of each
configuration on rank 0; if that build is absent, this repository's fp32
restatement of it (``oracle/fgmm_oracle.c``) is timed instead and labelled
"port".
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

from flashgmm_amd.configs import CONFIGS, Config, make_problem, make_shape  # noqa: E402

HBM_PEAK = 8.0e12        # B/s, MI355X
FP32_PEAK = 157.3e12     # FLOP/s, MI355X dense fp32 (vector = matrix)
FP64_PEAK = 78.6e12      # FLOP/s, MI355X dense fp64 (vector = matrix)
BF16_PEAK = 2.5e15       # FLOP/s, MI355X dense bf16 matrix cores
METRIC = "EM iters/s (N=65536,K=256,d=128 fp32) + % of HBM / fp32-MFMA roofline"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    ap.add_argument("--configs", default=",".join(str(c) for c in sorted(CONFIGS)),
                    help="configurations reported in the line's `configs` array")
    ap.add_argument("--variant", default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=4.0,
                    help="target CPU time per configuration for the baseline sample")
    ap.add_argument("--stream-chunk", type=int, default=0,
                    help="instead of the resident benchmark, time the streaming iteration "
                         "(X in pinned host memory, chunks of this many rows copied while "
                         "the previous chunk computes) on --config")
    ap.add_argument("--shape", default=None,
                    help="N,K,d: instead of the five configurations, time this shape "
                         "(configs.make_shape; one JSON line of its own)")
    ap.add_argument("--overlap", action="store_true",
                    help="with --shape: all components nearly identical (the sparse "
                         "variant's worst case: every point takes the dense path)")
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


def arithmetic_type(variant: str) -> str:
    """What the variant computes in (inputs and outputs are fp32 throughout)."""
    if variant == "sparse":
        return ("f64 (pairs near each point's maximum, statistics, reduction) + "
                "bf16x3 matrix-core bound sweep with fp32 accumulation")
    if variant == "x32":
        return "f32 matrix-core sweeps with error bounds + f64 window pairs and reduction"
    if variant in ("mfma", "mixed"):
        return ("f64 matrix cores (distance, sum gamma x^2, reduction) + f32 (gamma, sum gamma x)"
                + (" + f32 matrix-core Pass-1 bound sweep" if variant == "mixed" else ""))
    if variant == "small":
        return "f64 (vector ALU; every stage of an iteration in one launch)"
    return "f64 (vector ALU)"


def padded(cfg, variant):
    """(Kp, dp, dpb) as the library pads them for the matrix-core kernels."""
    Kp = (cfg.K + 31) // 32 * 32
    dp = (cfg.d + 15) // 16 * 16
    return Kp, dp, (dp + 31) // 32 * 32


def pass_work(cfg, variant, which):
    """(issued flops per launch, peak FLOP/s of that instruction mix, unit)
    of Pass 1 or Pass 2 over the padded problem (Kp, dp / dpb).

    Pass 1: sparse issues 3 bf16 products (lo*hi, hi*lo, hi*hi of the split
    operands) per fp32-class product, 2 flops each, over the Kp x 2dpb
    contraction; x32 / mixed one fp32 product over Kp x 2dp; mfma one fp64
    product.  Pass 2 (dense): the distance recompute (Kp x 2dp) plus
    sum gamma x (dp) and sum gamma x^2 (dp) per pair -- mfma / mixed: the
    distance and sum gamma x^2 on fp64, sum gamma x on fp32 matrix cores;
    x32: distance and sum gamma x on fp32, sum gamma x^2 on fp64.  The peak of
    a mix is its time-weighted one.  valu: 4NKd (Pass 1) or 8NKd (Pass 2) on
    the fp64 vector ALU."""
    N = float(cfg.N)
    Kp, dp, dpb = padded(cfg, variant)
    if variant == "small":   # one launch: distance (4) + statistics (4) per (n, k, j), fp64
        return 8.0 * N * cfg.K * cfg.d, FP64_PEAK, "fp64 vector ALU, one launch per iteration"
    if variant == "valu":
        f = (4.0 if which == 1 else 8.0) * N * cfg.K * cfg.d
        return f, FP64_PEAK, "fp64 vector ALU"
    if which == 1:
        if variant == "sparse":
            return 3 * 2 * N * Kp * 2 * dpb, BF16_PEAK, "bf16 matrix cores"
        if variant in ("x32", "mixed"):
            return 2 * N * Kp * 2 * dp, FP32_PEAK, "fp32 matrix cores"
        return 2 * N * Kp * 2 * dp, FP64_PEAK, "fp64 matrix cores"
    dist, half = 2 * N * Kp * 2 * dp, 2 * N * Kp * dp
    if variant == "x32":
        f32, f64 = dist + half, half
    else:
        f32, f64 = half, dist + half
    return f32 + f64, (f32 + f64) / (f32 / FP32_PEAK + f64 / FP64_PEAK), "fp64/fp32 matrix cores"


def dominant_roofline(cfg, variant, kernels):
    """Utilisation of the kernel that takes the most time per iteration: its
    issued work per launch (pass_work) over its average launch duration,
    against the peak of the units that execute it.  The sparse variant's
    Pass 2 works on the listed pairs only and is never the dense sweep, so
    Pass 1 is its kernel."""
    nkd = float(cfg.N) * cfg.K * cfg.d
    t1 = kernels["pass1"]["ms_avg"] / 1e3
    t2 = kernels["pass2"]["ms_avg"] / 1e3
    which = 1 if (variant in ("sparse", "small") or t1 >= t2) else 2
    t = t1 if which == 1 else t2
    issued, peak, unit = pass_work(cfg, variant, which)
    name = ("fused iteration (all stages" if variant == "small"
            else "pass1 (log-normalizer sweep" if which == 1
            else "pass2 (gamma recompute + sufficient statistics")
    achieved = issued / t if t > 0 else 0.0
    out = {"kernel": f"{name}, {unit})", "bound": "mfma", "achieved": achieved / 1e12,
           "peak": peak / 1e12, "unit": "TFLOP/s", "frac": achieved / peak,
           "flops_per_launch": issued, "launch_ms": t * 1e3}
    if which == 1 and variant in ("sparse", "x32", "mixed") and t > 0:
        out["fp32_class_tflops"] = 4 * nkd / t / 1e12
        out["t_fp32_roofline_over_t"] = (4 * nkd / FP32_PEAK) / t
    return out


def work_model(cfg, variant, ms_per_step, counts):
    """Executed work of one iteration priced at the units' peaks.

    sparse: the bf16 sweep (3 x 2 x N x Kp x 2dpb), fp64 work on the listed
    entries (Pass 1 evaluates each exactly: ~4 flops per feature; Pass 2
    accumulates gamma, gamma x, gamma x^2: 4 flops per feature), the dense
    fp64 pass over the components the reduction flagged (8 x N x 16 x dp
    per 16-component subtile), and HBM bytes: X read by both passes, the
    lists written and read (12 B per entry), the log-normalizer and
    parameters.  Dense variants: both passes' issued work (pass_work)."""
    N = float(cfg.N)
    Kp, dp, dpb = padded(cfg, variant)
    B = cfg.bytes_per_iter()
    if variant == "sparse":
        E = float(counts.get("entries", 0))
        flagged = float(counts.get("flagged", 0))
        t_mfma = 3 * 2 * N * Kp * 2 * dpb / BF16_PEAK
        f64 = E * 4 * cfg.d * 2 + ((flagged + 15) // 16) * 16 * 8 * N * dp
        t_f64 = f64 / FP64_PEAK
        B += 2 * 12 * E
        parts = {"bf16_sweep_us": t_mfma * 1e6, "fp64_us": t_f64 * 1e6,
                 "listed_entries": int(E), "flagged_components": int(flagged)}
        t_c = t_mfma + t_f64
    elif variant == "small":
        f1, p1, _ = pass_work(cfg, variant, 1)
        t_c = f1 / p1
        parts = {"fused_us": t_c * 1e6}
    else:
        f1, p1, _ = pass_work(cfg, variant, 1)
        f2, p2, _ = pass_work(cfg, variant, 2)
        t_c = f1 / p1 + f2 / p2
        parts = {"pass1_us": f1 / p1 * 1e6, "pass2_us": f2 / p2 * 1e6}
    t_b = B / HBM_PEAK
    t_model = max(t_c, t_b)
    t = ms_per_step / 1e3
    return {"t_model_us": t_model * 1e6, "bound": "compute" if t_c >= t_b else "hbm",
            "compute_us": t_c * 1e6, "hbm_us": t_b * 1e6, "hbm_bytes": B,
            "frac": t_model / t if t > 0 else 0.0, **parts}


def sparse_counts(lib, cfg, variant, ws):
    """Counts of the last timed iteration, read from the workspace."""
    import torch
    if variant != "sparse":
        return {}
    out = {}
    vcode = 5
    for name in ("pcnt", "nflag"):
        off, nb = ctypes.c_size_t(), ctypes.c_size_t()
        if lib.fgmm_workspace_region(cfg.N, cfg.K, cfg.d, vcode, name.encode(),
                                     ctypes.byref(off), ctypes.byref(nb)) != 0:
            return {}
        view = ws[off.value:off.value + nb.value].view(torch.int32)
        if name == "pcnt":
            cap = min(cfg.K, 16)
            out["entries"] = int(view.clamp(max=cap).sum().item())
            out["overflow_points"] = int((view > cap).sum().item())
        else:
            out["flagged"] = int(view[0].item())
    return out


def run_gpu(cfg, problem, steps, warmup, variant):
    import torch
    from flashgmm_amd import _lib
    from flashgmm_amd import flash_gmm_native as C

    dev = torch.device("cuda:0")
    X, mu0, var0, lp0 = problem
    Xd = torch.from_numpy(X).to(dev)
    mu = torch.from_numpy(mu0).to(dev)
    var = torch.from_numpy(var0).to(dev)
    lp = torch.from_numpy(lp0).to(dev)
    lib = _lib.load()
    vname = C.resolve_variant(cfg.N, cfg.K, cfg.d, variant)
    wsb = lib.fgmm_em_fused_workspace_bytes(cfg.N, cfg.K, cfg.d, _lib.variant_code(variant))

    if warmup > 0:   # also builds the workspace
        C.em_fit(Xd, mu, var, lp, warmup, variant=variant)
    torch.cuda.synchronize()
    # clean run: the headline
    t0 = time.perf_counter()
    _, _, _, traj = C.em_fit(Xd, mu, var, lp, steps, variant=variant)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    switched = int(lib.fgmm_em_fit_switch_iteration())
    counts = sparse_counts(lib, cfg, vname, _lib.workspace(dev, wsb))
    # profiled run: per-pass HIP events on the launch stream
    _lib.check(lib.fgmm_profile_enable(1))
    ms = (ctypes.c_double * 4)()
    cnt = (ctypes.c_long * 4)()
    _lib.check(lib.fgmm_profile_read(ms, cnt))  # reset
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    C.em_fit(Xd, mu, var, lp, steps, variant=variant)
    torch.cuda.synchronize()
    elapsed_prof = time.perf_counter() - t0
    _lib.check(lib.fgmm_profile_read(ms, cnt))
    _lib.check(lib.fgmm_profile_enable(0))
    ll = traj.cpu().numpy()
    kern = {name: {"ms_avg": ms[i] / max(cnt[i], 1), "launches": int(cnt[i]),
                   "ms_per_step": ms[i] / steps}
            for i, name in enumerate(["precompute", "pass1", "pass2", "reduce_mstep"])}
    del Xd, mu, var, lp
    return {"elapsed": elapsed, "elapsed_profiled": elapsed_prof, "kernels": kern,
            "ll_first": float(ll[0]), "ll_last": float(ll[-1]), "variant": vname,
            "workspace_bytes": int(wsb), "counts": counts, "dense_from_iteration": switched}


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
    """Times the reference's standard E+M on the host (bounded sample: one
    warm-up iteration, then iterations until the budget is spent, at least
    one; past the configuration's iteration count it stops once a second
    has been sampled, so that short iterations (C1) still time a stable
    sample)."""
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
        el = time.perf_counter() - t_start
        if el > budget_s or (len(times) >= cfg.iters and el > min(1.0, budget_s)):
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


def measure(cid, args, with_cpu):
    cfg = CONFIGS[cid]
    steps = cfg.iters if cid == 5 else args.steps
    print(f"[bench] C{cid}: N={cfg.N} K={cfg.K} d={cfg.d}, {steps} steps", file=sys.stderr,
          flush=True)
    r = run_gpu(cfg, make_problem(cid), steps, args.warmup, args.variant)
    sec = r["elapsed"]
    ms_step = sec * 1e3 / steps
    roof = dominant_roofline(cfg, r["variant"], r["kernels"])
    roof["traffic"] = measured_traffic(cid, r["variant"], roof["kernel"])
    roof["traffic_unit"] = ("HBM bytes/launch (rocprofv3 FETCH_SIZE and WRITE_SIZE, scaled "
                            "by a plain copy's reading; profiles/)")
    ev_sum = sum(k["ms_per_step"] for k in r["kernels"].values())
    out = {
        "config": cid, "N": cfg.N, "K": cfg.K, "d": cfg.d, "variant": r["variant"],
        "steps": steps, "value": steps / sec, "ms_per_step": ms_step,
        "roofline": roof,
        "work_model": work_model(cfg, r["variant"], ms_step, r["counts"]),
        "timing": {
            "profiled_run_ms_per_step": r["elapsed_profiled"] * 1e3 / steps,
            "event_sum_ms_per_step": ev_sum,
            "kernels_ms_per_launch": {k: v["ms_avg"] for k, v in r["kernels"].items()},
            "note": "events are recorded in the profiled run only; their sum per step is "
                    "part of that run's wall time (the rest is host queueing and the gaps "
                    "between launches); value comes from the clean run",
        },
        "workspace_bytes": r["workspace_bytes"],
        "dense_from_iteration": r["dense_from_iteration"],
        "x_bytes": cfg.N * cfg.d * 4,
        "ll_first": r["ll_first"], "ll_last": r["ll_last"],
    }
    if with_cpu:
        out["cpu_baseline"] = cpu_baseline(cid, args.cpu_seconds)
        out["gpu_over_cpu"] = out["value"] / out["cpu_baseline"]["value"]
    return out


def measure_shape(args):
    """--shape N,K,d [--overlap]: the device loop on configs.make_shape's
    problem, timed as the configurations are (clean run for the value,
    profiled run for the per-pass durations); no CPU baseline."""
    N, K, d = (int(v) for v in args.shape.split(","))
    cfg = Config(0, N, K, d, -5.0, 5.0, "uniform", 0.5, 1.5, None, 0.0, args.steps,
                 "overlapping components" if args.overlap else "custom shape")
    r = run_gpu(cfg, make_shape(N, K, d, args.overlap), args.steps, args.warmup, args.variant)
    ms_step = r["elapsed"] * 1e3 / args.steps
    return {
        "metric": f"EM iters/s (N={N},K={K},d={d} fp32{', overlapping components' if args.overlap else ''})",
        "value": args.steps / r["elapsed"], "unit": "EM iters/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": arithmetic_type(r["variant"]), "data": "synthetic (configs.make_shape)",
        "config": {"workload": f"diag-cov GMM EM N={N} K={K} d={d} fp32"
                               + (" (all components within 0.02)" if args.overlap else ""),
                   "N": N, "K": K, "d": d, "kernel_variant": r["variant"]},
        "roofline": dominant_roofline(cfg, r["variant"], r["kernels"]),
        "timing": {"profiled_run_ms_per_step": r["elapsed_profiled"] * 1e3 / args.steps,
                   "kernels_ms_per_launch": {k: v["ms_avg"] for k, v in r["kernels"].items()}},
        "counts": r["counts"], "workspace_bytes": r["workspace_bytes"],
        "dense_from_iteration": r["dense_from_iteration"],
        "ll_first": r["ll_first"], "ll_last": r["ll_last"],
    }


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
    if args.shape:
        if rank == 0:
            print(json.dumps(measure_shape(args)), flush=True)
        return
    with_cpu = rank == 0 and not args.no_cpu_baseline
    cids = [int(c) for c in args.configs.split(",") if c.strip()]
    if args.config not in cids:
        cids.insert(0, args.config)
    per = {cid: measure(cid, args, with_cpu) for cid in cids}
    h = per[args.config]
    cfg = CONFIGS[args.config]
    line = {
        "metric": METRIC,
        "value": h["value"],
        "unit": "EM iters/s",
        "n_gpus": 1,
        "steps": h["steps"],
        "warmup": args.warmup,
        "ms_per_step": h["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": arithmetic_type(h["variant"]),
        "data": "synthetic (seeded mixture generator, flashgmm_amd/configs.py)",
        "config": {"workload": f"C{args.config}: diag-cov GMM EM N={cfg.N} K={cfg.K} "
                               f"d={cfg.d} fp32",
                   "N": cfg.N, "K": cfg.K, "d": cfg.d, "kernel_variant": h["variant"]},
        "roofline": h["roofline"],
        "work_model": h["work_model"],
        "timing": h["timing"],
        "workspace_bytes": h["workspace_bytes"],
    }
    if "cpu_baseline" in h:
        line["cpu_baseline"] = h["cpu_baseline"]
    line["configs"] = [per[c] for c in sorted(per)]
    if rank == 0:
        print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
