"""Benchmark of the batched LM fitter on the headline configuration.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C2] [--cpu-sample S]

One step = one full LM fit (all iterations, on-device accept/reject) of the
synthetic C2 population: 16,384 seeded expressions, depth <= 6, <= 31 nodes,
K uniform 1..8, D = 3, N = 1,024, 50 iterations, forward AD, fp64. The
population is uploaded before timing (inputs resident in HBM); each timed step
re-fits it from the same starting constants. Prints one JSON line.

roofline: the dominant launch is the fit kernel of the K bin that runs
longest; its algorithmic HBM bytes (cusr_amd/benchmark/accounting.py: per LM
iteration of each active expression two point-passes that each read y, X once
per pass, the bytecode) over its duration from HIP events recorded around
that launch on the stream it runs on. The same object carries the fp64 VALU
figure (algorithmic flops over the same duration), the roof this kernel is
actually under. traffic: measured HBM bytes of that launch, from the
rocprofv3 FETCH_SIZE / WRITE_SIZE summary committed under profiles/, when it
was taken on this workload. cpu_baseline: the reference CPU path (scipy LM per
expression over a process pool) on the same population, repeated to 10-30 s,
on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
FP64_VECTOR_PEAK_TFLOPS = 78.6


def cpu_baseline(pop, sample, min_seconds=10.0, max_seconds=30.0):
    """scipy LM (the reference CPU path, restated in oracle/scipy_pop.py) on
    the first `sample` expressions, repeated until at least `min_seconds` of
    wall time (never starting a repeat that would pass `max_seconds`)."""
    from cusr_amd.benchmark import popio
    from oracle.scipy_pop import ScipyPop

    nproc = min(16, os.cpu_count() or 1)
    sp = ScipyPop(nproc=nproc)
    try:
        warm = popio.slice_pop(pop, min(2 * nproc, pop["M"]))
        sp.fit_pop(warm)                       # pool start-up + imports
        sub = popio.slice_pop(pop, min(sample, pop["M"]))
        fits, wall, reps = 0, 0.0, 0
        while True:
            t0 = time.perf_counter()
            r = sp.fit_pop(sub)
            dt = time.perf_counter() - t0
            fits += r["n_fit"]
            wall += dt
            reps += 1
            if wall >= min_seconds or wall + dt > max_seconds:
                break
    finally:
        sp.close()
    return {"value": fits / wall, "unit": "fits/s", "cores": nproc, "kind": "port",
            "sample": (f"first {sub['M']} expressions of the same C2 population "
                       f"({r['n_fit']} with K>0) x {reps}, scipy least_squares lm "
                       f"xtol=ftol=1e-10 max_nfev=200, {wall:.1f} s wall on {nproc} processes"),
            "wall_s": wall}


def copy_calibration(co, pop):
    """One plain copy kernel of known size for scaling rocprofv3 FETCH_SIZE /
    WRITE_SIZE: the reference's fp32 entry point (co_optimize, zero
    iterations) widens y on the device with one elementwise kernel that reads
    4*M*N and writes 8*M*N bytes (widen_kernel, the largest of its launches)."""
    n = int(pop["M"]) * int(pop["N"])
    co.optimize(pop, 0)
    print(f"[bench] copy calibration: widen_kernel over {n} values, {4 * n} bytes read, "
          f"{8 * n} bytes written", file=sys.stderr, flush=True)


def load_traffic(workload_key, kernel):
    """HBM bytes per launch of `kernel`, from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE scaled by a copy kernel), when that
    summary was taken on this workload."""
    p = REPO / "profiles" / "lm_fit_c2_traffic.json"
    if not p.exists():
        return None
    d = json.loads(p.read_text())
    if d.get("workload_key") != workload_key:
        return None
    for name, v in d["kernels"].items():
        if kernel in name:
            return v["bytes_per_launch"]
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", default="C2")
    ap.add_argument("--cpu-sample", type=int, default=16384)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one copy kernel of known size (for rocprofv3 --pmc scaling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}); this build measures "
              "one GPU's share and does not launch multi-GPU runs.", file=sys.stderr)
        sys.exit(2)

    from cusr_amd.benchmark import accounting, gen_synth
    from cusr_amd.kernel import co_inproc

    cfg = gen_synth.CONFIGS[args.config]
    co = co_inproc.get_inproc_co(0, "ad")

    def gpu_eval(p, c, xs):
        return co.evaluate(p, c, xs)

    t_gen = time.perf_counter()
    pop, _ = gen_synth.generate(cfg, gpu_eval)
    t_gen = time.perf_counter() - t_gen
    print(f"[bench] generated {cfg.name}: M={pop['M']} N={pop['N']} nodes={pop['total_nodes']} "
          f"K_max={pop['K_max']} in {t_gen:.1f}s", file=sys.stderr, flush=True)
    if args.copy_calibration:
        copy_calibration(co, pop)
    fit_kw = dict(ad_mode=cfg.ad_mode, precision=cfg.precision)
    co.upload(pop)
    for _ in range(args.warmup):
        co.fit_resident(cfg.max_iter, outputs=False, **fit_kw)
    fit_ms, bin_ms = [], []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        co.fit_resident(cfg.max_iter, outputs=False, **fit_kw)
        fit_ms.append(co.last_kernel_ms())
        bin_ms.append(co.last_bin_ms())
    wall = time.perf_counter() - t0
    ms_per_step = 1e3 * wall / args.steps
    res = co.fit_resident(cfg.max_iter, **fit_kw)
    # end-to-end from host buffers (upload over PCIe + fit + read-back), untimed above
    t_e2e = time.perf_counter()
    co.optimize_ex(pop, cfg.max_iter, **fit_kw)
    e2e_ms = 1e3 * (time.perf_counter() - t_e2e)
    K = pop["metas"][:, 3]
    n_fit = int(np.count_nonzero(K > 0))
    value = n_fit / (ms_per_step / 1e3)
    kms = float(np.mean(fit_ms))
    bins = np.mean(np.asarray(bin_ms), axis=0)
    kdom = int(np.argmax(bins))                       # dominant launch: longest K bin
    wdom = accounting.algorithmic_work(pop, res["iters"], cfg.ad_mode, subset=(K == kdom))
    wall_fit = accounting.algorithmic_work(pop, res["iters"], cfg.ad_mode)
    dom_s = bins[kdom] / 1e3
    achieved = wdom["bytes"] / dom_s / 1e9
    rname = "double" if cfg.precision == 0 else "float"
    kname = f"lm_fit_kernel<{kdom}, {rname}, {cfg.ad_mode}>"
    status_counts = np.bincount(res["status"], minlength=5).tolist()
    print(f"[bench] {args.steps} steps: {ms_per_step:.2f} ms/step, device {kms:.2f} ms/fit, "
          f"{value:.0f} fits/s, statuses {status_counts}, mean iters {res['iters'].mean():.1f}",
          file=sys.stderr, flush=True)
    print("[bench] per-bin kernel ms: " + " ".join(f"K{k}={v:.2f}" for k, v in enumerate(bins)
                                                  if v >= 0), file=sys.stderr, flush=True)
    workload_key = f"{cfg.name}:{pop['M']}x{pop['N']}:seed{cfg.seed}:it{cfg.max_iter}"
    traffic = load_traffic(workload_key, kname)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(pop, args.cpu_sample)
        print(f"[bench] cpu baseline {cpu['value']:.1f} fits/s on {cpu['cores']} cores",
              file=sys.stderr, flush=True)
        cpu.pop("wall_s", None)

    line = {
        "metric": "expressions fitted/sec (16k exprs, K=1-8, N=1024, fp64) + achieved HBM GB/s",
        "value": value,
        "unit": "fits/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64" if cfg.precision == 0 else "f32+f64",
        "data": "synthetic: seeded C2 population, targets from the true constants + noise",
        "config": {"workload": (f"{cfg.name}: {pop['M']} expressions, depth<={cfg.depth}, "
                                f"<={cfg.max_nodes} nodes, K {cfg.k_lo}-{cfg.k_hi}, D={cfg.D}, "
                                f"N={cfg.N}, {cfg.max_iter} LM iterations, "
                                f"{'reverse' if cfg.ad_mode else 'forward'} AD, "
                                f"{'mixed' if cfg.precision else 'fp64'}"),
                   "expressions": int(pop["M"]), "points": int(pop["N"]),
                   "max_iter": cfg.max_iter, "seed": cfg.seed},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": traffic,
                     "kernel": kname, "expressions_in_launch": int(np.sum(K == kdom)),
                     "launch_ms": float(bins[kdom]),
                     "algorithmic_bytes_per_launch": wdom["bytes"],
                     "valu": {"achieved": wdom["flops"] / dom_s / 1e12,
                              "peak": FP64_VECTOR_PEAK_TFLOPS, "unit": "TFLOP/s",
                              "frac": wdom["flops"] / dom_s / 1e12 / FP64_VECTOR_PEAK_TFLOPS,
                              "algorithmic_flops_per_launch": wdom["flops"]}},
        "cpu_baseline": cpu,
        "fit": {"status_counts": status_counts, "mean_iters": float(res["iters"].mean()),
                "device_ms_per_fit": kms, "fits_per_s_device": n_fit / (kms / 1e3),
                "hbm_gbs_whole_fit": wall_fit["bytes"] / (kms / 1e3) / 1e9,
                "e2e_ms_from_host": e2e_ms, "fits_per_s_from_host": n_fit / (e2e_ms / 1e3),
                "fp64_tflops_whole_fit": wall_fit["flops"] / (kms / 1e3) / 1e12,
                "bin_ms": {str(k): float(v) for k, v in enumerate(bins) if v >= 0}},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
