"""Benchmark of the batched LM fitter.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C2] [--no-cpu]
                    [--rounds R] [--tiled] [--copy-calibration] [--configs C3,C4,C5]

Default (the headline metric): one step = one full LM fit (all iterations,
on-device accept/reject) of the synthetic C2 population: 16,384 seeded
expressions, depth <= 6, <= 31 nodes, K uniform 1..8, D = 3, N = 1,024,
50 iterations, forward AD, fp64. The population is uploaded before timing
(inputs resident in HBM); each timed step re-fits it from the same starting
constants. Prints one JSON line. --config C1/C3/C4 measure the other resident
configurations the same way (and G1 / G1F, a GP generation shaped like the
reference's operon4000_g100 snapshot, with and without its K >= 17 expressions
that run in the general kernel); --config C5 runs the GP inner-solver shape: R
rounds of fresh 65,536-expression populations (generated untimed), each timed
end to end from host buffers (upload, 10 mixed-precision iterations,
read-back), the per-round latency being the step; the round's one target goes
over as a shared row (pop.bin v2), or tiled per expression with --tiled.

configs: the default (C2) run also measures the other configurations after
the headline line's own work, each briefly and without a CPU leg -- C3 and C4
resident (1 warm-up, 2 timed fits), C5 as 2 rounds from host buffers -- and
adds them as a `configs` block of the same JSON line: per configuration the
ms per step, fits/s, the dominant launch's kernel, its duration alone and
beside the other bins, and its algorithmic TFLOP/s against the vector peak.
`--configs ""` leaves the block out.

roofline: the roof that binds the dominant launch (the K bin whose fit
kernel runs longest) is VALU issue ("bound": "valu"): its algorithmic flops
(cusr_amd/benchmark/accounting.py; a lower bound, a transcendental counts 2)
over its duration running ALONE, against the MI355X fp64 vector peak. That
duration comes from a leg after the timed steps that fits only the dominant
bin's expressions (the same launch: the same expressions and iterations, no
other bin beside it), timed with HIP events recorded around the launch on the
stream it runs on; the contended duration inside the timed steps (the bins
share the GPU over 4 streams) is reported beside it. `measured_valu_busy`
gives SQ_ACTIVE_INST_VALU over the machine's VALU cycles for that kernel alone
and for the whole fit, from the committed rocprofv3 counter summary
(profiles/lm_fit_<config>_valu.json) when it was taken on this workload. The
`hbm` block keeps the HBM figure: algorithmic bytes (per LM iteration of each
active expression two point-passes that each read y, X once per pass, the
bytecode) over the same alone duration against 8 TB/s, and `traffic` the
measured HBM bytes of that launch from the rocprofv3 FETCH_SIZE / WRITE_SIZE
summary under profiles/. cpu_baseline: the reference CPU path (scipy LM per
expression over a process pool, oracle/scipy_pop.py) on a sample of the same
population, on every core granted to this process (within its cgroup CPU
quota), the median of >= 3 repeats; with the host (lscpu, versions) and the
quality of the CPU and GPU constants against the serial scipy oracle (tier-A/B
of cusr_amd/benchmark/runner.py) on a prefix of the sample.
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
FP32_VECTOR_PEAK_TFLOPS = 157.3
MI355X_SIMDS = 256 * 4          # CUs x SIMDs; a wave64 VALU op issues in 4 cycles
MI355X_CLOCK_HZ = 2.4e9         # peak engine clock
HEADLINE_METRIC = "expressions fitted/sec (16k exprs, K=1-8, N=1024, fp64) + achieved HBM GB/s"


def _say(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_cores():
    """(cores used, host description): every core in this process's affinity
    mask, within its cgroup CPU quota when one is set."""
    import platform
    import subprocess

    import scipy

    granted = len(os.sched_getaffinity(0))
    info = {"affinity_cores": granted, "os_cpu_count": os.cpu_count(),
            "python": platform.python_version(), "numpy": np.__version__,
            "scipy": scipy.__version__}
    quota = None
    try:
        q, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        info["cgroup_cpu_max"] = f"{q} {period}"
        if q != "max":
            quota = max(1, int(int(q) // int(period)))
    except (OSError, ValueError):
        pass
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        keep = ("Model name", "CPU(s)", "Thread(s) per core", "Core(s) per socket",
                "Socket(s)", "NUMA node(s)", "CPU max MHz")
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in keep:
                info["lscpu " + k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    cores = min(granted, quota) if quota else granted
    return cores, info


def cpu_baseline(pop, gpu_c_final, repeats=3, target_s=15.0, quality_s=8.0):
    """scipy LM (the reference CPU path, restated in oracle/scipy_pop.py) on
    the first expressions of the population: a warm-up slice measures the
    rate, the sample is sized so `repeats` fits of it take about target_s,
    and the value is the median rate of the repeats. Quality: the serial
    scipy oracle (cached by population hash) on a prefix of the sample sized
    to about quality_s, and tier-A/B of the pool's and the GPU's constants
    against it, all rescored by the numpy fp64 scorer (oracle/interp.py)."""
    import statistics

    from cusr_amd.benchmark import popio, runner
    from oracle import interp
    from oracle.scipy_pop import ScipyPop

    cores, host = cpu_cores()
    sp = ScipyPop(nproc=cores)
    try:
        warm = popio.slice_pop(pop, min(2 * cores, pop["M"]))
        sp.fit_pop(warm)                       # pool start-up + imports
        t0 = time.perf_counter()
        r = sp.fit_pop(warm)
        rate = max(r["n_fit"], 1) / max(time.perf_counter() - t0, 1e-3)
        n = int(min(pop["M"], max(cores, rate * target_s / repeats)))
        sub = popio.slice_pop(pop, n)
        rates, walls = [], []
        for _ in range(repeats):
            t0 = time.perf_counter()
            r = sp.fit_pop(sub)
            dt = time.perf_counter() - t0
            rates.append(r["n_fit"] / dt)
            walls.append(dt)
    finally:
        sp.close()
    value = statistics.median(rates)
    # quality on a prefix of the sample (the serial oracle runs on one core)
    q = int(min(n, max(16, value / cores * quality_s)))
    qpop = popio.slice_pop(pop, q)
    nc = int(np.sum(qpop["metas"][:, 3]))
    serial = ScipyPop(nproc=1)
    try:
        orc = runner.cached_oracle(qpop, lambda p: serial.fit_pop(p)["c_final"],
                                   lambda c: interp.loss_pop(qpop, c))
    finally:
        serial.close()
    K = qpop["metas"][:, 3]
    quality = {"expressions": q, "oracle": "serial scipy least_squares lm (the same settings), "
               f"{orc['wall']:.1f} s" + (" (cached)" if orc["cached"] else "")}
    for name, c in (("cpu", r["c_final"][:nc]), ("gpu", np.asarray(gpu_c_final)[:nc])):
        loss = interp.loss_pop(qpop, c)
        ta, tb, el = runner.classify_tiers(loss, orc["loss_star"], K)
        quality[name] = {"tier_a": runner.tier_rate(ta, el), "tier_b": runner.tier_rate(tb, el),
                         "eligible": int(np.sum(el)),
                         "spearman": runner.selection_fidelity(loss, orc["loss_star"],
                                                               el)["spearman"]}
    return {"value": value, "unit": "fits/s", "cores": cores, "kind": "port",
            "sample": (f"first {sub['M']} expressions of the same population "
                       f"({r['n_fit']} with K>0), {repeats} repeats (median; rates "
                       + ", ".join(f"{x:.1f}" for x in rates) + " fits/s; "
                       + ", ".join(f"{w:.1f}" for w in walls) + " s wall) on "
                       f"{cores} processes, scipy least_squares lm xtol=ftol=1e-10 "
                       "max_nfev=200"),
            "host": host, "quality": quality}


def copy_calibration(co, pop):
    """One plain copy kernel of known size for scaling rocprofv3 FETCH_SIZE /
    WRITE_SIZE: the reference's fp32 entry point (co_optimize, zero
    iterations) widens y on the device with one elementwise kernel that reads
    4*M*N and writes 8*M*N bytes (widen_kernel, the largest of its launches)."""
    n = int(pop["M"]) * int(pop["N"])
    co.optimize(pop, 0)
    _say(f"copy calibration: widen_kernel over {n} values, {4 * n} bytes read, "
         f"{8 * n} bytes written")


def _profile(workload_key, what):
    """profiles/lm_fit_<config>_<what>.json for the configuration named in
    the workload key (C1..C5)."""
    return REPO / "profiles" / f"lm_fit_{workload_key.split(':')[0].lower()}_{what}.json"


def load_traffic(workload_key, kernel):
    """HBM bytes per launch of `kernel`, from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE scaled by a copy kernel), when that
    summary was taken on this workload."""
    p = _profile(workload_key, "traffic")
    if not p.exists():
        return None
    d = json.loads(p.read_text())
    if d.get("workload_key") != workload_key:
        return None
    # instances chosen by N carry one more template argument (<K, R, AD, 1>)
    for name, v in d["kernels"].items():
        if kernel.rstrip(">") in name:
            return v["bytes_per_launch"]
    return None


def load_valu(workload_key):
    """Per-kernel SQ counters (SQ_ACTIVE_INST_VALU: quad-cycles of VALU issue,
    summed over waves) from the committed rocprofv3 --pmc summary, when that
    summary was taken on this workload."""
    p = _profile(workload_key, "valu")
    if not p.exists():
        return None
    d = json.loads(p.read_text())
    if d.get("workload_key") != workload_key:
        return None
    return d["kernels"]


def valu_issue(workload_key, kname_of, bins, device_ms, kdom, rounds=0):
    """Measured VALU busy fraction: SQ_ACTIVE_INST_VALU x 4 cycles over the
    machine's VALU cycles (1024 SIMDs at the 2.4 GHz peak clock, so a lower
    bound) -- for the whole fit (all K bins over the fit's device time) and
    for the dominant kernel running alone (its counter-run dispatch)."""
    ctr = load_valu(workload_key)
    if not ctr:
        return None
    cyc = 4.0 / (MI355X_SIMDS * MI355X_CLOCK_HZ)
    if kname_of(kdom).startswith("lm_pass_kernel"):
        # the split path: a bin is `rounds` pass launches, each followed by a
        # step launch; the summary holds per-launch means over each kernel's
        # last `rounds` dispatches (one fit of the bin; the step kernel's are
        # the last bin's), so the whole fit is those means times the launches
        dom = next((e for n, e in ctr.items() if kname_of(kdom).rstrip(">") in n), None)
        if dom is None:
            return None
        step = next((e for n, e in ctr.items() if n.startswith("cusr::lm_step_kernel")), None)
        tot, nb, whole = 0.0, 0, None
        for k, v in enumerate(bins):
            if v < 0:
                continue
            e = next((e for n, e in ctr.items() if kname_of(k).rstrip(">") in n), None)
            if e is None:
                tot = None
                break
            tot += e["SQ_ACTIVE_INST_VALU"] * rounds
            nb += 1
        if tot is not None and step is not None and rounds:
            tot += step["SQ_ACTIVE_INST_VALU"] * rounds * nb
            whole = tot * cyc / (device_ms / 1e3)
        return {"whole_fit_frac": whole,
                "dominant_alone_frac": dom["SQ_ACTIVE_INST_VALU"] * cyc / (dom["alone_ms"] / 1e3),
                "dominant_alone_ms": dom["alone_ms"],
                "per": "a pass launch of the bin, the mean over one fit's launches",
                "clock_ghz": MI355X_CLOCK_HZ / 1e9, "simds": MI355X_SIMDS,
                "source": str(_profile(workload_key, "valu").relative_to(REPO))}
    tot, missing = 0.0, []
    for k, v in enumerate(bins):
        if v < 0:
            continue
        e = next((e for n, e in ctr.items() if kname_of(k).rstrip(">") in n), None)
        if e is None:
            missing.append(k)
            continue
        tot += e["SQ_ACTIVE_INST_VALU"]
    dom = next((e for n, e in ctr.items() if kname_of(kdom).rstrip(">") in n), None)
    if missing or dom is None:
        return None
    return {"whole_fit_frac": tot * cyc / (device_ms / 1e3),
            "dominant_alone_frac": dom["SQ_ACTIVE_INST_VALU"] * cyc / (dom["alone_ms"] / 1e3),
            "dominant_alone_ms": dom["alone_ms"], "clock_ghz": MI355X_CLOCK_HZ / 1e9,
            "simds": MI355X_SIMDS, "source": str(_profile(workload_key, "valu").relative_to(REPO))}


def workload_text(cfg, pop):
    return (f"{cfg.name}: {pop['M']} expressions, depth<={cfg.depth}, <={cfg.max_nodes} nodes, "
            f"K {cfg.k_lo}-{cfg.k_hi}, D={cfg.D}, N={cfg.N}, {cfg.max_iter} LM iterations, "
            f"{'reverse' if cfg.ad_mode else 'forward'} AD, "
            f"{'mixed fp32/fp64' if cfg.precision else 'fp64'}")


def launch_bins(pop):
    """The launch bin of every expression: its K on the fast kernels, or
    CO_GENERAL_BIN (include/cusr_co.h co_fast_path)."""
    from cusr_amd.kernel import co_inproc

    rc, *_, route = co_inproc.decode(pop, "ad", full=True)
    if rc != 0:
        raise RuntimeError(f"co_decode failed ({rc})")
    K = np.asarray(pop["metas"])[:, 3]
    return np.where(route != 0, co_inproc.CO_GENERAL_BIN, K)


def dominant_bin(args, bins, bin_of):
    """The bin whose launch alone the roofline measures: the longest beside the
    others, or the one --roofline-bin names (refused when no expression is in it)."""
    if args.roofline_bin is None:
        return int(np.argmax(bins))
    k = int(args.roofline_bin)
    if not 0 <= k < len(bins) or not np.any(bin_of == k):
        sys.exit(f"bench.py: --roofline-bin {k}: no expression of this workload is in that bin")
    return k


def kernel_name(cfg, pop, k, parts=0):
    """Kernel name (as rocprofv3 shows it, without the last template
    arguments) of bin k's fit with `parts` point partitions (0: the default
    for N and the AD mode): lm_fit_kernel / lm_fit_gen_kernel, or the split
    path's lm_pass_kernel, which the step kernel follows."""
    from cusr_amd.kernel import co_inproc

    rname = "double" if cfg.precision == 0 else "float"
    gen = k == co_inproc.CO_GENERAL_BIN
    G = parts or co_inproc.co_partitions_for(int(pop["N"]), cfg.ad_mode)
    if G > co_inproc.CO_MAX_PARTITIONS:
        return (f"lm_pass_kernel<{co_inproc.CO_MAX_K if gen else k}, {rname}, "
                f"{cfg.ad_mode}")
    if gen:
        return f"lm_fit_gen_kernel<{rname}, {cfg.ad_mode}"
    return f"lm_fit_kernel<{k}, {rname}, {cfg.ad_mode}"


def alone_leg(fit_alone, pop, bin_of, kdom, reps):
    """Duration of bin kdom's launch with no other bin beside it: fit only
    its expressions, `reps` times, and read the bin's HIP-event time."""
    from cusr_amd.benchmark import popio

    sub = popio.select_pop(pop, np.flatnonzero(bin_of == kdom))
    ms = [float(fit_alone(sub)[kdom]) for _ in range(reps)]
    return float(np.mean(ms)), ms


def roofline(pop, cfg, iters, bins, kdom, alone_ms, alone_runs, bin_of, device_ms=None,
             parts=0):
    """Dominant launch against the fp64 (fp32 for mixed) vector peak, with
    the HBM figure as a secondary block."""
    from cusr_amd.benchmark import accounting

    w = accounting.algorithmic_work(pop, iters, cfg.ad_mode, subset=(bin_of == kdom))
    dom_s = alone_ms / 1e3
    vpeak = FP64_VECTOR_PEAK_TFLOPS if cfg.precision == 0 else FP32_VECTOR_PEAK_TFLOPS
    tflops = w["flops"] / dom_s / 1e12
    gbs = w["bytes"] / dom_s / 1e9
    kname = kernel_name(cfg, pop, kdom, parts)
    key = f"{cfg.name}:{pop['M']}x{pop['N']}:seed{cfg.seed}:it{cfg.max_iter}"
    out = {"bound": "valu", "achieved": tflops, "peak": vpeak, "unit": "TFLOP/s",
           "frac": tflops / vpeak, "traffic": load_traffic(key, kname),
           "kernel": kname + ", ...>", "bin": int(kdom),
           "expressions_in_launch": int(np.sum(bin_of == kdom)),
           "launch_ms": alone_ms, "launch_ms_runs": alone_runs,
           "launch_ms_concurrent": float(bins[kdom]),
           "algorithmic_flops_per_launch": w["flops"],
           "hbm": {"achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                   "frac": gbs / HBM_PEAK_GBS, "algorithmic_bytes_per_launch": w["bytes"]}}
    if device_ms:
        out["measured_valu_busy"] = valu_issue(key, lambda k: kernel_name(cfg, pop, k, parts), bins,
                                               device_ms, kdom,
                                               1 + cfg.max_iter + (2 if cfg.precision else 0))
    return out


def run_resident(args, cfg, co, pop):
    """C1-C4: fit the HBM-resident population `steps` times."""
    from cusr_amd.benchmark import accounting

    fit_kw = dict(ad_mode=cfg.ad_mode, precision=cfg.precision, partitions=args.partitions)
    if args.copy_calibration:
        copy_calibration(co, pop)
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
    e2e_ms = float("nan")
    if not args.no_e2e:
        # end to end from host buffers (upload over PCIe + fit + read-back), untimed above
        t_e2e = time.perf_counter()
        co.optimize_ex(pop, cfg.max_iter, **fit_kw)
        e2e_ms = 1e3 * (time.perf_counter() - t_e2e)
    K = pop["metas"][:, 3]
    n_fit = int(np.count_nonzero(K > 0))
    value = n_fit / (ms_per_step / 1e3)
    kms = float(np.mean(fit_ms))
    bins = np.mean(np.asarray(bin_ms), axis=0)
    bin_of = launch_bins(pop)
    kdom = dominant_bin(args, bins, bin_of)

    def fit_alone(sub):
        co.upload(sub)
        co.fit_resident(cfg.max_iter, outputs=False, **fit_kw)
        return co.last_bin_ms()

    alone_ms, alone_runs = alone_leg(fit_alone, pop, bin_of, kdom, args.alone_reps)
    roof = roofline(pop, cfg, res["iters"], bins, kdom, alone_ms, alone_runs, bin_of,
                    device_ms=kms, parts=args.partitions)
    whole = accounting.algorithmic_work(pop, res["iters"], cfg.ad_mode)
    status_counts = np.bincount(res["status"], minlength=5).tolist()
    _say(f"{args.steps} steps: {ms_per_step:.2f} ms/step, device {kms:.2f} ms/fit, "
         f"{value:.0f} fits/s, statuses {status_counts}, mean iters {res['iters'].mean():.1f}")
    _say("per-bin kernel ms: " + " ".join(f"K{k}={v:.2f}" for k, v in enumerate(bins) if v >= 0))
    _say(f"dominant bin {kdom} alone: {alone_ms:.3f} ms ({len(alone_runs)} launches), "
         f"{bins[kdom]:.3f} ms beside the other bins")
    fit = {"status_counts": status_counts, "mean_iters": float(res["iters"].mean()),
           "device_ms_per_fit": kms, "fits_per_s_device": n_fit / (kms / 1e3),
           "hbm_gbs_whole_fit": whole["bytes"] / (kms / 1e3) / 1e9,
           "tflops_whole_fit": whole["flops"] / (kms / 1e3) / 1e12,
           "e2e_ms_from_host": None if np.isnan(e2e_ms) else e2e_ms,
           "fits_per_s_from_host": None if np.isnan(e2e_ms) else n_fit / (e2e_ms / 1e3),
           "bin_ms": {str(k): float(v) for k, v in enumerate(bins) if v >= 0}}
    return value, ms_per_step, roof, fit, res


def run_rounds(args, cfg, co, gen):
    """C5: fresh populations per round, each timed from host buffers. The
    round's one target goes over as the shared row of pop.bin v2 unless
    --tiled sends it once per expression, as the reference does."""
    from cusr_amd.benchmark import popio

    lat, fits, rounds, last = [], 0, [], None
    for r in range(args.rounds):
        pop = gen(r)
        if not args.tiled:
            pop = popio.share_y(pop)
        if r == 0:
            co.optimize_ex(pop, 0, precision=cfg.precision)     # first-use costs, untimed
        t0 = time.perf_counter()
        res = co.optimize_ex(pop, cfg.max_iter, ad_mode=cfg.ad_mode, precision=cfg.precision)
        dt = 1e3 * (time.perf_counter() - t0)
        n_fit = int(np.count_nonzero(pop["metas"][:, 3] > 0))
        lat.append(dt)
        fits += n_fit
        setup_ms, loop_ms = co.last_split()
        rounds.append({"round": r, "ms": dt, "device_ms": co.last_kernel_ms(),
                       "setup_ms": setup_ms, "fit_and_readback_ms": loop_ms, "fits": n_fit,
                       "status_counts": np.bincount(res["status"], minlength=5).tolist()})
        _say(f"round {r}: {dt:.1f} ms end to end, device {co.last_kernel_ms():.1f} ms, "
             f"{n_fit} fits")
        last = (pop, res, co.last_bin_ms())
    value = fits / (sum(lat) / 1e3)
    pop, res, bins = last
    bin_of = launch_bins(pop)
    kdom = dominant_bin(args, bins, bin_of)

    def fit_alone(sub):
        co.optimize_ex(sub, cfg.max_iter, ad_mode=cfg.ad_mode, precision=cfg.precision)
        return co.last_bin_ms()

    alone_ms, alone_runs = alone_leg(fit_alone, pop, bin_of, kdom, args.alone_reps)
    _say(f"dominant bin {kdom} alone: {alone_ms:.3f} ms, {bins[kdom]:.3f} ms beside the others")
    roof = roofline(pop, cfg, res["iters"], bins, kdom, alone_ms, alone_runs, bin_of,
                    device_ms=rounds[-1]["device_ms"])
    fit = {"rounds": rounds, "mean_round_ms": float(np.mean(lat)),
           "p50_round_ms": float(np.median(lat)),
           "target": "tiled [M][N]" if args.tiled else "shared row [N] (pop.bin v2)"}
    return value, float(np.mean(lat)), roof, fit, pop, res


def make_gen(cfg, co):
    """Population generator of a configuration, targets from the device evaluator."""
    from cusr_amd.benchmark import gen_synth

    def gen(round_index=0):
        t = time.perf_counter()
        pop, _ = gen_synth.generate(cfg, lambda p, c, xs: co.evaluate(p, c, xs),
                                    round_index=round_index)
        _say(f"generated {cfg.name} round {round_index}: M={pop['M']} N={pop['N']} "
             f"nodes={pop['total_nodes']} K_max={pop['K_max']} in {time.perf_counter() - t:.1f}s")
        return pop

    return gen


def config_block(co, names, base_args):
    """The other configurations, measured briefly beside the headline (no CPU
    leg): C1-C4 resident, 1 warm-up and 2 timed fits; C5 2 rounds from host
    buffers. Returns {name: summary}."""
    from cusr_amd.benchmark import gen_synth

    out = {}
    for name in names:
        cfg = gen_synth.CONFIGS[name]
        a = argparse.Namespace(**vars(base_args))
        a.steps, a.warmup, a.rounds, a.no_e2e = 2, 1, 2, True
        a.alone_reps, a.partitions, a.copy_calibration, a.tiled = 3, 0, False, False
        t0 = time.perf_counter()
        gen = make_gen(cfg, co)
        if cfg.rounds > 1:
            value, ms, roof, fit, pop, res = run_rounds(a, cfg, co, gen)
            steps, what = a.rounds, "rounds from host buffers (upload, fit, read-back)"
        else:
            pop = gen()
            value, ms, roof, fit, res = run_resident(a, cfg, co, pop)
            steps, what = a.steps, "fits of the HBM-resident population"
        out[name] = {
            "workload": workload_text(cfg, pop), "steps": steps, "warmup": 1, "timed": what,
            "ms_per_step": ms, "value": value, "unit": "fits/s",
            "dtype": "f64" if cfg.precision == 0 else "f32+f64",
            "dominant_kernel": roof["kernel"], "dominant_bin": roof["bin"],
            "dominant_alone_ms": roof["launch_ms"],
            "dominant_concurrent_ms": roof["launch_ms_concurrent"],
            "achieved_tflops": roof["achieved"], "peak_tflops": roof["peak"],
            "frac": roof["frac"],
            "status_counts": np.bincount(res["status"], minlength=5).tolist(),
            "mean_iters": float(res["iters"].mean()),
            "wall_s": time.perf_counter() - t0}
        _say(f"config {name}: {ms:.2f} ms per step, {value:.0f} fits/s, dominant "
             f"{roof['kernel']} alone {roof['launch_ms']:.3f} ms, {roof['achieved']:.2f} TFLOP/s")
        del pop, res
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", default="C2", choices=["C1", "C2", "C3", "C4", "C5", "G1", "G1F"])
    ap.add_argument("--rounds", type=int, default=3, help="C5 rounds (the spec runs 20)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--ad-mode", type=int, default=None, choices=[0, 1],
                    help="override the configuration's AD mode (0 forward, 1 reverse)")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the end-to-end fit from host buffers (profiling runs)")
    ap.add_argument("--tiled", action="store_true",
                    help="C5: send the target tiled per expression, as the reference does")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one copy kernel of known size (for rocprofv3 --pmc scaling)")
    ap.add_argument("--alone-reps", type=int, default=3,
                    help="launches of the dominant bin alone (the roofline's duration)")
    ap.add_argument("--roofline-bin", type=int, default=None,
                    help="the bin whose launch alone the roofline measures (default: the "
                         "longest beside the others; counter runs fix it, since under the "
                         "profiler the bins' concurrent times reorder)")
    ap.add_argument("--configs", default=None,
                    help="comma-separated configurations measured briefly after the main "
                         "one (default: C3,C4,C5 when --config is C2; '' for none)")
    ap.add_argument("--partitions", type=int, default=0,
                    help="point partitions per expression (0: by N and AD mode, co_partitions_for; "
                         "above 4 the split path)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}); this build measures "
              "one GPU's share and does not launch multi-GPU runs.", file=sys.stderr)
        sys.exit(2)

    from cusr_amd.benchmark import gen_synth
    from cusr_amd.kernel import co_inproc

    cfg = gen_synth.CONFIGS[args.config]
    if args.ad_mode is not None:
        cfg = gen_synth.scaled(cfg)
        cfg.ad_mode = args.ad_mode
    co = co_inproc.get_inproc_co(0, "ad")
    gen = make_gen(cfg, co)

    if cfg.rounds > 1:
        value, ms_per_step, roof, fit, pop, res = run_rounds(args, cfg, co, gen)
        steps, warmup = args.rounds, 1
    else:
        pop = gen()
        value, ms_per_step, roof, fit, res = run_resident(args, cfg, co, pop)
        steps, warmup = args.steps, args.warmup

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(pop, res["c_final"])
        _say(f"cpu baseline {cpu['value']:.1f} fits/s on {cpu['cores']} cores; quality "
             + json.dumps(cpu["quality"]))

    names = args.configs
    if names is None:
        names = "C3,C4,C5" if args.config == "C2" and args.ad_mode is None else ""
    others = config_block(co, [n for n in names.split(",") if n], args) if names else None

    metric = HEADLINE_METRIC if cfg.name == "C2" else \
        f"expressions fitted/sec ({cfg.name}) + achieved HBM GB/s"
    line = {
        "metric": metric,
        "value": value,
        "unit": "fits/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64" if cfg.precision == 0 else "f32+f64",
        "data": f"synthetic: seeded {cfg.name} population, targets from true constants + noise",
        "config": {"workload": workload_text(cfg, pop), "expressions": int(pop["M"]),
                   "points": int(pop["N"]), "max_iter": cfg.max_iter, "seed": cfg.seed},
        "roofline": roof,
        "cpu_baseline": cpu,
        "fit": fit,
    }
    if others:
        line["configs"] = others
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
