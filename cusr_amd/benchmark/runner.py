"""Quality and throughput harness with the reference benchmark's protocol
(cusr/benchmark/runner.py:55-376): every backend fits the same population,
its constants are rescored in fp64, and each expression is classified against
a tight reference fit ("oracle") and, for synthetic data, against the noise
floor of the true constants.

    tier-A: loss <= max(1.005 loss*, loss* + 1e-10)
    tier-B: loss <= max(1.05 loss*,  loss* + 1e-10)      (K > 0, finite loss*)
    selection fidelity: Spearman rank correlation of backend vs oracle losses
        and the overlap of their best 10 / 25 / 50 % (what GP selection uses)

The protocol math is restated here in code of its own; the thresholds and
panels are kept identical so the numbers compare with the reference's. The
harness is generic over its inputs: `run_quality` takes the backends (objects
with fit_pop(pop) -> FitResult), the oracle fit and a scoring function
(constants -> per-expression fp64 loss), so the reference-side tools (a serial
scipy oracle, a numpy scorer) are supplied by whoever runs it.
"""
from __future__ import annotations

import hashlib
import json
import os
import socket
import time
from datetime import datetime
from pathlib import Path

import numpy as np

from . import popio

PROTOCOL_VERSION = 2
TIER_ABS_FLOOR = 1e-10
TIER_A_MULT, TIER_B_MULT = 1.005, 1.05


def classify_tiers(loss_b, loss_star, K):
    """(tier_a, tier_b, eligible) boolean arrays; K = 0 or non-finite loss*
    expressions are not eligible."""
    loss_b = np.asarray(loss_b, np.float64)
    loss_star = np.asarray(loss_star, np.float64)
    eligible = (np.asarray(K) > 0) & np.isfinite(loss_star)
    with np.errstate(invalid="ignore", over="ignore"):
        thr_a = np.maximum(TIER_A_MULT * loss_star, loss_star + TIER_ABS_FLOOR)
        thr_b = np.maximum(TIER_B_MULT * loss_star, loss_star + TIER_ABS_FLOOR)
        tier_a = eligible & (loss_b <= thr_a)
        tier_b = eligible & (loss_b <= thr_b)
    return tier_a, tier_b, eligible


def tier_rate(tier, eligible) -> float:
    n = int(np.sum(eligible))
    return float(np.sum(tier) / n) if n else float("nan")


def selection_fidelity(loss_b, loss_star, eligible) -> dict:
    """Rank agreement of backend and oracle losses over eligible expressions
    with both losses finite."""
    loss_b = np.asarray(loss_b, np.float64)
    loss_star = np.asarray(loss_star, np.float64)
    ok = np.asarray(eligible) & np.isfinite(loss_b) & np.isfinite(loss_star)
    idx = np.flatnonzero(ok)
    out = {"n": int(idx.size), "spearman": None, "top10": None, "top25": None, "top50": None}
    if idx.size < 3:
        return out
    rank_b = np.argsort(np.argsort(loss_b[idx]))
    rank_o = np.argsort(np.argsort(loss_star[idx]))
    out["spearman"] = float(np.corrcoef(rank_b, rank_o)[0, 1])
    for frac, key in ((0.10, "top10"), (0.25, "top25"), (0.50, "top50")):
        k = max(1, int(frac * idx.size))
        best_o = set(idx[np.argsort(loss_star[idx])[:k]].tolist())
        best_b = set(idx[np.argsort(loss_b[idx])[:k]].tolist())
        out[key] = len(best_o & best_b) / k
    return out


def pop_sha(pop: dict) -> str:
    """sha1 (16 hex digits) of everything a fit reads: programs, metas,
    starting constants, X and the target rows."""
    h = hashlib.sha1()
    for a in (pop["nt"], pop["nv"], pop["ci"], pop["metas"], pop["c_init"], pop["xs"],
              popio.y_rows(pop)):
        a = np.ascontiguousarray(a)
        h.update(str((a.dtype.str, a.shape)).encode())
        h.update(a.tobytes())
    return h.hexdigest()[:16]


def default_cache_dir() -> Path:
    """Where the harness keeps its serial-oracle cache: $CUSR_CACHE_DIR, else
    $XDG_CACHE_HOME/cusr_amd/oracle, else ~/.cache/cusr_amd/oracle. Outside
    the repository, so results and scratch folders never hold it."""
    if os.environ.get("CUSR_CACHE_DIR"):
        return Path(os.environ["CUSR_CACHE_DIR"])
    base = os.environ.get("XDG_CACHE_HOME") or str(Path.home() / ".cache")
    return Path(base) / "cusr_amd" / "oracle"


def cached_oracle(pop: dict, fit_serial, score, cache_dir=None, limit: int | None = None) -> dict:
    """The tight serial oracle of a population, cached by (population sha1,
    limit) as the reference caches it by file sha1 (cusr/benchmark/runner.py:
    111-128): fit_serial(pop) -> c_final (a serial fit, reproducible bit for
    bit, which a process pool is not on degenerate expressions), score(c) ->
    per-expression fp64 loss. Returns loss_star, c_star, wall (of the fit that
    filled the cache) and cached."""
    if limit is not None:
        pop = popio.slice_pop(pop, limit)
    cache_dir = Path(cache_dir) if cache_dir is not None else default_cache_dir()
    path = cache_dir / f"oracle_{pop_sha(pop)}_L{limit or 'all'}_serial.npz"
    if path.exists():
        z = np.load(path)
        return {"loss_star": z["loss_star"], "c_star": z["c_star"], "wall": float(z["wall"]),
                "cached": True}
    t0 = time.perf_counter()
    c_star = np.asarray(fit_serial(pop), np.float64)
    loss_star = np.asarray(score(c_star), np.float64)
    wall = time.perf_counter() - t0
    cache_dir.mkdir(parents=True, exist_ok=True)
    tmp = path.with_suffix(".tmp.npz")
    np.savez(tmp, loss_star=loss_star, c_star=c_star, wall=wall)
    tmp.replace(path)
    return {"loss_star": loss_star, "c_star": c_star, "wall": wall, "cached": False}


def run_quality(pop: dict, backends: dict, loss_star: np.ndarray, score, *, repeats: int = 3,
                c_true: np.ndarray | None = None, label: str = "population") -> dict:
    """Fit `pop` with each backend (`repeats` timed runs after a warm-up on a
    small slice), rescore the last run's constants with `score(c) -> loss[M]`
    and classify against `loss_star` (and the noise floor score(c_true))."""
    K = np.asarray(pop["metas"])[:, 3]
    results = {"meta": {"hostname": socket.gethostname(), "protocol_version": PROTOCOL_VERSION,
                        "timestamp": datetime.now().isoformat(timespec="seconds")},
               "pop": {"label": label, "M": int(pop["M"]), "N": int(pop["N"]),
                       "n_vars": int(pop["n_vars"]), "K_max": int(pop["K_max"]),
                       "repeats": repeats},
               "oracle": {"n_eligible": int(np.sum((K > 0) & np.isfinite(loss_star)))},
               "backends": {}}
    floor = None
    if c_true is not None:
        floor = score(np.asarray(c_true, np.float64))
        fa, fb, fe = classify_tiers(loss_star, floor, K)
        results["noise_floor"] = {"median": float(np.median(floor[fe])) if fe.any() else None,
                                  "n": int(fe.sum()), "oracle_reach_a": tier_rate(fa, fe),
                                  "oracle_reach_b": tier_rate(fb, fe)}
    kpos = int(np.argmax(K > 0)) if np.any(K > 0) else 0
    warm = popio.slice_pop(pop, min(int(pop["M"]), max(2, kpos + 1)))
    for name, be in backends.items():
        be.fit_pop(warm)
        walls, res = [], None
        for _ in range(repeats):
            res = be.fit_pop(pop)
            walls.append(res.wall_e2e)
        loss_b = score(res.c_final)
        ta, tb, el = classify_tiers(loss_b, loss_star, K)
        wall = float(np.median(walls))
        entry = {"wall_e2e": wall, "wall_e2e_runs": walls, "wall_core": res.wall_core,
                 "tier_a_rate": tier_rate(ta, el), "tier_b_rate": tier_rate(tb, el),
                 "tier_a_n": int(ta.sum()), "tier_b_n": int(tb.sum()), "n_eligible": int(el.sum()),
                 "tput_a": float(ta.sum() / wall), "tput_b": float(tb.sum() / wall),
                 "selection_fidelity": selection_fidelity(loss_b, loss_star, el),
                 "status_counts": {s: int(np.sum(res.status == c)) for s, c in
                                   (("converged", 0), ("iter_limit", 1), ("failed", 2), ("k0", 3))},
                 "n_iter_median": (int(np.median(res.n_iter[res.n_iter >= 0]))
                                   if np.any(res.n_iter >= 0) else None),
                 "dtype": res.meta.get("dtype", "?")}
        if floor is not None:
            fa, fb, fe = classify_tiers(loss_b, floor, K)
            entry["floor_a_rate"] = tier_rate(fa, fe)
            entry["floor_b_rate"] = tier_rate(fb, fe)
        results["backends"][name] = entry
    return results


def report_markdown(results: dict) -> str:
    p = results["pop"]
    lines = [f"# Quality and throughput — {p['label']} (M={p['M']}, N={p['N']}, "
             f"repeats={p['repeats']})", "",
             f"* protocol v{results['meta']['protocol_version']} @ {results['meta']['timestamp']} "
             f"on {results['meta']['hostname']}",
             f"* oracle: eligible {results['oracle']['n_eligible']} expressions", "",
             "| backend | dtype | e2e (s) | core (s) | tier-A | tier-B | tput-A (fits/s) | "
             "tput-B (fits/s) | conv/lim/fail | iters (median) |",
             "|---|---|---:|---:|---:|---:|---:|---:|---|---:|"]
    for name, r in results["backends"].items():
        sc = r["status_counts"]
        it = r["n_iter_median"] if r["n_iter_median"] is not None else "—"
        lines.append(f"| {name} | {r['dtype']} | {r['wall_e2e']:.3f} | {r['wall_core']:.3f} | "
                     f"{100 * r['tier_a_rate']:.1f}% | {100 * r['tier_b_rate']:.1f}% | "
                     f"{r['tput_a']:.0f} | {r['tput_b']:.0f} | "
                     f"{sc['converged']}/{sc['iter_limit']}/{sc['failed']} | {it} |")
    lines += ["", "Selection fidelity (backend loss ranking against the oracle's):", "",
              "| backend | Spearman | top-10% | top-25% | top-50% |", "|---|---:|---:|---:|---:|"]

    def pct(x):
        return f"{100 * x:.0f}%" if isinstance(x, float) else "—"

    for name, r in results["backends"].items():
        sf = r["selection_fidelity"]
        sp = f"{sf['spearman']:.3f}" if sf["spearman"] is not None else "—"
        lines.append(f"| {name} | {sp} | {pct(sf['top10'])} | {pct(sf['top25'])} | "
                     f"{pct(sf['top50'])} |")
    nf = results.get("noise_floor")
    if nf:
        lines += ["", f"Noise floor (loss at the true constants): median {nf['median']:.3e} over "
                      f"{nf['n']} expressions; the oracle reaches it within 1.005x for "
                      f"{100 * nf['oracle_reach_a']:.1f}% and within 1.05x for "
                      f"{100 * nf['oracle_reach_b']:.1f}%.", "",
                  "| backend | reaches floor (1.005x) | reaches floor (1.05x) |", "|---|---:|---:|"]
        for name, r in results["backends"].items():
            if "floor_a_rate" in r:
                lines.append(f"| {name} | {100 * r['floor_a_rate']:.1f}% | "
                             f"{100 * r['floor_b_rate']:.1f}% |")
    return "\n".join(lines) + "\n"


def write_outputs(results: dict, out_dir: Path, stem: str) -> tuple[Path, Path]:
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    js = out_dir / f"{stem}.json"
    md = out_dir / f"{stem}.md"
    js.write_text(json.dumps(results, indent=2, default=str))
    md.write_text(report_markdown(results))
    return js, md


def timed(fn, *a, **kw):
    t0 = time.perf_counter()
    out = fn(*a, **kw)
    return out, time.perf_counter() - t0
