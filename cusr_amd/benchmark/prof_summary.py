"""Summarise a rocprofv3 database (rocpd SQLite) as a markdown table.

    python -m cusr_amd.benchmark.prof_summary trace  <run_results.db> [--match lm_fit]
           [--skip W --take T]
    python -m cusr_amd.benchmark.prof_summary pmc    <run_results.db> [--match lm_fit]
    python -m cusr_amd.benchmark.prof_summary valu   <run_results.db> [--match lm_fit]
           [--out JSON --workload-key KEY] [--last]
    python -m cusr_amd.benchmark.prof_summary resources [--match lm_] [--resources JSON]
    python -m cusr_amd.benchmark.prof_summary traffic <fetch.db> <write.db> --kernel NAME
           --calib-fetch-bytes F --calib-write-bytes W [--out JSON --workload-key KEY]
           [--last]

trace: per kernel, calls and average / min / max / total duration plus the
grid of the dispatch and the kernel's registers, spills and scratch bytes per
lane from the compiler's resource-usage remarks of the build
(cusr_amd/kernel/kernel_resources.json, written by cusr_amd/build.py; rocpd's
register figures count the gfx950 VGPR allocation in granules of 4 where the
hardware allocates 8, so the code object's figure is taken from the build).
resources: that table for the fit and pass kernels alone. pmc: per kernel, the average of
every counter per dispatch. valu: the same as JSON, with each kernel's
dispatch duration (counter runs serialise dispatches). traffic: HBM bytes per dispatch of each matching kernel from
a FETCH_SIZE run and a WRITE_SIZE run, each scaled by the ratio of the known
bytes of the copy calibration kernel (bench.py --copy-calibration: the
widen_kernel dispatch with the largest grid) to what the same counter read
for it.
"""
from __future__ import annotations

import argparse
import collections
import json
import sqlite3
import statistics
from pathlib import Path

RESOURCES = Path(__file__).resolve().parents[1] / "kernel" / "kernel_resources.json"


def load_resources(path=None) -> dict:
    """{demangled kernel name: resource fields} of the build (empty if absent)."""
    p = Path(path) if path else RESOURCES
    if not p.exists():
        return {}
    return {v["name"]: v for v in json.loads(p.read_text()).values()}


def _res_for(res: dict, name: str):
    if name in res:
        return res[name]
    for k, v in res.items():          # rocpd may drop the return type or arguments
        if name in k or k in name:
            return v
    return None


def _rows(db, sql):
    con = sqlite3.connect(db)
    try:
        return con.execute(sql).fetchall()
    finally:
        con.close()


def trace(db, match=None, skip=0, take=None, resources=None):
    """skip / take: per kernel, drop its first `skip` dispatches and keep the
    next `take` (a benchmark's timed steps after its warm-up)."""
    res = load_resources(resources)
    rows = _rows(db, "select name, duration, vgpr_count, accum_vgpr_count, sgpr_count, "
                     "scratch_size, lds_size, grid_x, workgroup_x from kernels "
                     "order by dispatch_id")
    by = collections.defaultdict(list)
    seen = collections.Counter()
    meta = {}
    for name, dur, vg, ag, sg, scr, lds, gx, wx in rows:
        if match and match not in name:
            continue
        seen[name] += 1
        if seen[name] <= skip or (take is not None and seen[name] > skip + take):
            continue
        by[name].append(dur / 1e6)
        meta[name] = (vg, ag, sg, scr, lds, gx // max(wx, 1))
    out = ["| kernel | calls | avg ms | min ms | max ms | total ms | VGPR | AGPR | SGPR "
           "| VGPR spill | scratch B/lane | waves/SIMD | LDS B | workgroups |", "|" + "---|" * 14]
    for name in sorted(by, key=lambda n: -sum(by[n])):
        d = by[name]
        vg, ag, sg, scr, lds, wg = meta[name]
        r = _res_for(res, name)
        if r:
            vg, ag, sg = r.get("vgpr", vg), r.get("agpr", ag), r.get("sgpr", sg)
            sp, scr, occ = r.get("vgpr_spill", "?"), r.get("scratch_bytes_per_lane", scr), \
                r.get("waves_per_simd", "?")
        else:
            sp, occ = "?", "?"
        out.append(f"| `{name}` | {len(d)} | {statistics.mean(d):.3f} | {min(d):.3f} | "
                   f"{max(d):.3f} | {sum(d):.2f} | {vg} | {ag} | {sg} | {sp} | {scr} | {occ} "
                   f"| {lds} | {wg} |")
    return "\n".join(out)


def resources_table(match=None, resources=None):
    """The build's per-kernel registers, spills, scratch and occupancy."""
    res = load_resources(resources)
    out = ["| kernel | VGPR | AGPR | SGPR | VGPR spill | SGPR spill | scratch B/lane | "
           "waves/SIMD | static LDS B |", "|" + "---|" * 9]
    for name in sorted(res):
        if match and match not in name:
            continue
        r = res[name]
        out.append(f"| `{name}` | {r.get('vgpr')} | {r.get('agpr')} | {r.get('sgpr')} | "
                   f"{r.get('vgpr_spill')} | {r.get('sgpr_spill')} | "
                   f"{r.get('scratch_bytes_per_lane')} | {r.get('waves_per_simd')} | "
                   f"{r.get('static_lds_bytes')} |")
    return "\n".join(out)


def _tail_ids(pairs, tail):
    """{kernel: the ids of its last `tail` dispatches} from (kernel, id) pairs."""
    ids = collections.defaultdict(set)
    for name, disp in pairs:
        ids[name].add(disp)
    return {k: set(sorted(v)[-tail:]) for k, v in ids.items()}


def pmc_per_dispatch(db, match=None, last=False, tail=0):
    """Per kernel, each counter's mean over its dispatches (last: the value of
    the kernel's last dispatch only; tail: the mean over its last `tail`
    dispatches, e.g. one whole split-path fit of a bin)."""
    rows = _rows(db, "select kernel_name, dispatch_id, counter_name, sum(value) "
                     "from counters_collection group by kernel_name, dispatch_id, counter_name")
    acc = collections.defaultdict(lambda: collections.defaultdict(list))
    tail = 1 if last and not tail else tail
    if tail:
        keep = _tail_ids(((r[0], r[1]) for r in rows), tail)
        rows = [r for r in rows if r[1] in keep[r[0]]]
    for name, _disp, ctr, val in rows:
        if match and match not in name:
            continue
        acc[name][ctr].append(val)
    return {k: {c: statistics.mean(v) for c, v in d.items()} for k, d in acc.items()}


def pmc(db, match=None):
    d = pmc_per_dispatch(db, match)
    ctrs = sorted({c for v in d.values() for c in v})
    out = ["| kernel | " + " | ".join(ctrs) + " |", "|" + "---|" * (len(ctrs) + 1)]
    for name in sorted(d):
        out.append(f"| `{name}` | " + " | ".join(f"{d[name].get(c, float('nan')):.6g}"
                                                 for c in ctrs) + " |")
    return "\n".join(out)


def valu(db, match=None, workload_key=None, last=False, tail=0):
    """Per kernel: the average per dispatch of every collected counter and
    the dispatch duration (counter runs serialise dispatches, so these are
    the kernels running alone); last: the kernel's last dispatch only; tail:
    the averages over its last `tail` dispatches."""
    d = pmc_per_dispatch(db, match, last, tail)
    durs = collections.defaultdict(list)
    rows = _rows(db, "select name, dispatch_id, duration from kernels")
    tail = 1 if last and not tail else tail
    keep = _tail_ids(((r[0], r[1]) for r in rows), tail) if tail else None
    for name, disp, dur in rows:
        if name in d and (keep is None or disp in keep[name]):
            durs[name].append(dur / 1e6)
    out = {"kernels": {}}
    for name in sorted(d):
        e = dict(d[name])
        e["alone_ms"] = statistics.mean(durs[name]) if durs[name] else None
        out["kernels"][name] = e
    if workload_key:
        out["workload_key"] = workload_key
    return out


def _calib(db, counter):
    """Counter value of the largest widen_kernel dispatch."""
    rows = _rows(db, "select dispatch_id, max(grid_size), sum(value) from counters_collection "
                     f"where kernel_name like '%widen_kernel%' and counter_name = '{counter}' "
                     "group by dispatch_id order by max(grid_size) desc limit 1")
    if not rows:
        raise SystemExit("no copy calibration kernel (widen_kernel) in " + db)
    return rows[0][2]


def traffic(fetch_db, write_db, kernel, calib_fetch, calib_write, last=False):
    """Per kernel whose name contains `kernel`: HBM bytes per dispatch (last:
    the kernel's last dispatch only, leaving out the calibration call's)."""
    f = pmc_per_dispatch(fetch_db, kernel, last)
    w = pmc_per_dispatch(write_db, kernel, last)
    if not f or sorted(f) != sorted(w):
        raise SystemExit(f"kernel {kernel!r} matches {sorted(f)} / {sorted(w)}")
    # FETCH_SIZE and WRITE_SIZE are in KiB per dispatch
    cf, cw = _calib(fetch_db, "FETCH_SIZE"), _calib(write_db, "WRITE_SIZE")
    f_scale = calib_fetch / (1024.0 * cf)
    w_scale = calib_write / (1024.0 * cw)
    out = {"calib_kernel": "widen_kernel", "calib_fetch_bytes": calib_fetch,
           "calib_write_bytes": calib_write, "calib_fetch_kib_raw": cf,
           "calib_write_kib_raw": cw, "fetch_scale": f_scale, "write_scale": w_scale,
           "kernels": {}}
    for name in sorted(f):
        fetch_b = 1024.0 * f[name]["FETCH_SIZE"] * f_scale
        write_b = 1024.0 * w[name]["WRITE_SIZE"] * w_scale
        out["kernels"][name] = {"fetch_bytes": fetch_b, "write_bytes": write_b,
                                "bytes_per_launch": fetch_b + write_b,
                                "fetch_kib_raw": f[name]["FETCH_SIZE"],
                                "write_kib_raw": w[name]["WRITE_SIZE"]}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("mode", choices=["trace", "pmc", "traffic", "valu", "resources"])
    ap.add_argument("dbs", nargs="*")
    ap.add_argument("--resources", default=None,
                    help="trace, resources: the build's kernel_resources.json (default: "
                         "the one next to the library)")
    ap.add_argument("--match", default=None)
    ap.add_argument("--kernel", default=None)
    ap.add_argument("--calib-fetch-bytes", type=float, default=None)
    ap.add_argument("--calib-write-bytes", type=float, default=None)
    ap.add_argument("--out", default=None)
    ap.add_argument("--workload-key", default=None)
    ap.add_argument("--skip", type=int, default=0,
                    help="trace: drop each kernel's first SKIP dispatches")
    ap.add_argument("--take", type=int, default=None,
                    help="trace: then keep TAKE dispatches per kernel")
    ap.add_argument("--last", action="store_true",
                    help="valu, traffic: each kernel's last dispatch only (runs whose "
                         "earlier dispatches are warm-ups or calibration calls)")
    ap.add_argument("--tail", type=int, default=0,
                    help="valu: averages over each kernel's last TAIL dispatches (the "
                         "split path: 1 + max_iter pass launches are one fit of a bin)")
    a = ap.parse_args()
    if a.mode == "resources":
        print(resources_table(a.match, a.resources))
    elif a.mode == "trace":
        print(trace(a.dbs[0], a.match, a.skip, a.take, a.resources))
    elif a.mode == "pmc":
        print(pmc(a.dbs[0], a.match))
    elif a.mode == "valu":
        t = valu(a.dbs[0], a.match, a.workload_key, a.last, a.tail)
        print(json.dumps(t, indent=1))
        if a.out:
            with open(a.out, "w") as fh:
                json.dump(t, fh, indent=1)
    else:
        t = traffic(a.dbs[0], a.dbs[1], a.kernel, a.calib_fetch_bytes, a.calib_write_bytes,
                    a.last)
        if a.workload_key:
            t["workload_key"] = a.workload_key
        print(json.dumps(t, indent=1))
        if a.out:
            with open(a.out, "w") as fh:
                json.dump(t, fh, indent=1)


if __name__ == "__main__":
    main()
