"""Mutation gate of the oracle's pins (test infrastructure only).

    python oracle/mutation_gate.py [--only NAME ...] [--list] [--md OUT.md]
    python oracle/mutation_gate.py --device-build DIR     (CPU: build the device mutants)
    python oracle/mutation_gate.py --device-run DIR [--md OUT.md]   (GPU box: run them)

The device and the CPU oracle share include/cusr_math.h and the routing and
partition rules of include/cusr_co.h, so a mistake made in both is invisible
to the bit-exact GPU-vs-oracle comparison. What guards against it are the
oracle's independent pins: the reference's golden losses and Jacobians,
closed forms, central differences, textbook solves, exact-rational sums,
libm accuracy bounds and the truth fixtures (tests/test_oracle.py,
tests/test_math.py). This gate shows that those pins bite: each mutant is
one behaviour-changing edit of oracle/lm_oracle.c or include/cusr_math.h,
made in a copy in a temporary directory and compiled with the oracle's own
flags; the two test files then run against the mutant library
(CUSR_ORACLE_LIB). A mutant is killed when they fail. The unmutated copy must
pass first. The reference gates its reverse-AD kernel the same way, with
behaviour-changing mutants its tests must catch
(experiments/revad_v5/mutation_test.py:1-40, docs/kernel/REVAD_V5.md:97).

The device half: each device mutant is one edit of the HIP source
(cusr_amd/csrc/lm_device.h), built as a redirected library from a copy of
the sources (cusr_amd/build.py src_root); on the GPU box
tests/test_gpu_parity.py runs once against each (CUSR_CO_LIB), and a mutant
is killed when the device-vs-oracle comparison fails. The edits change
arithmetic only (a sign, an operand, a seed, an order, a factor), so no
mutant can reach memory the unmutated kernel does not.

Exit status 0 when every mutant is killed.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import tempfile
import time
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]
CFLAGS = ["-O2", "-fPIC", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-shared"]
TESTS = ["tests/test_oracle.py", "tests/test_math.py"]

# name, file (relative to the repo), text to replace, replacement, occurrence
# (0-based, among the exact matches), what the edit breaks
MUTANTS = [
    ("sin-partial-sign", "oracle/lm_oracle.c",
     "case OP_SIN: cm_sincos(a, &r, d); break;",
     "case OP_SIN: cm_sincos(a, &r, d); *d = -*d; break;", 0,
     "d sin(a)/da = -cos(a)"),
    ("div-partials-swapped", "oracle/lm_oracle.c",
     "o = l / rv; *d1 = 1.0 / rv; *d2 = -(o * *d1); break;",
     "o = l / rv; *d2 = 1.0 / rv; *d1 = -(o * *d2); break;", 0,
     "the partials of l / r exchanged"),
    ("mul-partials-swapped", "oracle/lm_oracle.c",
     "case OP_MUL: o = l * rv; *d1 = rv; *d2 = l; break;",
     "case OP_MUL: o = l * rv; *d1 = l; *d2 = rv; break;", 0,
     "d(l r)/dl = l"),
    ("adjoint-seed", "oracle/lm_oracle.c",
     "sa[asp++] = 1.0;", "sa[asp++] = 2.0;", 0,
     "the reverse sweep starts from adjoint 2"),
    ("reverse-push-order", "oracle/lm_oracle.c",
     "sa[asp++] = safe_mul64(adj, tape2[i]);\n                sa[asp++] = safe_mul64(adj, tape1[i]);",
     "sa[asp++] = safe_mul64(adj, tape1[i]);\n                sa[asp++] = safe_mul64(adj, tape2[i]);",
     0, "a binary node's operand adjoints pushed in the wrong order"),
    ("safe-mul-plain", "oracle/lm_oracle.c",
     "static double safe_mul64(double a, double b) { return (a == 0.0 || b == 0.0) ? 0.0 : a * b; }",
     "static double safe_mul64(double a, double b) { return a * b; }", 0,
     "0 * inf leaks NaN into the reverse sweep"),
    ("flat-branch-select", "oracle/lm_oracle.c",
     "g[j] = mode ? ((d1 != 0.0) ? g[j] : 0.0) : g[j] * d1;",
     "g[j] = g[j] * d1;", 0,
     "a flat branch's tangent multiplied instead of zeroed"),
    ("lambda-decrease", "oracle/lm_oracle.c",
     "lambda = lambda * 0.1;", "lambda = lambda * 0.5;", 0,
     "lambda / 2 instead of / 10 after an accept"),
    ("accept-strict", "oracle/lm_oracle.c",
     "accept = tri->loss <= cur->loss;", "accept = tri->loss < cur->loss;", 0,
     "an equal loss rejected"),
    ("pivot-zero-accepted", "oracle/lm_oracle.c",
     "} else if (s <= 0.0) {\n            return -1;",
     "} else if (s < 0.0) {\n            return -1;", 0,
     "a zero pivot does not fail the solve"),
    ("damping-absolute", "oracle/lm_oracle.c",
     "else L[i * K + i] = L[i * K + i] * (1.0 + lambda);",
     "else L[i * K + i] = L[i * K + i] + lambda;", 0,
     "absolute instead of relative damping"),
    ("trust-region-diagonal", "oracle/lm_oracle.c",
     "if (damp == CO_DAMP_TRUST_REGION) L[i * K + i] = L[i * K + i] + lambda;",
     "if (damp == CO_DAMP_TRUST_REGION) L[i * K + i] = L[i * K + i] * (1.0 + lambda);", 0,
     "relative instead of absolute damping in the trust-region variant"),
    ("trust-region-rescue", "oracle/lm_oracle.c",
     "if (s <= 0.0) s = lambda;", "if (s <= 0.0) s = 2.0 * lambda;", 0,
     "a trust-region pivot <= 0 replaced by 2 lambda"),
    ("guard-ignores-worse", "oracle/lm_oracle.c",
     "if (!isfinite(lf) || (isfinite(li) && lf > li)) {",
     "if (!isfinite(lf)) {", 0,
     "the fp64 guard keeps a final loss worse than the start"),
    ("partition-order", "oracle/lm_oracle.c",
     "    for (int part = 1; part < G; part++) {\n"
     "        const double *pp = sums + (size_t)part * width;\n"
     "        for (int w = 0; w < width; w++) sums[w] = sums[w] + pp[w];\n    }",
     "    for (int part = G - 2; part >= 0; part--) {\n"
     "        const double *pp = sums + (size_t)part * width;\n"
     "        double *dd = sums + (size_t)(G - 1) * width;\n"
     "        for (int w = 0; w < width; w++) dd[w] = dd[w] + pp[w];\n    }\n"
     "    for (int w = 0; G > 1 && w < width; w++) sums[w] = sums[(size_t)(G - 1) * width + w];",
     0, "partition sums added last partition first"),
    ("butterfly-order", "oracle/lm_oracle.c",
     "for (int s = ORC_LANES / 2; s >= 1; s >>= 1) {",
     "for (int s = 1; s < ORC_LANES; s <<= 1) {", 0,
     "the 64 lanes combined at strides 1..32 instead of 32..1"),
    ("exp-coefficient", "include/cusr_math.h", None, None, 0,
     "one polynomial coefficient of exp changed in its 8th digit"),
    ("log-coefficient", "include/cusr_math.h", None, None, 0,
     "one polynomial coefficient of log changed in its 8th digit"),
    ("cos-quadrant-sign", "include/cusr_math.h",
     "co = ((q + 1) & 2) ? -co : co;", "co = (q & 2) ? -co : co;", 0,
     "the sign of cos taken from the sine's quadrant rule"),
]


# device mutants of the HIP source: name, file, text, replacement, occurrence,
# what the edit breaks, the GPU parity tests that run against it (-k)
DEVICE_MUTANTS = [
    ("dev-sin-partial-sign", "cusr_amd/csrc/lm_device.h",
     "case OP_SIN: CUSR_MATH_V(sincos_v, a + c0, r + c0, d + c0); break;",
     "case OP_SIN: CUSR_MATH_V(sincos_v, a + c0, r + c0, d + c0); CUSR_FOR_P d[p] = -d[p]; break;",
     0, "d sin(a)/da = -cos(a) on the device", "c1 or c2_small"),
    ("dev-pdiv-partials-swapped", "cusr_amd/csrc/lm_device.h",
     "            d1[p] = prot ? zero : inv;\n            d2[p] = prot ? zero : -(q * inv);",
     "            d2[p] = prot ? zero : inv;\n            d1[p] = prot ? zero : -(q * inv);",
     0, "the partials of the protected l / r exchanged on the device", "c1 or c2_small"),
    ("dev-adjoint-seed", "cusr_amd/csrc/lm_device.h",
     "CUSR_FOR_P accadj[p] = R(1);", "CUSR_FOR_P accadj[p] = R(2);", 0,
     "the device's reverse sweep starts from adjoint 2", "c1"),
    ("dev-partition-order", "cusr_amd/csrc/lm_device.h",
     "            double v = a.part[q];\n"
     "            for (int g = 1; g < a.parts; ++g) v = v + a.part[g * W + q];",
     "            double v = a.part[(a.parts - 1) * W + q];\n"
     "            for (int g = a.parts - 2; g >= 0; --g) v = v + a.part[g * W + q];",
     0, "in-workgroup partition sums added last first", "partitions"),
    ("dev-lambda-decrease", "cusr_amd/csrc/lm_device.h",
     "lambda = lambda * 0.1;", "lambda = lambda * 0.5;", 0,
     "lambda / 2 after an accept on the device", "c1 or c2_small"),
]

# (table, index) of the coefficient each coefficient mutant scales: a term
# whose change moves the function by well over an ulp somewhere on its
# reduced range (the r^4 term of exp's polynomial, the z^3 term of log's R)
COEFFICIENT_MUTANTS = {"exp-coefficient": ("cm_exp_tab", 10),
                       "log-coefficient": ("cm_log_tab", 4)}


def _coefficient_edit(text: str, table: str, index: int):
    """(old, new): coefficient `index` of the C table `table` of cusr_math.h
    scaled by (1 + 1e-8), written with 17 significant digits."""
    start = text.index(f" {table}[")
    body_start = text.index("{", start) + 1
    body_end = text.index("};", body_start)
    body = text[body_start:body_end]
    vals = [v.strip() for v in body.split(",")]
    old = vals[index]
    new = repr(float(old.rstrip("f")) * (1.0 + 1e-8))
    vals2 = list(vals)
    vals2[index] = new
    return body, ", ".join(vals2)


def _apply(root: Path, name, rel, old, new, occ) -> None:
    p = root / rel
    text = p.read_text()
    if old is None:
        table, idx = COEFFICIENT_MUTANTS[name]
        old, new = _coefficient_edit(text, table, idx)
    hits, at = [], text.find(old)
    while at >= 0:
        hits.append(at)
        at = text.find(old, at + 1)
    if len(hits) <= occ:
        raise SystemExit(f"mutant {name}: anchor not found in {rel} ({len(hits)} matches)")
    at = hits[occ]
    p.write_text(text[:at] + new + text[at + len(old):])


def _copy_tree(dst: Path) -> None:
    (dst / "oracle").mkdir(parents=True)
    shutil.copy2(REPO / "oracle" / "lm_oracle.c", dst / "oracle" / "lm_oracle.c")
    shutil.copytree(REPO / "include", dst / "include")


def _build(root: Path) -> Path:
    lib = root / "liblm_oracle.so"
    subprocess.run(["gcc", *CFLAGS, "-o", str(lib), str(root / "oracle" / "lm_oracle.c"), "-lm"],
                   check=True, capture_output=True, text=True)
    return lib


def _run_tests(lib: Path, timeout: float):
    """(passed, first failing test id or '', seconds)."""
    env = dict(os.environ, CUSR_ORACLE_LIB=str(lib), PYTHONDONTWRITEBYTECODE="1")
    t0 = time.perf_counter()
    r = subprocess.run([sys.executable, "-m", "pytest", *TESTS, "-x", "-q", "-rf", "-m", "not gpu",
                        "-p", "no:cacheprovider"], cwd=REPO, env=env, capture_output=True,
                       text=True, timeout=timeout)
    dt = time.perf_counter() - t0
    failed = ""
    for line in r.stdout.splitlines():
        if line.startswith("FAILED "):
            failed = line[len("FAILED "):].split(" - ")[0]
            break
    return r.returncode == 0, failed, dt


def run(names=None, timeout=600.0):
    rows = []
    with tempfile.TemporaryDirectory(prefix="cusr_mut_") as tmp:
        base = Path(tmp) / "base"
        _copy_tree(base)
        ok, failed, dt = _run_tests(_build(base), timeout)
        print(f"unmutated copy: {'pass' if ok else 'FAIL ' + failed} ({dt:.1f} s)", flush=True)
        if not ok:
            raise SystemExit("the unmutated oracle fails its own tests; gate not run")
        for name, rel, old, new, occ, what in MUTANTS:
            if names and name not in names:
                continue
            root = Path(tmp) / name
            _copy_tree(root)
            _apply(root, name, rel, old, new, occ)
            try:
                lib = _build(root)
            except subprocess.CalledProcessError as e:
                raise SystemExit(f"mutant {name} does not compile:\n{e.stderr}")
            ok, failed, dt = _run_tests(lib, timeout)
            rows.append((name, what, not ok, failed, dt))
            print(f"{name}: {'killed by ' + failed if not ok else 'SURVIVED'} ({dt:.1f} s)",
                  flush=True)
    return rows


def _device_copy(dst: Path) -> None:
    shutil.copytree(REPO / "cusr_amd" / "csrc", dst / "cusr_amd" / "csrc")
    shutil.copytree(REPO / "include", dst / "include")


def device_build(outdir: Path, names=None) -> None:
    """Build every device mutant as outdir/<name>.so (from a mutated copy of
    the sources; the objects go to cusr_amd/_build/<name>/)."""
    sys.path.insert(0, str(REPO))
    from cusr_amd import build as cbuild

    outdir = Path(outdir)
    outdir.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory(prefix="cusr_devmut_") as tmp:
        for name, rel, old, new, occ, what, _k in DEVICE_MUTANTS:
            if names and name not in names:
                continue
            root = Path(tmp) / name
            _device_copy(root)
            _apply(root, name, rel, old, new, occ)
            t0 = time.perf_counter()
            cbuild.build(out=outdir / f"{name}.so", src_root=root, cli=False)
            print(f"built {name} ({time.perf_counter() - t0:.0f} s): {what}", flush=True)


def device_run(libdir: Path, names=None, timeout: float = 300.0):
    """On the GPU box: tests/test_gpu_parity.py once against each mutant
    library; rows as run()'s."""
    rows = []
    for name, _rel, _old, _new, _occ, what, sel in DEVICE_MUTANTS:
        if names and name not in names:
            continue
        lib = Path(libdir) / f"{name}.so"
        if not lib.exists():
            raise SystemExit(f"{lib} is not built (--device-build)")
        print(f"device mutant {name}: {what}", flush=True)
        env = dict(os.environ, CUSR_CO_LIB=str(lib), PYTHONDONTWRITEBYTECODE="1")
        t0 = time.perf_counter()
        r = subprocess.run([sys.executable, "-m", "pytest", "tests/test_gpu_parity.py", "-x", "-q",
                            "-rf", "-m", "gpu", "-k", sel, "-p", "no:cacheprovider",
                            "--timeout", "120", "--timeout-method", "thread"],
                           cwd=REPO, env=env, capture_output=True, text=True, timeout=timeout)
        dt = time.perf_counter() - t0
        failed = next((ln[len("FAILED "):].split(" - ")[0] for ln in r.stdout.splitlines()
                       if ln.startswith("FAILED ")), "")
        # a failure is a kill only when a test failed its assertions (not a
        # crash or an import error of the run itself)
        killed = r.returncode == 1 and bool(failed)
        if r.returncode not in (0, 1):
            print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
            raise SystemExit(f"device mutant {name}: pytest exited {r.returncode}")
        rows.append((name, what, killed, failed, dt))
        print(f"{name}: {'killed by ' + failed if killed else 'SURVIVED'} ({dt:.1f} s)",
              flush=True)
    return rows


def markdown(rows) -> str:
    out = ["| mutant | edit | killed | first failing test |", "|---|---|---|---|"]
    for name, what, killed, failed, _ in rows:
        out.append(f"| `{name}` | {what} | {'yes' if killed else '**no**'} | "
                   f"`{failed or '-'}` |")
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", nargs="*", default=None)
    ap.add_argument("--list", action="store_true")
    ap.add_argument("--md", default=None, help="write the table as markdown")
    ap.add_argument("--device-build", default=None, metavar="DIR",
                    help="build the device mutant libraries into DIR")
    ap.add_argument("--device-run", default=None, metavar="DIR",
                    help="run the GPU parity tests against the device mutants in DIR")
    a = ap.parse_args()
    if a.list:
        for m in MUTANTS + DEVICE_MUTANTS:
            print(f"{m[0]}: {m[5]}")
        return 0
    if a.device_build:
        device_build(a.device_build, a.only)
        return 0
    rows = device_run(a.device_run, a.only) if a.device_run else run(a.only)
    md = markdown(rows)
    print(md)
    if a.md:
        Path(a.md).write_text(md + "\n")
    return 0 if all(r[2] for r in rows) else 1


if __name__ == "__main__":
    sys.exit(main())
