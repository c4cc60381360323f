"""Build the gfx950 fitter library and CLI in-tree.

    python -m cusr_amd.build [--jobs N]

Outputs (next to the ctypes loader, like the reference's make targets,
cusr/kernel/Makefile:77-81):
    cusr_amd/kernel/libcusr_co_ad.so   C ABI of include/cusr_co.h, AD variant LM ordering
    cusr_amd/kernel/libcusr_co_fd.so   same kernels, the FD variant's LM ordering by default
    cusr_amd/kernel/batch_lm_ad        CLI with the reference's arguments/blobs (AD ordering)
    cusr_amd/kernel/batch_lm           the same CLI over libcusr_co_fd.so
    cusr_amd/kernel/kernel_resources.json
                                       per kernel: VGPRs, AGPRs, SGPRs, spills, scratch
                                       bytes per lane, occupancy and static LDS, from the
                                       compiler's resource-usage remarks
Objects go to cusr_amd/_build/. Every call recompiles.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
REPO = ROOT.parent
CSRC = ROOT / "csrc"
BUILD = ROOT / "_build"
KDIR = ROOT / "kernel"
LIB = KDIR / "libcusr_co_ad.so"
LIB_FD = KDIR / "libcusr_co_fd.so"
CLI = KDIR / "batch_lm_ad"
CLI_FD = KDIR / "batch_lm"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# offload target; CUSR_OFFLOAD_ARCH selects a feature variant (e.g. gfx950:xnack-)
ARCH = os.environ.get("CUSR_OFFLOAD_ARCH", "gfx950")

# -ffp-contract=off: fused multiply-adds only where fma() is written, so the
# device arithmetic order is the one the CPU oracle reproduces.
# -packed-fp32-ops off: no v_pk_*_f32 generated from float code.
# -structurizecfg-skip-uniform-regions: regions whose branches are wave-uniform
# (the interpreter's dispatch on scalar-loaded instruction words) keep their
# scalar branches instead of being rewritten into structured form with
# flow-flag blocks; per interpreter step about a quarter fewer scalar and
# branch instructions and fewer register copies (C2 -9 %, C3 -15 %, C4 -11 %,
# C5 -12 %, bit-identical results). Divergent regions are structurized as
# before.
DEVICE_FLAGS = ["-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}", "-ffp-contract=off",
                "-fno-fast-math", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                "-mllvm", "-structurizecfg-skip-uniform-regions=1",
                f"-I{REPO / 'include'}", "-Wall", "-Wno-unused-function"]

FIT_VARIANTS = [("double", 0, "f64_fwd"), ("double", 1, "f64_rev"),
                ("float", 0, "f32_fwd"), ("float", 1, "f32_rev")]
RESOURCES = KDIR / "kernel_resources.json"
# the compiler reports each kernel's registers, spills, scratch and occupancy
REMARKS = "-Rpass-analysis=kernel-resource-usage"
_REMARK = re.compile(r"remark: +(Function Name|[A-Za-z ]+?)(?: \[[^\]]*\])?: (\S+) \[-Rpass")
_FIELDS = {"TotalSGPRs": "sgpr", "VGPRs": "vgpr", "AGPRs": "agpr",
           "ScratchSize": "scratch_bytes_per_lane", "Occupancy": "waves_per_simd",
           "SGPRs Spill": "sgpr_spill", "VGPRs Spill": "vgpr_spill", "LDS Size": "static_lds_bytes"}


def parse_resource_remarks(text: str) -> dict:
    """{mangled kernel name: {field: int}} from -Rpass-analysis=kernel-resource-usage output."""
    out, cur = {}, None
    for line in text.splitlines():
        m = _REMARK.search(line)
        if not m:
            continue
        key, val = m.group(1).strip(), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {})
        elif cur is not None and key in _FIELDS:
            cur[_FIELDS[key]] = int(val) if val.lstrip("-").isdigit() else val
    return out


def _demangle(names):
    try:
        r = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True,
                           check=True)
        return r.stdout.splitlines()
    except (OSError, subprocess.CalledProcessError):
        return list(names)


_RES_SINK: dict = {}


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in (r.stderr or "").splitlines()
                    if "packed-fp32-ops" not in l and "kernel-resource-usage" not in l)
    res = parse_resource_remarks(r.stderr or "")
    if res:
        _RES_SINK.update(res)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(map(str, cmd))}\n{err}")
    return err


def build(jobs: int | None = None, verbose: bool = False, defines=(), out: Path | None = None,
          cli: bool = True, src_root: Path | None = None) -> Path:
    """Compile everything; `defines` adds -D flags (tuning variants) and `out`
    redirects the library (the CLI is only built for the default library).
    `src_root` (with `out` only) compiles a copy of the sources laid out as
    the repository's (src_root/cusr_amd/csrc, src_root/include), such as the
    device mutants of oracle/mutation_gate.py."""
    if src_root is not None and out is None:
        raise ValueError("a build from another source tree needs its own output")
    csrc = CSRC if src_root is None else Path(src_root) / "cusr_amd" / "csrc"
    flags = DEVICE_FLAGS if src_root is None else \
        [f if not f.startswith("-I") else f"-I{Path(src_root) / 'include'}" for f in DEVICE_FLAGS]
    extra = [f"-D{d}" for d in defines]
    # CUSR_EXTRA_HIPCC_FLAGS: more device-compile flags, for redirected (tuning)
    # builds only; the shipped libraries never pick them up from the environment
    if out is not None:
        extra += os.environ.get("CUSR_EXTRA_HIPCC_FLAGS", "").split()
    lib = Path(out) if out is not None else LIB
    # a redirected build keeps its objects apart, so builds can run side by side
    bdir = BUILD if out is None else BUILD / Path(out).stem
    bdir.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    compiles = []
    for rtype, ad, name in FIT_VARIANTS:
        obj = bdir / f"fit_launch_fit_{name}.o"
        compiles.append([HIPCC, *flags, *extra, REMARKS, "-x", "hip",
                         f"-DCUSR_FIT_R={rtype}",
                         f"-DCUSR_FIT_AD={ad}", f"-DCUSR_FIT_LAUNCH=launch_fit_{name}",
                         f"-DCUSR_PASS_LAUNCH=launch_pass_{name}", "-c",
                         str(csrc / "fit_kernels.hip"), "-o", str(obj)])
    compiles.append([HIPCC, *flags, *extra, REMARKS, "-x", "hip", "-c",
                     str(csrc / "co_lib.hip"), "-o", str(bdir / "co_lib.o")])
    compiles.append([HIPCC, *flags, "-x", "hip", "-c", str(csrc / "program.cpp"),
                     "-o", str(bdir / "program.o")])
    default = out is None
    if default:
        compiles.append([HIPCC, *flags, *extra, "-x", "hip", "-DCUSR_DEFAULT_ORDER=1", "-c",
                         str(csrc / "co_lib.hip"), "-o", str(bdir / "co_lib_fd.o")])
    _RES_SINK.clear()
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for err in ex.map(_run, compiles):
            if verbose and err.strip():
                print(err, file=sys.stderr)
    names = sorted(_RES_SINK)
    table = {m: dict(_RES_SINK[m], name=d) for m, d in zip(names, _demangle(names))}
    res_path = RESOURCES if out is None else Path(out).with_suffix(".resources.json")
    res_path.write_text(json.dumps(table, indent=1, sort_keys=True) + "\n")
    objs = [str(c[c.index("-o") + 1]) for c in compiles]
    fit_objs = [o for o in objs if "co_lib" not in Path(o).name]
    links = [(lib, fit_objs + [str(bdir / "co_lib.o")])]
    if default:
        links.append((LIB_FD, fit_objs + [str(bdir / "co_lib_fd.o")]))
    for target, lobjs in links:
        tmp = target.with_suffix(".so.tmp")
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *lobjs])
        os.replace(tmp, target)
    if cli and default:
        for exe, name in ((CLI, "cusr_co_ad"), (CLI_FD, "cusr_co_fd")):
            _run(["g++", "-O2", "-std=c++17", f"-I{REPO / 'include'}", "-o", str(exe),
                  str(csrc / "batch_lm_main.cpp"), f"-L{KDIR}", f"-l{name}",
                  "-Wl,-rpath,$ORIGIN"])
    return lib


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("-D", dest="defines", action="append", default=[])
    ap.add_argument("--out", default=None)
    a = ap.parse_args()
    print(build(a.jobs, a.verbose, a.defines, a.out))
