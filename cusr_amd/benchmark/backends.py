"""Benchmark backends over the MI355X fitter, with the reference benchmark's
result contract (cusr/benchmark/backends.py:80-89, 740-785).

    FitResult(backend, c_final, status, n_iter, wall_e2e, wall_core, meta)

status uses the benchmark's codes: 0 converged, 1 iteration limit, 2 failed,
3 K = 0 (the library's FAIL_CHOLESKY 4 counts as failed, backends.py:746).

KernelPop fits in process through the C ABI (fp64 in and out);
CudaKernelPop runs the CLI on a pop.bin in a temporary directory and parses
its completion line, as the reference's subprocess backend does.
"""
from __future__ import annotations

import re
import subprocess
import tempfile
import time
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from . import popio

STATUS_MAP = {0: 0, 1: 1, 2: 2, 3: 3, 4: 2}
_TIME_RE = re.compile(r"总耗时 ([\d.]+) 秒")
KERNEL_DIR = Path(__file__).resolve().parents[1] / "kernel"


@dataclass
class FitResult:
    backend: str
    c_final: np.ndarray          # (total_c,) float64
    status: np.ndarray           # (M,) int32, benchmark codes above
    n_iter: np.ndarray           # (M,) int32, -1 where the backend does not report it
    wall_e2e: float              # seconds from fit_pop entry to constants in host memory
    wall_core: float             # seconds of the backend's own core section (nan if unknown)
    meta: dict = field(default_factory=dict)


class KernelRunError(RuntimeError):
    pass


def _map_status(raw):
    return np.asarray([STATUS_MAP.get(int(s), 2) for s in raw], np.int32)


class KernelPop:
    """In-process fit (co_optimize_ex). wall_core is the device time of the
    fit kernels (HIP events)."""

    def __init__(self, variant: str = "ad", max_iter: int | None = None, device_id: int = 0,
                 ad_mode: int = 0, precision: int = 0, name: str | None = None):
        self.variant = variant
        self.max_iter = 50 if max_iter is None else int(max_iter)
        self.device_id = int(device_id)
        self.ad_mode = int(ad_mode)
        self.precision = int(precision)
        self.name = name or f"mi355x:{variant}"

    def fit_pop(self, pop: dict) -> FitResult:
        from cusr_amd.kernel import co_inproc

        co = co_inproc.get_inproc_co(self.device_id, self.variant)
        t0 = time.perf_counter()
        r = co.optimize_ex(pop, self.max_iter, ad_mode=self.ad_mode, precision=self.precision)
        wall = time.perf_counter() - t0
        raw = r["status"]
        return FitResult(self.name, r["c_final"].astype(np.float64), _map_status(raw),
                         r["iters"].astype(np.int32), wall, co.last_kernel_ms() / 1e3,
                         meta=dict(dtype="float64" if self.precision == 0 else "mixed",
                                   ad_mode=self.ad_mode, variant=self.variant,
                                   loss_final=r["loss_final"],
                                   raw_status_counts={int(k): int(v) for k, v in
                                                      zip(*np.unique(raw, return_counts=True))},
                                   criteria=f"xtol=1e-6 max_iter={self.max_iter}"))


class CudaKernelPop:
    """The CLI as a subprocess (pop.bin written to a temporary directory);
    wall_core is the time the CLI reports on its completion line."""

    def __init__(self, binary: Path | str | None = None, max_iter: int | None = None,
                 name: str | None = None):
        self.binary = Path(binary) if binary is not None else KERNEL_DIR / "batch_lm_ad"
        self.max_iter = max_iter
        self.name = name or f"kernel:{self.binary.name}"

    def fit_pop(self, pop: dict) -> FitResult:
        if not self.binary.exists():
            raise KernelRunError(f"binary not found: {self.binary}")
        t0 = time.perf_counter()
        with tempfile.TemporaryDirectory(prefix="cusr_amd_kernel_") as td:
            path = Path(td) / "pop.bin"
            popio.save_pop_bin(pop, path)
            cmd = [str(self.binary), str(path), td]
            if self.max_iter is not None:
                cmd += ["--max-iter", str(self.max_iter)]
            r = subprocess.run(cmd, capture_output=True, encoding="utf-8")
            if r.returncode != 0:
                raise KernelRunError(f"exit={r.returncode}: {(r.stderr or r.stdout)[-500:]}")
            raw = np.fromfile(Path(td) / "status.bin", dtype=np.int32)
            c_final = np.fromfile(Path(td) / "c_final.bin", dtype=np.float32).astype(np.float64)
        m = _TIME_RE.search(r.stdout or "")
        return FitResult(self.name, c_final, _map_status(raw), np.full(int(pop["M"]), -1, np.int32),
                         time.perf_counter() - t0, float(m.group(1)) if m else float("nan"),
                         meta=dict(dtype="float32", binary=str(self.binary),
                                   raw_status_counts={int(k): int(v) for k, v in
                                                      zip(*np.unique(raw, return_counts=True))}))
