"""The reference CPU path: scipy Levenberg-Marquardt per expression, process pool.

Test / baseline infrastructure only (bench.py's cpu_baseline leg, tests).
Restates ScipyPop (cusr/benchmark/backends.py:97-162): one
scipy.optimize.least_squares(method='lm', xtol=1e-10, ftol=1e-10,
max_nfev=200) per K > 0 expression, fp64 residual from the numpy interpreter
with non-finite residuals replaced by 1e6, a spawn-context process pool with
one worker per core; K = 0 expressions are skipped (status 3).
Status: 0 converged (least_squares status >= 1), 1 iteration limit,
2 failed, 3 K0 (backends.py:102-120).
"""
from __future__ import annotations

import multiprocessing as mp
import os
import time

import numpy as np

from . import interp

SETTINGS = dict(xtol=1e-10, ftol=1e-10, max_nfev=200)


def _worker(payload):
    from scipy.optimize import least_squares

    m, nt, nv, ci, xs, y, c0 = payload
    y64 = np.asarray(y, np.float64)

    def residual(c):
        r = interp.eval_tree_arrays(nt, nv, ci, xs, c) - y64
        return np.where(np.isfinite(r), r, 1e6)

    try:
        res = least_squares(residual, np.asarray(c0, np.float64), method="lm", **SETTINGS)
        c = np.asarray(res.x, np.float64)
        if not np.all(np.isfinite(c)):
            return m, np.asarray(c0, np.float64), 2, int(res.nfev)
        return m, c, (0 if res.status >= 1 else 1), int(res.nfev)
    except Exception:  # noqa: BLE001 -- one expression must not fail the batch
        return m, np.asarray(c0, np.float64), 2, 0


class ScipyPop:
    """fit_pop(pop) -> dict(c_final, status, n_iter, wall_e2e, wall_core, nproc)."""

    name = "scipy"

    def __init__(self, nproc: int | None = None, timeout: float = 120.0):
        self.nproc = nproc or (os.cpu_count() or 1)
        self.timeout = timeout
        self._pool = None

    def pool(self):
        if self._pool is None:
            self._pool = mp.get_context("spawn").Pool(processes=self.nproc)
        return self._pool

    def close(self):
        if self._pool is not None:
            self._pool.terminate()
            self._pool = None

    def fit_pop(self, pop: dict, c_init=None) -> dict:
        t0 = time.perf_counter()
        M = int(pop["M"])
        c_src = pop["c_init"] if c_init is None else c_init
        c_final = np.asarray(c_src, np.float64).copy()
        status = np.full(M, 3, np.int32)
        n_iter = np.zeros(M, np.int32)
        xs = np.asarray(pop["xs"], np.float64)
        payloads = []
        for m in range(M):
            off, n, c_off, K = (int(v) for v in pop["metas"][m])
            if K == 0:
                continue
            status[m] = 2
            payloads.append((m, pop["nt"][off:off + n], pop["nv"][off:off + n],
                             pop["ci"][off:off + n], xs, interp.y_row(pop, m),
                             np.asarray(c_src[c_off:c_off + K], np.float64)))
        pool = self.pool() if payloads else None
        t_core = time.perf_counter()
        if payloads:
            # a per-result timeout, like backends._imap_drain (backends.py:46-68):
            # a pool whose workers died would otherwise wait forever
            it = pool.imap_unordered(_worker, payloads, chunksize=1)
            for _ in range(len(payloads)):
                try:
                    m, c, st, nfev = it.next(self.timeout)
                except mp.TimeoutError:
                    self.close()
                    raise RuntimeError("scipy worker pool stalled")
                off, n, c_off, K = (int(v) for v in pop["metas"][m])
                c_final[c_off:c_off + K] = c
                status[m] = st
                n_iter[m] = nfev
        wall_core = time.perf_counter() - t_core
        return dict(c_final=c_final, status=status, n_iter=n_iter,
                    wall_e2e=time.perf_counter() - t0, wall_core=wall_core,
                    nproc=self.nproc, n_fit=len(payloads))
