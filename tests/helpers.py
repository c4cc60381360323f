"""Shared test helpers: fixture paths and seeded populations (targets from the oracle)."""
from __future__ import annotations

import functools
from pathlib import Path

import numpy as np

from cusr_amd.benchmark import gen_synth, popio
from oracle import lm_oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
REF_FIX = GOLDEN / "ref_fixtures"


def oracle_evaluator(pop, c, xs):
    return lm_oracle.eval_pop(pop, c=c, xs=xs)


@functools.lru_cache(maxsize=None)
def synth(name: str, M: int, N: int | None = None, seed: int | None = None):
    cfg = gen_synth.scaled(gen_synth.CONFIGS[name], M=M, N=N)
    if seed is not None:
        cfg.seed = seed
    return gen_synth.generate(cfg, oracle_evaluator)


def ref_pop(name: str) -> dict:
    return popio.load_pop_bin(REF_FIX / name)


def f64(pop):
    """fp64 copies of the pop's fp32 inputs (exact promotion)."""
    return (pop["c_init"].astype(np.float64), pop["xs"].astype(np.float64),
            pop["ym"].astype(np.float64))


def rel_diff(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    both_nan = ~np.isfinite(a) & ~np.isfinite(b)
    d = np.abs(a - b) / np.maximum(np.maximum(np.abs(a), np.abs(b)), 1e-300)
    d[both_nan] = 0.0
    d[(a == b)] = 0.0
    return d
