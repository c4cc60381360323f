"""Seeded synthetic populations for the benchmark configurations.

Role of the reference generator (cusr/benchmark/workload/gen_synth.py:46-153),
with the benchmark's own op sets and shapes:

  C1  1,024 expr, depth<=4, K in 1..4,  D=2, N=256,     x~U[-3,3], sigma 0.01, init sd 0.5
  C2 16,384 expr, depth<=6, <=31 nodes, K in 1..8,  D=3, N=1,024, x~U[-3,3], sigma 0.01, init sd 0.5
  C3  8,192 expr, depth<=8, <=63 nodes, K in 4..16, D=4, N=2,048, x~U[-2,2], sigma 0.01, init sd 1.0
  C4  4,096 expr, depth<=6, <=31 nodes, K in 1..8,  D=5, N=100,000, x~U[-3,3], sigma 0.05, init sd 0.5
  C5 65,536 expr per round, depth<=7, <=63 nodes, K in 0..8, D=4, N=2,048, one shared target
  G1  4,000 expr, depth<=9, <=127 nodes, K in 1..28, D=2, N=1,000: a GP generation shaped
      like the header of the reference's operon4000_g100 snapshot (M 4,000, N 1,000,
      n_vars 2, K_max 28, mean K 14.4; cusr/kernel/tests/golden/manifest.json), whose
      K >= 17 expressions run in the general kernel (not a BASELINE configuration)
  G1F the same generation with K in 1..16: every expression on the fast kernels, for
      comparing the general kernel's cost with theirs

Draw order (numpy default_rng(seed)): x for all points; then per expression
slot: K, the tree shape and ops, the constant/variable leaf assignment,
c_true ~ N(0,1), c_init = c_true + N(0, init_sd^2), noise. Slots whose target
is non-finite or exceeds 1e6 in magnitude are redrawn from the same stream
(the rejection rule of gen_synth.py:137-140). x, y and c_init are rounded to
float32 before use, so a pop.bin file carries the exact inputs of a fit.

Targets need an evaluator: a callable (pop_dict, c float64, xs float64) ->
y float64 [M, N]. The product passes the HIP evaluator (co_eval_ex); CPU tests
pass the oracle's.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import popio

OPS_C1 = dict(binary=(1, 2, 3, 32), unary=(14, 15, 33, 34))
OPS_FULL = dict(binary=(1, 2, 3, 32), unary=(14, 15, 33, 35, 28, 34))


@dataclass
class SynthConfig:
    name: str
    M: int
    N: int
    D: int
    depth: int
    max_nodes: int
    k_lo: int
    k_hi: int
    x_lo: float
    x_hi: float
    sigma: float
    init_sd: float
    max_iter: int
    seed: int
    ad_mode: int = 0       # 0 forward, 1 reverse
    precision: int = 0     # 0 fp64, 1 mixed
    ops: dict = field(default_factory=lambda: OPS_FULL)
    shared_target: bool = False
    rounds: int = 1


CONFIGS = {
    "C1": SynthConfig("C1", 1024, 256, 2, 4, 31, 1, 4, -3.0, 3.0, 0.01, 0.5, 20, 101, ops=OPS_C1),
    "C2": SynthConfig("C2", 16384, 1024, 3, 6, 31, 1, 8, -3.0, 3.0, 0.01, 0.5, 50, 201),
    "C3": SynthConfig("C3", 8192, 2048, 4, 8, 63, 4, 16, -2.0, 2.0, 0.01, 1.0, 50, 301, ad_mode=1),
    "C4": SynthConfig("C4", 4096, 100000, 5, 6, 31, 1, 8, -3.0, 3.0, 0.05, 0.5, 30, 401),
    "C5": SynthConfig("C5", 65536, 2048, 4, 7, 63, 0, 8, -3.0, 3.0, 0.01, 0.5, 10, 501,
                      precision=1, shared_target=True, rounds=20),
    "G1": SynthConfig("G1", 4000, 1000, 2, 9, 127, 1, 28, -3.0, 3.0, 0.01, 0.5, 50, 601),
    "G1F": SynthConfig("G1F", 4000, 1000, 2, 9, 127, 1, 16, -3.0, 3.0, 0.01, 0.5, 50, 601),
}


def scaled(cfg: SynthConfig, M: int | None = None, N: int | None = None) -> SynthConfig:
    """Same config with fewer expressions / points (parity-test sizes)."""
    d = dict(cfg.__dict__)
    if M is not None:
        d["M"] = M
    if N is not None:
        d["N"] = N
    return SynthConfig(**d)


def _grow(rng, cfg: SynthConfig, ops):
    """One random shape in prefix order: list of (kind, op) with kind 'u','b','l'."""
    out = []

    def rec(depth):
        if len(out) > cfg.max_nodes:
            return
        leaf = depth >= cfg.depth or (depth > 0 and rng.random() < 0.3)
        if leaf:
            out.append(("l", 0))
        elif rng.random() < 0.6:
            out.append(("b", int(rng.choice(ops["binary"]))))
            rec(depth + 1)
            rec(depth + 1)
        else:
            out.append(("u", int(rng.choice(ops["unary"]))))
            rec(depth + 1)

    rec(0)
    return out


def random_tree(rng, cfg: SynthConfig, ops=None):
    """(nt, nv, ci, K): a tree with exactly K constants and >= 1 variable leaf."""
    ops = ops or cfg.ops
    K = int(rng.integers(cfg.k_lo, cfg.k_hi + 1))
    for _ in range(10000):
        shape = _grow(rng, cfg, ops)
        n_leaf = sum(1 for k, _ in shape if k == "l")
        if len(shape) > cfg.max_nodes or n_leaf < K + 1:
            continue
        leaf_is_const = np.zeros(n_leaf, bool)
        leaf_is_const[rng.choice(n_leaf, size=K, replace=False)] = True
        nt, nv, ci = [], [], []
        li = rank = 0
        for kind, op in shape:
            if kind == "b":
                nt.append(popio.NODE_BFUNC); nv.append(float(op)); ci.append(-1)
            elif kind == "u":
                nt.append(popio.NODE_UFUNC); nv.append(float(op)); ci.append(-1)
            else:
                if leaf_is_const[li]:
                    nt.append(popio.NODE_CONST); nv.append(0.0); ci.append(rank); rank += 1
                else:
                    nt.append(popio.NODE_VAR); nv.append(float(rng.integers(0, cfg.D))); ci.append(-1)
                li += 1
        return (np.asarray(nt, np.int32), np.asarray(nv, np.float32),
                np.asarray(ci, np.int32), K)
    raise RuntimeError("could not draw a tree with the requested K")


def _draw_slot(rng, cfg: SynthConfig, N: int):
    nt, nv, ci, K = random_tree(rng, cfg)
    c_true = rng.standard_normal(K)
    c_init = (c_true + cfg.init_sd * rng.standard_normal(K)).astype(np.float32)
    noise = cfg.sigma * rng.standard_normal(N)
    return (nt, nv, ci, c_init), c_true, noise


def generate(cfg: SynthConfig, evaluator, round_index: int = 0, max_rounds: int = 50):
    """Population dict plus the true constants (float64, pop c_offset layout)."""
    rng = np.random.default_rng(cfg.seed + round_index)
    N, M = cfg.N, cfg.M
    xs = rng.uniform(cfg.x_lo, cfg.x_hi, size=(N, cfg.D)).astype(np.float32)
    xs64 = xs.astype(np.float64)
    shared_y = None
    if cfg.shared_target:
        # one seeded target expression, tiled to every row as the reference's
        # GP bridge does (cusr/demonstrator/kernel_bridge.py:202)
        tcfg = scaled(cfg)
        tcfg.k_lo = max(cfg.k_lo, 1)
        for _ in range(max_rounds * 10):
            (tnt, tnv, tci, _), tc, tnoise = _draw_slot(rng, tcfg, N)
            tp = popio.build_pop([(tnt, tnv, tci, tc.astype(np.float32))], xs, np.zeros((1, N)))
            ty = evaluator(tp, tc.astype(np.float64), xs64)[0]
            if np.all(np.isfinite(ty)) and np.max(np.abs(ty)) <= 1e6:
                shared_y = (ty + tnoise).astype(np.float32)
                break
        if shared_y is None:
            raise RuntimeError("no finite shared target")
    slots = [None] * M
    truth = [None] * M
    noises = [None] * M
    todo = np.arange(M)
    for _ in range(max_rounds):
        for m in todo:
            slots[m], truth[m], noises[m] = _draw_slot(rng, cfg, N)
        if cfg.shared_target:
            bad = np.zeros(len(todo), bool)   # any expression is a valid GP candidate
            for j, m in enumerate(todo):
                noises[m] = None
        else:
            cand = popio.build_pop([slots[m] for m in todo], xs, np.zeros((len(todo), N)))
            c64 = np.concatenate([truth[m] for m in todo]) if cand["total_c"] else np.zeros(0)
            y = evaluator(cand, c64, xs64)
            bad = ~np.all(np.isfinite(y) & (np.abs(y) <= 1e6), axis=1)
            for j, m in enumerate(todo):
                if not bad[j]:
                    noises[m] = (y[j] + noises[m]).astype(np.float32)
        todo = todo[bad]
        if len(todo) == 0:
            break
    if len(todo):
        raise RuntimeError(f"{len(todo)} slots still invalid after {max_rounds} rounds")
    ym = np.tile(shared_y, (M, 1)) if cfg.shared_target else np.stack(noises)
    pop = popio.build_pop(slots, xs, ym)
    c_true = np.concatenate(truth) if pop["total_c"] else np.zeros(0)
    return pop, c_true
