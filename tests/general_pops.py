"""Seeded populations for the general kernel (expressions outside co_fast_path):
K 17..32, value stacks 17..64, more than 255 nodes, more than 8 variables --
all within the reference's bounds (K <= 32, stack <= 64,
cusr/kernel/ad_interp.cuh:34-39), which its GP bridge sends to the library
(cusr/demonstrator/kernel_bridge.py:45-46,66-71).

Shapes:
  highk  random trees (depth <= 8, <= 127 nodes) with K uniform in 17..32
  deep   left spines: op(op(...op(x, l1)..., l_{S-1}), l_S) has a value stack
         of S + 1; S uniform in 17..63, leaves constants or variables
  long   right spines: op(l1, op(l2, ...)) of 128..200 operators: stack 2,
         more than 255 nodes
  wide   C2-shaped trees (K 1..8) over 12 variables
  mixed  C2-shaped trees and highk trees in one population
Targets come from the CPU oracle's evaluator at c_true ~ N(0, 1) plus noise;
c_init = c_true + N(0, 0.3^2); non-finite or huge targets are redrawn.
"""
from __future__ import annotations

import functools

import numpy as np

from cusr_amd.benchmark import gen_synth, popio
from oracle import lm_oracle

ADD, SUB, MUL, SIN, COS, SQUARE = 1, 2, 3, 14, 15, 34


def _leaf(rng, D, want_const, rank):
    if want_const:
        return popio.NODE_CONST, 0.0, rank
    return popio.NODE_VAR, float(rng.integers(0, D)), -1


def deep_tree(rng, S, D, K):
    """Left spine of S binary operators; K of its S right leaves are constants."""
    ops = rng.choice([ADD, SUB, MUL, ADD], size=S)
    const_at = set(rng.choice(S, size=min(K, S), replace=False).tolist())
    nt = [popio.NODE_BFUNC] * S
    nv = [float(o) for o in ops[::-1]]
    ci = [-1] * S
    # innermost left operand: sin(x_v) keeps the spine's values bounded
    nt += [popio.NODE_UFUNC, popio.NODE_VAR]
    nv += [float(SIN), float(rng.integers(0, D))]
    ci += [-1, -1]
    rank = 0
    for j in range(S):
        t, v, c = _leaf(rng, D, j in const_at, rank)
        rank += t == popio.NODE_CONST
        nt.append(t); nv.append(v); ci.append(c)
    return nt, nv, ci, rank


def long_tree(rng, S, D, K):
    """Right spine of S operators (binary, with an occasional cos): stack 2."""
    nt, nv, ci = [], [], []
    slots = S          # one leaf per binary operator, plus the last leaf
    const_at = set(rng.choice(slots + 1, size=min(K, slots + 1), replace=False).tolist())
    rank = leaf = 0
    for _ in range(S):
        if rng.random() < 0.15:
            nt.append(popio.NODE_UFUNC); nv.append(float(COS)); ci.append(-1)
        op = int(rng.choice([ADD, SUB, ADD, MUL]))
        nt.append(popio.NODE_BFUNC); nv.append(float(op)); ci.append(-1)
        t, v, c = _leaf(rng, D, leaf in const_at, rank)
        rank += t == popio.NODE_CONST
        leaf += 1
        nt.append(t); nv.append(v); ci.append(c)
    t, v, c = _leaf(rng, D, leaf in const_at, rank)
    rank += t == popio.NODE_CONST
    nt.append(t); nv.append(v); ci.append(c)
    return nt, nv, ci, rank


HIGHK = gen_synth.SynthConfig("G", 0, 0, 4, 8, 127, 17, 32, -2.0, 2.0, 0.01, 0.3, 15, 0)


def _draw(rng, kind, D):
    if kind == "highk":
        cfg = gen_synth.scaled(HIGHK)
        cfg.D = D
        nt, nv, ci, K = gen_synth.random_tree(rng, cfg)
        return list(nt), list(nv), list(ci), K
    if kind == "deep":
        S = int(rng.integers(17, 64))
        return deep_tree(rng, S, D, int(rng.integers(1, 33)))
    if kind == "long":
        S = int(rng.integers(128, 201))
        return long_tree(rng, S, D, int(rng.integers(1, 17)))
    cfg = gen_synth.scaled(gen_synth.CONFIGS["C2"])
    cfg.D = D
    nt, nv, ci, K = gen_synth.random_tree(rng, cfg)
    return list(nt), list(nv), list(ci), K


@functools.lru_cache(maxsize=None)
def general_pop(kind: str, M: int, N: int, seed: int = 7):
    """(pop, c_true); kind in highk, deep, long, wide, mixed."""
    rng = np.random.default_rng(seed)
    D = 12 if kind == "wide" else 4
    xs = rng.uniform(-2.0, 2.0, size=(N, D)).astype(np.float32)
    xs64 = xs.astype(np.float64)
    trees, truth, ys = [], [], []
    while len(trees) < M:
        k = kind
        if kind == "mixed":
            k = "highk" if len(trees) % 3 == 0 else "c2"
        elif kind == "wide":
            k = "c2"
        nt, nv, ci, K = _draw(rng, k, D)
        c_true = rng.standard_normal(K)
        c_init = (c_true + 0.3 * rng.standard_normal(K)).astype(np.float32)
        one = popio.build_pop([(nt, nv, ci, c_init)], xs, np.zeros((1, N)))
        y = lm_oracle.eval_pop(one, c=c_true, xs=xs64)[0]
        if not (np.all(np.isfinite(y)) and np.max(np.abs(y)) <= 1e4):
            continue
        trees.append((nt, nv, ci, c_init))
        truth.append(c_true)
        ys.append((y + 0.01 * rng.standard_normal(N)).astype(np.float32))
    pop = popio.build_pop(trees, xs, np.stack(ys))
    return pop, np.concatenate(truth)
