"""Vectorised numpy fp64 interpreter and loss: the scoring oracle.

Test infrastructure only. Restates cusr/benchmark/interp.py:32-102 (stack of
(N,) arrays, last node first, LOOSE_* with the numpy meanings, non-finite
values propagate) and adds the benchmark's protected/clamped operators with
the definitions of include/pop_format.h. `loss_pop` recomputes 0.5 * sum r^2
per expression from returned constants, inf when non-finite (interp.py:81-95,
docs/PROTOCOL.md:37-38).
"""
from __future__ import annotations

import numpy as np

NODE_VAR, NODE_CONST, NODE_UFUNC, NODE_BFUNC = 0, 1, 2, 3


def _pdiv(l, r):
    prot = np.abs(r) < 1e-9
    with np.errstate(all="ignore"):
        q = l / np.where(prot, 1.0, r)
    return np.where(prot, 1.0, q)


def _cexp(a):
    with np.errstate(all="ignore"):
        return np.where(a > 20.0, 485165195.4097903, np.exp(np.minimum(a, 20.0)))


UNARY = {
    14: np.sin, 15: np.cos, 16: np.tan, 17: np.sinh, 18: np.cosh, 19: np.tanh,
    20: np.log, 21: lambda a: np.log(np.abs(a)), 22: np.exp,
    23: lambda a: 1.0 / a, 24: lambda a: 1.0 / a, 25: np.negative, 26: np.abs,
    27: np.sqrt, 28: lambda a: np.sqrt(np.abs(a)),
    33: _cexp, 34: lambda a: a * a, 35: lambda a: np.log(np.abs(a) + 1e-9),
}

BINARY = {
    1: np.add, 2: np.subtract, 3: np.multiply, 4: np.divide, 5: np.divide,
    6: np.power, 7: lambda l, r: np.abs(l) ** r, 8: np.maximum, 9: np.minimum,
    10: lambda l, r: (l < r).astype(float), 11: lambda l, r: (l > r).astype(float),
    12: lambda l, r: (l <= r).astype(float), 13: lambda l, r: (l >= r).astype(float),
    32: _pdiv,
}


def eval_tree_arrays(nt, nv, ci, xs, c):
    """One expression at all N points (interp.py:52-76): xs (N, D), c (K,) -> (N,)."""
    xs = np.asarray(xs, np.float64)
    c = np.asarray(c, np.float64)
    N = xs.shape[0]
    stack = []
    with np.errstate(all="ignore"):
        for i in range(len(nt) - 1, -1, -1):
            t = int(nt[i])
            if t == NODE_VAR:
                stack.append(xs[:, int(nv[i])])
            elif t == NODE_CONST:
                stack.append(np.full(N, c[int(ci[i])]))
            elif t == NODE_UFUNC:
                stack.append(UNARY[int(nv[i])](stack.pop()))
            elif t == NODE_BFUNC:
                l = stack.pop()
                r = stack.pop()
                stack.append(BINARY[int(nv[i])](l, r))
            else:
                raise ValueError(f"unsupported node type {t} at node {i}")
    if len(stack) != 1:
        raise RuntimeError(f"malformed expression: stack depth {len(stack)}")
    return stack[0]


def y_row(pop, m, ym=None):
    """Target of expression m: row m of ym, or its one row when the
    population has a shared target (pop.bin v2 flag)."""
    ym = pop["ym"] if ym is None else ym
    return ym[0] if pop.get("shared_y") and len(ym) == 1 else ym[m]


def tree_view(pop, m):
    off, n, c_off, K = (int(v) for v in pop["metas"][m])
    sl = slice(off, off + n)
    return pop["nt"][sl], pop["nv"][sl], pop["ci"][sl], y_row(pop, m), K


def loss_pop(pop, c_final, xs=None, ym=None) -> np.ndarray:
    """fp64 0.5 * sum r^2 per expression at c_final; inf when non-finite."""
    xs = pop["xs"] if xs is None else xs
    ym = pop["ym"] if ym is None else ym
    out = np.full(int(pop["M"]), np.inf)
    for m in range(int(pop["M"])):
        off, n, c_off, K = (int(v) for v in pop["metas"][m])
        nt, nv, ci = pop["nt"][off:off + n], pop["nv"][off:off + n], pop["ci"][off:off + n]
        y = eval_tree_arrays(nt, nv, ci, xs, np.asarray(c_final[c_off:c_off + K], np.float64))
        if np.all(np.isfinite(y)):
            r = y - np.asarray(y_row(pop, m, ym), np.float64)
            out[m] = 0.5 * float(np.sum(r * r))
    return out
