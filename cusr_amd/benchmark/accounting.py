"""Algorithmic work of one LM fit: compulsory HBM bytes and flops.

The unit of work is a point-pass (one expression, one data point). An LM
iteration of an active expression costs two point-passes over its N points:
the Jacobian / J^T J pass at the accepted constants and the trial evaluation
at c + delta (cusr/kernel/batch_lm_ad.cu:363-372 and :400-412). The count is
fixed at two whatever the implementation does (this one re-uses the trial
pass's Jacobian after an accept), and an expression stops counting at the
iteration it finished on.

Bytes (compulsory): every point-pass reads y once; X is read once per pass for
the whole population; the bytecode and constants of an active expression once
per pass (12 bytes per node and 8 per constant, the pop.bin sizes). B_stream
adds X re-read per expression, the upper figure when nothing stays in cache.

Flops per point-pass, by opcode (forward AD, K constants):
    value: 1 for a binary node, 2 for a unary node (f and f')
    tangent: K for + - max min and comparisons, 3K for * / pow, K for unary
    residual and normal equations: 1 + 2 * (K(K+1)/2 + K + 1)
Reverse AD replaces the tangent terms with a backward sweep of 4 flops per
binary and 2 per unary node. The trial pass costs the value flops plus 3
(residual and its square). Transcendental functions count 2, so the figure
is a lower bound on the VALU work.
"""
from __future__ import annotations

import numpy as np

ADDITIVE = {1, 2, 8, 9, 10, 11, 12, 13}     # ADD SUB MAX MIN LT GT LE GE
PASSES_PER_ITER = 2


def _node_counts(pop):
    """Per expression: (binary additive, binary multiplicative, unary) counts."""
    nt = np.asarray(pop["nt"])
    nv = np.asarray(pop["nv"]).astype(np.int64)
    metas = np.asarray(pop["metas"]).astype(np.int64)
    M = metas.shape[0]
    owner = np.full(len(nt), -1, np.int64)
    for m in range(M):
        owner[metas[m, 0]:metas[m, 0] + metas[m, 1]] = m
    is_bin = nt == 3
    is_add = is_bin & np.isin(nv, list(ADDITIVE))
    counts = []
    for mask in (is_add, is_bin & ~is_add, nt == 2):
        counts.append(np.bincount(owner[mask & (owner >= 0)], minlength=M).astype(np.int64))
    return tuple(counts)


def flops_per_point_pass(pop, ad_mode: int = 0):
    """(pass A, pass B) flops per point for every expression."""
    K = np.asarray(pop["metas"])[:, 3].astype(np.int64)
    add, mul, una = _node_counts(pop)
    value = add + mul + 2 * una
    normal = 1 + 2 * (K * (K + 1) // 2 + K + 1)
    if ad_mode == 0:
        tangent = K * add + 3 * K * mul + K * una
    else:
        tangent = 4 * (add + mul) + 2 * una
    return value + tangent + normal, value + 3


def algorithmic_work(pop, iters, ad_mode: int = 0, s_y: int = 8, s_x: int = 8, subset=None):
    """Compulsory bytes, streaming bytes and flops of one fit.

    iters: iterations each expression ran (K = 0 expressions run none).
    subset: optional boolean mask or index array of expressions (one launch)."""
    metas = np.asarray(pop["metas"])
    K = metas[:, 3].astype(np.int64)
    n_nodes = metas[:, 1].astype(np.int64)
    it = np.where(K > 0, np.asarray(iters, np.int64), 0)
    fa, fb = flops_per_point_pass(pop, ad_mode)
    sel = np.ones(len(K), bool) if subset is None else np.zeros(len(K), bool)
    if subset is not None:
        sel[subset] = True
    it = np.where(sel, it, 0)
    N, D = int(pop["N"]), int(pop["n_vars"])
    P = PASSES_PER_ITER
    y_bytes = P * N * s_y * int(it.sum())
    x_bytes = P * N * D * s_x * int(it.max() if it.size else 0)
    code_bytes = P * int(np.sum(it * (12 * n_nodes + 8 * K)))
    stream = P * N * (s_y + D * s_x) * int(it.sum()) + code_bytes
    flops = N * int(np.sum(it * (fa + fb)))
    return {"bytes": y_bytes + x_bytes + code_bytes, "bytes_stream": stream, "flops": flops,
            "point_passes": P * N * int(it.sum())}
