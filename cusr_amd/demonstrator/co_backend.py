"""Constant-optimisation backend for a GP inner loop, with the reference
demonstrator's contract (cusr/demonstrator/co_backend.py:25-47, 250-285;
cusr/demonstrator/kernel_bridge.py:140-238):

    fit_batch(skeletons, inits, X, y, *, max_iter, native) -> [COResult]

Every candidate shares one problem's (X, y). `native[j]` is candidate j's
expression in prefix form, (nt, nv, ci) arrays of pop.bin node types, values
and constant ranks (the reference extracts the same arrays from its EvoGP
trees; that extraction belongs to the GP system, not to this library).
`skeletons[j]` is only consulted for `n_constants` when it has one. (X, y)
goes to the device once and stays there while later calls pass the same
values; the reference re-sends X with y tiled per candidate on every call
(kernel_bridge.py:200-206).

Candidates the device cannot take (more than 16 constants, a value stack
deeper than 16, more than 255 nodes, more than 8 variables) go to the
`fallback` backend when one is given; without one they raise, since this
library has no CPU path of its own. Results stay aligned with the input
order; final_loss is mean(r^2) = 2 * loss / N in fp64; converged is
status == CONVERGED (kernel_bridge.py:216).
"""
from __future__ import annotations

import hashlib
from collections import OrderedDict
from dataclasses import dataclass

import numpy as np

from cusr_amd.benchmark import popio


@dataclass
class COResult:
    constants: np.ndarray   # fitted constants, shape (n_consts,)
    n_iter: int
    converged: bool
    final_loss: float       # mean(residual ** 2)


def _eligible(nt, n_vars):
    from cusr_amd.kernel import co_inproc as ci

    nt = np.asarray(nt)
    K = int(np.sum(nt == popio.NODE_CONST))
    # the reference bridge's rule (kernel_bridge.py:45-46,66-71): K and the
    # value stack within the library's bounds
    return (K <= ci.CO_MAX_K and n_vars <= ci.CO_MAX_VARS
            and popio.stack_depth(nt) <= ci.CO_MAX_STACK and not np.any(nt > popio.NODE_BFUNC))


def fit_natives(skeletons, inits, natives, X, y, *, max_iter: int = 50, fallback=None,
                variant: str = "ad", device_id: int = 0, ad_mode: int = 0,
                precision: int = 0):
    """(results aligned with skeletons, stats) -- kernel_bridge.py:140-238."""
    from cusr_amd.kernel import co_inproc

    X = np.asarray(X, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64).ravel()
    n_vars = X.shape[1]
    M = len(natives)
    results = [None] * M
    take, fb, n_overflow, n_kmismatch = [], [], 0, 0
    for j, nat in enumerate(natives):
        nt, nv, ci = (np.asarray(a) for a in nat)
        K = int(np.sum(nt == popio.NODE_CONST))
        skel = skeletons[j] if skeletons is not None else None
        if skel is not None and hasattr(skel, "n_constants") and skel.n_constants != K:
            n_kmismatch += 1
            fb.append(j)
        elif not _eligible(nt, n_vars):
            n_overflow += 1
            fb.append(j)
        else:
            take.append(j)
    if fb and fallback is None:
        raise ValueError(f"{len(fb)} candidates are beyond the device limits and no fallback "
                         "backend was given")
    if take:
        trees = []
        for j in take:
            nt, nv, ci = (np.asarray(a) for a in natives[j])
            c0 = np.asarray(inits[j], np.float64)
            trees.append((nt, nv, ci, c0))
        # programs only: (X, y) stays on the device across calls while it is
        # unchanged (co_data_upload), instead of X and y tiled per candidate
        pop = popio.build_pop(trees, np.zeros((len(y), n_vars), np.float32),
                              np.broadcast_to(np.float32(0), (len(take), len(y))))
        c0_64 = np.concatenate([np.asarray(inits[j], np.float64) for j in take]) \
            if pop["total_c"] else np.zeros(0)
        co = co_inproc.get_inproc_co(device_id, variant)
        with co.lock:
            if not co.data_matches(X, y):
                co.upload_data(X, y)
            r = co.optimize_data(pop, max_iter, ad_mode=ad_mode, precision=precision,
                                 c_init=c0_64)
        N = len(y)
        for slot, j in enumerate(take):
            _, _, c_off, K = (int(v) for v in pop["metas"][slot])
            loss = float(r["loss_final"][slot])
            results[j] = COResult(np.asarray(r["c_final"][c_off:c_off + K], np.float64),
                                  int(r["iters"][slot]),
                                  bool(int(r["status"][slot]) == co_inproc.STATUS_CONVERGED),
                                  2.0 * loss / N if np.isfinite(loss) else float("inf"))
    if fb:
        fb_res = fallback.fit_batch([skeletons[j] for j in fb] if skeletons is not None else None,
                                    [inits[j] for j in fb], X, y, max_iter=max_iter,
                                    native=[natives[j] for j in fb])
        for j, res in zip(fb, fb_res):
            results[j] = res
    stats = dict(n_total=M, n_kernel=len(take), n_fallback=len(fb), n_overflow=n_overflow,
                 n_kmismatch=n_kmismatch)
    return results, stats


def data_key(X, y) -> bytes:
    """Digest of one problem's (X, y) as fp64 values."""
    h = hashlib.blake2b(digest_size=16)
    for a in (np.ascontiguousarray(X, np.float64), np.ascontiguousarray(y, np.float64).ravel()):
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.digest()


def structure_key(nt, nv, ci) -> bytes:
    """Digest of an expression's prefix arrays (its structure, constants aside)."""
    h = hashlib.blake2b(digest_size=16)
    for a, dt in ((nt, np.int32), (nv, np.float32), (ci, np.int32)):
        h.update(np.ascontiguousarray(a, dt).tobytes())
        h.update(b"|")
    return h.digest()


class WarmStartCache:
    """Best constants found so far per (data set, expression structure), LRU
    bounded. In a GP loop the same structure comes back generation after
    generation (elites, unchanged copies, converging populations); starting it
    from its best fitted constants instead of the inherited ones turns a fresh
    LM fit into a few polishing iterations. This is the warm start the
    reference plans (docs/kernel/OPTIMIZATION_BACKLOG.md:124-126,
    docs/PAPER.md:24: 50 iterations down to 5-10), whose missing piece there
    is writing fitted constants back for reuse."""

    def __init__(self, capacity: int = 200_000):
        self.capacity = int(capacity)
        self._d: OrderedDict[bytes, tuple[np.ndarray, float]] = OrderedDict()

    def __len__(self):
        return len(self._d)

    def get(self, dkey: bytes, skey: bytes):
        v = self._d.get(dkey + skey)
        if v is not None:
            self._d.move_to_end(dkey + skey)
        return v

    def put(self, dkey: bytes, skey: bytes, constants, loss: float) -> None:
        """Keep constants if they beat what is stored (finite losses only)."""
        if not np.isfinite(loss):
            return
        key = dkey + skey
        old = self._d.get(key)
        if old is None or loss < old[1]:
            self._d[key] = (np.array(constants, np.float64), float(loss))
        self._d.move_to_end(key)
        while len(self._d) > self.capacity:
            self._d.popitem(last=False)


class KernelLM:
    """The fitter behind the demonstrator's ConstantOptimizer protocol.

    warm_start=True starts every candidate whose structure was fitted before
    on the same (X, y) from the best constants found for it (WarmStartCache)
    instead of its passed initial values; last_stats["n_warm"] counts them."""

    name = "cuda_kernel_lm"

    def __init__(self, max_iter: int = 50, fallback=None, variant: str = "ad", device_id: int = 0,
                 ad_mode: int = 0, precision: int = 0, warm_start: bool = False,
                 cache_capacity: int = 200_000):
        self.max_iter = int(max_iter)
        self.fallback = fallback
        self.variant = variant
        self.device_id = int(device_id)
        self.ad_mode = int(ad_mode)
        self.precision = int(precision)
        self.warm_start = bool(warm_start)
        self.cache = WarmStartCache(cache_capacity) if warm_start else None
        self.last_stats: dict = {}
        self.cum_stats: dict = {}

    def fit_batch(self, skeletons, inits, X, y, *, max_iter=100, native=None) -> list[COResult]:
        if native is None:
            raise ValueError("KernelLM needs the prefix arrays of every candidate via native=")
        n_warm = 0
        keys = None
        if self.cache is not None:
            dkey = data_key(X, y)
            keys = [structure_key(*nat) for nat in native]
            inits = list(inits)
            for j, sk in enumerate(keys):
                hit = self.cache.get(dkey, sk)
                if hit is not None and len(hit[0]) == len(np.atleast_1d(inits[j])):
                    inits[j] = hit[0].copy()
                    n_warm += 1
        results, stats = fit_natives(skeletons, inits, native, X, y, max_iter=self.max_iter,
                                     fallback=self.fallback, variant=self.variant,
                                     device_id=self.device_id, ad_mode=self.ad_mode,
                                     precision=self.precision)
        if self.cache is not None:
            for sk, r in zip(keys, results):
                self.cache.put(dkey, sk, r.constants, r.final_loss)
        stats["n_warm"] = n_warm
        self.last_stats = stats
        for k, v in stats.items():
            self.cum_stats[k] = self.cum_stats.get(k, 0) + v
        return results
