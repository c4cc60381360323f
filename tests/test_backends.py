"""Benchmark and demonstrator backends (reference contracts:
cusr/benchmark/backends.py:80-89,740-785; cusr/demonstrator/co_backend.py:25-47;
cusr/demonstrator/kernel_bridge.py:140-238)."""
import numpy as np
import pytest

from cusr_amd.benchmark import backends, popio
from cusr_amd.demonstrator import co_backend
from oracle import interp, lm_oracle
from tests.helpers import synth


def _candidates(n, seed=3):
    """Prefix arrays of simple candidates over X with 2 variables."""
    rng = np.random.default_rng(seed)
    forms = [([3, 3, 1, 0, 1], [1, 3, 0, 0, 0], [-1, -1, 0, -1, 1]),          # c0*x0 + c1
             ([2, 3, 1, 0], [14, 3, 0, 1], [-1, -1, 0, -1]),                   # sin(c0*x1)
             ([3, 3, 1, 2, 0, 1], [1, 3, 0, 34, 1, 0], [-1, -1, 0, -1, -1, 1])]  # c0*sq(x1)+c1
    nat, inits = [], []
    for j in range(n):
        nt, nv, ci = forms[j % len(forms)]
        K = int(np.sum(np.asarray(nt) == 1))
        nat.append((np.asarray(nt, np.int32), np.asarray(nv, np.float32), np.asarray(ci, np.int32)))
        inits.append(rng.normal(size=K))
    return nat, inits


def test_ineligible_without_fallback_raises():
    nat, inits = _candidates(3)
    nt = np.asarray([3] * 32 + [1] * 33, np.int32)                  # 33 constants > 32
    nat.append((nt, np.asarray([1.0] * 32 + [0.0] * 33, np.float32),
                np.asarray([-1] * 32 + list(range(33)), np.int32)))
    inits.append(np.zeros(33))
    X = np.zeros((8, 2))
    with pytest.raises(ValueError):
        co_backend.fit_natives(None, inits, nat, X, np.zeros(8))


def test_status_map_matches_reference():
    assert backends.STATUS_MAP == {0: 0, 1: 1, 2: 2, 3: 3, 4: 2}


@pytest.mark.gpu
def test_kernel_pop_and_cli_pop():
    pop, _ = synth("C1", 96, 128)
    a = backends.KernelPop(max_iter=20).fit_pop(pop)
    b = backends.CudaKernelPop(max_iter=20).fit_pop(pop)
    o = lm_oracle.fit(pop, max_iter=20)
    assert a.c_final.dtype == np.float64 and a.status.dtype == np.int32
    assert np.array_equal(a.c_final, o["c_final"])
    assert np.array_equal(a.n_iter, o["iters"])
    assert np.array_equal(a.status, backends._map_status(o["status"]))
    # the CLI writes float32 blobs of a fit with constants held in fp32
    from cusr_amd.kernel import co_inproc
    n = co_inproc.narrow_fp32(pop, lm_oracle.fit(pop, max_iter=20, f32_range=1))
    assert np.array_equal(b.status, backends._map_status(n["status"]))
    assert np.array_equal(b.c_final, n["c_final"].astype(np.float64))
    assert np.isfinite(b.wall_core) and b.wall_core >= 0 and np.all(b.n_iter == -1)


@pytest.mark.gpu
def test_kernel_lm_fit_batch_aligned_with_fallback():
    nat, inits = _candidates(12)
    rng = np.random.default_rng(9)
    X = rng.uniform(-2, 2, size=(300, 2))
    y = 1.5 * X[:, 0] - 0.25 + 0.01 * rng.normal(size=300)
    big = np.asarray([3] * 32 + [1] * 33, np.int32)                 # 33 constants > 32
    nat.insert(5, (big, np.asarray([1.0] * 32 + [0.0] * 33, np.float32),
                   np.asarray([-1] * 32 + list(range(33)), np.int32)))
    inits.insert(5, np.zeros(33))

    class Stub:
        def fit_batch(self, skeletons, inits, X, y, *, max_iter=100, native=None):
            return [co_backend.COResult(np.asarray(c), -7, False, float("nan")) for c in inits]

    lm = co_backend.KernelLM(max_iter=30, fallback=Stub())
    res = lm.fit_batch(None, inits, X, y, native=nat)
    assert len(res) == 13 and res[5].n_iter == -7
    assert lm.last_stats == dict(n_total=13, n_kernel=12, n_fallback=1, n_overflow=1,
                                 n_kmismatch=0, n_warm=0)
    for j, r in enumerate(res):
        if j == 5:
            continue
        nt, nv, ci = nat[j]
        pred = interp.eval_tree_arrays(nt, nv, ci, X, r.constants)
        assert r.final_loss == pytest.approx(np.mean((pred - y) ** 2), rel=1e-9)
    # c0*x0 + c1 recovers the line
    assert np.allclose(res[0].constants, [1.5, -0.25], atol=5e-3) and res[0].converged


@pytest.mark.gpu
def test_fit_natives_reuses_resident_data():
    """Two calls with the same (X, y) fit against the data set uploaded by the
    first; a changed y is uploaded again. Results equal a plain fp64 fit of
    the same candidates with y tiled per expression."""
    from cusr_amd.kernel import co_inproc

    rng = np.random.default_rng(4)
    X = rng.uniform(-2, 2, size=(257, 2))
    y = np.sin(0.7 * X[:, 1]) + 0.5 * X[:, 0] + 0.01 * rng.normal(size=257)
    co = co_inproc.get_inproc_co(0, "ad")
    for n, seed, yy in ((9, 1, y), (14, 2, y), (9, 1, 2.0 * y)):
        nat, inits = _candidates(n, seed)
        res, stats = co_backend.fit_natives(None, inits, nat, X, yy, max_iter=25)
        assert stats["n_kernel"] == n and co.data_matches(X, yy)
        trees = [(nt, nv, ci, np.asarray(c0, np.float32)) for (nt, nv, ci), c0 in zip(nat, inits)]
        pop = popio.build_pop(trees, X, np.tile(yy, (n, 1)))
        ref = co.optimize_ex(pop, 25, c_init=np.concatenate(inits), xs=X, ym=np.tile(yy, (n, 1)))
        got = np.concatenate([r.constants for r in res])
        assert np.array_equal(got, ref["c_final"])
        assert [r.n_iter for r in res] == ref["iters"].tolist()


def test_warm_start_cache_keys_and_policy():
    nat, _ = _candidates(3)
    k0 = co_backend.structure_key(*nat[0])
    assert k0 == co_backend.structure_key(*(np.array(a) for a in nat[0]))
    assert k0 != co_backend.structure_key(*nat[1])
    nt, nv, ci = nat[0]
    assert k0 != co_backend.structure_key(nt, nv + np.float32(1), ci)   # another operator
    X = np.arange(12.0).reshape(6, 2)
    d = co_backend.data_key(X, np.ones(6))
    assert d == co_backend.data_key(X.copy(), np.ones(6)) != co_backend.data_key(X, np.zeros(6))
    cache = co_backend.WarmStartCache(capacity=2)
    cache.put(d, k0, [1.0, 2.0], 0.5)
    cache.put(d, k0, [9.0, 9.0], 0.7)            # worse: kept the better one
    assert cache.get(d, k0)[0].tolist() == [1.0, 2.0]
    cache.put(d, k0, [3.0, 4.0], 0.1)            # better: replaced
    assert cache.get(d, k0)[0].tolist() == [3.0, 4.0]
    cache.put(d, k0, [5.0, 6.0], float("inf"))   # non-finite: ignored
    assert cache.get(d, k0)[1] == 0.1
    k1, k2 = co_backend.structure_key(*nat[1]), co_backend.structure_key(*nat[2])
    cache.put(d, k1, [1.0], 1.0)
    cache.get(d, k0)                             # k0 most recently used
    cache.put(d, k2, [1.0, 1.0], 1.0)            # evicts k1
    assert len(cache) == 2 and cache.get(d, k1) is None and cache.get(d, k0) is not None
    assert cache.get(co_backend.data_key(X, np.zeros(6)), k0) is None   # other data set


@pytest.mark.gpu
def test_kernel_lm_warm_start_reuses_fitted_constants():
    """A second generation of the same structures starts from the constants
    the first fitted: every candidate is warm, none gets worse, and the LM
    loops are much shorter."""
    rng = np.random.default_rng(7)
    X = rng.uniform(-2, 2, size=(400, 2))
    y = np.sin(0.7 * X[:, 1]) * 1.3 + 0.5 * X[:, 0] - 0.2 + 0.01 * rng.normal(size=400)
    nat, inits = _candidates(30, seed=5)
    lm = co_backend.KernelLM(max_iter=50, warm_start=True)
    first = lm.fit_batch(None, inits, X, y, native=nat)
    assert lm.last_stats["n_warm"] == 0
    fresh = [rng.normal(size=len(c)) for c in inits]       # the next generation's inherited values
    second = lm.fit_batch(None, fresh, X, y, native=nat)
    assert lm.last_stats["n_warm"] == 30
    it1 = np.mean([r.n_iter for r in first])
    it2 = np.mean([r.n_iter for r in second])
    print(f"warm start: mean iterations {it1:.1f} -> {it2:.1f}", flush=True)
    assert it2 < 0.5 * it1
    for a, b in zip(first, second):
        assert b.final_loss <= a.final_loss * (1 + 1e-12) + 1e-300
    # the cold path ignores the cache
    cold = co_backend.KernelLM(max_iter=50).fit_batch(None, fresh, X, y, native=nat)
    assert np.mean([r.n_iter for r in cold]) > it2


class _Skel:
    """A skeleton with the reference's protocol (n_constants, residual,
    jacobian) over prefix arrays, scored by the numpy interpreter."""

    def __init__(self, nt, nv, ci):
        self.nt, self.nv, self.ci = nt, nv, ci
        self.n_constants = int(np.sum(np.asarray(nt) == 1))

    def residual(self, c, X, y):
        return interp.eval_tree_arrays(self.nt, self.nv, self.ci, X, np.asarray(c)) - y


def test_scipy_lm_fits_through_the_skeleton():
    nat, inits = _candidates(3, seed=2)
    rng = np.random.default_rng(5)
    X = rng.uniform(-2, 2, size=(200, 2))
    y = 1.5 * X[:, 0] - 0.25
    skels = [_Skel(*n) for n in nat]
    res = co_backend.ScipyLM().fit_batch(skels, inits, X, y, max_iter=200)
    assert np.allclose(res[0].constants, [1.5, -0.25], atol=1e-8) and res[0].converged
    for r, s in zip(res, skels):
        assert r.final_loss == pytest.approx(np.mean(s.residual(r.constants, X, y) ** 2))
    with pytest.raises(ValueError):
        co_backend.ScipyLM().fit_batch(None, inits, X, y)


def test_cuda_kernel_lm_constructor_and_cpu_routing():
    """The reference constructor (co_backend.py:250-263) and its defaults; a
    batch of candidates beyond the device bounds goes to the default ScipyLM
    without touching the device."""
    lm = co_backend.CudaKernelLM()
    assert (lm.binary, lm.max_iter, lm.fallback, lm.inproc, lm.device_id) == \
        (None, 50, None, False, 0)
    assert co_backend.variant_for_binary(co_backend.DEFAULT_BINARY) == "fd"
    assert co_backend.variant_for_binary("/x/batch_lm_ad") == "ad"
    nt = np.asarray([3] * 32 + [1] * 33, np.int32)            # 33 constants
    big = (nt, np.asarray([1.0] * 32 + [0.0] * 33, np.float32),
           np.asarray([-1] * 32 + list(range(33)), np.int32))
    X = np.random.default_rng(1).uniform(-1, 1, size=(50, 2))
    y = np.full(50, 3.0)
    res = lm.fit_batch([_Skel(*big)], [np.zeros(33)], X, y, native=[big], max_iter=50)
    assert lm.last_stats == dict(n_total=1, n_kernel=0, n_fallback=1, n_overflow=1,
                                 n_kmismatch=0)
    # y = 3 = c0 * c1 * ... : the fit reaches the target
    assert res[0].final_loss < 1e-12
    with pytest.raises(ValueError):
        lm.fit_batch(None, [], X, y)
