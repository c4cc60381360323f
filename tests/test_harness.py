"""Quality harness (cusr_amd/benchmark/runner.py) with the reference's protocol
(cusr/benchmark/runner.py:55-376): tier thresholds, selection fidelity, and an
end-to-end run with the serial scipy oracle and the numpy scorer."""
import numpy as np
import pytest

from cusr_amd.benchmark import backends, runner
from oracle import interp
from tests.helpers import synth


def test_tier_thresholds():
    star = np.array([1.0, 1.0, 1.0, 0.0, np.inf, 1.0])
    got = np.array([1.004, 1.04, 1.2, 5e-11, 1.0, 1.0])
    K = np.array([1, 1, 1, 1, 1, 0])
    a, b, e = runner.classify_tiers(got, star, K)
    assert e.tolist() == [True, True, True, True, False, False]
    assert a.tolist() == [True, False, False, True, False, False]
    assert b.tolist() == [True, True, False, True, False, False]
    assert runner.tier_rate(a, e) == 0.5


def test_selection_fidelity():
    rng = np.random.default_rng(1)
    star = rng.uniform(1, 2, 200)
    e = np.ones(200, bool)
    same = runner.selection_fidelity(star * 3.0, star, e)
    assert same["spearman"] == pytest.approx(1.0) and same["top10"] == 1.0
    rev = runner.selection_fidelity(-star, star, e)
    assert rev["spearman"] == pytest.approx(-1.0) and rev["top50"] == 0.0


class _Scipy:
    """The reference CPU path as a FitResult backend (test adapter)."""

    def __init__(self, nproc):
        from oracle.scipy_pop import ScipyPop
        self.sp = ScipyPop(nproc=nproc, timeout=120)

    def fit_pop(self, pop):
        import time
        t0 = time.perf_counter()
        r = self.sp.fit_pop(pop)
        return backends.FitResult("scipy", r["c_final"], r["status"], r["n_iter"],
                                  time.perf_counter() - t0, float("nan"),
                                  meta=dict(dtype="float64"))


@pytest.mark.gpu
def test_quality_run_end_to_end(tmp_path):
    pop, c_true = synth("C1", 96, 128)
    oracle, par = _Scipy(1), _Scipy(4)
    try:
        star = interp.loss_pop(pop, oracle.fit_pop(pop).c_final)
        res = runner.run_quality(
            pop, {"mi355x": backends.KernelPop(max_iter=50), "scipy": par}, star,
            lambda c: interp.loss_pop(pop, c), repeats=1, c_true=c_true, label="C1-96")
    finally:
        oracle.sp.close()
        par.sp.close()
    js, md = runner.write_outputs(res, tmp_path, "c1")
    assert js.exists() and "tier-A" in md.read_text()
    g = res["backends"]["mi355x"]
    print(runner.report_markdown(res), flush=True)
    assert g["tier_b_rate"] >= 0.9 and g["selection_fidelity"]["spearman"] > 0.9
    assert res["noise_floor"]["n"] > 0


def _harness_run(pop, label, c_true=None, nproc=16, repeats=3):
    """run_quality with the GPU (fp64 in process, the CLI) and the scipy port,
    against the serial scipy oracle cached by population hash."""
    import os
    from oracle.scipy_pop import ScipyPop

    serial = ScipyPop(nproc=1, timeout=300)
    try:
        orc = runner.cached_oracle(pop, lambda p: serial.fit_pop(p)["c_final"],
                                   lambda c: interp.loss_pop(pop, c))
    finally:
        serial.close()
    par = _Scipy(min(nproc, len(os.sched_getaffinity(0))))
    try:
        res = runner.run_quality(
            pop, {"mi355x:fp64": backends.KernelPop(max_iter=50),
                  "mi355x:cli-fp32": backends.CudaKernelPop(max_iter=50), "scipy": par},
            orc["loss_star"], lambda c: interp.loss_pop(pop, c), repeats=repeats,
            c_true=c_true, label=label)
    finally:
        par.sp.close()
    print(f"\n[harness] oracle wall {orc['wall']:.1f} s (cached: {orc['cached']})\n"
          + runner.report_markdown(res), flush=True)
    return res


@pytest.mark.gpu
def test_quality_pop1000_reference_forest():
    """The harness on the reference's real 1,000-tree forest (N = 1,000)."""
    from tests.helpers import ref_pop
    res = _harness_run(ref_pop("pop1000.bin"), "pop1000")
    g = res["backends"]["mi355x:fp64"]
    assert g["selection_fidelity"]["spearman"] > 0.9
    assert g["tier_b_rate"] >= 0.8


@pytest.mark.gpu
def test_quality_c2_sample_with_noise_floor():
    """The harness on 2,048 expressions of the C2 configuration, with the noise
    floor of the true constants."""
    pop, c_true = synth("C2", 2048)
    res = _harness_run(pop, "C2-2048", c_true=c_true)
    g = res["backends"]["mi355x:fp64"]
    assert g["selection_fidelity"]["spearman"] > 0.8
    assert res["noise_floor"]["n"] > 0


def test_cached_oracle_hits_by_population_hash(tmp_path):
    """The serial oracle is cached by (population sha1, limit): a second call
    on the same population reads the cache, any changed input misses it
    (cusr/benchmark/runner.py:111-128)."""
    pop, _ = synth("C1", 8, 32)
    calls = []

    def fit(p):
        calls.append(p["M"])
        return np.asarray(p["c_init"], np.float64) * 2.0

    def score(c):
        return np.asarray(c, np.float64) + 1.0

    a = runner.cached_oracle(pop, fit, score, tmp_path)
    b = runner.cached_oracle(pop, fit, score, tmp_path)
    assert calls == [8] and not a["cached"] and b["cached"]
    assert np.array_equal(a["c_star"], b["c_star"]) and np.array_equal(a["loss_star"], b["loss_star"])
    other = dict(pop)
    other["c_init"] = np.asarray(pop["c_init"]) + np.float32(1)
    assert runner.pop_sha(other) != runner.pop_sha(pop)
    runner.cached_oracle(other, fit, score, tmp_path)
    assert calls == [8, 8]
    c = runner.cached_oracle(pop, fit, score, tmp_path, limit=4)
    assert not c["cached"] and calls == [8, 8, 4] and len(c["c_star"]) == int(
        np.sum(pop["metas"][:4, 3]))


def test_bench_host_description_and_launch_bins():
    """bench.py's CPU-baseline host record and the launch bin of every
    expression (the fast kernel of its K, or the general kernel)."""
    import bench
    from cusr_amd.kernel import co_inproc as ci
    from tests.general_pops import general_pop
    cores, host = bench.cpu_cores()
    assert 1 <= cores <= host["affinity_cores"] and host["numpy"] and host["scipy"]
    pop, _ = general_pop("mixed", 24, 64)
    b = bench.launch_bins(pop)
    K = pop["metas"][:, 3]
    gen = b == ci.CO_GENERAL_BIN
    assert gen.any() and (~gen).any()
    assert np.array_equal(b[~gen], K[~gen]) and np.all(K[gen] > ci.CO_FAST_MAX_K)


def test_bench_roofline_bin_choice():
    """The roofline's bin: the longest beside the others by default, the one
    --roofline-bin names when an expression is in it, and a clear exit otherwise."""
    import argparse
    import bench
    bins = np.array([0.0, 1.0, 3.0, 2.0])
    bin_of = np.array([1, 2, 2, 3])
    free = argparse.Namespace(roofline_bin=None)
    assert bench.dominant_bin(free, bins, bin_of) == 2
    assert bench.dominant_bin(argparse.Namespace(roofline_bin=3), bins, bin_of) == 3
    for k in (0, 4, -1):
        with pytest.raises(SystemExit, match="roofline-bin"):
            bench.dominant_bin(argparse.Namespace(roofline_bin=k), bins, bin_of)
