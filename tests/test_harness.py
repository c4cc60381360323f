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
    from pathlib import Path
    from oracle.scipy_pop import ScipyPop

    serial = ScipyPop(nproc=1, timeout=300)
    try:
        cache = Path(os.environ.get("GRAFT_REPO_ROOT", ".")) / "gpurun_out" / "oracle_cache"
        orc = runner.cached_oracle(pop, lambda p: serial.fit_pop(p)["c_final"],
                                   lambda c: interp.loss_pop(pop, c), cache)
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
