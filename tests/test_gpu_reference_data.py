"""The reference's own populations and fixtures through the HIP path.

Each case restates one of the reference's own tests, run on the data the
reference holds (tests/golden/ref_fixtures, copied from cusr/kernel/tests and
data/fixtures):
  * pop1000.bin, the real EvoGP forest (M = 1,000, N = 1,000, D = 3,
    K_max = 8, max_stack 11): fp64 forward and reverse fits against the CPU
    oracle at the north star's tolerance, and the release gate of
    cusr/kernel/tests/test_parity_gate.py:39-97 against the scipy CPU path;
  * pop_fixture_op.bin (cusr/kernel/tests/test_fixture_op.py:24-57);
  * pop_fixture_scale_*.bin (cusr/kernel/tests/test_fixture_scale.py:44-75);
  * the 17 fp32-honesty fixtures
    (cusr/kernel/tests/fp32_honesty_regression/check_fp32_honesty.py:44-100).
Fits go through co_optimize, the fp32 reference ABI, where the reference test
runs its fp32 binary, and through co_optimize_ex (fp64) where the oracle is
the check. Constants are always rescored in fp64 by the numpy interpreter, as
the reference rescores every backend (cusr/kernel/verify.py:181-215).
"""
import json

import numpy as np
import pytest

from cusr_amd.benchmark import popio
from oracle import interp, lm_oracle
from tests.helpers import GOLDEN, REF_FIX, ref_pop, rel_diff, synth

pytestmark = pytest.mark.gpu

STATUS_NAMES = ("CONVERGED", "MAXITER", "FAIL_NAN", "K0_SKIP", "FAIL_CHOLESKY")


def _say(msg):
    print(msg, flush=True)


def _dist(status):
    c = np.bincount(np.asarray(status), minlength=5)
    return " ".join(f"{n}={v}" for n, v in zip(STATUS_NAMES, c))


@pytest.mark.parametrize("ad_mode", [0, 1])
def test_pop1000_fp64_matches_oracle(co, ad_mode):
    """The real forest, 50 iterations, fp64: final losses within 1e-9 and
    statuses equal on >= 99.9 % of the trees."""
    pop = ref_pop("pop1000.bin")
    _say(f"pop1000 fp64 ad_mode={ad_mode} M={pop['M']} N={pop['N']}")
    g = co.optimize_ex(pop, 50, ad_mode=ad_mode)
    o = lm_oracle.fit(pop, max_iter=50, ad_mode=ad_mode)
    d = rel_diff(g["loss_final"], o["loss_final"])
    st = float(np.mean(g["status"] == o["status"]))
    _say(f"  loss within 1e-9 {np.mean(d <= 1e-9):.4f} (exact {np.mean(d == 0):.4f}); "
         f"statuses equal {st:.4f}")
    _say(f"  GPU   {_dist(g['status'])}")
    ref = np.fromfile(REF_FIX / "golden_ad_pop1000" / "status.bin", np.int32)
    _say(f"  reference fp32 AD kernel (golden_ad_pop1000/status.bin, information only): "
         f"{_dist(ref)}")
    assert np.mean(d <= 1e-9) >= 0.999
    assert st >= 0.999


def test_pop1000_release_gate():
    """test_parity_gate.py:39-97 on the fp32 ABI: loss-down rate (K > 0) >= 93 %,
    and over the trees both converged, GPU loss <= 1.05x scipy on >= 90 % and
    <= 10x on >= 99 % (the envelope keeps verify.py's +1e-10 floor)."""
    from cusr_amd.kernel import co_inproc as ci
    co = ci.get_inproc_co(0, "fd")   # the reference gate runs its default (FD-variant) binary
    pop = ref_pop("pop1000.bin")
    sc = np.load(GOLDEN / "scipy_pop1000.npz")
    _say("pop1000 release gate through co_optimize (fp32 ABI), 50 iterations")
    g = co.optimize(pop, 50)
    K = pop["metas"][:, 3]
    gl = interp.loss_pop(pop, g["c_final"].astype(np.float64))
    gi = interp.loss_pop(pop, pop["c_init"].astype(np.float64))
    elig = (K > 0) & np.isfinite(gl) & np.isfinite(gi)
    down = float(np.mean(gl[elig] < gi[elig]))
    both = (K > 0) & (g["status"] == 0) & (sc["status"] == 0)
    fin = both & np.isfinite(gl) & np.isfinite(sc["loss"])

    def env(k):
        ok = fin & (gl <= np.maximum(k * sc["loss"], sc["loss"] + 1e-10))
        return float(ok.sum() / max(both.sum(), 1))

    e105, e10 = env(1.05), env(10.0)
    _say(f"  loss-down {100 * down:.1f}% (>= 93); both converged {both.sum()}; "
         f"within 1.05x {100 * e105:.1f}% (>= 90); within 10x {100 * e10:.1f}% (>= 99)")
    assert down >= 0.93
    assert e105 >= 0.90
    assert e10 >= 0.99


def test_fixture_op_converges_to_truth(co):
    """Eight trees covering TAN/SIN/COS/EXP/LOG/SQRT/... and several
    variables: every tree converges with ||c - c_true|| / ||c_true|| < 5e-3."""
    pop = ref_pop("pop_fixture_op.bin")
    truth = json.loads((REF_FIX / "pop_fixture_op_truth.json").read_text())["fixtures"]
    g = co.optimize(pop, 50)
    for i, fx in enumerate(truth):
        K, off = fx["K"], fx["c_offset"]
        c_true = np.asarray(fx["c_true"], np.float32)
        c = g["c_final"][off:off + K]
        rel = float(np.linalg.norm(c - c_true) / np.linalg.norm(c_true))
        _say(f"  {fx['name']:20s} K={K} status={g['status'][i]} c_rel={rel:.3e}")
        assert g["status"][i] == 0 and rel < 5e-3


def test_fixture_scale_tier1(co):
    """Magnitude sweep 1e-6 .. 1e6: every tier-1 tree converges with each
    constant within 5e-3 relative; tier 2 is reported only, as in the reference."""
    files = json.loads((REF_FIX / "pop_fixture_scale_truth.json").read_text())["files"]
    t1 = t1_ok = t2 = t2_ok = 0
    for entry in files:
        pop = popio.load_pop_bin(REF_FIX / entry["bin"])
        g = co.optimize(pop, 50)
        for i, fx in enumerate(entry["fixtures"]):
            K, off = fx["K"], fx["c_offset"]
            c_true = np.asarray(fx["c_true"], np.float64)
            c = g["c_final"][off:off + K].astype(np.float64)
            rel = float(np.max(np.abs(c - c_true) / np.maximum(np.abs(c_true), 1e-30)))
            ok = bool(g["status"][i] == 0 and rel < 5e-3)
            if fx["tier"] == 1:
                t1 += 1
                t1_ok += ok
            else:
                t2 += 1
                t2_ok += ok
    _say(f"  tier 1 {t1_ok}/{t1}; tier 2 {t2_ok}/{t2} (diagnostic)")
    assert t1 > 0 and t1_ok == t1


def test_fp32_honesty_fixtures():
    """The reference's offender trees (257 in 17 fixtures), 1,000 iterations
    like check_fp32_honesty.py: no tree reported converged is worse in exact
    fp64 than its start (the reference gate counts those > 2x worse and
    requires 0; this build has none at all), and no converged tree's fp64
    loss at c_final exceeds the manifest's loss_start_fp64."""
    from cusr_amd.kernel import co_inproc as ci
    man = json.loads((REF_FIX / "honesty" / "manifest.json").read_text())
    total = worse = serious = 0
    for variant in ("fd", "ad"):
        co = ci.get_inproc_co(0, variant)
        for fx in man["fixtures"].values():
            pop = popio.load_pop_bin(REF_FIX / "honesty" / fx["file"])
            g = co.optimize(pop, 1000)
            s0 = interp.loss_pop(pop, pop["c_init"].astype(np.float64))
            sf = interp.loss_pop(pop, g["c_final"].astype(np.float64))
            for tr in fx["trees"]:
                m = tr["fixture_index"]
                total += 1
                if g["status"][m] != 0:
                    continue
                bad = not np.isfinite(sf[m]) or sf[m] > s0[m] * (1 + 1e-6) + 1e-9
                worse += bad
                ratio = np.inf if not np.isfinite(sf[m]) else sf[m] / s0[m]
                serious += bool(bad and ratio > 2.0)
                assert sf[m] <= tr["loss_start_fp64"] * (1 + 1e-6) + 1e-9, (fx["file"], m)
    _say(f"  honesty: {total} tree fits; converged-but-worse {worse}; serious {serious}")
    assert total == 2 * man["total_trees"]
    assert serious == 0 and worse == 0


def test_full_c1_matches_oracle(co):
    """C1 at its full size: 1,024 expressions, N = 256, 20 iterations, fp64
    forward AD."""
    pop, _ = synth("C1", 1024, 256)
    _say(f"C1 full size M={pop['M']} N={pop['N']}")
    g = co.optimize_ex(pop, 20)
    o = lm_oracle.fit(pop, max_iter=20)
    d = rel_diff(g["loss_final"], o["loss_final"])
    st = float(np.mean(g["status"] == o["status"]))
    _say(f"  loss within 1e-9 {np.mean(d <= 1e-9):.4f}; statuses equal {st:.4f}")
    assert np.mean(d <= 1e-9) >= 0.999
    assert st >= 0.999
