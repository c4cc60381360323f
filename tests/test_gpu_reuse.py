"""Parity under reuse through the library, with the reference's design
(cusr/kernel/tests/test_inproc_reuse.py): one persistent handle per variant
runs a sequence of populations whose M, K_max and sizes grow and shrink, and
every co_optimize call must equal, byte for byte, the CLI's fit of the same
population in a fresh process (batch_lm_ad for the AD variant, batch_lm for
the FD one: the same library code behind the reference's standalone binary).
A persistent context that kept a larger earlier population's constants,
statuses or partial sums would hand finite wrong values to a later call;
only a comparison against a fresh process catches that.

Populations: the reference's pop1000 forest (K <= 8), slices and tilings of
it, a seeded high-K population (K 17..32, the general kernel; its fits end in
FAIL_CHOLESKY often, the reference's operon snapshot's role, which is not in
the reference tree), the reference's scale fixtures (magnitude span) and a
four-expression population that reaches CONVERGED, MAXITER, FAIL_NAN and
K0_SKIP (test_inproc_reuse.py:400-466).
"""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from cusr_amd.benchmark import popio
from cusr_amd.kernel import co_inproc as ci
from tests.general_pops import general_pop
from tests.helpers import REF_FIX, ref_pop

pytestmark = pytest.mark.gpu

MAX_ITER = 50
KDIR = Path(ci.__file__).resolve().parent
CLI = {"ad": KDIR / "batch_lm_ad", "fd": KDIR / "batch_lm"}
BLOBS = (("c_final", np.float32), ("status", np.int32), ("loss_init", np.float32),
         ("loss_final", np.float32))
SCALE_BINS = sorted(REF_FIX.glob("pop_fixture_scale_*.bin"))


def _say(msg):
    print(f"[reuse] {msg}", file=sys.stderr, flush=True)


def _cli(variant, pop, td, tag):
    """The CLI's blobs for pop, in a fresh process."""
    d = Path(td) / f"{variant}_{tag}"
    d.mkdir()
    popio.save_pop_bin(pop, d / "pop.bin")
    r = subprocess.run([str(CLI[variant]), str(d / "pop.bin"), str(d), "--quiet",
                        "--max-iter", str(MAX_ITER)], capture_output=True, text=True,
                       timeout=600)
    assert r.returncode == 0, r.stderr[-500:]
    return {k: np.fromfile(d / f"{k}.bin", dtype=dt) for k, dt in BLOBS}


def _same(got, ref, what):
    for k, dt in BLOBS:
        a = np.asarray(got[k], dt)
        assert a.shape == ref[k].shape and a.tobytes() == ref[k].tobytes(), \
            f"{what}: {k} differs from the fresh-process CLI"


def _tile(pop, reps):
    return popio.select_pop(pop, np.tile(np.arange(pop["M"]), reps))


def _run_sequence(variant, seq, tmp_path):
    refs = {}
    for tag, pop in seq:
        key = tag.rstrip("0123456789")
        if key not in refs:
            _say(f"{variant} CLI {tag}: M={pop['M']} K_max={pop['K_max']}")
            refs[key] = _cli(variant, pop, tmp_path, key)
    co = ci.InProcessCO(device_id=0, variant=variant)
    try:
        for tag, pop in seq:
            _say(f"{variant} in-process {tag}: M={pop['M']} K_max={pop['K_max']}")
            _same(co.optimize(pop, MAX_ITER), refs[tag.rstrip("0123456789")],
                  f"{variant}/{tag}")
    finally:
        co.teardown()


@pytest.fixture(scope="module")
def pops():
    base = ref_pop("pop1000.bin")
    highk, _ = general_pop("highk", 300, 256)
    return {"base": base, "small": popio.slice_pop(base, 50), "highk": highk}


@pytest.mark.parametrize("variant", ["ad", "fd"])
def test_parity_under_reuse(variant, pops, tmp_path):
    """A -> larger B -> smaller C -> A again (test_inproc_reuse.py:200-246)."""
    seq = [("base", pops["base"]), ("big", _tile(pops["base"], 3)),
           ("small", pops["small"]), ("base2", pops["base"])]
    _run_sequence(variant, seq, tmp_path)


@pytest.mark.parametrize("variant", ["ad", "fd"])
def test_parity_under_reuse_mixed_k(variant, pops, tmp_path):
    """K_max mixing within one context: K 8 -> K up to 32 -> K 8 (M = 50) ->
    K up to 32 again (test_inproc_reuse.py:249-300)."""
    seq = [("base", pops["base"]), ("highk", pops["highk"]), ("small", pops["small"]),
           ("highk2", pops["highk"])]
    kmax = [int(p["K_max"]) for _, p in seq]
    assert max(kmax) >= 28 and min(kmax) <= 8, kmax
    _run_sequence(variant, seq, tmp_path)


@pytest.mark.parametrize("variant", ["ad", "fd"])
def test_parity_under_reuse_shrink_m_grow_k(variant, pops, tmp_path):
    """A larger-M, low-K population first, then a smaller-M, high-K one: a
    buffer sized by M alone would be too small for the second
    (test_inproc_reuse.py:303-367)."""
    seq = [("bigm", _tile(pops["base"], 8)), ("highk", pops["highk"])]
    assert seq[0][1]["M"] > seq[1][1]["M"] and seq[0][1]["K_max"] < seq[1][1]["K_max"]
    _run_sequence(variant, seq, tmp_path)


def test_parity_under_reuse_large_then_shrink(pops, tmp_path):
    """66,000 -> 1,000 -> 66,000 -> 1,000 (test_inproc_reuse.py:370-397): the
    shrink must not read past the current M."""
    big = _tile(pops["base"], 66)
    assert big["M"] >= 65536
    seq = [("big", big), ("base", pops["base"]), ("big2", big), ("base2", pops["base"])]
    _run_sequence("fd", seq, tmp_path)


def _status_branch_pop():
    """CONVERGED, K0_SKIP, FAIL_NAN and MAXITER from four expressions over
    one variable (the reference's construction, test_inproc_reuse.py:403-451)."""
    xs = np.linspace(0.5, 3.0, 64).astype(np.float32).reshape(-1, 1)
    x = xs[:, 0].astype(np.float64)
    V, C, U, B = popio.NODE_VAR, popio.NODE_CONST, popio.NODE_UFUNC, popio.NODE_BFUNC
    ADD, MUL, SIN, EXP = 1, 3, 14, 22
    trees = [([B, C, B, C, V], [ADD, 0, MUL, 0, 0], [-1, 0, -1, 1, -1], [1.9, -0.45]),
             ([V], [0], [-1], []),
             ([U, B, C, V], [EXP, MUL, 0, 0], [-1, -1, 0, -1], [90.0]),
             ([B, U, B, C, V, C], [MUL, SIN, MUL, 0, 0, 0], [-1, -1, -1, 0, -1, 1], [0.3, 0.2])]
    ys = [2.0 - 0.5 * x, x.copy(), np.exp(0.3 * x), np.sin(4.7 * x) * 2.3]
    trees = [(np.asarray(nt), np.asarray(nv, np.float32), np.asarray(c_i),
              np.asarray(c0, np.float32)) for nt, nv, c_i, c0 in trees]
    return popio.build_pop(trees, xs, np.stack(ys).astype(np.float32))


@pytest.mark.parametrize("variant", ["ad", "fd"])
def test_status_branch_coverage(variant, tmp_path):
    pop = _status_branch_pop()
    ref = _cli(variant, pop, tmp_path, "branch")
    got = set(int(s) for s in ref["status"])
    _say(f"{variant} status branches {sorted(got)}")
    for code in (ci.STATUS_CONVERGED, ci.STATUS_MAXITER, ci.STATUS_FAIL_NAN, ci.STATUS_K0_SKIP):
        assert code in got, f"the fixture no longer reaches status {code}: {sorted(got)}"
    co = ci.InProcessCO(device_id=0, variant=variant)
    try:
        _same(co.optimize(pop, MAX_ITER), ref, f"{variant}/status-branch")
    finally:
        co.teardown()


@pytest.mark.parametrize("variant", ["ad", "fd"])
def test_fail_cholesky_high_k(variant, pops, tmp_path):
    """High K drives the Cholesky breakdown branch (test_inproc_reuse.py:505-532)."""
    ref = _cli(variant, pops["highk"], tmp_path, "highk")
    n4 = int(np.sum(ref["status"] == ci.STATUS_FAIL_CHOLESKY))
    _say(f"{variant} high-K FAIL_CHOLESKY: {n4} of {pops['highk']['M']}")
    assert n4 > 0
    co = ci.InProcessCO(device_id=0, variant=variant)
    try:
        _same(co.optimize(pops["highk"], MAX_ITER), ref, f"{variant}/high-K")
    finally:
        co.teardown()


@pytest.mark.parametrize("variant", ["ad", "fd"])
@pytest.mark.parametrize("path", SCALE_BINS, ids=[p.stem for p in SCALE_BINS])
def test_magnitude_span(variant, path, tmp_path):
    """The reference's scale fixtures (constants from 1e-6 to 1e6) through
    both routes (test_inproc_reuse.py:535-556)."""
    pop = popio.load_pop_bin(path)
    ref = _cli(variant, pop, tmp_path, path.stem)
    co = ci.InProcessCO(device_id=0, variant=variant)
    try:
        _same(co.optimize(pop, MAX_ITER), ref, f"{variant}/{path.stem}")
    finally:
        co.teardown()
