"""The fp32 carrier of the reference ABI (co_optimize, the CLI's float32 blobs)
on fp64 fits, host only (co_narrow_fp32; no device needed).

The reference fits in fp32 (cusr/kernel/co_lib.h:55-61), so any constant it
commits is representable in fp32; a loss that turns non-finite rejects the
step. An fp64 fit can keep a finite constant beyond FLT_MAX while its loss
stays finite. The carrier then treats the expression as the fp64 guard treats
a non-finite loss (cusr/kernel/lm_core.cuh:299-351): c_init back, the initial
loss reported, CONVERGED demoted to MAXITER.
"""
import numpy as np

from cusr_amd.kernel import co_inproc as ci
from oracle import lm_oracle
from tests.helpers import synth


def _expected(pop, fit):
    """The carrier rule restated on the fp64 results."""
    with np.errstate(over="ignore"):
        c32 = fit["c_final"].astype(np.float32)
    st = fit["status"].copy()
    lf32 = fit["loss_final"].astype(np.float32)
    demoted = []
    with np.errstate(over="ignore"):
        for m, (_, _, off, K) in enumerate(pop["metas"]):
            if K == 0:
                continue
            c = fit["c_final"][off:off + K]
            lost = np.any(np.isfinite(c) & ~np.isfinite(c.astype(np.float32)))
            lf = fit["loss_final"][m]
            lost |= bool(np.isfinite(lf) and not np.isfinite(np.float32(lf)))
            if lost:
                demoted.append(m)
                c32[off:off + K] = pop["c_init"][off:off + K]
                lf32[m] = np.float32(fit["loss_init"][m])
                if st[m] == ci.STATUS_CONVERGED:
                    st[m] = ci.STATUS_MAXITER
    return c32, st, lf32, demoted


def test_fp32_carrier_hands_back_no_overflowed_constant():
    pop, _ = synth("C1", 128, 256)
    fit = lm_oracle.fit(pop, max_iter=20)
    with np.errstate(over="ignore"):
        big = [m for m, (_, _, off, K) in enumerate(pop["metas"])
               if K and np.any(~np.isfinite(fit["c_final"][off:off + K].astype(np.float32)))]
    # fits whose fp64 constants run past FLT_MAX with a finite loss
    assert len(big) >= 2 and all(np.isfinite(fit["loss_final"][m]) for m in big)
    r = ci.narrow_fp32(pop, fit)
    c32, st, lf32, demoted = _expected(pop, fit)
    assert r["demoted"] == len(demoted) and set(big) <= set(demoted)
    fin = np.isfinite(fit["c_final"])
    assert np.all(np.isfinite(r["c_final"][fin]))
    assert np.array_equal(r["c_final"], c32)
    assert np.array_equal(r["status"], st)
    assert np.array_equal(r["loss_final"], lf32, equal_nan=True)
    assert np.array_equal(r["loss_init"], fit["loss_init"].astype(np.float32), equal_nan=True)
    for m in demoted:
        assert r["status"][m] != ci.STATUS_CONVERGED
        assert r["loss_final"][m] == r["loss_init"][m]


def test_fp32_carrier_is_a_plain_cast_otherwise():
    pop, _ = synth("C2", 64, 256)
    fit = lm_oracle.fit(pop, max_iter=10)
    r = ci.narrow_fp32(pop, fit)
    if r["demoted"] == 0:
        assert np.array_equal(r["c_final"], fit["c_final"].astype(np.float32))
        assert np.array_equal(r["status"], fit["status"])
    c32, st, _, demoted = _expected(pop, fit)
    assert r["demoted"] == len(demoted)
    assert np.array_equal(r["c_final"], c32) and np.array_equal(r["status"], st)


def test_fits_held_in_fp32_need_no_narrowing():
    """With f32_range (co_optimize, the CLI on float32 files) trial constants
    are rounded to fp32 and one beyond its range ends the fit (FAIL_NAN, the
    last accepted constants kept, batch_lm_ad.cu:437-443): every delivered
    constant is finite and exactly representable, so the carrier is a plain
    cast; the fits that ran off to +-1e80 in fp64 stop short of it."""
    pop, _ = synth("C1", 128, 256)
    fit = lm_oracle.fit(pop, max_iter=20, f32_range=1)
    c = fit["c_final"]
    assert np.all(np.isfinite(c)) and np.array_equal(c, c.astype(np.float32).astype(np.float64))
    r = ci.narrow_fp32(pop, fit)
    assert r["demoted"] == 0 and np.array_equal(r["c_final"], c.astype(np.float32))
    free = lm_oracle.fit(pop, max_iter=20)
    with np.errstate(over="ignore"):
        ran_off = [m for m, (_, _, off, K) in enumerate(pop["metas"])
                   if K and np.any(~np.isfinite(free["c_final"][off:off + K].astype(np.float32)))]
    assert ran_off
    for m in ran_off:
        assert fit["status"][m] != ci.STATUS_CONVERGED
        assert fit["loss_final"][m] <= fit["loss_init"][m]
