"""The general kernel on the GPU against the CPU oracle: expressions outside
co_fast_path (K 17..32, value stacks 17..64, more than 255 nodes, more than
8 variables) -- what the reference's bridge sends within its bounds
(cusr/demonstrator/kernel_bridge.py:45-46,66-71; cusr/kernel/ad_interp.cuh:34-39)
-- fitted forward and reverse, fp64 and mixed, alone and mixed with fast-kernel
expressions in one call, through the C ABI.
"""
import numpy as np
import pytest

from cusr_amd.kernel import co_inproc as ci
from oracle import lm_oracle
from tests.general_pops import general_pop
from tests.helpers import assert_parity, f64, rel_diff

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _both(co, pop, max_iter, **kw):
    _say(f"case M={pop['M']} N={pop['N']} K_max={pop['K_max']} stack={pop['max_stack']} "
         f"D={pop['n_vars']} max_iter={max_iter} {kw}")
    g = co.optimize_ex(pop, max_iter, **kw)
    o = lm_oracle.fit(pop, max_iter=max_iter, **kw)
    d = rel_diff(g["loss_final"], o["loss_final"])
    st = float(np.mean(g["status"] == o["status"]))
    _say(f"  statuses equal {st:.4f}; loss exact {np.mean(d == 0):.4f}; within 1e-9 "
         f"{np.mean(d <= 1e-9):.4f}; max rel {d.max():.3e}; iters {np.bincount(g['iters'])[:6]}")
    return g, o, d, st


@pytest.mark.parametrize("kind,ad_mode", [("highk", 0), ("highk", 1), ("deep", 0), ("deep", 1),
                                          ("long", 0), ("long", 1), ("wide", 0)])
def test_general_fp64_bit_exact(co, kind, ad_mode):
    """fp64, the north star's bar: every final loss and status equal to the
    oracle's (the arithmetic order is the oracle's, so the bits agree)."""
    pop, _ = general_pop(kind, 48, 700)
    rc, *_, route = ci.decode(pop, full=True)
    assert rc == 0 and route.all()
    g, o, d, st = _both(co, pop, 15, ad_mode=ad_mode)
    assert_parity(g, o, 1e-9, f"general {kind} ad={ad_mode}", exact=True)
    assert np.array_equal(g["iters"], o["iters"])


def test_general_mixed_with_fast_and_partitions(co):
    """Fast and general expressions in one population (their launches run
    concurrently), with 1, 2 and 4 point partitions."""
    pop, _ = general_pop("mixed", 96, 1100)
    for parts in (1, 2, 4):
        g, o, d, st = _both(co, pop, 12, partitions=parts)
        assert_parity(g, o, 1e-9, f"general mixed parts={parts}", exact=True)


def test_general_mixed_precision(co):
    """fp32 interpreter and Jacobian, fp64 sums and solve: 1e-4 on the final loss."""
    pop, _ = general_pop("highk", 48, 600)
    g, o, d, st = _both(co, pop, 12, precision=1)
    assert_parity(g, o, 1e-4, "general mixed precision")


def test_general_tail_segments(co):
    """The tail (a second launch resuming paused fits) on the general kernel."""
    pop, _ = general_pop("mixed", 64, 700)
    g, o, d, st = _both(co, pop, 14, tail_iter=4, tail_partitions=4)
    assert_parity(g, o, 1e-9, "general tail", exact=True)


def test_general_eval_matches_oracle(co):
    pop, _ = general_pop("mixed", 48, 300)
    c0, xs, _ = f64(pop)
    yg = co.evaluate(pop, c0, xs)
    yo = lm_oracle.eval_pop(pop, c=c0, xs=xs)
    scale = np.maximum(np.max(np.abs(yo), axis=1, keepdims=True), 1e-300)
    assert np.array_equal(np.isfinite(yg), np.isfinite(yo))
    assert np.nanmax(np.abs(yg - yo) / scale) < 1e-13


def test_reference_abi_k_max_28(co):
    """co_optimize (the fp32 reference ABI) on a header with K_max = 28 returns
    0 and fits every expression, where a K <= 16 build refused the population."""
    pop, _ = general_pop("mixed", 48, 256)
    assert pop["K_max"] >= 17
    hi = [m for m in range(pop["M"]) if pop["metas"][m][3] >= 17]
    sub_pop = dict(pop)
    sub_pop["K_max"] = 28 if pop["K_max"] <= 28 else pop["K_max"]
    g = co.optimize(sub_pop, 20)          # raises COError on a non-zero code
    fit = lm_oracle.fit(pop, max_iter=20, f32_range=1)
    o = ci.narrow_fp32(pop, fit)
    _say(f"co_optimize K_max={sub_pop['K_max']}: statuses equal "
         f"{np.mean(g['status'] == o['status']):.4f} ({len(hi)} expressions K >= 17)")
    assert np.array_equal(g["status"], o["status"])
    assert np.array_equal(g["c_final"], o["c_final"])


def test_bounds_refused_before_any_copy(co):
    """Headers beyond K 32 / stack 64 return CO_ERR_BOUNDS (co_lib.cu:211-212)
    and leave the handle usable."""
    pop, _ = general_pop("highk", 8, 64)
    for key, v in (("K_max", 33), ("max_stack", 65)):
        bad = dict(pop)
        bad[key] = v
        with pytest.raises(ci.COError) as e:
            co.optimize_ex(bad, 5)
        assert e.value.code == ci.CO_ERR_BOUNDS
    g = co.optimize_ex(pop, 5)
    assert len(g["status"]) == pop["M"]
