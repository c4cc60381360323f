"""Parity at the benchmark configurations' full sizes (C2-C5), through the C ABI.

The whole population is fitted on the GPU exactly as bench.py fits it; the CPU
oracle then refits a seeded random sample of its expressions. Expressions are
independent and the device's arithmetic order depends only on the expression
and N (point partitions by N), so every sampled expression must agree with the
oracle as in the small-population tests: final loss within 1e-9 relative for
fp64 fits and 1e-4 for the mixed-precision C5, statuses equal.

Targets are synthesised by the device evaluator (as in bench.py) and rounded to
fp32 as pop.bin carries them; both sides read the same rounded inputs.
"""
import numpy as np
import pytest

from cusr_amd.benchmark import gen_synth, popio
from oracle import lm_oracle
from tests.helpers import rel_diff

pytestmark = pytest.mark.gpu

# configuration -> (sample size, loss tolerance)
CASES = {"C2": (256, 1e-9), "C3": (48, 1e-9), "C4": (12, 1e-9), "C5": (256, 1e-4)}


def _say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("name", sorted(CASES))
def test_full_size_population_sample_matches_oracle(co, name):
    cfg = gen_synth.CONFIGS[name]
    sample, tol = CASES[name]
    _say(f"full size {name}: generating (device evaluator)")
    pop, _ = gen_synth.generate(cfg, lambda p, c, xs: co.evaluate(p, c, xs))
    M = int(pop["M"])
    _say(f"full size {name}: M={M} N={pop['N']} K_max={pop['K_max']} "
         f"ad={cfg.ad_mode} prec={cfg.precision} max_iter={cfg.max_iter}: GPU fit")
    g = co.optimize_ex(pop, cfg.max_iter, ad_mode=cfg.ad_mode, precision=cfg.precision)
    idx = np.sort(np.random.default_rng(7).choice(M, size=min(sample, M), replace=False))
    sub = popio.select_pop(pop, idx)
    _say(f"full size {name}: oracle on {len(idx)} sampled expressions")
    o = lm_oracle.fit(sub, max_iter=cfg.max_iter, ad_mode=cfg.ad_mode,
                      precision=cfg.precision)
    st = float(np.mean(g["status"][idx] == o["status"]))
    d = rel_diff(g["loss_final"][idx], o["loss_final"])
    _say(f"full size {name}: status agree {st:.4f}; loss rel max {d.max():.3e}; "
         f"exact {np.mean(d == 0):.4f}")
    assert np.mean(d <= tol) == 1.0
    assert st == 1.0
