"""co_optimize of a large population from host buffers decodes and uploads it
in ranges of expressions, each range launched while the host decodes the next
(the upload pipeline of cusr_amd/csrc/co_lib.hip, from M = 16,384 on). Every
expression's fit is independent of how the population is cut, so the
pipelined call must equal, bit for bit, the one-piece upload and resident fit
of the same population; a resident refit after a pipelined call plans its
bins range by range and must equal both. A decode error in the last range
returns its code after the earlier ranges have run, and the handle fits the
next population normally."""
import numpy as np
import pytest

from cusr_amd.kernel import co_inproc as ci
from tests.helpers import synth

pytestmark = pytest.mark.gpu

KEYS = ("c_final", "status", "loss_init", "loss_final", "iters")


@pytest.fixture(scope="module")
def co():
    return ci.get_inproc_co(0, "ad")


def _same(a, b, what):
    for k in KEYS:
        x, y = np.asarray(a[k]), np.asarray(b[k])
        assert x.shape == y.shape, (what, k)
        assert x.tobytes() == y.tobytes(), (what, k, int(np.count_nonzero(x != y)))


@pytest.mark.parametrize("name,M,ad_mode,precision", [
    ("C2", 20000, ci.CO_AD_FORWARD, ci.CO_PREC_FP64),
    ("C5", 33000, ci.CO_AD_FORWARD, ci.CO_PREC_MIXED),
    ("C3", 16500, ci.CO_AD_REVERSE, ci.CO_PREC_FP64),
])
def test_pipelined_equals_one_piece(co, name, M, ad_mode, precision):
    pop, _ = synth(name, M, 64)
    kw = dict(ad_mode=ad_mode, precision=precision)
    piped = co.optimize_ex(pop, 20, **kw)
    setup_ms, loop_ms = co.last_split()
    assert setup_ms is not None and loop_ms is not None and setup_ms >= 0 and loop_ms >= 0
    # the refit of the population the pipelined call left resident
    co._resident = (int(pop["M"]), int(pop["total_c"]))
    refit = co.fit_resident(20, **kw)
    co.upload(pop)
    whole = co.fit_resident(20, **kw)
    _same(piped, whole, f"{name} pipelined vs one piece")
    _same(refit, whole, f"{name} refit after the pipeline vs one piece")
    assert np.count_nonzero(piped["status"] == 0) > M // 10   # the fits did run


def test_error_in_last_range(co):
    pop, _ = synth("C2", 20000, 64)
    bad = dict(pop)
    bad["nv"] = pop["nv"].copy()
    metas = pop["metas"]
    # the last expression whose root is an operator gets an unknown operator id
    m = next(m for m in range(int(pop["M"]) - 1, -1, -1) if pop["nt"][metas[m, 0]] >= 2)
    bad["nv"][metas[m, 0]] = 29.0
    with pytest.raises(ci.COError) as e:
        co.optimize_ex(bad, 20)
    assert e.value.code == ci.CO_ERR_PROGRAM
    # the handle is usable and fits the good population as a fresh upload does
    good = co.optimize_ex(pop, 20)
    co.upload(pop)
    _same(good, co.fit_resident(20), "after a failed pipelined call")
