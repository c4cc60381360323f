"""co_fit_resident_static, the entry point that allocates nothing: its fit
against co_fit_resident's through the C ABI, bit for bit, on two calls in a
row (the second with a smaller population), with scratch in use -- the loop
state of tail segments and the split path's partition sums -- and the
refusal of a fit whose scratch exceeds the fixed array."""
import numpy as np
import pytest

from cusr_amd.kernel import co_inproc as ci
from tests.general_pops import general_pop
from tests.helpers import synth

pytestmark = pytest.mark.gpu

KEYS = ("c_final", "status", "loss_init", "loss_final", "iters")


def _say(msg):
    print(msg, flush=True)


def _same(a, b):
    for k in KEYS:
        assert np.array_equal(a[k], b[k], equal_nan=True), k


@pytest.mark.parametrize("opts", [dict(partitions=16), dict(partitions=32, ad_mode=1),
                                  dict(partitions=16, precision=1),
                                  dict(tail_iter=3, tail_partitions=4)])
def test_static_scratch_equals_allocating_entry(co, opts):
    big, _ = synth("C2", 192, 3000)
    small, _ = general_pop("mixed", 40, 1500)
    for pop in (big, small):
        _say(f"no-alloc M={pop['M']} N={pop['N']} {opts}")
        co.upload(pop)
        want = co.fit_resident(12, **opts)
        got = co.fit_resident(12, static_scratch=True, **opts)
        _same(got, want)
        again = co.fit_resident(12, static_scratch=True, **opts)
        _same(again, want)


def test_static_scratch_without_scratch_use(co):
    """A fit that needs no scratch (in-workgroup partitions, no tail) runs the
    same through both entry points."""
    pop, _ = synth("C1", 128, 256)
    co.upload(pop)
    _same(co.fit_resident(15, static_scratch=True), co.fit_resident(15))


def test_static_scratch_refuses_beyond_its_size(co):
    """State rows of a split fit: 5 KiB per expression plus the partition
    sums; 16,384 expressions at 256 partitions need far more than the array."""
    pop, _ = synth("C1", 16384, 64)
    co.upload(pop)
    need = 16384 * 256 * 15 * 8
    assert need > ci.CO_STATIC_SCRATCH_BYTES
    with pytest.raises(ci.COError) as e:
        co.fit_resident(3, static_scratch=True, partitions=256)
    assert e.value.code == ci.CO_ERR_BOUNDS
    # the handle and the array stay usable
    small, _ = synth("C1", 64, 64)
    co.upload(small)
    _same(co.fit_resident(5, static_scratch=True, partitions=8), co.fit_resident(5, partitions=8))
