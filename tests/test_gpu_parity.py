"""HIP path vs the CPU oracle on the same seeded inputs (called through the C ABI).

Tolerances: final loss relative 1e-9 for fp64 fits and
1e-4 for mixed-precision fits; statuses agree on >= 99.9% of expressions.
"""
import numpy as np
import pytest

from oracle import lm_oracle
from tests.helpers import assert_parity, f64, ref_pop, rel_diff, synth

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _fit_both(co, pop, max_iter, ad_mode=0, precision=0, partitions=0, **kw):
    c0, xs, ym = f64(pop)
    _say(f"case M={pop['M']} N={pop['N']} ad={ad_mode} prec={precision} max_iter={max_iter} "
         f"partitions={partitions} {kw}")
    g = co.optimize_ex(pop, max_iter, ad_mode=ad_mode, precision=precision, partitions=partitions,
                       **kw)
    o = lm_oracle.fit(pop, max_iter=max_iter, ad_mode=ad_mode, precision=precision,
                      partitions=partitions, **kw)
    return g, o


@pytest.mark.parametrize("name,M,N", [("C1", 256, 256), ("C2", 128, 512)])
def test_eval_matches_oracle(co, name, M, N):
    pop, c_true = synth(name, M, N)
    c0, xs, _ = f64(pop)
    _say(f"eval {name} M={M} N={N}")
    yg = co.evaluate(pop, c0, xs)
    yo = lm_oracle.eval_pop(pop, c=c0, xs=xs)
    # libm and ROCm transcendentals may differ in the last bit; compare each
    # value against the scale of its row so cancellation does not inflate it
    scale = np.maximum(np.max(np.abs(yo), axis=1, keepdims=True), 1e-300)
    d = np.abs(yg - yo) / scale
    _say(f"eval exact fraction {np.mean(yg == yo):.6f} max scaled diff {d.max():.3e}")
    assert np.array_equal(np.isfinite(yg), np.isfinite(yo))
    assert np.nanmax(d) < 1e-13


@pytest.mark.parametrize("ad_mode", [0, 1])
def test_fit_fp64_c1(co, ad_mode):
    pop, _ = synth("C1", 512, 256)
    g, o = _fit_both(co, pop, 20, ad_mode=ad_mode)
    assert_parity(g, o, 1e-9, f"C1 ad={ad_mode}", exact=True)


def test_fit_fp64_c2_small(co):
    pop, _ = synth("C2", 256, 1024)
    g, o = _fit_both(co, pop, 50)
    assert_parity(g, o, 1e-9, "C2 small", exact=True)


def test_fit_mixed_c5_small(co):
    pop, _ = synth("C5", 256, 512)
    g, o = _fit_both(co, pop, 10, precision=1)
    assert_parity(g, o, 1e-4, "C5 small mixed")


def test_reference_fixture_recovers_truth(co):
    import json
    from tests.helpers import REF_FIX
    pop = ref_pop("pop_fixture.bin")
    truth = json.loads((REF_FIX / "pop_fixture_truth.json").read_text())
    _say("pop_fixture.bin")
    r = co.optimize(pop, 50)
    for fx in truth["fixtures"]:
        k0, K = fx["c_offset"], fx["K"]
        got = r["c_final"][k0:k0 + K].astype(np.float64)
        want = np.asarray(fx["c_true"])
        assert np.all(np.abs(got - want) / np.abs(want) < 5e-3), (fx["name"], got, want)
    assert list(r["status"]) == [0, 0, 0]


def test_stress_fixture_statuses(co):
    import json
    from tests.helpers import REF_FIX
    pop = ref_pop("pop_fixture_stress.bin")
    truth = json.loads((REF_FIX / "pop_fixture_stress_truth.json").read_text())
    _say("pop_fixture_stress.bin")
    r = co.optimize(pop, 50)
    assert list(r["status"]) == [f["expect_status"] for f in truth["fixtures"]]


def _op_pop(N, seed):
    """One expression per operator applied to inputs x0 (and x1), K = 0."""
    from cusr_amd.benchmark import popio
    rng = np.random.default_rng(seed)
    unary = [14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26, 27, 28, 33, 34, 35]
    binary = [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 32]
    trees = []
    for f in unary:
        trees.append(([2, 0], [f, 0], [-1, -1], []))
    for f in binary:
        trees.append(([3, 0, 0], [f, 0, 1], [-1, -1, -1], []))
    # wide magnitudes, both signs, some exact zeros and tiny values
    mag = 10.0 ** rng.uniform(-12, 3, size=(N, 2))
    xs = (mag * rng.choice([-1.0, 1.0], size=(N, 2))).astype(np.float32)
    xs[::17, 1] = 0.0
    xs[::23, 0] = 0.0
    pop = popio.build_pop(trees, xs, np.zeros((len(trees), N)))
    return pop, unary + binary


@pytest.mark.parametrize("precision", [0, 1])
def test_operators_bit_exact(co, precision):
    """Every operator, device vs oracle, on wide-range inputs: identical bits."""
    pop, ops = _op_pop(4096, 7)
    xs = pop["xs"].astype(np.float64)
    _say(f"operators precision={precision}")
    yg = co.evaluate(pop, np.zeros(1), xs, precision=precision)
    yo = lm_oracle.eval_pop(pop, c=np.zeros(1), xs=xs, precision=precision)
    same = (yg == yo) | (np.isnan(yg) & np.isnan(yo))
    bad = [(ops[m], int(np.sum(~same[m]))) for m in range(len(ops)) if not same[m].all()]
    _say(f"mismatching ops (id, count): {bad}")
    assert not bad


def _edge_inputs():
    """fp64 arguments at the special ranges of the elementary functions: exp's
    overflow and subnormal-result ends, log's subnormal, zero, negative and
    infinite arguments, trigonometric arguments near multiples of pi/2, at the
    Payne-Hanek switch (2^30) and huge, fp32's reduction switch (2^17), NaN."""
    rng = np.random.default_rng(11)
    v = [0.0, -0.0, np.inf, -np.inf, np.nan, 5e-324, -5e-324, 1e-310, 2.2250738585072014e-308,
         np.nextafter(2.2250738585072014e-308, 0), 1.0, -1.0, np.nextafter(1.0, 2),
         np.nextafter(1.0, 0), 2.0 ** 30, np.nextafter(2.0 ** 30, 0), 2.0 ** 17,
         np.nextafter(2.0 ** 17, 0), 1e22, -1e22, 1e300, 20.0, np.nextafter(20.0, 30)]
    v += list(rng.uniform(-746.0, -706.0, 600)) + list(rng.uniform(706.0, 711.0, 200))
    v += list(rng.uniform(87.0, 89.5, 100)) + list(rng.uniform(-105.0, -86.0, 200))
    v += list(np.ldexp(rng.uniform(0.5, 1.0, 300), rng.integers(-1074, -1020, 300)))
    v += list(np.ldexp(rng.uniform(0.5, 1.0, 200), rng.integers(-149, -120, 200)))
    k = rng.integers(-10 ** 6, 10 ** 6, 400).astype(np.float64)
    v += list(k * (np.pi / 2) + rng.uniform(-1e-6, 1e-6, 400))
    v += list(rng.uniform(-1.0, 1.0, 200) * 2.0 ** rng.integers(16, 64, 200))
    x = np.asarray(v, np.float64)
    return np.concatenate([x, -x])


@pytest.mark.parametrize("precision", [0, 1])
def test_operators_edge_values_bit_exact(co, precision):
    """The unary operators at the special ranges of exp, log, sin and cos,
    fp64 inputs (fp32 in mixed precision), device vs oracle: identical bits."""
    from cusr_amd.benchmark import popio
    unary = [14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26, 27, 28, 33, 34, 35]
    x = _edge_inputs()
    xs = np.stack([x, np.ones_like(x)], axis=1)
    trees = [([2, 0], [f, 0], [-1, -1], []) for f in unary]
    pop = popio.build_pop(trees, xs.astype(np.float32), np.zeros((len(trees), len(x))))
    _say(f"edge values precision={precision} N={len(x)}")
    yg = co.evaluate(pop, np.zeros(1), xs, precision=precision)
    yo = lm_oracle.eval_pop(pop, c=np.zeros(1), xs=xs, precision=precision)
    same = (yg == yo) | (np.isnan(yg) & np.isnan(yo))
    bad = [(unary[m], int(np.sum(~same[m]))) for m in range(len(unary)) if not same[m].all()]
    _say(f"mismatching ops (id, count): {bad}")
    assert not bad


@pytest.mark.parametrize("parts,ad_mode,precision", [(2, 0, 0), (4, 0, 0), (4, 1, 0), (2, 0, 1)])
def test_point_partitions_match_oracle(co, parts, ad_mode, precision):
    """Several wavefronts per expression: granule g of 64 points goes to
    partition g mod G, partition sums are added in order (N = 1000: the last
    granule is ragged and partitions hold different granule counts)."""
    pop, _ = synth("C2", 96, 1000)
    g, o = _fit_both(co, pop, 15, ad_mode=ad_mode, precision=precision, partitions=parts)
    tol = 1e-9 if precision == 0 else 1e-4
    assert_parity(g, o, tol, f"partitions {parts}", exact=precision == 0)


def test_large_n_auto_partitions(co):
    """C4-shaped expressions (D = 5, N = 20,000 -> 4 partitions by N). From
    N = 16,384 the K = 1..8 bins run the large-N kernel instances (two points
    per lane instead of four); points per pass leave every summation order
    unchanged, so those expressions must match the oracle exactly, past the
    first accept/reject decisions of the LM loop."""
    pop, _ = synth("C4", 32, 20000)
    assert pop["N"] >= 16384
    K = pop["metas"][:, 3]
    ln = (K >= 1) & (K <= 8)
    assert ((K == 5) | (K == 6)).sum() >= 6 and ((K == 7) | (K == 8)).sum() >= 4
    g, o = _fit_both(co, pop, 20)
    _say(f"large-N instances: iters {g['iters'][ln].tolist()}")
    assert np.mean(g["iters"][ln] >= 2) >= 0.75
    assert_parity(g, o, 1e-9, "large-N instances", exact=True, mask=ln)
    assert_parity(g, o, 1e-9, "large N", exact=True)


@pytest.mark.parametrize("ad_mode,parts", [(1, 0), (0, 0), (1, 2)])
def test_high_k_matrix_sums(co, ad_mode, parts):
    """K >= CO_SUMS_MATRIX_MIN_K: sums from the fp64 matrix instruction (one fma
    chain per entry over the points in order) and the LDS Cholesky; K up to 16
    (C3 shapes: depth <= 8, <= 63 nodes)."""
    pop, _ = synth("C3", 128, 700)
    assert pop["K_max"] >= 13
    g, o = _fit_both(co, pop, 15, ad_mode=ad_mode, partitions=parts)
    assert_parity(g, o, 1e-9, f"high K ad={ad_mode} parts={parts}", exact=True)


@pytest.mark.parametrize("parts", [0, 8])
def test_high_k_reverse_mixed_matrix_sums(co, parts):
    """Mixed precision in reverse AD up to K = 16: from K = 12
    (CO_SUMS_MATRIX_MIN_K_REV) the fp32 Jacobian rows are staged as doubles
    over the fp32 tape's LDS for the matrix-instruction sums; in-workgroup
    (parts 0) and on the split path (parts 8, one workgroup per partition)."""
    pop, _ = synth("C3", 128, 700)
    K = np.array([int(m[3]) for m in pop["metas"]])
    assert np.sum(K >= 12) >= 8
    g, o = _fit_both(co, pop, 12, ad_mode=1, precision=1, partitions=parts)
    hk = K >= 12
    assert_parity(g, o, 1e-4, f"mixed reverse parts {parts}")
    # the staged rows over the fp32 tape: the oracle models the same sums, so
    # the K >= 12 expressions agree to the bit (a stale column or an LDS
    # overlap would not)
    assert_parity(g, o, 1e-4, f"mixed reverse K >= 12 parts {parts}", exact=True, mask=hk)
    c_off = np.concatenate([[0], np.cumsum(K)])
    for m in np.nonzero(hk)[0]:
        a, b = c_off[m], c_off[m + 1]
        assert np.array_equal(g["c_final"][a:b], o["c_final"][a:b]), m


@pytest.mark.parametrize("ad_mode,precision,tail_iter,tail_parts,lm_order", [
    (0, 0, 0, 0, 0), (0, 0, 3, 2, 0), (1, 0, 5, 4, 0), (0, 1, 4, 4, 0), (0, 0, 6, 4, 1),
    (0, 0, -1, 0, 0)])
def test_tail_segment_matches_oracle(co, ad_mode, precision, tail_iter, tail_parts, lm_order):
    """Active-set compaction: after tail_iter iterations the expressions still
    running resume in a second launch with tail_parts partitions (one wavefront
    each) from their saved loop state; passes after tail_iter, and the fp64
    audit of an expression finishing after it, sum with the tail's partitions
    in the oracle too. tail_iter 0 is the default rule, -1 one launch."""
    pop, _ = synth("C2", 160, 700)
    g, o = _fit_both(co, pop, 25, ad_mode=ad_mode, precision=precision, tail_iter=tail_iter,
                     tail_partitions=tail_parts, lm_order=lm_order)
    _say(f"iters > tail {np.mean(g['iters'] > max(tail_iter, 0)):.2f}")
    assert np.array_equal(g["iters"] > 0, o["iters"] > 0)
    tol = 1e-9 if precision == 0 else 1e-4
    assert_parity(g, o, tol, f"tail {tail_iter}/{tail_parts}", exact=precision == 0)


def test_tail_high_k_matrix_sums(co):
    """The tail with the matrix-instruction sums (forward AD, K >= 13)."""
    pop, _ = synth("C3", 96, 700)
    g, o = _fit_both(co, pop, 15, tail_iter=4, tail_partitions=4)
    assert_parity(g, o, 1e-9, "tail high K", exact=True)


@pytest.mark.parametrize("damping", [1, 2])
@pytest.mark.parametrize("case", ["fast", "reverse", "matrix", "split", "general", "mixed"])
def test_damping_variants_match_oracle(co, damping, case):
    """CoOptions.damping -- trust region (absolute damping, a pivot <= 0
    replaced by lambda) and the pivot floor (cusr/kernel/batch_lm_ad.cu:149-172)
    -- in every solve of the device: the register solve of the fast kernels
    (forward and reverse AD), the LDS solve of the matrix-sum bins, the split
    path's step kernel, the general kernel and a mixed-precision fit. Final
    constants, losses and statuses equal the oracle's (fp64) or agree to the
    mixed tolerance, and the variant changes the fit (against the oracle's
    relative damping), so its own rule is what is compared."""
    from tests.general_pops import general_pop
    lam0 = lm_oracle.CO_TRUST_REGION_LAMBDA0 if damping == 1 else 1e-3
    kw = dict(damping=damping, lambda0=lam0)
    prec = 1 if case == "mixed" else 0
    if case == "fast":
        pop, _ = synth("C2", 256, 512)
    elif case == "reverse":
        pop, _ = synth("C2", 128, 512)
        kw["ad_mode"] = 1
    elif case == "matrix":
        pop, _ = synth("C3", 96, 700)
        assert pop["K_max"] >= 13
    elif case == "split":
        pop, _ = synth("C3", 64, 1024)
        kw["partitions"] = 8
    elif case == "general":
        pop, _ = general_pop("highk", 32, 700)
    else:
        pop, _ = synth("C5", 128, 512)
    g, o = _fit_both(co, pop, 30, precision=prec, **kw)
    assert_parity(g, o, 1e-9 if prec == 0 else 1e-4, f"damping {damping} {case}",
                  exact=prec == 0)
    rel = lm_oracle.fit(pop, max_iter=30, precision=prec,
                        **{k: v for k, v in kw.items() if k not in ("damping", "lambda0")})
    assert not np.array_equal(o["c_final"], rel["c_final"])


def test_damping_out_of_range_refused(co):
    from cusr_amd.kernel import co_inproc as ci
    pop, _ = synth("C1", 8, 64)
    with pytest.raises(ci.COError) as e:
        co.optimize_ex(pop, 5, damping=3)
    assert e.value.code == ci.CO_ERR_NULLARG
