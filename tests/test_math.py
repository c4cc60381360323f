"""include/cusr_math.h against the C library (numpy's libm), no GPU.

The device and the CPU oracle both compile these functions, so device/oracle
agreement is by construction (tests/test_gpu_parity.py checks it on the GPU);
what this file pins is their accuracy: the largest error in units of the last
place against libm over wide argument ranges, and the special values.
"""
import numpy as np
import pytest

from oracle import lm_oracle

# (name, arguments, max ulp fp64, max ulp fp32)
RNG = np.random.default_rng(2024)


def _logu(lo, hi, n):
    return np.exp(RNG.uniform(np.log(lo), np.log(hi), n))


def _sym(a):
    return np.concatenate([a, -a])


CASES = {
    "exp": (np.concatenate([RNG.uniform(-700, 700, 20000), RNG.uniform(-1, 1, 5000)]), 1, 2),
    "log": (np.concatenate([_logu(1e-300, 1e300, 20000), RNG.uniform(0.5, 2, 5000)]), 1, 2),
    "sin": (_sym(np.concatenate([_logu(1e-8, 1e5, 20000), RNG.uniform(0, 10, 5000)])), 1, 2),
    "cos": (_sym(np.concatenate([_logu(1e-8, 1e5, 20000), RNG.uniform(0, 10, 5000)])), 1, 2),
    "tan": (_sym(np.concatenate([_logu(1e-8, 1e4, 20000), RNG.uniform(0, 1.5, 5000)])), 3, 3),
    "sinh": (_sym(np.concatenate([_logu(1e-8, 700, 20000), RNG.uniform(0, 2, 5000)])), 2, 3),
    "cosh": (_sym(_logu(1e-8, 700, 20000)), 2, 3),
    "tanh": (_sym(np.concatenate([_logu(1e-8, 20, 20000), RNG.uniform(0, 2, 5000)])), 4, 3),
}


def _ulps(got, want, dtype):
    got = got.astype(dtype).astype(np.float64)
    want_t = want.astype(dtype)
    sp = np.spacing(np.abs(want_t)).astype(np.float64)
    fin = np.isfinite(want_t) & (want_t != 0)
    return np.abs(got[fin] - want_t[fin].astype(np.float64)) / sp[fin]


@pytest.mark.parametrize("name", sorted(CASES))
def test_fp64_accuracy(name):
    x, ulp64, _ = CASES[name]
    got = lm_oracle.math_fn(name, x)
    want = getattr(np, name)(x)
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin), name
    e = _ulps(got, want, np.float64)
    assert e.max() <= ulp64, (name, e.max())


@pytest.mark.parametrize("name", sorted(CASES))
def test_fp32_accuracy(name):
    x, _, ulp32 = CASES[name]
    x = x[np.abs(x) < (88.0 if name in ("exp", "sinh", "cosh") else 3e38)]
    x32 = x.astype(np.float32)
    if name == "log":
        x32 = x32[x32 > 0]
    got = lm_oracle.math_fn(name, x32.astype(np.float64), fp32=True)
    want = getattr(np, name)(x32.astype(np.float64))      # the exact fp32 argument, in fp64
    e = _ulps(got, want, np.float32)
    assert e.max() <= ulp32, (name, e.max())


def test_pow_accuracy():
    a = _logu(1e-3, 1e3, 20000)
    b = RNG.uniform(-20, 20, 20000)
    got = lm_oracle.math_fn("pow", a, b)
    want = np.power(a, b)
    # exp(y log x) without an extra-precision log: the error of log x is
    # amplified by |y log x| (documented in include/cusr_math.h)
    amp = np.abs(b * np.log(a))
    fin = np.isfinite(want) & (want != 0)
    e = np.abs(got[fin] - want[fin]) / np.spacing(np.abs(want[fin]))
    assert np.all(e <= 2.0 * (1.0 + amp[fin])), (e / (1.0 + amp[fin])).max()
    small = fin & (amp < 1.0)
    assert (np.abs(got[small] - want[small]) / np.spacing(np.abs(want[small]))).max() <= 6
    # negative base with integral exponent keeps the sign; fractional gives NaN
    neg = lm_oracle.math_fn("pow", np.array([-2.0, -2.0, -8.0]), np.array([3.0, 2.0, 0.5]))
    assert neg[0] == -8.0 and neg[1] == 4.0 and np.isnan(neg[2])


def test_special_values():
    nan, inf = np.nan, np.inf
    f = lm_oracle.math_fn
    assert np.isnan(f("exp", np.array([nan])))[0]
    assert f("exp", np.array([inf]))[0] == inf and f("exp", np.array([-inf]))[0] == 0.0
    assert f("exp", np.array([710.0]))[0] == inf and f("exp", np.array([-746.0]))[0] == 0.0
    assert f("log", np.array([0.0]))[0] == -inf and np.isnan(f("log", np.array([-1.0])))[0]
    assert f("log", np.array([inf]))[0] == inf and f("log", np.array([1.0]))[0] == 0.0
    assert f("log", np.array([5e-324]))[0] == pytest.approx(np.log(5e-324), rel=1e-15)
    for name in ("sin", "cos", "tan"):
        assert np.all(np.isnan(f(name, np.array([nan, inf, -inf]))))
    assert f("sin", np.array([0.0]))[0] == 0.0 and f("cos", np.array([0.0]))[0] == 1.0
    assert f("tanh", np.array([inf]))[0] == 1.0 and f("tanh", np.array([-inf]))[0] == -1.0


def test_exact_small_cases():
    """Values every correct implementation must give exactly."""
    f = lm_oracle.math_fn
    assert f("exp", np.array([0.0]))[0] == 1.0
    assert f("exp", np.array([1.0]))[0] == np.exp(1.0)
    assert f("log", np.array([2.0]))[0] == np.log(2.0)
    assert f("pow", np.array([2.0]), np.array([10.0]))[0] == 1024.0
    assert f("pow", np.array([3.0]), np.array([-2.0]))[0] == 1.0 / 9.0
    assert f("pow", np.array([1.5]), np.array([2.0]))[0] == 2.25
    x = RNG.uniform(-3, 3, 1000)
    assert np.array_equal(f("pow", x, np.full(1000, 2.0)), x * x)
    assert f("sinh", np.array([0.0]))[0] == 0.0 and f("cosh", np.array([0.0]))[0] == 1.0


@pytest.mark.parametrize("name,ulp", [("sin", 1), ("cos", 1), ("tan", 3)])
def test_huge_arguments_reduced_exactly(name, ulp):
    """|x| from 2^20 to the largest double: the Payne-Hanek reduction (fp64
    from 2^50) keeps sin/cos within 1 ulp of the C library and tan within 3,
    as below; fp32 arguments from 2^21 are reduced in fp64. A fit cannot
    exploit a flattened sin/cos where constants drive arguments huge."""
    f = lm_oracle.math_fn
    e = RNG.uniform(20, 1023, 40000)
    x = _sym(RNG.uniform(1, 2, 40000) * 2.0 ** e)
    got = f(name, x)
    assert _ulps(got, getattr(np, name)(x), np.float64).max() <= ulp
    # near multiples of pi/2: a large k with the tiny remainder resolved
    k = RNG.integers(2 ** 40, 2 ** 52, 2000).astype(np.float64)
    near = np.nextafter(k * (np.pi / 2), np.inf)
    assert _ulps(f(name, near), getattr(np, name)(near), np.float64).max() <= ulp
    x32 = _sym(RNG.uniform(1, 2, 20000) * 2.0 ** RNG.uniform(21, 127, 20000)).astype(np.float32)
    got32 = f(name, x32.astype(np.float64), fp32=True)
    assert _ulps(got32, getattr(np, name)(x32.astype(np.float64)), np.float32).max() <= ulp + 1


@pytest.mark.parametrize("name", ["sin", "cos"])
def test_reduction_quotient_rounding_ranges(name):
    """Below the Payne-Hanek (fp64, 2^30) and fp64-reduction (fp32, 2^17)
    thresholds the quotient k = rint(x 2/pi) comes from x 2/pi rounded once,
    so the remainder can pass pi/4 by up to 2^-24 pi/2 (fp32: 2^-8 pi/2); the
    polynomials are fitted on ranges widened for it. Dense arguments where
    that rounding is largest keep sin/cos within 1 ulp (fp32: 2)."""
    f = lm_oracle.math_fn
    x = _sym(RNG.uniform(1, 2, 40000) * 2.0 ** RNG.uniform(20, 30, 40000))
    assert _ulps(f(name, x), getattr(np, name)(x), np.float64).max() <= 1
    x32 = _sym(RNG.uniform(1, 2, 40000) * 2.0 ** RNG.uniform(10, 17, 40000)).astype(np.float32)
    got = f(name, x32.astype(np.float64), fp32=True)
    assert _ulps(got, getattr(np, name)(x32.astype(np.float64)), np.float32).max() <= 2


def test_p_wide_forms_equal_scalar(tmp_path):
    """The interpreter evaluates exp, log, sin and cos P points at a time
    (cm_*_v<P> of include/cusr_math.h); each element must get the scalar
    function's bits, which the CPU oracle uses. tests/pwide_check.hip,
    compiled for the host with the device flags, compares both on 1.6 M
    random, huge, tiny, subnormal and special arguments for P = 1, 2, 4 in
    both precisions."""
    import shutil
    import subprocess
    from pathlib import Path

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    src = Path(__file__).resolve().parent / "pwide_check.hip"
    exe = tmp_path / "pwide_check"
    subprocess.run([hipcc, "-x", "hip", "--offload-arch=gfx950", "-O2", "-std=c++17",
                    "-ffp-contract=off", "-fno-fast-math", "-Xclang", "-target-feature",
                    "-Xclang", "-packed-fp32-ops", str(src), "-o", str(exe)],
                   check=True, capture_output=True, timeout=300)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "pwide ok" in r.stdout, r.stdout[-2000:]
