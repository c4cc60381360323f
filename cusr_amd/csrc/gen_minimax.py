"""Minimax polynomial coefficients of include/cusr_math.h (provenance of the tables).

    python cusr_amd/csrc/gen_minimax.py

Each elementary function reduces its argument, then evaluates a polynomial
for the smooth part that is left. The polynomial is the minimax (best
uniform) approximation of that smooth part on the reduced range, found with
the Remez exchange algorithm (E. Ya. Remez, 1934; e.g. Muller, "Elementary
Functions", 3rd ed., ch. 3) at 60 decimal digits with mpmath, then rounded to
the target precision. The smooth parts and ranges:

  exp   e^r = 1 + r + r^2 G(r),    G(r) = (e^r - 1 - r) / r^2,  |r| <= ln2/2
  log   log((1+s)/(1-s)) = 2s + s z P(z), z = s^2, P(z) = (2 atanh(s) - 2s) / (s z),
        0 <= z <= ((sqrt2 - 1)/(sqrt2 + 1))^2
  sin   sin r = r + r^3 S(z),      S(z) = (sin r - r) / r^3,     0 <= z <= (pi/4)^2
  cos   cos r = 1 - z/2 + z^2 C(z), C(z) = (cos r - 1 + z/2) / z^2

Each table is printed highest degree first, the order Horner's rule uses, with
the bound of the approximation error on the function itself (relative, in
units of 2^-53 or 2^-24) after the coefficients are rounded. The reduced
ranges are widened for the rounding of the reduction's quotient k: by 2^-20
relative for fp64 (sin/cos reduce by Cody-Waite below 2^30, where x 2/pi has
an ulp of at most 2^-23, so |r| exceeds pi/4 by at most 2^-24 pi/2), and by
1 % for fp32 (below 2^17, |r| exceeds pi/4 by at most 2^-8 pi/2 = 0.8 %).
"""
from __future__ import annotations

import mpmath as mp

mp.mp.dps = 60
WIDEN = {64: 1 + mp.mpf(2) ** -20, 32: mp.mpf("1.01")}


def _G(r):
    if abs(r) < mp.mpf("1e-12"):
        return mp.mpf(1) / 2 + r / 6 + r * r / 24
    return (mp.exp(r) - 1 - r) / (r * r)


def _P(z):
    if z < mp.mpf("1e-24"):
        return mp.mpf(2) / 3 + 2 * z / 5
    s = mp.sqrt(z)
    return (2 * mp.atanh(s) - 2 * s) / (s * z)


def _S(z):
    if z < mp.mpf("1e-24"):
        return -mp.mpf(1) / 6 + z / 120
    r = mp.sqrt(z)
    return (mp.sin(r) - r) / (r * z)


def _C(z):
    if z < mp.mpf("1e-24"):
        return mp.mpf(1) / 24 - z / 720
    r = mp.sqrt(z)
    return (mp.cos(r) - 1 + z / 2) / (z * z)


def _peval(c, x):
    """c[0] + c[1] x + ... (lowest degree first)."""
    acc = mp.mpf(0)
    for v in reversed(c):
        acc = acc * x + v
    return acc


def remez(f, a, b, n, iters=40, grid=3000):
    """Minimax polynomial of degree n of f on [a, b]: coefficients lowest
    degree first, and the levelled error |E|."""
    a, b = mp.mpf(a), mp.mpf(b)
    ref = sorted((a + b) / 2 + (b - a) / 2 * mp.cos(mp.pi * i / (n + 1)) for i in range(n + 2))
    xs = [a + (b - a) * mp.mpf(i) / (grid - 1) for i in range(grid)]
    fx = [f(x) for x in xs]
    E_prev = None
    c = None
    for _ in range(iters):
        A = mp.matrix(n + 2, n + 2)
        rhs = mp.matrix(n + 2, 1)
        for i, x in enumerate(ref):
            for j in range(n + 1):
                A[i, j] = x ** j
            A[i, n + 1] = (-1) ** i
            rhs[i] = f(x)
        sol = mp.lu_solve(A, rhs)
        c = [sol[j] for j in range(n + 1)]
        E = abs(sol[n + 1])
        err = [fv - _peval(c, x) for x, fv in zip(xs, fx)]
        # the extremum of each run of one sign, refined by golden-section search
        ext = []
        i = 0
        while i < grid:
            j = i
            while j + 1 < grid and (err[j + 1] >= 0) == (err[i] >= 0):
                j += 1
            k = max(range(i, j + 1), key=lambda t: abs(err[t]))
            lo = xs[max(k - 1, 0)]
            hi = xs[min(k + 1, grid - 1)]
            g = lambda x: -abs(f(x) - _peval(c, x))  # noqa: E731
            for _r in range(40):
                m1 = lo + (hi - lo) * mp.mpf("0.381966")
                m2 = lo + (hi - lo) * mp.mpf("0.618034")
                if g(m1) < g(m2):
                    hi = m2
                else:
                    lo = m1
            xm = (lo + hi) / 2
            if abs(f(xm) - _peval(c, xm)) < abs(err[k]):
                xm = xs[k]
            ext.append(xm)
            i = j + 1
        while len(ext) > n + 2:       # drop the smaller end extremum
            e0 = abs(f(ext[0]) - _peval(c, ext[0]))
            e1 = abs(f(ext[-1]) - _peval(c, ext[-1]))
            ext = ext[1:] if e0 < e1 else ext[:-1]
        if len(ext) < n + 2:
            raise RuntimeError(f"Remez: {len(ext)} alternations for degree {n}")
        ref = ext
        if E_prev is not None and abs(E - E_prev) <= E * mp.mpf("1e-12"):
            break
        E_prev = E
    return c, E


def _round(c, prec):
    if prec == 64:
        return [float(v) for v in c]
    import numpy as np
    return [float(np.float32(float(v))) for v in c]


def _bound(name, c, prec, samples=4000):
    """Largest relative error of the assembled function (rounded coefficients,
    exact arithmetic) on the reduced range, in units of 2^-53 / 2^-24."""
    w = WIDEN[prec]
    cm = [mp.mpf(v) for v in c]
    unit = mp.mpf(2) ** (-53 if prec == 64 else -24)
    worst = mp.mpf(0)
    for i in range(samples + 1):
        t = mp.mpf(i) / samples
        if name == "exp":
            h = mp.log(2) / 2 * w
            r = -h + 2 * h * t
            v = 1 + r + r * r * _peval(cm, r)
            e = abs(v - mp.exp(r)) / mp.exp(r)
        elif name == "log":
            smax = (mp.sqrt(2) - 1) / (mp.sqrt(2) + 1) * w
            s = smax * t
            if s == 0:
                continue
            z = s * s
            v = 2 * s + s * z * _peval(cm, z)
            e = abs(v - 2 * mp.atanh(s)) / (2 * mp.atanh(s))
        elif name == "sin":
            r = mp.pi / 4 * w * t
            if r == 0:
                continue
            z = r * r
            v = r + r * z * _peval(cm, z)
            e = abs(v - mp.sin(r)) / mp.sin(r)
        else:
            r = mp.pi / 4 * w * t
            z = r * r
            v = 1 - z / 2 + z * z * _peval(cm, z)
            e = abs(v - mp.cos(r)) / mp.cos(r)
        worst = max(worst, e)
    return float(worst / unit)


SPECS = {
    # name: (smooth part, range of its variable, degree for fp64, degree for fp32)
    # (one degree less leaves more than 6 x 2^-53 for every fp64 form, and
    # 7 x 2^-24 for fp32 exp)
    "exp": (_G, lambda w: (-mp.log(2) / 2 * w, mp.log(2) / 2 * w), 9, 4),
    "log": (_P, lambda w: (0, ((mp.sqrt(2) - 1) / (mp.sqrt(2) + 1) * w) ** 2), 6, 2),
    "sin": (_S, lambda w: (0, (mp.pi / 4 * w) ** 2), 5, 2),
    "cos": (_C, lambda w: (0, (mp.pi / 4 * w) ** 2), 5, 2),
}


def tables():
    """{(name, prec): (coefficients highest degree first, levelled error, bound)}."""
    out = {}
    for name, (f, rng, n64, n32) in SPECS.items():
        for prec, n in ((64, n64), (32, n32)):
            a, b = rng(WIDEN[prec])
            c, E = remez(f, a, b, n)
            cr = _round(c, prec)
            out[(name, prec)] = (list(reversed(cr)), float(E), _bound(name, cr, prec))
    return out


def main():
    for (name, prec), (c, E, bound) in tables().items():
        fmt = repr if prec == 64 else (lambda v: repr(v) + "f")
        print(f"/* {name} fp{prec}: degree {len(c) - 1} minimax of the smooth part, levelled "
              f"error {E:.3e}; relative error of the function from the polynomial <= "
              f"{bound:.4f} x 2^-{53 if prec == 64 else 24} */")
        print("    " + ", ".join(fmt(v) for v in c) + ",")


if __name__ == "__main__":
    main()
