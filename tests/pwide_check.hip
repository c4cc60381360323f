// Host check behind tests/test_math.py::test_p_wide_forms_equal_scalar: the
// P-wide forms of include/cusr_math.h (the interpreter's, P points at a time)
// give every element the bits of the scalar function, for P = 1, 2, 4 and
// both precisions, on random, huge, tiny, subnormal and special arguments.
// Prints "pwide ok <checked>" or the first mismatches; exit status 1 on any.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../include/cusr_math.h"

static uint64_t g_state = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64() {   // splitmix64
    uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static double uni01() { return (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0); }

static double arg(int i) {
    static const double special[] = {0.0, -0.0, 1.0, -1.0, 0.5, 2.0, 1e-300, 4.9e-324,
                                     2.2250738585072014e-308, 1e300, 709.78, -745.1,
                                     710.0, -750.0, 1.4142135623730951, 0.7071067811865476,
                                     0.7853981633974483, 1.5707963267948966, 1073741824.0,
                                     1073741823.0, 131072.0, 131071.9, 1e22, 88.7, -104.0};
    const int ns = (int)(sizeof(special) / sizeof(special[0]));
    if (i < ns) return special[i];
    if (i == ns) return CM_INF;
    if (i == ns + 1) return -CM_INF;
    if (i == ns + 2) return CM_NAN;
    const double s = (next_u64() & 1) ? -1.0 : 1.0;
    switch (i % 4) {
    case 0: return s * uni01() * 10.0;
    case 1: return s * CM_LDEXP(1.0 + uni01(), (int)(uni01() * 2040.0) - 1020);
    case 2: return s * CM_LDEXP(1.0 + uni01(), (int)(uni01() * 40.0));
    default: {
        uint64_t b = next_u64();   // any bit pattern
        return cm_dbl(b);
    }
    }
}

static long g_bad = 0;
static int same64(double a, double b) { return cm_bits(a) == cm_bits(b) || (a != a && b != b); }
static int same32(float a, float b) { return cm_bitsf(a) == cm_bitsf(b) || (a != a && b != b); }
static void report(const char *what, double x, double a, double b) {
    if (g_bad++ < 10) printf("mismatch %s x=%.17g wide=%.17g scalar=%.17g\n", what, x, a, b);
}

template <int P>
static void check(const double *x) {
    double e[P], l[P], s[P], c[P], ax[P];
    float xf[P], ef[P], lf[P], sf[P], cf[P], axf[P];
    for (int p = 0; p < P; ++p) {
        ax[p] = cm_fabs(x[p]);
        xf[p] = (float)x[p];
        axf[p] = cm_fabsf(xf[p]);
    }
    cm_exp_v<P>(x, e);
    cm_log_v<P>(ax, l);
    cm_sincos_v<P>(x, s, c);
    cm_expf_v<P>(xf, ef);
    cm_logf_v<P>(axf, lf);
    cm_sincosf_v<P>(xf, sf, cf);
    for (int p = 0; p < P; ++p) {
        double ss, cc;
        float ssf, ccf;
        cm_sincos(x[p], &ss, &cc);
        cm_sincosf(xf[p], &ssf, &ccf);
        if (!same64(e[p], cm_exp(x[p]))) report("exp", x[p], e[p], cm_exp(x[p]));
        if (!same64(l[p], cm_log(ax[p]))) report("log", ax[p], l[p], cm_log(ax[p]));
        if (!same64(s[p], ss)) report("sin", x[p], s[p], ss);
        if (!same64(c[p], cc)) report("cos", x[p], c[p], cc);
        if (!same32(ef[p], cm_expf(xf[p]))) report("expf", xf[p], ef[p], cm_expf(xf[p]));
        if (!same32(lf[p], cm_logf(axf[p]))) report("logf", axf[p], lf[p], cm_logf(axf[p]));
        if (!same32(sf[p], ssf)) report("sinf", xf[p], sf[p], ssf);
        if (!same32(cf[p], ccf)) report("cosf", xf[p], cf[p], ccf);
    }
}

int main() {
    const int n = 1600000;
    static double xs[4];
    long checked = 0;
    for (int i = 0; i < n; i += 4) {
        for (int p = 0; p < 4; ++p) xs[p] = arg(i + p);
        check<4>(xs);
        check<2>(xs);
        check<2>(xs + 2);
        check<1>(xs + 3);
        checked += 4;
    }
    if (g_bad) {
        printf("pwide FAILED: %ld mismatches\n", g_bad);
        return 1;
    }
    printf("pwide ok %ld\n", checked);
    return 0;
}
