/* cusr_math.h -- portable fp64 / fp32 elementary functions.
 *
 * One implementation, compiled unchanged as C (host) and as HIP (gfx950
 * device), so an expression evaluates to the same bits on the CPU and on the
 * GPU. The fitter needs that: LM accept/reject decisions on near-ties follow
 * the last bit, and a 1-ulp difference between two math libraries is enough
 * to send a trajectory to another minimum.
 *
 * Only IEEE-exact building blocks are used: +, -, *, /, sqrt, fma (all
 * correctly rounded on both sides), rint, frexp and ldexp (exact, ldexp
 * correctly rounded where its result is subnormal), exponent bit
 * manipulation, and integer rounding by the 1.5*2^52 (1.5*2^23) shift.
 * Callers must compile with -ffp-contract=off so no other operation is fused.
 * Methods (all published):
 *   exp   Cody-Waite reduction x = k ln2 + r, |r| <= ln2/2 (ln2 split into a
 *         32-bit head and a tail), e^r = 1 + r (1 + r G(r)) with G the degree-9
 *         minimax polynomial of (e^r - 1 - r)/r^2 (fp32: degree 4), scaling by
 *         2^k with ldexp.
 *   log   x = 2^e m (frexp), m in (sqrt(1/2), sqrt(2)], f = m - 1, s = f/(2+f),
 *         log(1+f) = f - (f^2/2 - s (f^2/2 + R)) with R = z P(z), z = s^2,
 *         the atanh form rearranged as in Sun's fdlibm e_log.c; P is the
 *         degree-6 minimax polynomial of (2 atanh(s) - 2s)/(s z) (fp32: 2).
 *   sin/cos  k = rint(x 2/pi), r = x - k pi/2 with pi/2 split into three
 *         doubles subtracted by fma (Cody-Waite); on [-pi/4, pi/4]
 *         sin r = r + r^3 S(z), cos r = 1 - z/2 + z^2 C(z), z = r^2, with S and
 *         C the degree-5 minimax polynomials of their parts (fp32: 2); cos
 *         uses the compensated 1 - z/2 step of fdlibm k_cos.c; quadrant by
 *         k mod 4.
 *   The minimax coefficients come from cusr_amd/csrc/gen_minimax.py (Remez
 *         exchange at 60 digits); each polynomial's approximation error is
 *         below 0.19 x 2^-53 (fp32: 0.22 x 2^-24) relative on its range.
 *         For |x| >= 2^30 the reduction is Payne and Hanek's ("Radian
 *         reduction for trigonometric functions", SIGNUM Newsletter 18,
 *         1983): x = M 2^E, and only the 192 bits of 2/pi from weight
 *         2^-(E-1) on matter for x 2/pi mod 4, a 53 x 192-bit integer
 *         product. fp32 arguments from 2^17 are reduced in fp64.
 *   tan   sin/cos of the same reduction.
 *   sinh, cosh, tanh  Taylor series for |x| < 1 (sinh), exp otherwise.
 *   pow   integral |y| <= 64: binary powering (x^2, x^3 exact when
 *         representable); otherwise exp(y log|x|) with no extra-precision
 *         log, so the error stays below 2 (1 + |y ln x|) ulp. The sign of x
 *         is kept for odd integral y.
 * Accuracy against the C library is checked by tests/test_math.py.
 */
#ifndef CUSR_MATH_H
#define CUSR_MATH_H

#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define CM_FN static inline __host__ __device__
#else
#define CM_FN static inline
#endif

/* Coefficient tables. The device pass keeps them in constant memory, read
 * only from __device__ accessors: a __constant__ variable referenced from a
 * __host__ __device__ function is made host-visible and addressed through the
 * GOT (one more dependent scalar load per use). The accessor hands out a
 * pointer the optimizer cannot see through (an empty asm that "changes" it),
 * so each call loads its coefficients into scalar registers with scalar loads
 * instead of the compiler keeping every coefficient of every function resident
 * in vector registers for the whole kernel. Every other compile (the host pass
 * of hipcc, gcc for the oracle) sees plain static arrays of the same values. */
#if defined(__HIP_DEVICE_COMPILE__) && !defined(CUSR_MATH_FOLD_TABLES)
typedef const __attribute__((address_space(4))) double *cm_dtab;
typedef const __attribute__((address_space(4))) float *cm_ftab;
typedef const __attribute__((address_space(4))) uint64_t *cm_utab;
#define CM_TABLE static __constant__ const
#define CM_ACCESSOR(T, name)                                              \
    static __device__ __forceinline__ T name##_ptr() {                    \
        T t_ = (T)(name);                                                 \
        __asm__ volatile("" : "+s"(t_));                                  \
        return t_;                                                        \
    }
#define CM_TAB(T, name) (name##_ptr())
#else
typedef const double *cm_dtab;
typedef const float *cm_ftab;
typedef const uint64_t *cm_utab;
#if defined(__HIP_DEVICE_COMPILE__)
#define CM_TABLE static __constant__ const
#else
#define CM_TABLE static const
#endif
#define CM_ACCESSOR(T, name)
#define CM_TAB(T, name) ((T)(name))
#endif

#ifdef __cplusplus
#define CM_FMA ::fma
#define CM_FMAF ::fmaf
#define CM_SQRT ::sqrt
#define CM_SQRTF ::sqrtf
#else
#include <math.h>
#define CM_FMA fma
#define CM_FMAF fmaf
#define CM_SQRT sqrt
#define CM_SQRTF sqrtf
#endif

/* Horner step p * z + c with c a table coefficient. On the device the
 * coefficient sits in scalar registers after its scalar load; the VOP3 fma
 * takes it from there, where the compiler's two-address fmac form would first
 * copy it into a vector register pair. Same IEEE fused multiply-add. */
#if defined(__HIP_DEVICE_COMPILE__)
static __device__ __forceinline__ double cm_fma_sd(double a, double b, double c) {
    double r;
    __asm__("v_fma_f64 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(c));
    return r;
}
static __device__ __forceinline__ float cm_fma_sf(float a, float b, float c) {
    float r;
    __asm__("v_fma_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(c));
    return r;
}
#define CM_HORNER(p, z, c) cm_fma_sd((p), (z), (c))
#define CM_HORNERF(p, z, c) cm_fma_sf((p), (z), (c))
#else
#define CM_HORNER(p, z, c) CM_FMA((p), (z), (c))
#define CM_HORNERF(p, z, c) CM_FMAF((p), (z), (c))
#endif

/* ------------------------------------------------------------ bit helpers */

CM_FN uint64_t cm_bits(double x) { uint64_t u; __builtin_memcpy(&u, &x, 8); return u; }
CM_FN double cm_dbl(uint64_t u) { double x; __builtin_memcpy(&x, &u, 8); return x; }
CM_FN uint32_t cm_bitsf(float x) { uint32_t u; __builtin_memcpy(&u, &x, 4); return u; }
CM_FN float cm_flt(uint32_t u) { float x; __builtin_memcpy(&x, &u, 4); return x; }

#define CM_NAN cm_dbl(0x7ff8000000000000ULL)
#define CM_INF cm_dbl(0x7ff0000000000000ULL)
#define CM_NANF cm_flt(0x7fc00000u)
#define CM_INFF cm_flt(0x7f800000u)

CM_FN int cm_isnan(double x) { return x != x; }
CM_FN double cm_fabs(double x) { return cm_dbl(cm_bits(x) & 0x7fffffffffffffffULL); }
CM_FN float cm_fabsf(float x) { return cm_flt(cm_bitsf(x) & 0x7fffffffu); }

/* nearest integer (ties to even) of |t| < 2^51, as a double */
CM_FN double cm_rint_small(double t) {
    const double shift = 6755399441055744.0; /* 1.5 * 2^52 */
    double v = t + shift;
    return v - shift;
}
CM_FN float cm_rint_smallf(float t) {
    const float shift = 12582912.0f; /* 1.5 * 2^23 */
    float v = t + shift;
    return v - shift;
}

/* rint (ties to even), x 2^k and frexp: the hardware's v_rndne, v_ldexp and
 * v_frexp_mant / v_frexp_exp on the device, the C library's on the host; each
 * is exact (ldexp rounds once where the result is subnormal), so both sides
 * get the same bits. */
#define CM_RINT(x) __builtin_rint(x)
#define CM_LDEXP(x, k) __builtin_ldexp((x), (k))
#define CM_LDEXPF(x, k) __builtin_ldexpf((x), (k))
#define CM_FREXP(x, e) __builtin_frexp((x), (e))
#define CM_FREXPF(x, e) __builtin_frexpf((x), (e))

/* ------------------------------------------------------------------- exp */

/* 1/ln2, ln2 head (32 bits), ln2 tail, then G(r) highest degree first
 * (gen_minimax.py), then 1, 1: Horner over entries 3.. gives 1 + r (1 + r G) */
#define CM_EXP_N 15
CM_TABLE double cm_exp_tab[CM_EXP_N] = {
    1.4426950408889634, 0.6931471803691238, 1.9082149288430703e-10,
    2.5110039143068074e-08, 2.762007695623653e-07, 2.7557242364947015e-06,
    2.480152131981927e-05, 0.00019841269886566317, 0.0013888888917198605,
    0.008333333333322215, 0.04166666666662416, 0.16666666666666674,
    0.5000000000000001, 1.0, 1.0};
CM_ACCESSOR(cm_dtab, cm_exp_tab)

/* |x| at most this: no overflow, underflow or NaN, so no final select */
#define CM_EXP_PLAIN 709.782712893384
#define CM_EXP_LO -745.1332191019412

CM_FN double cm_exp(double x) {
    /* branch-free: out-of-range and NaN arguments reduce 0 and are selected
     * at the end */
    const int nan = cm_isnan(x);
    const int hi = x > CM_EXP_PLAIN;
    const int lo = x < CM_EXP_LO;
    const double xr = (nan || hi || lo) ? 0.0 : x;
    cm_dtab t = CM_TAB(cm_dtab, cm_exp_tab);
    double kf = CM_RINT(xr * t[0]);
    double r = CM_FMA(-kf, t[1], xr);
    r = CM_FMA(-kf, t[2], r);
    double p = t[3];
    for (int i = 4; i < CM_EXP_N; i++) p = CM_HORNER(p, r, t[i]);
    const double res = CM_LDEXP(p, (int)kf);
    return nan ? x : (hi ? CM_INF : (lo ? 0.0 : res));
}

/* 1/ln2, ln2 head (16 bits), ln2 tail, then G(r) highest degree first
 * (gen_minimax.py), then 1, 1 */
#define CM_EXPF_N 10
CM_TABLE float cm_expf_tab[CM_EXPF_N] = {
    1.4426950216293335f, 0.693145751953125f, 1.4285906217992306e-06f,
    0.0013942165533080697f, 0.008363775908946991f, 0.041666362434625626f,
    0.16666573286056519f, 0.5f, 1.0f, 1.0f};
CM_ACCESSOR(cm_ftab, cm_expf_tab)

#define CM_EXPF_PLAIN 88.72283f
#define CM_EXPF_LO -103.97208f

CM_FN float cm_expf(float x) {
    const int nan = x != x;
    const int hi = x > CM_EXPF_PLAIN;
    const int lo = x < CM_EXPF_LO;
    const float xr = (nan || hi || lo) ? 0.0f : x;
    cm_ftab t = CM_TAB(cm_ftab, cm_expf_tab);
    float kf = cm_rint_smallf(xr * t[0]);
    float r = CM_FMAF(-kf, t[1], xr);
    r = CM_FMAF(-kf, t[2], r);
    float p = t[3];
    for (int i = 4; i < CM_EXPF_N; i++) p = CM_HORNERF(p, r, t[i]);
    const float res = CM_LDEXPF(p, (int)kf);
    return nan ? x : (hi ? CM_INFF : (lo ? 0.0f : res));
}

/* ------------------------------------------------------------------- log */

/* P(z) highest degree first (gen_minimax.py), then ln2 head and tail */
#define CM_LOG_P 7
CM_TABLE double cm_log_tab[CM_LOG_P + 2] = {
    0.1461773941368345, 0.15331607753678703, 0.1818289289358215, 0.22222211077310847,
    0.28571428626371803, 0.39999999999898506, 0.666666666666667,
    0.6931471803691238, 1.9082149288430703e-10};
CM_ACCESSOR(cm_dtab, cm_log_tab)

CM_FN double cm_log(double x) {
    /* branch-free: NaN, negative, zero and +inf arguments are selected at the
     * end; frexp's m in [1/2, 1) is doubled below sqrt(1/2) */
    int e;
    double m = CM_FREXP(x, &e);
    const int dn = m <= 0.7071067811865476;
    m = dn ? m + m : m;
    e = dn ? e - 1 : e;
    double f = m - 1.0;
    double s = f / (2.0 + f);
    double z = s * s;
    cm_dtab t = CM_TAB(cm_dtab, cm_log_tab);
    double R = t[0];
    for (int i = 1; i < CM_LOG_P; i++) R = CM_HORNER(R, z, t[i]);
    R = R * z;
    double hfsq = 0.5 * (f * f);
    double dk = (double)e;
    double res = dk * t[CM_LOG_P] - ((hfsq - (s * (hfsq + R) + dk * t[CM_LOG_P + 1])) - f);
    return cm_isnan(x) ? x : (x < 0.0 ? CM_NAN : (x == 0.0 ? -CM_INF : (x == CM_INF ? x : res)));
}

/* P(z) highest degree first (gen_minimax.py), then ln2 head and tail */
#define CM_LOGF_P 3
CM_TABLE float cm_logf_tab[CM_LOGF_P + 2] = {
    0.29602980613708496f, 0.3998825252056122f, 0.6666668653488159f,
    0.693145751953125f, 1.4285906217992306e-06f};
CM_ACCESSOR(cm_ftab, cm_logf_tab)

CM_FN float cm_logf(float x) {
    int e;
    float m = CM_FREXPF(x, &e);
    const int dn = m <= 0.70710676908493042f;
    m = dn ? m + m : m;
    e = dn ? e - 1 : e;
    float f = m - 1.0f;
    float s = f / (2.0f + f);
    float z = s * s;
    cm_ftab t = CM_TAB(cm_ftab, cm_logf_tab);
    float R = t[0];
    for (int i = 1; i < CM_LOGF_P; i++) R = CM_HORNERF(R, z, t[i]);
    R = R * z;
    float hfsq = 0.5f * (f * f);
    float dk = (float)e;
    float res = dk * t[CM_LOGF_P] - ((hfsq - (s * (hfsq + R) + dk * t[CM_LOGF_P + 1])) - f);
    return (x != x) ? x : (x < 0.0f ? CM_NANF : (x == 0.0f ? -CM_INFF : (x == CM_INFF ? x : res)));
}

/* --------------------------------------------------------------- sin/cos */

/* S(z), then C(z), each highest degree first (gen_minimax.py); then 2/pi
 * and pi/2 as three doubles */
#define CM_TRIG_S 0
#define CM_TRIG_C 6
#define CM_TRIG_N 6
#define CM_TRIG_2PI 12
#define CM_TRIG_PIO2 13
CM_TABLE double cm_trig_tab[16] = {
    1.591814230329288e-10, -2.505113204602621e-08, 2.75573161036397e-06,
    -0.00019841269836760975, 0.00833333333333095, -0.16666666666666666,
    -1.1382639639006937e-11, 2.087614637990424e-09, -2.755731727233302e-07,
    2.480158729876702e-05, -0.0013888888888887398, 0.041666666666666664,
    0.6366197723675814, 1.5707963267948966, 6.123233995736766e-17, -1.4973849048591698e-33};
CM_ACCESSOR(cm_dtab, cm_trig_tab)

CM_FN double cm_sin_kernel(double r, cm_dtab t) {
    double z = r * r;
    double p = t[CM_TRIG_S];
    for (int i = 1; i < CM_TRIG_N; i++) p = CM_HORNER(p, z, t[CM_TRIG_S + i]);
    return CM_FMA(r * z, p, r);
}

CM_FN double cm_cos_kernel(double r, cm_dtab t) {
    double z = r * r;
    double p = t[CM_TRIG_C];
    for (int i = 1; i < CM_TRIG_N; i++) p = CM_HORNER(p, z, t[CM_TRIG_C + i]);
    double hz = 0.5 * z;
    double w = 1.0 - hz;
    return w + (((1.0 - w) - hz) + z * (z * p));
}

/* The bits of 2/pi (cusr_amd/csrc/gen_two_over_pi.py, exact integer
 * arithmetic): word 0 is zero, word j >= 1 holds the bits of weight
 * 2^-(64(j-1)+1) .. 2^-64j, most significant first. */
CM_TABLE uint64_t cm_two_over_pi[24] = {
    0x0000000000000000ull, 0xA2F9836E4E441529ull, 0xFC2757D1F534DDC0ull,
    0xDB6295993C439041ull, 0xFE5163ABDEBBC561ull, 0xB7246E3A424DD2E0ull,
    0x06492EEA09D1921Cull, 0xFE1DEB1CB129A73Eull, 0xE88235F52EBB4484ull,
    0xE99C7026B45F7E41ull, 0x3991D639835339F4ull, 0x9C845F8BBDF9283Bull,
    0x1FF897FFDE05980Full, 0xEF2F118B5A0A6D1Full, 0x6D367ECF27CB09B7ull,
    0x4F463F669E5FEA2Dull, 0x7527BAC7EBE5F17Bull, 0x3D0739F78A5292EAull,
    0x6BFB5FB11F8D5D08ull, 0x56033046FC7B6BABull, 0xF0CFBC209AF4361Dull,
    0xA9E391615EE61B08ull, 0x6599855F14A06840ull, 0x8DFFD8804D732731ull,
};
CM_ACCESSOR(cm_utab, cm_two_over_pi)

/* Arguments reduced by Payne-Hanek (fp64) and fp32 arguments reduced in fp64.
 * Below them the Cody-Waite quotient k = rint(x 2/pi) is formed from x 2/pi
 * rounded once: below 2^30 its ulp is at most 2^-23, so the remainder
 * exceeds pi/4 by at most 2^-24 pi/2, inside the range the polynomials are
 * fitted on (widened by 2^-20); in fp32 below 2^17 by at most 2^-8 pi/2
 * (fitted on a range widened by 1 %). */
#define CM_PH_MIN 1073741824.0      /* 2^30 */
#define CM_F64_RED_MINF 131072.0f   /* 2^17 */

/* Payne-Hanek reduction of a finite ax >= 2^30: returns r with |r| <= pi/4
 * and sets *q so that ax = (4n + *q) pi/2 + r. ax = M 2^E with M the 53-bit
 * integer significand (E >= -22). Bits of 2/pi of weight 2^-i with i <= E - 2
 * add multiples of 4 to ax 2/pi; the 192 bits W from weight 2^-(E-1) on give
 * ax 2/pi = M W 2^-190 (mod 4) with an error below 2^-137. Bits 190..191 of
 * the product are the quadrant, the 128 below the fraction; a fraction
 * >= 1/2 rounds the quadrant up and turns negative. The fraction goes to
 * double-double and is multiplied by pi/2 (two doubles) with one fma for
 * the product's rounding error. Integer steps are exact, so host and device
 * agree to the bit. */
CM_FN double cm_rem_pio2_huge(double ax, int *q, cm_dtab t) {
    const uint64_t b = cm_bits(ax);
    const int E = (int)((b >> 52) & 0x7ff) - 1075;
    const uint64_t M = (b & 0xfffffffffffffull) | 0x10000000000000ull;
    cm_utab w = CM_TAB(cm_utab, cm_two_over_pi);
    const int bit = E + 62;                     /* stream position of weight 2^-(E-1) */
    const int j = bit >> 6, sh = bit & 63;
    const uint64_t a0 = w[j], a1 = w[j + 1], a2 = w[j + 2], a3 = w[j + 3];
    const uint64_t w2 = sh ? (a0 << sh) | (a1 >> (64 - sh)) : a0;
    const uint64_t w1 = sh ? (a1 << sh) | (a2 >> (64 - sh)) : a1;
    const uint64_t w0 = sh ? (a2 << sh) | (a3 >> (64 - sh)) : a2;
    typedef unsigned __int128 u128;
    const u128 p0 = (u128)M * w0, p1 = (u128)M * w1, p2 = (u128)M * w2;
    const uint64_t lo = (uint64_t)p0;
    const u128 t1 = (p0 >> 64) + (u128)(uint64_t)p1;
    const uint64_t mid = (uint64_t)t1;
    const uint64_t hi = (uint64_t)(t1 >> 64) + (uint64_t)(p1 >> 64) + (uint64_t)p2;
    const u128 g = ((u128)hi << 66) | ((u128)mid << 2) | (u128)(lo >> 62);
    *q = (int)((hi >> 62) + (uint64_t)(g >> 127)) & 3;
    const int64_t gh = (int64_t)(uint64_t)(g >> 64);   /* signed fraction, 2^-64 units */
    const double fh = (double)gh;
    const double fl = (double)(gh - (int64_t)fh) + (double)(uint64_t)g * 5.421010862427522e-20;
    const double a = fh * 5.421010862427522e-20, bq = fl * 5.421010862427522e-20; /* 2^-64 */
    const double rh = a * t[CM_TRIG_PIO2];
    const double rl = CM_FMA(a, t[CM_TRIG_PIO2], -rh) +
                      CM_FMA(a, t[CM_TRIG_PIO2 + 1], bq * t[CM_TRIG_PIO2]);
    return rh + rl;
}

/* x - k pi/2 with k = rint(x 2/pi) for |x| < 2^30 (Cody-Waite, pi/2 in three
 * doubles subtracted by fma); *q = k mod 4. */
CM_FN double cm_rem_pio2_cw(double x, int *q, cm_dtab t) {
    double kf = cm_rint_small(x * t[CM_TRIG_2PI]);
    double r = CM_FMA(-kf, t[CM_TRIG_PIO2], x);
    r = CM_FMA(-kf, t[CM_TRIG_PIO2 + 1], r);
    r = CM_FMA(-kf, t[CM_TRIG_PIO2 + 2], r);
    *q = (int)kf & 3;                           /* kf mod 4, |kf| < 2^30 */
    return r;
}

/* sin and cos of x from one argument reduction: NaN and +-inf give NaN
 * (through the reduction of 0 and a final select); |x| >= 2^30 takes the
 * Payne-Hanek reduction; the quadrant swaps and negates. */
CM_FN void cm_sincos(double x, double *s, double *c) {
    const double ax = cm_fabs(x);
    const int bad = !(ax < CM_INF);
    const int huge = !bad && ax >= CM_PH_MIN;
    const double xr = (bad || huge) ? 0.0 : x;
    cm_dtab t = CM_TAB(cm_dtab, cm_trig_tab);
    int q;
    double r = cm_rem_pio2_cw(xr, &q, t);
    if (huge) {
        int qh;
        const double rh = cm_rem_pio2_huge(ax, &qh, t);
        r = x < 0.0 ? -rh : rh;
        q = (x < 0.0 ? -qh : qh) & 3;
    }
    double sr = cm_sin_kernel(r, t), cr = cm_cos_kernel(r, t);
    double so = (q & 1) ? cr : sr;
    double co = (q & 1) ? sr : cr;
    so = (q & 2) ? -so : so;
    co = ((q + 1) & 2) ? -co : co;
    *s = bad ? CM_NAN : so;
    *c = bad ? CM_NAN : co;
}

CM_FN double cm_sin(double x) { double s, c; cm_sincos(x, &s, &c); return s; }
CM_FN double cm_cos(double x) { double s, c; cm_sincos(x, &s, &c); return c; }
CM_FN double cm_tan(double x) { double s, c; cm_sincos(x, &s, &c); return s / c; }

/* S(z), then C(z), each highest degree first (gen_minimax.py); then 2/pi
 * and pi/2 as three floats */
#define CM_TRIGF_S 0
#define CM_TRIGF_C 3
#define CM_TRIGF_N 3
#define CM_TRIGF_2PI 6
#define CM_TRIGF_PIO2 7
CM_TABLE float cm_trigf_tab[10] = {
    -0.00019582953245844692f, 0.008332725614309311f, -0.166666641831398f,
    2.4542972823837772e-05f, -0.0013888280373066664f, 0.0416666641831398f,
    0.6366197466850281f, 1.5707963705062866f, -4.371138828673793e-08f, -1.7151245100058819e-15f};
CM_ACCESSOR(cm_ftab, cm_trigf_tab)

CM_FN float cm_sin_kernelf(float r, cm_ftab t) {
    float z = r * r;
    float p = t[CM_TRIGF_S];
    for (int i = 1; i < CM_TRIGF_N; i++) p = CM_HORNERF(p, z, t[CM_TRIGF_S + i]);
    return CM_FMAF(r * z, p, r);
}

CM_FN float cm_cos_kernelf(float r, cm_ftab t) {
    float z = r * r;
    float p = t[CM_TRIGF_C];
    for (int i = 1; i < CM_TRIGF_N; i++) p = CM_HORNERF(p, z, t[CM_TRIGF_C + i]);
    float hz = 0.5f * z;
    float w = 1.0f - hz;
    return w + (((1.0f - w) - hz) + z * (z * p));
}

/* fp32 sin and cos; arguments from 2^17 on are reduced in fp64 (exact
 * widening, then the fp64 reduction) and the reduced argument rounded to
 * fp32. */
CM_FN void cm_sincosf(float x, float *s, float *c) {
    const float ax = cm_fabsf(x);
    const int bad = !(ax < CM_INFF);
    const int huge = !bad && ax >= CM_F64_RED_MINF;
    const float xr = (bad || huge) ? 0.0f : x;
    cm_ftab t = CM_TAB(cm_ftab, cm_trigf_tab);
    float kf = cm_rint_smallf(xr * t[CM_TRIGF_2PI]);
    float r = CM_FMAF(-kf, t[CM_TRIGF_PIO2], xr);
    r = CM_FMAF(-kf, t[CM_TRIGF_PIO2 + 1], r);
    r = CM_FMAF(-kf, t[CM_TRIGF_PIO2 + 2], r);
    int q = (int)kf & 3;
    if (huge) {
        cm_dtab td = CM_TAB(cm_dtab, cm_trig_tab);
        const double axd = (double)ax;
        int qh;
        const double rd = axd >= CM_PH_MIN ? cm_rem_pio2_huge(axd, &qh, td)
                                                    : cm_rem_pio2_cw(axd, &qh, td);
        r = (float)(x < 0.0f ? -rd : rd);
        q = (x < 0.0f ? -qh : qh) & 3;
    }
    float sr = cm_sin_kernelf(r, t), cr = cm_cos_kernelf(r, t);
    float so = (q & 1) ? cr : sr;
    float co = (q & 1) ? sr : cr;
    so = (q & 2) ? -so : so;
    co = ((q + 1) & 2) ? -co : co;
    *s = bad ? CM_NANF : so;
    *c = bad ? CM_NANF : co;
}

CM_FN float cm_sinf(float x) { float s, c; cm_sincosf(x, &s, &c); return s; }
CM_FN float cm_cosf(float x) { float s, c; cm_sincosf(x, &s, &c); return c; }
CM_FN float cm_tanf(float x) { float s, c; cm_sincosf(x, &s, &c); return s / c; }

/* ----------------------------------------------- P-wide forms (HIP only) */

/* The interpreter evaluates an operator for P points per lane at once. These
 * forms give each of the P elements the bits of the scalar function (cm_exp,
 * cm_log, cm_sincos, cm_expf, cm_logf, cm_sincosf), interleaved statement by
 * statement: the P polynomial chains are independent, and the coefficient
 * table is loaded once for the P elements instead of once per element. When
 * every argument of the wavefront is ordinary (a finite argument of exp that
 * neither overflows nor underflows, a positive finite argument of log, a
 * trigonometric argument below the Payne-Hanek range) one uniform branch skips
 * the special-value selects, which then would pass every value through
 * unchanged; otherwise the wavefront runs the operations of the scalar
 * function with its selects. */
#if defined(__cplusplus) && (defined(__HIPCC__) || defined(__HIP__))
#define CM_FORP _Pragma("unroll") for (int p = 0; p < P; ++p)
#if defined(__HIP_DEVICE_COMPILE__)
#define CM_ANY(v) (__builtin_amdgcn_ballot_w64((v) != 0) != 0)
#else
#define CM_ANY(v) ((v) != 0)
#endif

template <int P>
CM_FN void cm_exp_v(const double *x, double *res) {
    int odd = 0;
    CM_FORP odd |= !(cm_fabs(x[p]) <= CM_EXP_PLAIN);
    if (CM_ANY(odd)) {
        CM_FORP res[p] = cm_exp(x[p]);
        return;
    }
    cm_dtab t = CM_TAB(cm_dtab, cm_exp_tab);
    double kf[P], r[P], q[P];
    CM_FORP {
        kf[p] = CM_RINT(x[p] * t[0]);
        r[p] = CM_FMA(-kf[p], t[1], x[p]);
        r[p] = CM_FMA(-kf[p], t[2], r[p]);
        q[p] = t[3];
    }
    _Pragma("unroll") for (int i = 4; i < CM_EXP_N; i++) CM_FORP q[p] = CM_HORNER(q[p], r[p], t[i]);
    CM_FORP res[p] = CM_LDEXP(q[p], (int)kf[p]);
}

template <int P>
CM_FN void cm_log_v(const double *x, double *res) {
    int odd = 0;
    CM_FORP odd |= !(x[p] > 0.0 && x[p] < CM_INF);
    if (CM_ANY(odd)) {
        CM_FORP res[p] = cm_log(x[p]);
        return;
    }
    double f[P], s[P], z[P], R[P], dk[P];
    CM_FORP {
        int e;
        double m = CM_FREXP(x[p], &e);
        const int dn = m <= 0.7071067811865476;
        m = dn ? m + m : m;
        e = dn ? e - 1 : e;
        f[p] = m - 1.0;
        s[p] = f[p] / (2.0 + f[p]);
        z[p] = s[p] * s[p];
        dk[p] = (double)e;
    }
    cm_dtab t = CM_TAB(cm_dtab, cm_log_tab);
    CM_FORP R[p] = t[0];
    _Pragma("unroll") for (int i = 1; i < CM_LOG_P; i++) CM_FORP R[p] = CM_HORNER(R[p], z[p], t[i]);
    CM_FORP {
        const double Rz = R[p] * z[p];
        const double hfsq = 0.5 * (f[p] * f[p]);
        res[p] = dk[p] * t[CM_LOG_P] -
                 ((hfsq - (s[p] * (hfsq + Rz) + dk[p] * t[CM_LOG_P + 1])) - f[p]);
    }
}

template <int P>
CM_FN void cm_sincos_v(const double *x, double *so, double *co) {
    int odd = 0;
    CM_FORP odd |= !(cm_fabs(x[p]) < CM_PH_MIN);
    if (CM_ANY(odd)) {
        CM_FORP cm_sincos(x[p], &so[p], &co[p]);
        return;
    }
    cm_dtab t = CM_TAB(cm_dtab, cm_trig_tab);
    int q[P];
    double r[P], z[P], ps[P], pc[P];
    CM_FORP r[p] = cm_rem_pio2_cw(x[p], &q[p], t);
    CM_FORP {
        z[p] = r[p] * r[p];
        ps[p] = t[CM_TRIG_S];
        pc[p] = t[CM_TRIG_C];
    }
    _Pragma("unroll") for (int i = 1; i < CM_TRIG_N; i++) CM_FORP {
        ps[p] = CM_HORNER(ps[p], z[p], t[CM_TRIG_S + i]);
        pc[p] = CM_HORNER(pc[p], z[p], t[CM_TRIG_C + i]);
    }
    CM_FORP {
        const double sr = CM_FMA(r[p] * z[p], ps[p], r[p]);
        const double hz = 0.5 * z[p];
        const double w = 1.0 - hz;
        const double cr = w + (((1.0 - w) - hz) + z[p] * (z[p] * pc[p]));
        const double sv = (q[p] & 1) ? cr : sr;
        const double cv = (q[p] & 1) ? sr : cr;
        so[p] = (q[p] & 2) ? -sv : sv;
        co[p] = ((q[p] + 1) & 2) ? -cv : cv;
    }
}

template <int P>
CM_FN void cm_expf_v(const float *x, float *res) {
    int odd = 0;
    CM_FORP odd |= !(cm_fabsf(x[p]) <= CM_EXPF_PLAIN);
    if (CM_ANY(odd)) {
        CM_FORP res[p] = cm_expf(x[p]);
        return;
    }
    cm_ftab t = CM_TAB(cm_ftab, cm_expf_tab);
    float kf[P], r[P], q[P];
    CM_FORP {
        kf[p] = cm_rint_smallf(x[p] * t[0]);
        r[p] = CM_FMAF(-kf[p], t[1], x[p]);
        r[p] = CM_FMAF(-kf[p], t[2], r[p]);
        q[p] = t[3];
    }
    _Pragma("unroll") for (int i = 4; i < CM_EXPF_N; i++) CM_FORP q[p] = CM_HORNERF(q[p], r[p], t[i]);
    CM_FORP res[p] = CM_LDEXPF(q[p], (int)kf[p]);
}

template <int P>
CM_FN void cm_logf_v(const float *x, float *res) {
    int odd = 0;
    CM_FORP odd |= !(x[p] > 0.0f && x[p] < CM_INFF);
    if (CM_ANY(odd)) {
        CM_FORP res[p] = cm_logf(x[p]);
        return;
    }
    float f[P], s[P], z[P], R[P], dk[P];
    CM_FORP {
        int e;
        float m = CM_FREXPF(x[p], &e);
        const int dn = m <= 0.70710676908493042f;
        m = dn ? m + m : m;
        e = dn ? e - 1 : e;
        f[p] = m - 1.0f;
        s[p] = f[p] / (2.0f + f[p]);
        z[p] = s[p] * s[p];
        dk[p] = (float)e;
    }
    cm_ftab t = CM_TAB(cm_ftab, cm_logf_tab);
    CM_FORP R[p] = t[0];
    _Pragma("unroll") for (int i = 1; i < CM_LOGF_P; i++) CM_FORP R[p] = CM_HORNERF(R[p], z[p], t[i]);
    CM_FORP {
        const float Rz = R[p] * z[p];
        const float hfsq = 0.5f * (f[p] * f[p]);
        res[p] = dk[p] * t[CM_LOGF_P] -
                 ((hfsq - (s[p] * (hfsq + Rz) + dk[p] * t[CM_LOGF_P + 1])) - f[p]);
    }
}

template <int P>
CM_FN void cm_sincosf_v(const float *x, float *so, float *co) {
    int odd = 0;
    CM_FORP odd |= !(cm_fabsf(x[p]) < CM_F64_RED_MINF);
    if (CM_ANY(odd)) {
        CM_FORP cm_sincosf(x[p], &so[p], &co[p]);
        return;
    }
    cm_ftab t = CM_TAB(cm_ftab, cm_trigf_tab);
    int q[P];
    float r[P], z[P], ps[P], pc[P];
    CM_FORP {
        const float kf = cm_rint_smallf(x[p] * t[CM_TRIGF_2PI]);
        float rr = CM_FMAF(-kf, t[CM_TRIGF_PIO2], x[p]);
        rr = CM_FMAF(-kf, t[CM_TRIGF_PIO2 + 1], rr);
        r[p] = CM_FMAF(-kf, t[CM_TRIGF_PIO2 + 2], rr);
        q[p] = (int)kf & 3;
    }
    CM_FORP {
        z[p] = r[p] * r[p];
        ps[p] = t[CM_TRIGF_S];
        pc[p] = t[CM_TRIGF_C];
    }
    _Pragma("unroll") for (int i = 1; i < CM_TRIGF_N; i++) CM_FORP {
        ps[p] = CM_HORNERF(ps[p], z[p], t[CM_TRIGF_S + i]);
        pc[p] = CM_HORNERF(pc[p], z[p], t[CM_TRIGF_C + i]);
    }
    CM_FORP {
        const float sr = CM_FMAF(r[p] * z[p], ps[p], r[p]);
        const float hz = 0.5f * z[p];
        const float w = 1.0f - hz;
        const float cr = w + (((1.0f - w) - hz) + z[p] * (z[p] * pc[p]));
        const float sv = (q[p] & 1) ? cr : sr;
        const float cv = (q[p] & 1) ? sr : cr;
        so[p] = (q[p] & 2) ? -sv : sv;
        co[p] = ((q[p] + 1) & 2) ? -cv : cv;
    }
}
#undef CM_FORP
#undef CM_ANY
#endif

/* ------------------------------------------------------ hyperbolic, pow */

/* 1/19!, 1/17!, ..., 1/3! */
CM_TABLE double cm_sinh_tab[9] = {
    8.22063524662433e-18, 2.8114572543455206e-15, 7.647163731819816e-13,
    1.6059043836821613e-10, 2.505210838544172e-08, 2.7557319223985893e-06,
    0.0001984126984126984, 0.008333333333333333, 0.16666666666666666};
CM_ACCESSOR(cm_dtab, cm_sinh_tab)

CM_FN double cm_sinh(double x) {
    if (cm_isnan(x)) return x;
    double a = cm_fabs(x);
    double r;
    if (a < 1.0) {
        cm_dtab t = CM_TAB(cm_dtab, cm_sinh_tab);
        double z = a * a;
        double p = t[0];
        for (int i = 1; i < 9; i++) p = CM_HORNER(p, z, t[i]);
        r = CM_FMA(a * z, p, a);
    } else if (a < 709.0) {
        double e = cm_exp(a);
        r = 0.5 * (e - 1.0 / e);
    } else {
        r = 2.0 * cm_exp(a - 1.3862943611198906); /* e^a / 2 = 2 e^(a - 2 ln 2) */
    }
    return x < 0.0 ? -r : r;
}

CM_FN double cm_cosh(double x) {
    if (cm_isnan(x)) return x;
    double a = cm_fabs(x);
    if (a < 709.0) {
        double e = cm_exp(a);
        return 0.5 * (e + 1.0 / e);
    }
    return 2.0 * cm_exp(a - 1.3862943611198906);
}

CM_FN double cm_tanh(double x) {
    if (cm_isnan(x)) return x;
    double a = cm_fabs(x);
    double r;
    if (a < 0.55) {
        r = cm_sinh(a) / cm_cosh(a);
    } else if (a < 22.0) {
        double e = cm_exp(2.0 * a);
        r = 1.0 - 2.0 / (e + 1.0);
    } else {
        r = 1.0;
    }
    return x < 0.0 ? -r : r;
}

/* 1/11!, ..., 1/3! */
CM_TABLE float cm_sinhf_tab[5] = {
    2.5052107943679403e-08f, 2.7557318844628753e-06f, 0.00019841270113829523f,
    0.008333333767950535f, 0.1666666716337204f};
CM_ACCESSOR(cm_ftab, cm_sinhf_tab)

CM_FN float cm_sinhf(float x) {
    if (x != x) return x;
    float a = cm_fabsf(x);
    float r;
    if (a < 1.0f) {
        cm_ftab t = CM_TAB(cm_ftab, cm_sinhf_tab);
        float z = a * a;
        float p = t[0];
        for (int i = 1; i < 5; i++) p = CM_HORNERF(p, z, t[i]);
        r = CM_FMAF(a * z, p, a);
    } else if (a < 88.0f) {
        float e = cm_expf(a);
        r = 0.5f * (e - 1.0f / e);
    } else {
        r = 2.0f * cm_expf(a - 1.3862943611198906f);
    }
    return x < 0.0f ? -r : r;
}

CM_FN float cm_coshf(float x) {
    if (x != x) return x;
    float a = cm_fabsf(x);
    if (a < 88.0f) {
        float e = cm_expf(a);
        return 0.5f * (e + 1.0f / e);
    }
    return 2.0f * cm_expf(a - 1.3862943611198906f);
}

CM_FN float cm_tanhf(float x) {
    if (x != x) return x;
    float a = cm_fabsf(x);
    float r;
    if (a < 0.55f) {
        r = cm_sinhf(a) / cm_coshf(a);
    } else if (a < 9.0f) {
        float e = cm_expf(2.0f * a);
        r = 1.0f - 2.0f / (e + 1.0f);
    } else {
        r = 1.0f;
    }
    return x < 0.0f ? -r : r;
}

/* is y an integer, and if so is it odd */
CM_FN int cm_int_kind(double y) {
    double a = cm_fabs(y);
    if (a >= 9007199254740992.0) return 2;     /* 2^53: even integer */
    double t = cm_rint_small(a);
    if (t != a) return 0;                      /* not an integer */
    double h = cm_rint_small(a * 0.5);
    return (h * 2.0 == a) ? 2 : 1;             /* 2 even, 1 odd */
}

CM_FN double cm_pow(double x, double y) {
    if (y == 0.0) return 1.0;
    if (x == 1.0) return 1.0;
    if (cm_isnan(x) || cm_isnan(y)) return CM_NAN;
    int kind = cm_int_kind(y);
    double ax = cm_fabs(x);
    double sign = 1.0;
    if (x < 0.0 || (x == 0.0 && (cm_bits(x) >> 63))) {
        if (x != 0.0 && kind == 0) return CM_NAN;
        if (kind == 1) sign = -1.0;
    }
    if (ax == 0.0) return (y < 0.0) ? sign * CM_INF : sign * 0.0;
    if (ax == CM_INF) return (y < 0.0) ? sign * 0.0 : sign * CM_INF;
    if (y == CM_INF) return (ax < 1.0) ? 0.0 : CM_INF;
    if (y == -CM_INF) return (ax < 1.0) ? CM_INF : 0.0;
    if (kind != 0 && cm_fabs(y) <= 64.0) {
        /* small integral exponent: binary powering, exact when the result is
         * representable in a few products (x^2, x^3, ...) */
        int n = (int)cm_fabs(y);
        double b = ax, r = 1.0;
        while (n) {
            if (n & 1) r = r * b;
            b = b * b;
            n >>= 1;
        }
        return sign * ((y < 0.0) ? 1.0 / r : r);
    }
    return sign * cm_exp(y * cm_log(ax));
}

CM_FN int cm_int_kindf(float y) {
    float a = cm_fabsf(y);
    if (a >= 16777216.0f) return 2;
    float t = cm_rint_smallf(a);
    if (t != a) return 0;
    float h = cm_rint_smallf(a * 0.5f);
    return (h * 2.0f == a) ? 2 : 1;
}

CM_FN float cm_powf(float x, float y) {
    if (y == 0.0f) return 1.0f;
    if (x == 1.0f) return 1.0f;
    if (x != x || y != y) return CM_NANF;
    int kind = cm_int_kindf(y);
    float ax = cm_fabsf(x);
    float sign = 1.0f;
    if (x < 0.0f || (x == 0.0f && (cm_bitsf(x) >> 31))) {
        if (x != 0.0f && kind == 0) return CM_NANF;
        if (kind == 1) sign = -1.0f;
    }
    if (ax == 0.0f) return (y < 0.0f) ? sign * CM_INFF : sign * 0.0f;
    if (ax == CM_INFF) return (y < 0.0f) ? sign * 0.0f : sign * CM_INFF;
    if (y == CM_INFF) return (ax < 1.0f) ? 0.0f : CM_INFF;
    if (y == -CM_INFF) return (ax < 1.0f) ? CM_INFF : 0.0f;
    if (kind != 0 && cm_fabsf(y) <= 64.0f) {
        int n = (int)cm_fabsf(y);
        float b = ax, r = 1.0f;
        while (n) {
            if (n & 1) r = r * b;
            b = b * b;
            n >>= 1;
        }
        return sign * ((y < 0.0f) ? 1.0f / r : r);
    }
    return sign * cm_expf(y * cm_logf(ax));
}

#endif /* CUSR_MATH_H */
