// lm_device.h -- gfx950 kernels of the batched Levenberg-Marquardt fitter.
//
// One 64-lane wavefront owns one expression for the whole fit
// (cusr/kernel/batch_lm_ad.cu:350-495 runs one host loop over all trees
// instead). Lane l evaluates points l, l+64, l+128, ... of the expression;
// the opcode stream is wave-uniform, so every branch of the interpreter is a
// scalar branch and all 64 lanes stay converged. Per point a lane computes the
// value and the gradient row, and folds r^2, J^T r and the upper triangle of
// J^T J into registers; a butterfly over the 64 lanes then gives every lane
// the same sums, and every lane solves the same damped K x K system, so the
// accept/reject and lambda update run on the device with no host round trip.
//
// Arithmetic follows one fixed order, which the CPU oracle reproduces:
//   * lane l sums its points in ascending order from 0.0, fma(a, b, acc);
//   * lanes combine with strides 32, 16, 8, 4, 2, 1;
//   * operator values and partials use the formulas of op_unary/op_binary;
//   * no fma contraction except where fma() is written (-ffp-contract=off).
//
// A trial point is evaluated with its Jacobian: after an accept the J^T J of
// the new point is already there, after a reject the J^T J of the unchanged
// accepted point is reused. The reference recomputes both (batch_lm_ad.cu:363,
// :400); the numbers are identical because the Jacobian depends only on c.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/cusr_math.h"
#include "program.h"

namespace cusr {

constexpr int kLanes = 64;
constexpr double kCexpCap64 = 485165195.4097903;  // exp(20) rounded to double
constexpr float kCexpCap32 = 485165184.0f;         // exp(20) rounded to float

// ------------------------------------------------------------------ math

// Elementary functions come from include/cusr_math.h, the same code the CPU
// oracle compiles, so values agree to the bit; +, -, *, /, sqrt and fma are
// IEEE correctly rounded on both sides.
template <typename R> struct Fn;
template <> struct Fn<double> {
    static __device__ __forceinline__ void sincos_(double a, double *s, double *c) { cm_sincos(a, s, c); }
    static __device__ __forceinline__ double tan_(double a) { return cm_tan(a); }
    static __device__ __forceinline__ double sinh_(double a) { return cm_sinh(a); }
    static __device__ __forceinline__ double cosh_(double a) { return cm_cosh(a); }
    static __device__ __forceinline__ double tanh_(double a) { return cm_tanh(a); }
    static __device__ __forceinline__ double log_(double a) { return cm_log(a); }
    static __device__ __forceinline__ double exp_(double a) { return cm_exp(a); }
    static __device__ __forceinline__ double sqrt_(double a) { return ::sqrt(a); }
    static __device__ __forceinline__ double pow_(double a, double b) { return cm_pow(a, b); }
    static __device__ __forceinline__ double abs_(double a) { return ::fabs(a); }
    static __device__ __forceinline__ double max_(double a, double b) { return ::fmax(a, b); }
    static __device__ __forceinline__ double min_(double a, double b) { return ::fmin(a, b); }
    static constexpr double cexp_cap = kCexpCap64;
    static constexpr double pdiv_eps = 1e-9;
    static constexpr double plog_eps = 1e-9;
};
template <> struct Fn<float> {
    static __device__ __forceinline__ void sincos_(float a, float *s, float *c) { cm_sincosf(a, s, c); }
    static __device__ __forceinline__ float tan_(float a) { return cm_tanf(a); }
    static __device__ __forceinline__ float sinh_(float a) { return cm_sinhf(a); }
    static __device__ __forceinline__ float cosh_(float a) { return cm_coshf(a); }
    static __device__ __forceinline__ float tanh_(float a) { return cm_tanhf(a); }
    static __device__ __forceinline__ float log_(float a) { return cm_logf(a); }
    static __device__ __forceinline__ float exp_(float a) { return cm_expf(a); }
    static __device__ __forceinline__ float sqrt_(float a) { return ::sqrtf(a); }
    static __device__ __forceinline__ float pow_(float a, float b) { return cm_powf(a, b); }
    static __device__ __forceinline__ float abs_(float a) { return ::fabsf(a); }
    static __device__ __forceinline__ float max_(float a, float b) { return ::fmaxf(a, b); }
    static __device__ __forceinline__ float min_(float a, float b) { return ::fminf(a, b); }
    static constexpr float cexp_cap = kCexpCap32;
    static constexpr float pdiv_eps = 1e-9f;
    static constexpr float plog_eps = 1e-9f;
};

// Value of a unary operator and its derivative d. sel: the tangent is kept
// where d != 0 and zeroed elsewhere instead of multiplied (flat branches).
template <typename R>
__device__ __forceinline__ R op_unary(int f, R a, R &d, bool &sel) {
    typedef Fn<R> F;
    const R one = R(1), zero = R(0), two = R(2);
    R r;
    sel = false;
    switch (f) {
    case OP_SIN: F::sincos_(a, &r, &d); break;
    case OP_COS: { R sn; F::sincos_(a, &sn, &r); d = -sn; break; }
    case OP_TAN: r = F::tan_(a); d = one + r * r; break;
    case OP_SINH: r = F::sinh_(a); d = F::cosh_(a); break;
    case OP_COSH: r = F::cosh_(a); d = F::sinh_(a); break;
    case OP_TANH: r = F::tanh_(a); d = one - r * r; break;
    case OP_LOG: r = F::log_(a); d = one / a; break;
    case OP_LOOSE_LOG: r = F::log_(F::abs_(a)); d = one / a; break;
    case OP_EXP: r = F::exp_(a); d = r; break;
    case OP_INV: case OP_LOOSE_INV: r = one / a; d = -(r * r); break;
    case OP_NEG: r = -a; d = -one; break;
    case OP_ABS: r = F::abs_(a); d = (a > zero) ? one : ((a < zero) ? -one : zero); break;
    case OP_SQRT: r = F::sqrt_(a); d = one / (two * r); break;
    case OP_LOOSE_SQRT:
        r = F::sqrt_(F::abs_(a));
        d = (a > zero) ? one / (two * r) : ((a < zero) ? -one / (two * r) : zero);
        break;
    case OP_CEXP:
        if (a > R(20)) { r = F::cexp_cap; d = zero; sel = true; }
        else { r = F::exp_(a); d = r; }
        break;
    case OP_SQUARE: r = a * a; d = a + a; break;
    case OP_PLOG: {
        R t = F::abs_(a) + F::plog_eps;
        r = F::log_(t);
        d = (a > zero) ? one / t : ((a < zero) ? -one / t : zero);
        break;
    }
    default: r = zero; d = zero; break;
    }
    return r;
}

// Value of a binary operator l op rv and the partials d1 = dOut/dl,
// d2 = dOut/drv. want_d2 false skips log(l) of POW (no constant on the right).
template <typename R>
__device__ __forceinline__ R op_binary(int f, R l, R rv, bool want_d2, R &d1, R &d2, bool &sel) {
    typedef Fn<R> F;
    const R one = R(1), zero = R(0);
    R o;
    sel = false;
    switch (f) {
    case OP_ADD: o = l + rv; d1 = one; d2 = one; break;
    case OP_SUB: o = l - rv; d1 = one; d2 = -one; break;
    case OP_MUL: o = l * rv; d1 = rv; d2 = l; break;
    case OP_DIV: case OP_LOOSE_DIV: o = l / rv; d1 = one / rv; d2 = -o / rv; break;
    case OP_PDIV:
        if (F::abs_(rv) < F::pdiv_eps) { o = one; d1 = zero; d2 = zero; sel = true; }
        else { o = l / rv; d1 = one / rv; d2 = -o / rv; }
        break;
    case OP_POW:
        o = F::pow_(l, rv);
        d1 = rv * F::pow_(l, rv - one);
        d2 = want_d2 ? o * F::log_(l) : zero;
        break;
    case OP_LOOSE_POW: {
        R al = F::abs_(l);
        R s = (l > zero) ? one : ((l < zero) ? -one : zero);
        o = F::pow_(al, rv);
        d1 = s * (rv * F::pow_(al, rv - one));
        d2 = want_d2 ? o * F::log_(al) : zero;
        break;
    }
    case OP_MAX: o = F::max_(l, rv); d1 = (l >= rv) ? one : zero; d2 = (l >= rv) ? zero : one;
        sel = true; break;
    case OP_MIN: o = F::min_(l, rv); d1 = (l <= rv) ? one : zero; d2 = (l <= rv) ? zero : one;
        sel = true; break;
    case OP_LT: o = (l < rv) ? one : zero; d1 = zero; d2 = zero; sel = true; break;
    case OP_GT: o = (l > rv) ? one : zero; d1 = zero; d2 = zero; sel = true; break;
    case OP_LE: o = (l <= rv) ? one : zero; d1 = zero; d2 = zero; sel = true; break;
    case OP_GE: o = (l >= rv) ? one : zero; d1 = zero; d2 = zero; sel = true; break;
    default: o = zero; d1 = zero; d2 = zero; break;
    }
    return o;
}

template <typename R>
__device__ __forceinline__ R safe_mul(R a, R b) {
    return (a == R(0) || b == R(0)) ? R(0) : a * b;
}

// wave-uniform copies (values every lane already agrees on)
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ double uni(double v) {
    int2 p = *reinterpret_cast<int2 *>(&v);
    p.x = __builtin_amdgcn_readfirstlane(p.x);
    p.y = __builtin_amdgcn_readfirstlane(p.y);
    return *reinterpret_cast<double *>(&p);
}

// -------------------------------------------------------- one point

// Forward sweep over one expression at one point. JAC: 0 value only,
// 1 forward AD into T[0..K), 2 record partials on the tape (reverse AD).
// x: the point's inputs; cs: the wave's constants (LDS, fp64);
// tape: this wave's tape base, slot s of lane l at tape[s*64 + l].
template <int K, typename R, int JAC>
__device__ __forceinline__ R forward_point(const uint64_t *__restrict__ prog, int n,
                                           const R *x, const double *cs, R *T, R *tape,
                                           int lane) {
    R st[CO_MAX_STACK];
    for (int pc = 0; pc < n; ++pc) {
        const uint64_t w = prog[pc];
        const int kind = ins_kind(w);
        const int sp = ins_sp(w);
        if (kind == NODE_VAR) {
            st[sp] = x[ins_arg(w)];
        } else if (kind == NODE_CONST) {
            const int k = ins_arg(w);
            st[sp] = (R)cs[k];
            if (JAC == 1) T[k] = R(1);
        } else if (kind == NODE_UFUNC) {
            R d;
            bool sel;
            st[sp - 1] = op_unary<R>(ins_fid(w), st[sp - 1], d, sel);
            if (JAC == 1) {
                const int lo = ins_lo(w), hi = ins_hi(w);
                if (sel) { for (int j = lo; j < hi; ++j) T[j] = (d != R(0)) ? T[j] : R(0); }
                else { for (int j = lo; j < hi; ++j) T[j] = T[j] * d; }
            } else if (JAC == 2) {
                tape[ins_tape(w) * kLanes + lane] = d;
            }
        } else {
            R d1, d2;
            bool sel;
            const int lo = ins_lo(w), mid = ins_mid(w), hi = ins_hi(w);
            const bool want_d2 = (JAC == 2) || (mid < hi);
            const R o = op_binary<R>(ins_fid(w), st[sp - 1], st[sp - 2], want_d2, d1, d2, sel);
            st[sp - 2] = o;
            if (JAC == 1) {
                if (sel) {
                    for (int j = lo; j < mid; ++j) T[j] = (d1 != R(0)) ? T[j] : R(0);
                    for (int j = mid; j < hi; ++j) T[j] = (d2 != R(0)) ? T[j] : R(0);
                } else {
                    for (int j = lo; j < mid; ++j) T[j] = T[j] * d1;
                    for (int j = mid; j < hi; ++j) T[j] = T[j] * d2;
                }
            } else if (JAC == 2) {
                const int s = ins_tape(w);
                tape[s * kLanes + lane] = d1;
                tape[(s + 1) * kLanes + lane] = d2;
            }
        }
    }
    return st[0];
}

// Reverse sweep (prefix order = instructions from last to first) over the
// tape written by forward_point<..., 2>: g[k] = d f / d c_k
// (cusr/kernel/revad_interp.cuh:131-156).
template <int K, typename R>
__device__ __forceinline__ void reverse_point(const uint64_t *__restrict__ prog, int n,
                                              const R *tape, R *g, int lane) {
    R as[CO_MAX_STACK + 1];
    R tos = R(1);
    for (int pc = n - 1; pc >= 0; --pc) {
        const uint64_t w = prog[pc];
        const int kind = ins_kind(w);
        const int asp = ins_asp(w);
        const int apop = ins_apop(w);
        const R adj = apop ? as[asp - 1] : tos;
        if (kind == NODE_CONST) {
            g[ins_arg(w)] = R(0) + adj;
        } else if (kind == NODE_UFUNC) {
            tos = safe_mul<R>(adj, tape[ins_tape(w) * kLanes + lane]);
        } else if (kind == NODE_BFUNC) {
            const int s = ins_tape(w);
            as[asp - apop] = safe_mul<R>(adj, tape[(s + 1) * kLanes + lane]);
            tos = safe_mul<R>(adj, tape[s * kLanes + lane]);
        }
    }
}

// ------------------------------------------------------- one data pass

struct PassArgs {
    const uint64_t *prog;  // this expression's program
    int n;
    const double *X;       // [D][N] column-major
    const double *y;       // this expression's targets [N]
    int N, D;
    float *tape32;         // this wave's tape (reverse AD), lane-interleaved
    double *tape64;
};

constexpr int sums_width(int K) { return 1 + K + K * (K + 1) / 2; }

template <int W>
__device__ __forceinline__ void wave_allreduce(double (&a)[W]) {
#pragma unroll
    for (int s = kLanes / 2; s >= 1; s >>= 1) {
#pragma unroll
        for (int w = 0; w < W; ++w) a[w] = a[w] + __shfl_xor(a[w], s, kLanes);
    }
}

// One pass over all points at constants cs (LDS): sums[0] = sum r^2,
// sums[1..K] = J^T r, sums[1+K..] = upper triangle of J^T J (row-major),
// written to out (LDS) by lane 0. JAC: 0 value only, 1 forward, 2 reverse.
template <int K, typename R, int JAC>
__device__ void data_pass(const PassArgs &a, const double *cs, double *out, int lane) {
    constexpr int W = (JAC == 0) ? 1 : sums_width(K);
    double acc[W];
#pragma unroll
    for (int w = 0; w < W; ++w) acc[w] = 0.0;
    R *tape = nullptr;
    if constexpr (JAC == 2) {
        if constexpr (sizeof(R) == 8) tape = (R *)a.tape64; else tape = (R *)a.tape32;
    }
    for (int i = lane; i < a.N; i += kLanes) {
        R x[CO_MAX_VARS];
#pragma unroll
        for (int v = 0; v < CO_MAX_VARS; ++v)
            if (v < a.D) x[v] = (R)a.X[(size_t)v * a.N + i];
        const double yi = a.y[i];
        R T[K > 0 ? K : 1];
        const R f = forward_point<K, R, JAC>(a.prog, a.n, x, cs, T, tape, lane);
        if constexpr (JAC == 2) reverse_point<K, R>(a.prog, a.n, tape, T, lane);
        const double r = (double)f - yi;
        acc[0] = fma(r, r, acc[0]);
        if constexpr (JAC != 0) {
#pragma unroll
            for (int j = 0; j < K; ++j) acc[1 + j] = fma((double)T[j], r, acc[1 + j]);
            int q = 1 + K;
#pragma unroll
            for (int j1 = 0; j1 < K; ++j1)
#pragma unroll
                for (int j2 = j1; j2 < K; ++j2, ++q)
                    acc[q] = fma((double)T[j1], (double)T[j2], acc[q]);
        }
    }
    wave_allreduce<W>(acc);
    if (lane == 0) {
#pragma unroll
        for (int w = 0; w < W; ++w) out[w] = acc[w];
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

// ------------------------------------------------------------ the solve

// Relative-damped Cholesky solve of (J^T J + lambda diag(J^T J)) delta = -J^T r
// from pass sums s (cusr/kernel/batch_lm_ad.cu:149-191); false when a pivot is
// <= 0. Every lane computes the same result.
template <int K>
__device__ __forceinline__ bool damped_solve(const double *s, double lambda, double (&delta)[K]) {
    double L[K][K];
    double b[K];
#pragma unroll
    for (int i = 0; i < K; ++i) {
        b[i] = -s[1 + i];
#pragma unroll
        for (int j = 0; j <= i; ++j) {
            // upper-triangle element (j, i): row j starts at j*K - j*(j-1)/2
            L[i][j] = s[1 + K + j * K - (j * (j - 1)) / 2 + (i - j)];
        }
        L[i][i] = L[i][i] * (1.0 + lambda);
    }
    bool ok = true;
#pragma unroll
    for (int j = 0; j < K; ++j) {
        double sj = L[j][j];
#pragma unroll
        for (int k = 0; k < j; ++k) sj = fma(-L[j][k], L[j][k], sj);
        if (sj <= 0.0) ok = false;
        const double dj = ::sqrt(sj);
        L[j][j] = dj;
#pragma unroll
        for (int i = j + 1; i < K; ++i) {
            double t = L[i][j];
#pragma unroll
            for (int k = 0; k < j; ++k) t = fma(-L[i][k], L[j][k], t);
            L[i][j] = t / dj;
        }
    }
    if (!ok) return false;
#pragma unroll
    for (int i = 0; i < K; ++i) {
        double t = b[i];
#pragma unroll
        for (int k = 0; k < i; ++k) t = fma(-L[i][k], b[k], t);
        b[i] = t / L[i][i];
    }
#pragma unroll
    for (int i = K - 1; i >= 0; --i) {
        double t = b[i];
#pragma unroll
        for (int k = i + 1; k < K; ++k) t = fma(-L[k][i], b[k], t);
        b[i] = t / L[i][i];
    }
#pragma unroll
    for (int i = 0; i < K; ++i) delta[i] = b[i];
    return true;
}

// ------------------------------------------------------------- the fit

struct FitArgs {
    const uint64_t *prog;
    const ExprDesc *desc;   // by launch position
    const double *X;        // [D][N]
    const double *Y;        // [M][N]
    const double *C0;       // [total_c]
    double *C;              // [total_c] out
    int32_t *status;        // [M] out
    double *loss_init;      // [M] out
    double *loss_final;     // [M] out
    int32_t *iters;         // [M] out
    int N, D, max_iter, guard;
    double lambda0, xtol;
    int tape_slots;         // per-wave tape slots in dynamic LDS
};

// internal states, mapped to STATUS_* at the end (lm_core.cuh:46-56)
enum { ST_RUN = 0, ST_CONV = 1, ST_NAN = 2, ST_K0 = 3, ST_CHOL = 4 };

template <int K, typename R, int AD>
__device__ void fit_one(const FitArgs &fa, const ExprDesc &e, double *lds_c, double *lds_s,
                        void *lds_tape, int lane) {
    constexpr int JAC = (K == 0) ? 0 : (AD == CO_AD_REVERSE ? 2 : 1);
    PassArgs pa;
    pa.prog = fa.prog + e.prog_off;
    pa.n = e.n;
    pa.X = fa.X;
    pa.y = fa.Y + (size_t)e.y_row * fa.N;
    pa.N = fa.N;
    pa.D = fa.D;
    pa.tape32 = (float *)lds_tape;
    pa.tape64 = (double *)lds_tape;

    double *c_cur = lds_c, *c_try = lds_c + CO_MAX_K;
    double *s_cur = lds_s, *s_try = lds_s + sums_width(CO_MAX_K);
    if (lane < K) c_cur[lane] = fa.C0[e.c_off + lane];
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();

    data_pass<K, R, JAC>(pa, c_cur, s_cur, lane);
    double loss = uni(0.5 * s_cur[0]);
    double loss_init = loss;
    int st = (K == 0) ? ST_K0 : (isfinite(loss) ? ST_RUN : ST_NAN);
    double lambda = fa.lambda0;
    int it = 0;
    if constexpr (K > 0) {
        while (uni(st) == ST_RUN && it < fa.max_iter) {
            ++it;
            double delta[K];
            if (!damped_solve<K>(s_cur, lambda, delta)) {
                lambda = lambda * 10.0;
                if (lambda > 1e12) st = ST_CHOL;
                continue;
            }
            if (lane < K) {
#pragma unroll
                for (int j = 0; j < K; ++j)
                    if (j == lane) c_try[j] = c_cur[j] + delta[j];
            }
            __builtin_amdgcn_s_waitcnt(0);
            __builtin_amdgcn_wave_barrier();
            data_pass<K, R, JAC>(pa, c_try, s_try, lane);
            const double loss_try = uni(0.5 * s_try[0]);
            if (!isfinite(loss_try)) { st = ST_NAN; continue; }
            double dn2 = 0.0, cn2 = 0.0;
#pragma unroll
            for (int j = 0; j < K; ++j) {
                dn2 = fma(delta[j], delta[j], dn2);
                cn2 = fma(c_try[j], c_try[j], cn2);
            }
            const double dn = ::sqrt(dn2), cn = ::sqrt(cn2);
            if (loss_try <= loss) {
                double *t = c_cur; c_cur = c_try; c_try = t;
                t = s_cur; s_cur = s_try; s_try = t;
                loss = loss_try;
                if (dn < fa.xtol * (cn + fa.xtol)) st = ST_CONV;
                else {
                    lambda = lambda * 0.1;
                    if (lambda < 1e-12) lambda = 1e-12;
                }
            } else {
                lambda = lambda * 10.0;
                if (lambda > 1e12) st = ST_NAN;
            }
        }
    }
    double lf = loss, li = loss_init;
    if constexpr (sizeof(R) == 4) {
        // fp64 losses at the delivered point and at the start
        data_pass<K, double, 0>(pa, c_cur, s_try, lane);
        lf = uni(0.5 * s_try[0]);
        if (lane < K) c_try[lane] = fa.C0[e.c_off + lane];
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
        data_pass<K, double, 0>(pa, c_try, s_try, lane);
        li = uni(0.5 * s_try[0]);
    }
    bool revert = false;
    if (fa.guard && K > 0) revert = !isfinite(lf) || (isfinite(li) && lf > li);
    if (revert) {
        if (st == ST_CONV) st = ST_RUN;
        lf = li;
    }
    if (lane < K) fa.C[e.c_off + lane] = revert ? fa.C0[e.c_off + lane] : c_cur[lane];
    if (lane == 0) {
        // ST_RUN -> STATUS_MAXITER, ST_CONV -> STATUS_CONVERGED, the rest keep their code
        fa.status[e.y_row] = (st <= ST_CONV) ? (1 - st) : st;
        fa.loss_init[e.y_row] = li;
        fa.loss_final[e.y_row] = lf;
        fa.iters[e.y_row] = it;
    }
}

// One kernel per (K, precision, AD mode): each K gets its own register
// allocation, so small-K expressions are not held to the occupancy of K = 16.
// Launch position p of a K bin runs descriptor desc[p] (the host offsets desc
// to the bin's start).
template <int K, typename R, int AD>
__global__ void __launch_bounds__(kLanes) lm_fit_kernel(FitArgs fa) {
    __shared__ double lds_c[2 * CO_MAX_K];
    __shared__ double lds_s[2 * sums_width(CO_MAX_K)];
    extern __shared__ double lds_tape[];
    const ExprDesc e = fa.desc[blockIdx.x];
    fit_one<K, R, AD>(fa, e, lds_c, lds_s, lds_tape, (int)threadIdx.x);
}

hipError_t launch_fit_f64_fwd(int K, unsigned grid, size_t lds, hipStream_t s, const FitArgs &fa);
hipError_t launch_fit_f64_rev(int K, unsigned grid, size_t lds, hipStream_t s, const FitArgs &fa);
hipError_t launch_fit_f32_fwd(int K, unsigned grid, size_t lds, hipStream_t s, const FitArgs &fa);
hipError_t launch_fit_f32_rev(int K, unsigned grid, size_t lds, hipStream_t s, const FitArgs &fa);

// ------------------------------------------------------ plain evaluation

struct EvalArgs {
    const uint64_t *prog;
    const ExprDesc *desc;
    const double *X;   // [D][N]
    const double *C;   // [total_c]
    double *Yout;      // [M][N]
    int N, D;
};

template <typename R>
__global__ void __launch_bounds__(kLanes) eval_kernel(EvalArgs ea) {
    __shared__ double cs[CO_MAX_K];
    const int lane = threadIdx.x;
    const ExprDesc e = ea.desc[blockIdx.x];
    if (lane < e.K) cs[lane] = ea.C[e.c_off + lane];
    __syncthreads();
    for (int i = lane; i < ea.N; i += kLanes) {
        R x[CO_MAX_VARS];
#pragma unroll
        for (int v = 0; v < CO_MAX_VARS; ++v)
            if (v < ea.D) x[v] = (R)ea.X[(size_t)v * ea.N + i];
        R T[1];
        const R f = forward_point<0, R, 0>(ea.prog + e.prog_off, e.n, x, cs, T, nullptr, lane);
        ea.Yout[(size_t)e.y_row * ea.N + i] = (double)f;
    }
}

}  // namespace cusr
