// lm_device.h -- gfx950 kernels of the batched Levenberg-Marquardt fitter.
//
// One 64-lane wavefront owns one expression for the whole fit
// (cusr/kernel/batch_lm_ad.cu:350-495 runs one host loop over all trees
// instead). Lane l evaluates points l, l+64, l+128, ... of the expression, P
// of them per pass of the interpreter; the program (program.h) is read with
// scalar loads and every branch on it is a scalar branch, so the 64 lanes stay
// converged and the fetch/decode cost is shared by 64*P points. Per point a
// lane computes the value and the gradient row and folds r^2, J^T r and the
// upper triangle of J^T J into registers; a butterfly over the 64 lanes then
// gives every lane the same sums, and every lane solves the same damped
// K x K system, so accept/reject and the lambda update stay on the device.
//
// Arithmetic follows one fixed order, which the CPU oracle reproduces:
//   * lane l sums its points in ascending order from 0.0, fma(a, b, acc);
//   * lanes combine with strides 32, 16, 8, 4, 2, 1;
//   * operator values and partials use the formulas of unary_p/binary_p and
//     the elementary functions of include/cusr_math.h;
//   * no fma contraction except where fma() is written (-ffp-contract=off).
//
// A trial point is evaluated with its Jacobian: after an accept the J^T J of
// the new point is already there, after a reject the J^T J of the unchanged
// accepted point is reused. The reference recomputes both (batch_lm_ad.cu:363,
// :400); the numbers are identical because the Jacobian depends only on c.
//
// LDS per wavefront: the batch's inputs x[v][p][lane], the spill slots
// [s][p][lane], the constants and the pass sums; reverse AD adds its tape
// [t][p][lane]. All indices are uniform, so accesses are bank-conflict free.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/cusr_math.h"
#include "program.h"

namespace cusr {

constexpr int kLanes = 64;
constexpr double kCexpCap64 = 485165195.4097903;  // exp(20) rounded to double
constexpr float kCexpCap32 = 485165184.0f;         // exp(20) rounded to float

// Points per lane per interpreter pass: more amortises the scalar fetch and
// dispatch, fewer keeps registers (the J^T J sums dominate for large K) and
// the reverse-AD tape in LDS small.
// Per-K tables for fp64 forward AD, K = 0..16 (overridable for tuning).
#ifndef CUSR_P64_TABLE
#define CUSR_P64_TABLE 4, 4, 4, 4, 4, 4, 4, 4, 4, 1, 1, 1, 1, 1, 1, 1, 1
#endif
#ifndef CUSR_P32_TABLE
#define CUSR_P32_TABLE 4, 4, 4, 4, 4, 4, 4, 4, 4, 2, 2, 2, 2, 2, 2, 2, 2
#endif
#ifndef CUSR_PREV_TABLE
#define CUSR_PREV_TABLE 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1
#endif
// fp64 forward AD from kLargeN points on (C4's N = 100,000): each pass streams
// y from memory, and two points per lane with three waves per SIMD hide the
// loads better (C4 on the split path: 187 -> 179.5 ms with every K = 1..8 so,
// against K = 5, 6 only; at N = 1,024 four points measured faster). Points per
// pass do not change any summation order.
#ifndef CUSR_P64_LARGE_N_TABLE
#define CUSR_P64_LARGE_N_TABLE 2, 2, 2, 2, 2, 2, 2, 2, 2, 1, 1, 1, 1, 1, 1, 1, 1
#endif
constexpr int kLargeN = 16384;
constexpr int kP64[CO_FAST_MAX_K + 1] = {CUSR_P64_TABLE};
constexpr int kP64LargeN[CO_FAST_MAX_K + 1] = {CUSR_P64_LARGE_N_TABLE};
constexpr int kP32[CO_FAST_MAX_K + 1] = {CUSR_P32_TABLE};
constexpr int kPRev[CO_FAST_MAX_K + 1] = {CUSR_PREV_TABLE};   // reverse AD (tape in LDS)
template <typename R, int K, int AD, int LN = 0>
constexpr int points_per_pass() {
    return (AD == CO_AD_REVERSE) ? kPRev[K]
           : (sizeof(R) == 4)    ? kP32[K]
                                 : (LN ? kP64LargeN[K] : kP64[K]);
}

// Points per lane of the mixed-precision fit's fp64 guard passes: as many as
// fit the LDS bytes of the fit's own passes (fp32 at P points -> fp64 at P/2).
template <typename R, int K, int AD, int LN = 0>
constexpr int audit_points() {
    return points_per_pass<R, K, AD, LN>() * (int)sizeof(R) / 8 > 0
               ? points_per_pass<R, K, AD, LN>() * (int)sizeof(R) / 8
               : 1;
}

// Points per elementary-function call in the interpreter (the rest of an
// operator always runs P-wide): fp64 forward-AD kernels from
// CUSR_MATH_CHUNK_MIN_K constants on interleave two chains at a time, where
// four would push the kernel past 256 VGPRs.
#ifndef CUSR_MATH_CHUNK_MIN_K
#define CUSR_MATH_CHUNK_MIN_K 7
#endif
template <int K, typename R, int P, int JAC>
constexpr int math_chunk() {
    return (sizeof(R) == 8 && JAC == 1 && K >= CUSR_MATH_CHUNK_MIN_K && P > 2) ? 2 : P;
}

// scalar-cache view of the program (constant address space)
typedef const __attribute__((address_space(4))) uint64_t *ProgPtr;

// The two program formats of program.h, read by the same interpreter: one
// 64-bit word per instruction for the fast kernels, two for the general one.
// The word's high half rides beside it as an opaque copy: the compiler then
// tests a flag above bit 31 with one 32-bit bit test (on the 64-bit word it
// folds the same test into a mask and a 64-bit compare). The operator's arity
// is tested once per step, and each arm fetches its own operands.
struct FastWord {
    uint64_t w;
    uint32_t h;   // w >> 32
};
struct FastFmt {
    typedef FastWord W;
    static constexpr int kWords = 1;   // program words per instruction
    static __device__ __forceinline__ W load(ProgPtr p, int pc) {
        W r;
        r.w = p[pc];
        r.h = (uint32_t)(r.w >> 32);
        __asm__("" : "+s"(r.h));
        return r;
    }
    static __device__ __forceinline__ int fid(W w) { return ins_fid(w.w); }
    static __device__ __forceinline__ int binary(W w) { return ins_binary(w.w); }
    static __device__ __forceinline__ int akind(W w) { return ins_akind(w.w); }
    static __device__ __forceinline__ int aidx(W w) { return ins_aidx(w.w); }
    static __device__ __forceinline__ int bkind(W w) { return ins_bkind(w.w); }
    static __device__ __forceinline__ int bidx(W w) { return ins_bidx(w.w); }
    static __device__ __forceinline__ int toslot(W w) { return ins_toslot(w.w); }
    static __device__ __forceinline__ int didx(W w) { return ins_didx(w.w); }
    static __device__ __forceinline__ int lo(W w) { return ins_lo(w.w); }
    static __device__ __forceinline__ int mid(W w) { return ins_mid(w.w); }
    static __device__ __forceinline__ int hi(W w) { return (int)((w.h >> 2) & 31u); }
    static __device__ __forceinline__ int tape(W w) { return (int)((w.h >> 7) & 255u); }
    static __device__ __forceinline__ int sel(W w) { return (int)((w.h >> 15) & 1u); }
    static __device__ __forceinline__ int scale_a(W w) { return (int)((w.h >> 16) & 1u); }
    static __device__ __forceinline__ int scale_b(W w) { return (int)((w.h >> 17) & 1u); }
    static __device__ __forceinline__ int tape_a(W w) { return (int)((w.h >> 18) & 1u); }
    static __device__ __forceinline__ int tape_b(W w) { return (int)((w.h >> 19) & 1u); }
};
struct WideFmt {
    typedef Wide W;
    static constexpr int kWords = 2;
    static __device__ __forceinline__ W load(ProgPtr p, int pc) {
        W w;
        w.a = p[2 * pc];
        w.b = p[2 * pc + 1];
        return w;
    }
    static __device__ __forceinline__ int fid(W w) { return wins_fid(w.a); }
    static __device__ __forceinline__ int binary(W w) { return wins_binary(w.a); }
    static __device__ __forceinline__ int akind(W w) { return wins_akind(w.a); }
    static __device__ __forceinline__ int aidx(W w) { return wins_aidx(w.a); }
    static __device__ __forceinline__ int bkind(W w) { return wins_bkind(w.a); }
    static __device__ __forceinline__ int bidx(W w) { return wins_bidx(w.a); }
    static __device__ __forceinline__ int toslot(W w) { return wins_toslot(w.a); }
    static __device__ __forceinline__ int didx(W w) { return wins_didx(w.a); }
    static __device__ __forceinline__ int lo(W w) { return wins_lo(w.b); }
    static __device__ __forceinline__ int mid(W w) { return wins_mid(w.b); }
    static __device__ __forceinline__ int hi(W w) { return wins_hi(w.b); }
    static __device__ __forceinline__ int tape(W w) { return wins_tape(w.b); }
    static __device__ __forceinline__ int sel(W w) { return wins_sel(w.a); }
    static __device__ __forceinline__ int scale_a(W w) { return wins_scale_a(w.a); }
    static __device__ __forceinline__ int scale_b(W w) { return wins_scale_b(w.a); }
    static __device__ __forceinline__ int tape_a(W w) { return wins_tape_a(w.a); }
    static __device__ __forceinline__ int tape_b(W w) { return wins_tape_b(w.a); }
};

__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ double uni(double v) {
    int2 p = *reinterpret_cast<int2 *>(&v);
    p.x = __builtin_amdgcn_readfirstlane(p.x);
    p.y = __builtin_amdgcn_readfirstlane(p.y);
    return *reinterpret_cast<double *>(&p);
}

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
    template <int P>
    static __device__ __forceinline__ void sincos_v(const double *a, double *s, double *c) { cm_sincos_v<P>(a, s, c); }
    template <int P>
    static __device__ __forceinline__ void log_v(const double *a, double *r) { cm_log_v<P>(a, r); }
    template <int P>
    static __device__ __forceinline__ void exp_v(const double *a, double *r) { cm_exp_v<P>(a, r); }
    static constexpr double cexp_cap = kCexpCap64;
    static constexpr double eps9 = 1e-9;
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
    template <int P>
    static __device__ __forceinline__ void sincos_v(const float *a, float *s, float *c) { cm_sincosf_v<P>(a, s, c); }
    template <int P>
    static __device__ __forceinline__ void log_v(const float *a, float *r) { cm_logf_v<P>(a, r); }
    template <int P>
    static __device__ __forceinline__ void exp_v(const float *a, float *r) { cm_expf_v<P>(a, r); }
    static constexpr float cexp_cap = kCexpCap32;
    static constexpr float eps9 = 1e-9f;
};

#define CUSR_FOR_P _Pragma("unroll") for (int p = 0; p < P; ++p)

// Value r and derivative d of a unary operator for P points. z[p]: the
// tangent is zeroed instead of multiplied (a flat branch: derivative exactly
// 0 by definition, so 0 * inf must not leak a NaN).
// sin, cos, tan, log and exp take the P-wide forms of include/cusr_math.h
// (the scalar functions' bits, points interleaved), MC points at a time: the
// kernels whose registers are tight interleave fewer chains.
#define CUSR_MATH_V(fn, ...) \
    _Pragma("unroll") for (int c0 = 0; c0 < P; c0 += MC) F::template fn<MC>(__VA_ARGS__)
template <typename R, int P, int MC = P>
__device__ __forceinline__ void unary_p(int f, const R *a, R *r, R *d, uint64_t *zm) {
    typedef Fn<R> F;
    static_assert(P % MC == 0, "math chunks must divide the points per lane");
    const R one = R(1), zero = R(0), two = R(2);
    switch (f) {
    case OP_SIN: CUSR_MATH_V(sincos_v, a + c0, r + c0, d + c0); break;
    case OP_COS: {
        R s[P];
        CUSR_MATH_V(sincos_v, a + c0, s + c0, r + c0);
        CUSR_FOR_P d[p] = -s[p];
        break;
    }
    case OP_TAN: {
        R s[P], c[P];
        CUSR_MATH_V(sincos_v, a + c0, s + c0, c + c0);
        CUSR_FOR_P { r[p] = s[p] / c[p]; d[p] = one + r[p] * r[p]; }
        break;
    }
    case OP_SINH: CUSR_FOR_P { r[p] = F::sinh_(a[p]); d[p] = F::cosh_(a[p]); } break;
    case OP_COSH: CUSR_FOR_P { r[p] = F::cosh_(a[p]); d[p] = F::sinh_(a[p]); } break;
    case OP_TANH: CUSR_FOR_P { r[p] = F::tanh_(a[p]); d[p] = one - r[p] * r[p]; } break;
    case OP_LOG:
        CUSR_MATH_V(log_v, a + c0, r + c0);
        CUSR_FOR_P d[p] = one / a[p];
        break;
    case OP_LOOSE_LOG: {
        R aa[P];
        CUSR_FOR_P aa[p] = F::abs_(a[p]);
        CUSR_MATH_V(log_v, aa + c0, r + c0);
        CUSR_FOR_P d[p] = one / a[p];
        break;
    }
    case OP_EXP:
        CUSR_MATH_V(exp_v, a + c0, r + c0);
        CUSR_FOR_P d[p] = r[p];
        break;
    case OP_INV: case OP_LOOSE_INV: CUSR_FOR_P { r[p] = one / a[p]; d[p] = -(r[p] * r[p]); } break;
    case OP_NEG: CUSR_FOR_P { r[p] = -a[p]; d[p] = -one; } break;
    case OP_ABS:
        CUSR_FOR_P {
            r[p] = F::abs_(a[p]);
            d[p] = (a[p] > zero) ? one : ((a[p] < zero) ? -one : zero);
        }
        break;
    case OP_SQRT: CUSR_FOR_P { r[p] = F::sqrt_(a[p]); d[p] = one / (two * r[p]); } break;
    case OP_LOOSE_SQRT:
        CUSR_FOR_P {
            r[p] = F::sqrt_(F::abs_(a[p]));
            const R inv = one / (two * r[p]);      // -(1/x) == (-1)/x exactly
            d[p] = (a[p] > zero) ? inv : ((a[p] < zero) ? -inv : zero);
        }
        break;
    case OP_CEXP: {
        R xin[P], e[P];
        CUSR_FOR_P xin[p] = (a[p] > R(20)) ? zero : a[p];
        CUSR_MATH_V(exp_v, xin + c0, e + c0);
        CUSR_FOR_P {
            const bool flat = a[p] > R(20);
            r[p] = flat ? F::cexp_cap : e[p];
            d[p] = flat ? zero : e[p];
            zm[p] = __builtin_amdgcn_ballot_w64(flat);
        }
        break;
    }
    case OP_SQUARE: CUSR_FOR_P { r[p] = a[p] * a[p]; d[p] = a[p] + a[p]; } break;
    case OP_PLOG: {
        R t[P];
        CUSR_FOR_P t[p] = F::abs_(a[p]) + F::eps9;
        CUSR_MATH_V(log_v, t + c0, r + c0);
        CUSR_FOR_P {
            const R inv = one / t[p];
            d[p] = (a[p] > zero) ? inv : ((a[p] < zero) ? -inv : zero);
        }
        break;
    }
    case OP_IDENT: CUSR_FOR_P { r[p] = a[p]; d[p] = one; } break;
    default: CUSR_FOR_P { r[p] = zero; d[p] = zero; } break;
    }
}

#undef CUSR_MATH_V

// Value o = l op rv and partials d1 = do/dl, d2 = do/drv for P points.
// want_d2 false skips log(l) of POW when no constant is on the right.
// UNIT false leaves the partials that are exactly 1 (ADD's two, SUB's left)
// unset: the forward sweep never reads them, and a register left unset on
// that branch is not copied into at every ADD step.
// The flat-branch lanes (the points whose partial is a flat branch: zero, not
// d * tangent) leave as wave-uniform masks m1, m2 (bit = lane), set only by
// the operators the decoder marks sel (MAX, MIN, the comparisons, PDIV; CEXP
// in unary_p) and read only on their steps. As uniform scalars they need no
// default: per-lane flags left unset on the other operators' branches were
// merged with the execution mask at the join, and clearing them instead cost
// 2P scalar moves on every step.
template <typename R, int P, bool UNIT = true>
__device__ __forceinline__ void binary_p(int f, const R *l, const R *rv, bool want_d2, R *o,
                                         R *d1, R *d2, uint64_t *m1, uint64_t *m2) {
    typedef Fn<R> F;
    const R one = R(1), zero = R(0);
    switch (f) {
    case OP_ADD:
        CUSR_FOR_P {
            o[p] = l[p] + rv[p];
            if constexpr (UNIT) { d1[p] = one; d2[p] = one; }
        }
        break;
    case OP_SUB:
        CUSR_FOR_P {
            o[p] = l[p] - rv[p];
            if constexpr (UNIT) d1[p] = one;
            d2[p] = -one;
        }
        break;
    case OP_MUL: CUSR_FOR_P { o[p] = l[p] * rv[p]; d1[p] = rv[p]; d2[p] = l[p]; } break;
    // d(l/r)/dr = -(l/r) * (1/r): one division for the value, one for 1/r
    case OP_DIV: case OP_LOOSE_DIV:
        CUSR_FOR_P { o[p] = l[p] / rv[p]; d1[p] = one / rv[p]; d2[p] = -(o[p] * d1[p]); }
        break;
    case OP_PDIV:
        CUSR_FOR_P {
            const bool prot = F::abs_(rv[p]) < F::eps9;
            const R den = prot ? one : rv[p];
            const R q = l[p] / den;
            const R inv = one / den;
            o[p] = prot ? one : q;
            d1[p] = prot ? zero : inv;
            d2[p] = prot ? zero : -(q * inv);
            m1[p] = m2[p] = __builtin_amdgcn_ballot_w64(prot);
        }
        break;
    case OP_POW:
        CUSR_FOR_P {
            o[p] = F::pow_(l[p], rv[p]);
            d1[p] = rv[p] * F::pow_(l[p], rv[p] - one);
            d2[p] = want_d2 ? o[p] * F::log_(l[p]) : zero;
        }
        break;
    case OP_LOOSE_POW:
        CUSR_FOR_P {
            const R al = F::abs_(l[p]);
            const R s = (l[p] > zero) ? one : ((l[p] < zero) ? -one : zero);
            o[p] = F::pow_(al, rv[p]);
            d1[p] = s * (rv[p] * F::pow_(al, rv[p] - one));
            d2[p] = want_d2 ? o[p] * F::log_(al) : zero;
        }
        break;
    case OP_MAX:
        CUSR_FOR_P {
            const bool ge = l[p] >= rv[p];
            o[p] = F::max_(l[p], rv[p]);
            d1[p] = ge ? one : zero;
            d2[p] = ge ? zero : one;
            m1[p] = __builtin_amdgcn_ballot_w64(!ge);
            m2[p] = __builtin_amdgcn_ballot_w64(ge);
        }
        break;
    case OP_MIN:
        CUSR_FOR_P {
            const bool le = l[p] <= rv[p];
            o[p] = F::min_(l[p], rv[p]);
            d1[p] = le ? one : zero;
            d2[p] = le ? zero : one;
            m1[p] = __builtin_amdgcn_ballot_w64(!le);
            m2[p] = __builtin_amdgcn_ballot_w64(le);
        }
        break;
    case OP_LT:
        CUSR_FOR_P {
            o[p] = (l[p] < rv[p]) ? one : zero;
            d1[p] = zero;
            d2[p] = zero;
            m1[p] = m2[p] = __builtin_amdgcn_ballot_w64(true);
        }
        break;
    case OP_GT:
        CUSR_FOR_P {
            o[p] = (l[p] > rv[p]) ? one : zero;
            d1[p] = zero;
            d2[p] = zero;
            m1[p] = m2[p] = __builtin_amdgcn_ballot_w64(true);
        }
        break;
    case OP_LE:
        CUSR_FOR_P {
            o[p] = (l[p] <= rv[p]) ? one : zero;
            d1[p] = zero;
            d2[p] = zero;
            m1[p] = m2[p] = __builtin_amdgcn_ballot_w64(true);
        }
        break;
    case OP_GE:
        CUSR_FOR_P {
            o[p] = (l[p] >= rv[p]) ? one : zero;
            d1[p] = zero;
            d2[p] = zero;
            m1[p] = m2[p] = __builtin_amdgcn_ballot_w64(true);
        }
        break;
    default: CUSR_FOR_P { o[p] = zero; d1[p] = zero; d2[p] = zero; } break;
    }
}

template <typename R>
__device__ __forceinline__ R safe_mul(R a, R b) {
    return (a == R(0) || b == R(0)) ? R(0) : a * b;
}

// ----------------------------------------------------------- the wave state

// Per-wavefront LDS areas; every array is [index][p][lane].
template <typename R, int P>
struct WaveLds {
    R *x;      // [D][P][64] the batch's inputs
    R *slot;   // [slots][P][64] spilled right operands (adjoints in the reverse sweep)
    R *tape;   // [tape][P][64] reverse-AD partials
};

template <typename R, int P>
__device__ __forceinline__ R &lds_at(R *base, int idx, int p, int lane) {
    return base[(idx * P + p) * kLanes + lane];
}

// In-place tangent scaling. ScaleAsm<R, P>::run<J>(t, d, z, m, sel) multiplies
// the P tangents t[p] (entry J of point p) by d[p] when bit J of the
// wave-uniform mask m is set; when sel is non-zero it then sets the lanes of
// lane mask z[p] (the points whose partial is a flat branch) to exactly 0.
// Test, branches, multiplies and zeroing sit in one asm block whose tangent
// operands are read and written in the same registers: written as C++, the
// conditional update is a merge of old and new values, which the register
// allocator resolved with copies of the whole tangent array at every
// interpreter step. The arithmetic is the same IEEE v_mul_f64 / v_mul_f32; a
// zeroed lane is the select z ? 0 : t*d, done by masking exec to z around one
// move and restoring it. The blocks set SCC (declared clobbered).
#define CUSR_SKIP_HEAD "s_bitcmp1_b32 %[m], %[j]\n\ts_cbranch_scc0 .Lcusr_skip%=\n\t"
#define CUSR_SEL_TEST "s_cmp_lg_u32 %[sel], 0\n\ts_cbranch_scc0 .Lcusr_skip%=\n\t"
#define CUSR_SKIP_TAIL ".Lcusr_skip%=:"
#define CUSR_MUL(op, i) op " %[t" #i "], %[t" #i "], %[d" #i "]\n\t"
#define CUSR_ZERO(mov, i) \
    "s_and_saveexec_b64 %[sv], %[z" #i "]\n\t" mov " %[t" #i "], 0\n\ts_mov_b64 exec, %[sv]\n\t"
#define CUSR_T(i) [t##i] "+v"(t[i])
#define CUSR_D(i) [d##i] "v"(d[i])
#define CUSR_Z(i) [z##i] "s"(z[i])
#define CUSR_IN [m] "s"(m), [sel] "s"(sel), [j] "n"(J)

template <typename R, int P> struct ScaleAsm;
#define CUSR_SCALE_ASM(R, MUL, MOV)                                                              \
    template <> struct ScaleAsm<R, 1> {                                                          \
        template <int J>                                                                         \
        static __device__ __forceinline__ void run(R *t, const R *d, const uint64_t *z,          \
                                                   uint32_t m, uint32_t sel) {                   \
            uint64_t sv;                                                                         \
            __asm__ volatile(CUSR_SKIP_HEAD CUSR_MUL(MUL, 0) CUSR_SEL_TEST CUSR_ZERO(MOV, 0)     \
                                 CUSR_SKIP_TAIL                                                  \
                             : CUSR_T(0), [sv] "=&s"(sv)                                         \
                             : CUSR_IN, CUSR_D(0), CUSR_Z(0) : "scc");                                   \
        }                                                                                        \
    };                                                                                           \
    template <> struct ScaleAsm<R, 2> {                                                          \
        template <int J>                                                                         \
        static __device__ __forceinline__ void run(R *t, const R *d, const uint64_t *z,          \
                                                   uint32_t m, uint32_t sel) {                   \
            uint64_t sv;                                                                         \
            __asm__ volatile(CUSR_SKIP_HEAD CUSR_MUL(MUL, 0) CUSR_MUL(MUL, 1) CUSR_SEL_TEST      \
                                 CUSR_ZERO(MOV, 0) CUSR_ZERO(MOV, 1) CUSR_SKIP_TAIL              \
                             : CUSR_T(0), CUSR_T(1), [sv] "=&s"(sv)                              \
                             : CUSR_IN, CUSR_D(0), CUSR_D(1), CUSR_Z(0), CUSR_Z(1) : "scc");             \
        }                                                                                        \
    };                                                                                           \
    template <> struct ScaleAsm<R, 4> {                                                          \
        template <int J>                                                                         \
        static __device__ __forceinline__ void run(R *t, const R *d, const uint64_t *z,          \
                                                   uint32_t m, uint32_t sel) {                   \
            uint64_t sv;                                                                         \
            __asm__ volatile(CUSR_SKIP_HEAD CUSR_MUL(MUL, 0) CUSR_MUL(MUL, 1) CUSR_MUL(MUL, 2)   \
                                 CUSR_MUL(MUL, 3) CUSR_SEL_TEST CUSR_ZERO(MOV, 0)                \
                                     CUSR_ZERO(MOV, 1) CUSR_ZERO(MOV, 2) CUSR_ZERO(MOV, 3)       \
                                         CUSR_SKIP_TAIL                                          \
                             : CUSR_T(0), CUSR_T(1), CUSR_T(2), CUSR_T(3), [sv] "=&s"(sv)        \
                             : CUSR_IN, CUSR_D(0), CUSR_D(1), CUSR_D(2), CUSR_D(3), CUSR_Z(0),   \
                               CUSR_Z(1), CUSR_Z(2), CUSR_Z(3) : "scc");                                 \
        }                                                                                        \
    };                                                                                           \
    template <> struct ScaleAsm<R, 8> {                                                          \
        template <int J>                                                                         \
        static __device__ __forceinline__ void run(R *t, const R *d, const uint64_t *z,          \
                                                   uint32_t m, uint32_t sel) {                   \
            uint64_t sv;                                                                         \
            __asm__ volatile(CUSR_SKIP_HEAD CUSR_MUL(MUL, 0) CUSR_MUL(MUL, 1) CUSR_MUL(MUL, 2)   \
                                 CUSR_MUL(MUL, 3) CUSR_MUL(MUL, 4) CUSR_MUL(MUL, 5)              \
                                     CUSR_MUL(MUL, 6) CUSR_MUL(MUL, 7) CUSR_SEL_TEST             \
                                         CUSR_ZERO(MOV, 0) CUSR_ZERO(MOV, 1) CUSR_ZERO(MOV, 2)   \
                                             CUSR_ZERO(MOV, 3) CUSR_ZERO(MOV, 4)                 \
                                                 CUSR_ZERO(MOV, 5) CUSR_ZERO(MOV, 6)             \
                                                     CUSR_ZERO(MOV, 7) CUSR_SKIP_TAIL            \
                             : CUSR_T(0), CUSR_T(1), CUSR_T(2), CUSR_T(3), CUSR_T(4), CUSR_T(5), \
                               CUSR_T(6), CUSR_T(7), [sv] "=&s"(sv)                              \
                             : CUSR_IN, CUSR_D(0), CUSR_D(1), CUSR_D(2), CUSR_D(3), CUSR_D(4),   \
                               CUSR_D(5), CUSR_D(6), CUSR_D(7), CUSR_Z(0), CUSR_Z(1), CUSR_Z(2), \
                               CUSR_Z(3), CUSR_Z(4), CUSR_Z(5), CUSR_Z(6), CUSR_Z(7) : "scc");           \
        }                                                                                        \
    };
#define CUSR_PLAIN_ASM(R, MUL)                                                                   \
    template <> struct PlainAsm<R, 1> {                                                          \
        template <int J>                                                                         \
        static __device__ __forceinline__ void run(R *t, const R *d, uint32_t m) {               \
            __asm__ volatile(CUSR_SKIP_HEAD CUSR_MUL(MUL, 0) CUSR_SKIP_TAIL                      \
                             : CUSR_T(0) : [m] "s"(m), [j] "n"(J), CUSR_D(0) : "scc");            \
        }                                                                                        \
    };                                                                                           \
    template <> struct PlainAsm<R, 2> {                                                          \
        template <int J>                                                                         \
        static __device__ __forceinline__ void run(R *t, const R *d, uint32_t m) {               \
            __asm__ volatile(CUSR_SKIP_HEAD CUSR_MUL(MUL, 0) CUSR_MUL(MUL, 1) CUSR_SKIP_TAIL     \
                             : CUSR_T(0), CUSR_T(1) : [m] "s"(m), [j] "n"(J), CUSR_D(0), CUSR_D(1) \
                             : "scc");                                                           \
        }                                                                                        \
    };                                                                                           \
    template <> struct PlainAsm<R, 4> {                                                          \
        template <int J>                                                                         \
        static __device__ __forceinline__ void run(R *t, const R *d, uint32_t m) {               \
            __asm__ volatile(CUSR_SKIP_HEAD CUSR_MUL(MUL, 0) CUSR_MUL(MUL, 1) CUSR_MUL(MUL, 2)   \
                                 CUSR_MUL(MUL, 3) CUSR_SKIP_TAIL                                 \
                             : CUSR_T(0), CUSR_T(1), CUSR_T(2), CUSR_T(3)                        \
                             : [m] "s"(m), [j] "n"(J), CUSR_D(0), CUSR_D(1), CUSR_D(2), CUSR_D(3) \
                             : "scc");                                                           \
        }                                                                                        \
    };                                                                                           \
    template <> struct PlainAsm<R, 8> {                                                          \
        template <int J>                                                                         \
        static __device__ __forceinline__ void run(R *t, const R *d, uint32_t m) {               \
            __asm__ volatile(CUSR_SKIP_HEAD CUSR_MUL(MUL, 0) CUSR_MUL(MUL, 1) CUSR_MUL(MUL, 2)   \
                                 CUSR_MUL(MUL, 3) CUSR_MUL(MUL, 4) CUSR_MUL(MUL, 5)              \
                                     CUSR_MUL(MUL, 6) CUSR_MUL(MUL, 7) CUSR_SKIP_TAIL            \
                             : CUSR_T(0), CUSR_T(1), CUSR_T(2), CUSR_T(3), CUSR_T(4), CUSR_T(5), \
                               CUSR_T(6), CUSR_T(7)                                              \
                             : [m] "s"(m), [j] "n"(J), CUSR_D(0), CUSR_D(1), CUSR_D(2), CUSR_D(3), \
                               CUSR_D(4), CUSR_D(5), CUSR_D(6), CUSR_D(7) : "scc");              \
        }                                                                                        \
    };
// PlainAsm<R, P>::run<J>: the same block without the select rule (operators
// that are not flat-branch ones: no lane masks and no test of sel per entry).
template <typename R, int P> struct PlainAsm;
CUSR_PLAIN_ASM(double, "v_mul_f64")
CUSR_PLAIN_ASM(float, "v_mul_f32")
#undef CUSR_PLAIN_ASM
CUSR_SCALE_ASM(double, "v_mul_f64", "v_mov_b64")
CUSR_SCALE_ASM(float, "v_mul_f32", "v_mov_b32")
#undef CUSR_SCALE_ASM
#undef CUSR_SKIP_HEAD
#undef CUSR_SEL_TEST
#undef CUSR_SKIP_TAIL
#undef CUSR_MUL
#undef CUSR_ZERO
#undef CUSR_T
#undef CUSR_D
#undef CUSR_Z
#undef CUSR_IN

// Entries J..K-1 of the tangent rows, one asm block per entry. From K = 5 the
// entries go in groups (of 4 up to K = 8, of 8 beyond) behind one test of the
// group's mask bits, so a range costs the tests of the groups it touches
// instead of K tests (the general kernel's K = 32 chain: 64 bit tests per
// multiplicative step; G1 121.0 -> 103.8 ms; groups of 4 at K = 5..8: C4
// 144.3 -> 141.6 ms, C2 -0.5 %).
template <int K, int J, typename R, int P>
__device__ __forceinline__ void scale_entries(R *T, const R *d, const uint64_t *z, uint32_t m,
                                              uint32_t sel);
template <int K, int J, int E, typename R, int P>
__device__ __forceinline__ void scale_group(R *T, const R *d, const uint64_t *z, uint32_t m,
                                            uint32_t sel) {
    if constexpr (J < E) {
        R t[P];
        CUSR_FOR_P t[p] = T[p * K + J];
        ScaleAsm<R, P>::template run<J>(t, d, z, m, sel);
        CUSR_FOR_P T[p * K + J] = t[p];
        scale_group<K, J + 1, E, R, P>(T, d, z, m, sel);
    }
}
template <int K, int J, int E, typename R, int P>
__device__ __forceinline__ void plain_group(R *T, const R *d, uint32_t m) {
    if constexpr (J < E) {
        R t[P];
        CUSR_FOR_P t[p] = T[p * K + J];
        PlainAsm<R, P>::template run<J>(t, d, m);
        CUSR_FOR_P T[p * K + J] = t[p];
        plain_group<K, J + 1, E, R, P>(T, d, m);
    }
}
template <int K, int J, typename R, int P>
__device__ __forceinline__ void plain_entries(R *T, const R *d, uint32_t m) {
    constexpr int GS = K > 8 ? 8 : 4;
    constexpr unsigned GM = (1u << GS) - 1u;
    if constexpr (K <= 4) {
        plain_group<K, J, K, R, P>(T, d, m);
    } else if constexpr (J < K) {
        constexpr int E = (J + GS < K) ? J + GS : K;
        if ((m >> J) & GM) plain_group<K, J, E, R, P>(T, d, m);
        plain_entries<K, E, R, P>(T, d, m);
    }
}
template <int K, int J, typename R, int P>
__device__ __forceinline__ void scale_entries(R *T, const R *d, const uint64_t *z, uint32_t m,
                                              uint32_t sel) {
    constexpr int GS = K > 8 ? 8 : 4;
    constexpr unsigned GM = (1u << GS) - 1u;
    if constexpr (K <= 4) {
        scale_group<K, J, K, R, P>(T, d, z, m, sel);
    } else if constexpr (J < K) {
        constexpr int E = (J + GS < K) ? J + GS : K;
        if ((m >> J) & GM) scale_group<K, J, E, R, P>(T, d, z, m, sel);
        scale_entries<K, E, R, P>(T, d, z, m, sel);
    }
}

// T[p*K + j] *= d[p] for j in [lo, hi); with sel, zero where z[p] instead.
template <int K, typename R, int P>
__device__ __forceinline__ void scale_range(R *T, int lo, int hi, const R *d, const uint64_t *zm,
                                            bool sel) {
    uint32_t mask;
    if constexpr (K < 32) {
        mask = ((1u << hi) - 1u) & ~((1u << lo) - 1u);
    } else {   // hi up to 32: the shift is formed in 64 bits
        mask = (uint32_t)(((uint64_t)1 << hi) - 1u) & ~(uint32_t)(((uint64_t)1 << lo) - 1u);
    }
    // one uniform test of sel: the select rule's lane masks (a vector-to-scalar
    // transfer) and its per-entry test only on the flat-branch operators'
    // steps (C2 -3.5 %, C4 -3.3 %)
    if (sel) {
        scale_entries<K, 0, R, P>(T, d, zm, mask, 1u);
    } else {
        // an opaque copy: both paths open with the same group test, which the
        // compiler otherwise forms once above the branch as a 64-bit lane mask
        uint32_t m = mask;
        __asm__("" : "+s"(m));
        plain_entries<K, 0, R, P>(T, d, m);
    }
}

// T[p*K + k] += v[p] for a wave-uniform k, the add in the branch of entry k.
// The add sits in the asm of its branch: as plain C++ the compiler merges the
// K branches into one add at a selected address, which puts T in scratch
// memory. The arithmetic is the IEEE v_add_f64 / v_add_f32 of a plain add.
template <typename R> struct AddAsm;
template <> struct AddAsm<double> {
    static __device__ __forceinline__ void run(double &t, double v) {
        __asm__ volatile("v_add_f64 %0, %0, %1" : "+v"(t) : "v"(v));
    }
};
template <> struct AddAsm<float> {
    static __device__ __forceinline__ void run(float &t, float v) {
        __asm__ volatile("v_add_f32 %0, %0, %1" : "+v"(t) : "v"(v));
    }
};
// k is found by halving [0, K): log2(K) uniform tests instead of one per entry.
template <int K, int LO, int HI, typename R, int P>
__device__ __forceinline__ void add_tangent_in(R *T, int k, const R *v) {
    if constexpr (HI - LO == 1) {
        CUSR_FOR_P AddAsm<R>::run(T[p * K + LO], v[p]);
    } else {
        constexpr int MID = (LO + HI) / 2;
        if (k < MID) add_tangent_in<K, LO, MID, R, P>(T, k, v);
        else add_tangent_in<K, MID, HI, R, P>(T, k, v);
    }
}
template <int K, typename R, int P>
__device__ __forceinline__ void add_tangent(R *T, int k, const R *v) {
    if constexpr (K > 0) add_tangent_in<K, 0, K, R, P>(T, k, v);
}

// Fetch an operand of kind/idx for P points.
template <typename R, int P>
__device__ __forceinline__ void fetch(int kind, int idx, const R *acc, const WaveLds<R, P> &w,
                                      const double *cs, int lane, R *out) {
    // the running value first (one test), then bit 0 of the kind: a variable
    // or a spilled value, one per-lane LDS read from the row's base chosen
    // by bit 1 without a branch; else a constant. Bit tests, unlike equality
    // tests, are not merged into a balanced compare tree.
    if (kind == OPD_ACC) {
        CUSR_FOR_P out[p] = acc[p];
    } else if (kind & 1) {
        R *base = (kind & 2) ? w.slot : w.x;
        CUSR_FOR_P out[p] = lds_at<R, P>(base, idx, p, lane);
    } else {
        const R c = (R)cs[idx];
        CUSR_FOR_P out[p] = c;
    }
}

// Forward sweep of one program over P points whose inputs are in w.x.
// JAC: 0 value only, 1 forward AD into T[p*K + j] (which must hold 1.0 on
// entry: the tangent of constant k with respect to itself), 2 partials to the
// tape.
template <int K, typename R, int P, int JAC, typename F = FastFmt>
__device__ __forceinline__ void forward_pass(ProgPtr prog, int n, const WaveLds<R, P> &w,
                                             const double *cs, int lane, R *acc, R *T) {
    // the word's address advances by one increment and the loop ends on it,
    // instead of forming the address from a counter at every step
    const ProgPtr end = prog + F::kWords * n;
    for (ProgPtr q = prog; q != end; q += F::kWords) {
        const typename F::W ins = F::load(q, 0);
        const int fid = F::fid(ins);
        const int ak = F::akind(ins), ai = F::aidx(ins);
        R a[P], b[P], o[P], d1[P], d2[P];
        uint64_t z1[P], z2[P];
        // one arity test per step; a binary step fetches the right operand
        // first: the accumulator is then dead once the left one is fetched,
        // and the left operand can share its registers
        if (F::binary(ins)) {
            fetch<R, P>(F::bkind(ins), F::bidx(ins), acc, w, cs, lane, b);
            fetch<R, P>(ak, ai, acc, w, cs, lane, a);
            // POW's log(l) only where its right partial is read: the tape, or a
            // scaled right range (the decoder sets scale_b exactly where
            // hi > mid and the partial is not unit)
            binary_p<R, P, JAC != 1>(fid, a, b, JAC == 2 || (JAC == 1 && F::scale_b(ins)), o, d1,
                                     d2, z1, z2);
            if constexpr (JAC == 2) {
                const int t = F::tape(ins), ta = F::tape_a(ins);
                if (ta) CUSR_FOR_P lds_at<R, P>(w.tape, t, p, lane) = d1[p];
                if (F::tape_b(ins)) CUSR_FOR_P lds_at<R, P>(w.tape, t + ta, p, lane) = d2[p];
            }
        } else {
            fetch<R, P>(ak, ai, acc, w, cs, lane, a);
            // d2 and z2 stay unset: the decoder never sets scale_b on a unary step
            unary_p<R, P, math_chunk<K, R, P, JAC>()>(fid, a, o, d1, z1);
            if constexpr (JAC == 2) {
                if (F::tape_a(ins)) CUSR_FOR_P lds_at<R, P>(w.tape, F::tape(ins), p, lane) = d1[p];
            }
        }
        if constexpr (JAC == 1) {
            // a constant operand k owns the range [k, k+1) and its tangent
            // starts at 1, so one rule covers leaves and subtrees; the decode
            // sets scale_a / scale_b only where a partial is not exactly 1
            // (not for ADD, SUB's left operand or the identity) and the
            // range is non-empty, and sel for the flat-branch operators
            // the fields are read at each site: formed once before both, they
            // were computed on every step and the select flag was kept live
            // as a 64-bit lane mask
            if (F::scale_a(ins))
                scale_range<K, R, P>(T, F::lo(ins), F::mid(ins), d1, z1, F::sel(ins));
            if (F::scale_b(ins))
                scale_range<K, R, P>(T, F::mid(ins), F::hi(ins), d2, z2, F::sel(ins));
        }
        // the decoder spills a value only when its sibling subtree runs next,
        // and that subtree's first instruction reads leaves only: the old
        // accumulator is dead after a spill, so it takes o either way and the
        // loop carries one accumulator (no second copy for the loop's exit)
        const bool spill = F::toslot(ins);
        if (spill) {
            const int di = F::didx(ins);
            CUSR_FOR_P lds_at<R, P>(w.slot, di, p, lane) = o[p];
        }
        CUSR_FOR_P acc[p] = o[p];
    }
}

// Reverse sweep over the tape written by forward_pass<..., 2>:
// T[p*K + k] = d f / d c_k, T zero on entry (cusr/kernel/revad_interp.cuh:131-156). The
// adjoints of spilled values live in the slot area (their values are dead).
template <int K, typename R, int P, typename F = FastFmt>
__device__ __forceinline__ void reverse_pass(ProgPtr prog, int n, const WaveLds<R, P> &w,
                                             int lane, R *T) {
    R accadj[P];
    CUSR_FOR_P accadj[p] = R(1);
    for (int pc = n - 1; pc >= 0; --pc) {
        const typename F::W ins = F::load(prog, pc);
        R adj[P];
        if (F::toslot(ins)) {
            const int di = F::didx(ins);
            CUSR_FOR_P adj[p] = lds_at<R, P>(w.slot, di, p, lane);
        } else {
            CUSR_FOR_P adj[p] = accadj[p];
        }
        const int t = F::tape(ins), ta = F::tape_a(ins);
        const int nop = F::binary(ins) ? 2 : 1;
        for (int side = 0; side < nop; ++side) {
            const int kind = side ? F::bkind(ins) : F::akind(ins);
            const int idx = side ? F::bidx(ins) : F::aidx(ins);
            if (kind == OPD_VAR) continue;
            R g[P];
            if (side ? F::tape_b(ins) : ta) {
                const int slot = t + (side ? ta : 0);
                CUSR_FOR_P g[p] = safe_mul<R>(adj[p], lds_at<R, P>(w.tape, slot, p, lane));
            } else if (side && F::fid(ins) == OP_SUB) {
                // safe_mul(adj, -1) without the tape: -adj, and 0 for a zero adjoint
                CUSR_FOR_P g[p] = (adj[p] == R(0)) ? R(0) : -adj[p];
            } else {
                // safe_mul(adj, +1): ADD, SUB's left operand, the identity
                CUSR_FOR_P g[p] = (adj[p] == R(0)) ? R(0) : adj[p];
            }
            if (kind == OPD_ACC) {
                CUSR_FOR_P accadj[p] = g[p];
            } else if (kind == OPD_SLOT) {
                CUSR_FOR_P lds_at<R, P>(w.slot, idx, p, lane) = g[p];
            } else {
                add_tangent<K, R, P>(T, idx, g);   // T starts at 0: 0 + adjoint
            }
        }
    }
}

// ------------------------------------------------------- one data pass

struct PassArgs {
    ProgPtr prog;       // this expression's program
    int n;
    const double *X;    // [D][N] column-major
    const double *y;    // this expression's targets [N]
    int N, D;
    int parts;          // point partitions G (64-point granule g -> partition g mod G)
    int pwaves;         // wavefronts of the workgroup; wave w sums partitions w, w+pwaves, ...
    int wave;           // this wavefront
    double *part;       // [parts][sums_width(K)] partition sums (parts > 1): LDS, or
                        // HBM on the split path
    double *jt;         // LDS [64][17] augmented Jacobian rows of one slice (matrix sums)
    int split;          // 1: this workgroup sums one partition into part (HBM) and the
                        // step kernel adds the partitions; no combine here
    int part_stride;    // split: doubles between partitions in part (the launch's
                        // widest sums row, which the step kernel reads by)
};

// Matrix sums (forward AD, K >= CO_SUMS_MATRIX_MIN_K): v_mfma_f64_16x16x4 takes A[i][k]
// from lane i + 16k and B[k][j] from lane j + 16k, and returns D[i][j] in
// lane j + 16 (i mod 4), register i / 4; each output is the chain
// c = fma(a_k, b_k, c) over k = 0..3 (measured on gfx950). With A = B^T =
// 4 rows of [J | r], 16 instructions fold one 64-point slice into the
// 16 x 16 accumulator in ascending point order.
typedef double cusr_double4 __attribute__((ext_vector_type(4)));
constexpr int kJtStride = 17;                       // doubles per row (bank spread)
constexpr size_t kJtBytes = (size_t)kLanes * kJtStride * sizeof(double);
template <int K, int AD>
constexpr bool matrix_sums() {
    return AD == CO_AD_FORWARD ? K >= CO_SUMS_MATRIX_MIN_K : K >= CO_SUMS_MATRIX_MIN_K_REV;
}
// Reverse AD stages the rows (and the solve's K x K factor) in the tape's LDS:
// a batch's rows are written after its reverse sweep has read the tape, and
// the solve runs between passes. Every column the matrix instruction reads
// (0..15) is rewritten for each batch, the ones past r with zeros.
template <int K, int AD>
constexpr bool sums_over_tape() { return AD == CO_AD_REVERSE && matrix_sums<K, AD>(); }

constexpr int sums_width(int K) { return 1 + K + K * (K + 1) / 2; }

// Cross-lane exchange of a double with lane ^ S (S = 32, 16, 8, 4, 2, 1):
// ds_bpermute for 32, ds_swizzle (xor mask) for 16, DPP moves below: row_ror:8
// is the xor-8 partner within a row of 16, row_half_mirror then the reversed
// quad permutation is xor 4, quad_perm [2,3,0,1] / [1,0,3,2] are xor 2 / 1.
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int S>
__device__ __forceinline__ int xchg_i32(int v, int lane) {
    if constexpr (S == 32) return __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, v);
    else if constexpr (S == 16) return __builtin_amdgcn_ds_swizzle(v, (16 << 10) | 0x1F);
    else if constexpr (S == 8) return dpp_i32<0x128>(v);
    else if constexpr (S == 4) return dpp_i32<0x1B>(dpp_i32<0x141>(v));
    else if constexpr (S == 2) return dpp_i32<0x4E>(v);
    else return dpp_i32<0xB1>(v);
}
template <int S>
__device__ __forceinline__ double xchg(double v, int lane) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)xchg_i32<S>((int)(uint32_t)u, lane);
    const uint32_t hi = (uint32_t)xchg_i32<S>((int)(uint32_t)(u >> 32), lane);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// The butterfly of the sums over the 64 lanes: at strides 32, 16, ..., 1 lane
// l adds lane l ^ s, so every lane ends with the same sums, the ones the CPU
// oracle forms (p[l] + p[l ^ s]).
template <int W>
__device__ __forceinline__ void wave_allreduce(double (&a)[W], int lane) {
#pragma unroll
    for (int w = 0; w < W; ++w) a[w] = a[w] + xchg<32>(a[w], lane);
#pragma unroll
    for (int w = 0; w < W; ++w) a[w] = a[w] + xchg<16>(a[w], lane);
#pragma unroll
    for (int w = 0; w < W; ++w) a[w] = a[w] + xchg<8>(a[w], lane);
#pragma unroll
    for (int w = 0; w < W; ++w) a[w] = a[w] + xchg<4>(a[w], lane);
#pragma unroll
    for (int w = 0; w < W; ++w) a[w] = a[w] + xchg<2>(a[w], lane);
#pragma unroll
    for (int w = 0; w < W; ++w) a[w] = a[w] + xchg<1>(a[w], lane);
}

// One reduce-scatter step of the butterfly at stride S: a lane keeps the lower
// half of its entries when bit S of its index is clear, the upper half when
// set, and adds the partner's copy of the half it keeps -- the value the
// butterfly has in that lane for those entries.
template <int S, int H>
__device__ __forceinline__ void scatter_step(const double (&a)[2 * H], double (&b)[H], int lane) {
    const bool up = (lane & S) != 0;
#pragma unroll
    for (int j = 0; j < H; ++j) {
        const double keep = up ? a[H + j] : a[j];
        const double send = up ? a[j] : a[H + j];
        b[j] = keep + xchg<S>(send, lane);
    }
}

// The same sums written to dst[0..W): strides 32, 16 and 8 reduce-scatter
// (W padded to a multiple of 8; each lane ends with an eighth of the entries),
// strides 4, 2 and 1 finish the butterfly on those; lanes 0, 8, ..., 56 store.
// Every stored value is the butterfly's, bit for bit.
template <int W>
__device__ __forceinline__ void wave_reduce_store(const double (&acc)[W], double *dst, int lane) {
    if constexpr (W < 8) {
        double a[W];
#pragma unroll
        for (int q = 0; q < W; ++q) a[q] = acc[q];
        wave_allreduce<W>(a, lane);
        if (lane == 0) {
#pragma unroll
            for (int q = 0; q < W; ++q) dst[q] = a[q];
        }
    } else {
        constexpr int W8 = (W + 7) / 8 * 8;
        constexpr int H1 = W8 / 2, H2 = W8 / 4, H3 = W8 / 8;
        double a0[W8], a1[H1], a2[H2], a3[H3];
#pragma unroll
        for (int q = 0; q < W8; ++q) a0[q] = q < W ? acc[q] : 0.0;
        scatter_step<32, H1>(a0, a1, lane);
        scatter_step<16, H2>(a1, a2, lane);
        scatter_step<8, H3>(a2, a3, lane);
#pragma unroll
        for (int j = 0; j < H3; ++j) a3[j] = a3[j] + xchg<4>(a3[j], lane);
#pragma unroll
        for (int j = 0; j < H3; ++j) a3[j] = a3[j] + xchg<2>(a3[j], lane);
#pragma unroll
        for (int j = 0; j < H3; ++j) a3[j] = a3[j] + xchg<1>(a3[j], lane);
        if ((lane & 7) == 0) {
            const int start = ((lane & 32) ? H1 : 0) + ((lane & 16) ? H2 : 0) + ((lane & 8) ? H3 : 0);
#pragma unroll
            for (int j = 0; j < H3; ++j)
                if (start + j < W) dst[start + j] = a3[j];
        }
    }
}

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

// LDS visibility for every wavefront of the workgroup (pwaves uniform).
__device__ __forceinline__ void block_sync(int pwaves) {
    if (pwaves > 1) __syncthreads();
    else wave_sync_lds();
}

// One pass over all points at constants cs (LDS): sums[0] = sum r^2,
// sums[1..K] = J^T r, sums[1+K..] = upper triangle of J^T J (row-major),
// written to out (LDS) by lane 0. JAC: 0 value only, 1 forward, 2 reverse.
template <int K, typename R, int P, int JAC, typename F = FastFmt>
__device__ __forceinline__ void data_pass(const PassArgs &a, const WaveLds<R, P> &w, const double *cs,
                          double *out, int lane) {
    constexpr int W = (JAC == 0) ? 1 : sums_width(K);
    constexpr int KT = (K > 0) ? K : 1;
    constexpr bool MX = (JAC != 0) && matrix_sums<K, (JAC == 2 ? CO_AD_REVERSE : CO_AD_FORWARD)>();
    // per-lane accumulators: all sums, or (matrix sums, K = 16) r^2 and J^T r
    constexpr int WL = MX ? ((K < 16) ? 1 : 1 + K) : W;
    const int granules = (a.N + kLanes - 1) / kLanes;
    const int last = a.N - 1;
    for (int part = a.wave; part < a.parts; part += a.pwaves) {
    double acc[WL];
#pragma unroll
    for (int q = 0; q < WL; ++q) acc[q] = 0.0;
    cusr_double4 g4 = {0.0, 0.0, 0.0, 0.0};
    // granules part, part + G, part + 2G, ... of this partition, P per batch
    const int ng = (part < granules) ? (granules - part + a.parts - 1) / a.parts : 0;
    const int batches = (ng + P - 1) / P;
    for (int bt = 0; bt < batches; ++bt) {
        // Every load of the batch is issued before the first one is used:
        // points past N read point N-1 (in bounds, never accumulated), so no
        // load sits behind a branch and one memory latency covers the batch.
        double yv[P];
        bool valid[P];
        int ic[P];
        CUSR_FOR_P {
            const int gi = bt * P + p;
            const int i = (part + a.parts * gi) * kLanes + lane;
            valid[p] = gi < ng && i < a.N;
            ic[p] = valid[p] ? i : last;
        }
        CUSR_FOR_P yv[p] = a.y[ic[p]];
#pragma unroll 2
        for (int v = 0; v < a.D; ++v) {
            const double *col = a.X + (size_t)v * a.N;
            double xv[P];
            CUSR_FOR_P xv[p] = col[ic[p]];
            CUSR_FOR_P lds_at<R, P>(w.x, v, p, lane) = (R)xv[p];
        }
        R accv[P];
        R T[P * KT];
#pragma unroll
        for (int j = 0; j < P * KT; ++j) T[j] = (JAC == 1) ? R(1) : R(0);
        forward_pass<K, R, P, JAC, F>(a.prog, a.n, w, cs, lane, accv, T);
        if constexpr (JAC == 2) reverse_pass<K, R, P, F>(a.prog, a.n, w, lane, T);
        if constexpr (MX) {
            CUSR_FOR_P {
                const double r = valid[p] ? (double)accv[p] - yv[p] : 0.0;
                double *row = a.jt + lane * kJtStride;
#pragma unroll
                for (int j = 0; j < K; ++j) row[j] = valid[p] ? (double)T[p * KT + j] : 0.0;
                if constexpr (JAC == 2) {
                    // rows over the tape: the columns past r are rewritten too
#pragma unroll
                    for (int j = K + 1; j < 16; ++j) row[j] = 0.0;
                }
                if constexpr (K < 16) {
                    row[K] = r;
                } else if (valid[p]) {
                    acc[0] = fma(r, r, acc[0]);
#pragma unroll
                    for (int j = 0; j < K; ++j) acc[1 + j] = fma((double)T[p * KT + j], r, acc[1 + j]);
                }
                wave_sync_lds();
#pragma unroll
                for (int m = 0; m < 16; ++m) {
                    const double v = a.jt[(4 * m + (lane >> 4)) * kJtStride + (lane & 15)];
                    g4 = __builtin_amdgcn_mfma_f64_16x16x4f64(v, v, g4, 0, 0, 0);
                }
                wave_sync_lds();
            }
            continue;
        }
        CUSR_FOR_P {
            if (valid[p]) {
                const double r = (double)accv[p] - yv[p];
                acc[0] = fma(r, r, acc[0]);
                if constexpr (JAC != 0) {
#pragma unroll
                    for (int j = 0; j < K; ++j)
                        acc[1 + j] = fma((double)T[p * KT + j], r, acc[1 + j]);
                    int q = 1 + K;
#pragma unroll
                    for (int j1 = 0; j1 < K; ++j1)
#pragma unroll
                        for (int j2 = j1; j2 < K; ++j2, ++q)
                            acc[q] = fma((double)T[p * KT + j1], (double)T[p * KT + j2], acc[q]);
                }
            }
        }
    }
    double *dst = (a.parts == 1) ? out : a.part + part * (a.split ? a.part_stride : W);
    if constexpr (MX) {
        // the accumulator to LDS as G[16][16], then the sums vector by lane 0
        double *gt = a.jt;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) gt[(4 * r4 + (lane >> 4)) * 16 + (lane & 15)] = g4[r4];
        if constexpr (K == 16) wave_reduce_store<WL>(acc, dst, lane);
        wave_sync_lds();
        if (lane == 0) {
            if constexpr (K < 16) {
                dst[0] = gt[K * 16 + K];
#pragma unroll
                for (int j = 0; j < K; ++j) dst[1 + j] = gt[j * 16 + K];
            }
            int q = 1 + K;
#pragma unroll
            for (int j1 = 0; j1 < K; ++j1)
#pragma unroll
                for (int j2 = j1; j2 < K; ++j2, ++q) dst[q] = gt[j1 * 16 + j2];
        }
        wave_sync_lds();
    } else {
        wave_reduce_store<WL>(acc, dst, lane);
    }
    }
    if (a.parts == 1 || a.split) {
        wave_sync_lds();
        return;
    }
    // partition sums added in partition order, sum q by lane q mod 64 of the
    // first wavefront
    __syncthreads();
    if (a.wave == 0) {
        for (int q = lane; q < W; q += kLanes) {
            double v = a.part[q];
            for (int g = 1; g < a.parts; ++g) v = v + a.part[g * W + q];
            out[q] = v;
        }
    }
    __syncthreads();
}

// The general kernel's Jacobian pass (runtime K = Kr <= CO_MAX_K, one point
// per lane): sums[0] = sum r^2, sums[1..Kr] = J^T r, then the upper triangle
// of J^T J, every entry one fma chain over the partition's points in ascending
// order. The 64 augmented rows [J | r] of a slice go to LDS (jt, [64][kGenStride],
// r in column Kr); v_mfma_f64_16x16x4 then folds them four points at a time into
// the 16 x 16 blocks (a, b), a <= b, of [J | r]^T [J | r]: nb = ceil((Kr+1)/16)
// column blocks, nb (nb+1) / 2 accumulators. Columns past Kr read column Kr
// (so every operand is defined); the entries they produce are never read.
// The accumulators then go straight to the sums vector: register r4 of lane l
// holds entry (4 r4 + l / 16, l mod 16) of its block.
constexpr int kGenK = CO_MAX_K;
constexpr int kGenStride = kGenK + 1;   // doubles per staged row: [J | r]
constexpr size_t kGenJtBytes = (size_t)kLanes * kGenStride * sizeof(double);

// Entries (i, j), i <= j <= Kr, of the 16 x 16 block (ba, bb) of
// [J | r]^T [J | r] (accumulator g: register r4 of lane l holds entry
// (4 r4 + l / 16, l mod 16)) to their places in the sums vector.
__device__ __forceinline__ void put_block(double *dst, cusr_double4 g, int ba, int bb, int Kr,
                                          int lane) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
        const int i = 16 * ba + 4 * r4 + (lane >> 4), j = 16 * bb + (lane & 15);
        if (i > j || j > Kr) continue;
        const int q = (j == Kr) ? ((i == Kr) ? 0 : 1 + i)
                                : 1 + Kr + i * Kr - (i * (i - 1)) / 2 + (j - i);
        dst[q] = g[r4];
    }
}

template <typename R, int JAC, typename F>
__device__ __forceinline__ void data_pass_gen(const PassArgs &a, const WaveLds<R, 1> &w,
                                              const double *cs, double *out, int lane, int Kr) {
    constexpr int K = kGenK;
    const int W = sums_width(Kr);
    const int nb = (Kr + 16) / 16;
    const int granules = (a.N + kLanes - 1) / kLanes;
    const int last = a.N - 1;
    double *jt = a.jt;
    const int c16 = lane & 15;
    const int col0 = c16 < Kr ? c16 : Kr;
    const int col1 = 16 + c16 < Kr ? 16 + c16 : Kr;
    const int col2 = 32 + c16 < Kr ? 32 + c16 : Kr;
    for (int part = a.wave; part < a.parts; part += a.pwaves) {
        cusr_double4 g0 = {0.0, 0.0, 0.0, 0.0}, g1 = g0, g2 = g0, g3 = g0, g4 = g0, g5 = g0;
        const int ng = (part < granules) ? (granules - part + a.parts - 1) / a.parts : 0;
        for (int gi = 0; gi < ng; ++gi) {
            // points past N read point N-1 (in bounds) and stage a zero row
            const int i = (part + a.parts * gi) * kLanes + lane;
            const bool valid = i < a.N;
            const int ic = valid ? i : last;
            const double yv = a.y[ic];
            for (int v = 0; v < a.D; ++v)
                lds_at<R, 1>(w.x, v, 0, lane) = (R)a.X[(size_t)v * a.N + ic];
            R accv[1];
            R T[K];
#pragma unroll
            for (int j = 0; j < K; ++j) T[j] = (JAC == 1) ? R(1) : R(0);
            forward_pass<K, R, 1, JAC, F>(a.prog, a.n, w, cs, lane, accv, T);
            if constexpr (JAC == 2) reverse_pass<K, R, 1, F>(a.prog, a.n, w, lane, T);
            const double r = valid ? (double)accv[0] - yv : 0.0;
            double *row = jt + lane * kGenStride;
#pragma unroll
            for (int j = 0; j < K; ++j) row[j] = valid ? (double)T[j] : 0.0;
            row[Kr] = r;
            wave_sync_lds();
#pragma unroll
            for (int m = 0; m < 16; ++m) {
                const double *pr = jt + (4 * m + (lane >> 4)) * kGenStride;
                const double v0 = pr[col0];
                g0 = __builtin_amdgcn_mfma_f64_16x16x4f64(v0, v0, g0, 0, 0, 0);
                if (nb > 1) {
                    const double v1 = pr[col1];
                    g1 = __builtin_amdgcn_mfma_f64_16x16x4f64(v0, v1, g1, 0, 0, 0);
                    g2 = __builtin_amdgcn_mfma_f64_16x16x4f64(v1, v1, g2, 0, 0, 0);
                    if (nb > 2) {
                        const double v2 = pr[col2];
                        g3 = __builtin_amdgcn_mfma_f64_16x16x4f64(v0, v2, g3, 0, 0, 0);
                        g4 = __builtin_amdgcn_mfma_f64_16x16x4f64(v1, v2, g4, 0, 0, 0);
                        g5 = __builtin_amdgcn_mfma_f64_16x16x4f64(v2, v2, g5, 0, 0, 0);
                    }
                }
            }
            wave_sync_lds();
        }
        double *dst = (a.parts == 1) ? out : a.part + part * (a.split ? a.part_stride : W);
        put_block(dst, g0, 0, 0, Kr, lane);
        if (nb > 1) {
            put_block(dst, g1, 0, 1, Kr, lane);
            put_block(dst, g2, 1, 1, Kr, lane);
        }
        if (nb > 2) {
            put_block(dst, g3, 0, 2, Kr, lane);
            put_block(dst, g4, 1, 2, Kr, lane);
            put_block(dst, g5, 2, 2, Kr, lane);
        }
    }
    if (a.parts == 1 || a.split) {
        wave_sync_lds();
        return;
    }
    // partition sums added in partition order, sum q by lane q mod 64 of the
    // first wavefront
    __syncthreads();
    if (a.wave == 0) {
        for (int q = lane; q < W; q += kLanes) {
            double v = a.part[q];
            for (int g = 1; g < a.parts; ++g) v = v + a.part[g * W + q];
            out[q] = v;
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------ the solve

// The damping variants of the solve (cusr/kernel/batch_lm_ad.cu:149-172):
// the damped diagonal, and the rule for a pivot s_j (false: the step fails).
// CO_DAMP_RELATIVE: A_jj (1 + lambda), fail on s_j <= 0; CO_DAMP_TRUST_REGION:
// A_jj + lambda, s_j <= 0 becomes lambda; CO_DAMP_PIVOT_FLOOR: A_jj (1 + lambda),
// s_j below CO_PIVOT_FLOOR_EPS becomes it. A NaN pivot passes every rule (and
// its NaN step is a non-finite trial). REL: the relative rule alone, compiled
// as it stands; otherwise selects on the wave-uniform mode. The solve sits on
// each iteration's dependent chain: run-time tests in the default solve made
// the K = 7 fit kernel 1.5 % and C3's K = 15 bin 3.5 % slower, so callers
// branch once to a REL instance for the default.
template <bool REL>
__device__ __forceinline__ double damp_diag(double a, double lambda, int damp) {
    if constexpr (REL) {
        return a * (1.0 + lambda);
    } else {
        const double absolute = a + lambda, relative = a * (1.0 + lambda);
        return damp == CO_DAMP_TRUST_REGION ? absolute : relative;
    }
}
template <bool REL>
__device__ __forceinline__ bool damp_pivot(double &sj, double lambda, int damp) {
    if constexpr (REL) {
        return !(sj <= 0.0);
    } else {
        const bool fl = damp == CO_DAMP_PIVOT_FLOOR, rel = damp == CO_DAMP_RELATIVE;
        const bool low = (fl & (sj < CO_PIVOT_FLOOR_EPS)) | (!fl & (sj <= 0.0));
        const double repl = fl ? CO_PIVOT_FLOOR_EPS : lambda;
        sj = (low & !rel) ? repl : sj;
        return !(low & rel);
    }
}

// Damped Cholesky solve of (J^T J + damping) delta = -J^T r from pass sums s
// (cusr/kernel/batch_lm_ad.cu:149-191) under damping variant damp; false when
// the pivot rule fails the step. Every lane computes the same result.
template <int K, bool REL>
__device__ __forceinline__ bool damped_solve(const double *s, double lambda, int damp,
                                             double (&delta)[K]) {
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
        L[i][i] = damp_diag<REL>(L[i][i], lambda, damp);
    }
    bool ok = true;
#pragma unroll
    for (int j = 0; j < K; ++j) {
        double sj = L[j][j];
#pragma unroll
        for (int k = 0; k < j; ++k) sj = fma(-L[j][k], L[j][k], sj);
        if (!damp_pivot<REL>(sj, lambda, damp)) ok = false;
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

// The same solve with L in LDS, K at run time (the general kernel, and the
// fast kernels with matrix sums, where K(K+1)/2 doubles per lane of the
// register version would set the kernel's register count). Every element gets
// exactly the arithmetic of damped_solve: column j's pivot is computed by
// every lane, the entries below it by lane i; the substitutions run on every
// lane with L read by broadcast. The solution is left in L[K*K .. K*K+K).
template <bool REL>
__device__ __forceinline__ bool damped_solve_rt(const double *s, double lambda, int damp, int K,
                                                double *L, int lane) {
    double *b = L + K * K;   // right-hand side, then the solution (LDS, K doubles)
    // L[i][j] = upper-triangle element (j, i) of J^T J for j <= i; diagonal damped
    if (lane < K) {
        const int i = lane;
        for (int j = 0; j <= i; ++j) {
            double v = s[1 + K + j * K - (j * (j - 1)) / 2 + (i - j)];
            if (j == i) v = damp_diag<REL>(v, lambda, damp);
            L[i * K + j] = v;
        }
        b[i] = -s[1 + i];
    }
    wave_sync_lds();
    bool ok = true;
#pragma unroll 1
    for (int j = 0; j < K; ++j) {
        double sj = L[j * K + j];
        for (int k = 0; k < j; ++k) sj = fma(-L[j * K + k], L[j * K + k], sj);
        if (!damp_pivot<REL>(sj, lambda, damp)) ok = false;
        const double dj = ::sqrt(sj);
        if (lane > j && lane < K) {
            const int i = lane;
            double t = L[i * K + j];
            for (int k = 0; k < j; ++k) t = fma(-L[i * K + k], L[j * K + k], t);
            L[i * K + j] = t / dj;
        }
        wave_sync_lds();
        if (lane == j) L[j * K + j] = dj;
        wave_sync_lds();
    }
    if (!ok) return false;
#pragma unroll 1
    for (int i = 0; i < K; ++i) {
        double t = b[i];
        for (int k = 0; k < i; ++k) t = fma(-L[i * K + k], b[k], t);
        wave_sync_lds();
        if (lane == 0) b[i] = t / L[i * K + i];
        wave_sync_lds();
    }
#pragma unroll 1
    for (int i = K - 1; i >= 0; --i) {
        double t = b[i];
        for (int k = i + 1; k < K; ++k) t = fma(-L[k * K + i], b[k], t);
        wave_sync_lds();
        if (lane == 0) b[i] = t / L[i * K + i];
        wave_sync_lds();
    }
    return true;
}

template <int K, bool REL>
__device__ __forceinline__ bool damped_solve_lds(const double *s, double lambda, int damp,
                                                 double (&delta)[K], double *L, int lane) {
    if (!damped_solve_rt<REL>(s, lambda, damp, K, L, lane)) return false;
#pragma unroll
    for (int i = 0; i < K; ++i) delta[i] = L[K * K + i];
    return true;
}

// ------------------------------------------------------------- the fit

struct FitArgs {
    const uint64_t *prog;
    const ExprDesc *desc;   // by launch position (offset to the bin's start)
    const double *X;        // [D][N]
    const double *Y;        // [M][N], or [N] when shared_y
    const double *C0;       // [total_c]
    double *C;              // [total_c] out
    int32_t *status;        // [M] out
    double *loss_init;      // [M] out
    double *loss_final;     // [M] out
    int32_t *iters;         // [M] out
    int N, D, max_iter, guard, lm_order;
    int damp;               // CO_DAMP_* of the solve
    int shared_y;           // 1: Y is one row [N] shared by every expression
    int f32_range;          // 1: constants and losses held to the fp32 range
    double lambda0, xtol;
    int slots, tape;        // per-wave LDS rows of this launch ([row][P][64] each)
    int parts;              // point partitions per expression (1, 2 or 4)
    int pwaves;             // wavefronts of the workgroup (divides parts)
    int wave_bytes;         // dynamic LDS of one wavefront; partition sums follow
    // segments of the iteration loop: this launch runs iterations up to it_end
    // (<= max_iter); an expression still running there saves its loop state
    // to state[y_row * state_stride] (and its constants to C) for the next
    // launch, which resumes it (resume = 1) or, for expressions that
    // finished, exits
    int it_end, resume;
    int state_stride;       // doubles per state row, >= kStateSums + sums_width(K)
    double *state;          // [M][state_stride], null for single-launch fits
    // the split path: partition sums of the launch's expressions in HBM,
    // [launch position][parts][psum_width]
    double *psum;
    int psum_width;
};

// loop state of a paused fit, per expression: loss, loss_init, lambda,
// internal status (kStateDone once the outputs are written), iterations,
// then the sums at the current constants
constexpr int kStateSums = 8;
constexpr double kStateDone = -1.0;
constexpr int state_stride_for(int K) { return kStateSums + sums_width(K); }

// internal states, mapped to STATUS_* at the end (lm_core.cuh:46-56)
enum { ST_RUN = 0, ST_CONV = 1, ST_NAN = 2, ST_K0 = 3, ST_CHOL = 4 };

// A loss the fit may go on from (batch_lm_ad.cu:437-443): finite, and under
// f32_range finite in fp32 too, where the reference accumulates it.
__device__ __forceinline__ bool loss_ok(const FitArgs &fa, double loss) {
    return isfinite(loss) && (!fa.f32_range || isfinite((float)loss));
}

// Static LDS of a fit kernel: current and trial constants, current and trial
// sums, sized for the kernel family's largest K.
template <bool GEN>
struct FitStatic {
    static constexpr int KC = GEN ? CO_MAX_K : CO_FAST_MAX_K;
    static constexpr int SW = sums_width(KC);
};

// Points per lane of a fit's passes and of its fp64 audit passes: the
// general kernel runs one of each.
template <bool GEN, typename R, int K, int AD, int LN>
constexpr int fit_points() {
    if constexpr (GEN) return 1;
    else return points_per_pass<R, K, AD, LN>();
}
template <bool GEN, typename R, int K, int AD, int LN>
constexpr int fit_audit_points() {
    if constexpr (GEN) return 1;
    else return audit_points<R, K, AD, LN>();
}

template <int K, typename R, int AD, int LN, bool GEN = false>
__device__ __forceinline__ void fit_one(const FitArgs &fa, const ExprDesc &e, double *lds_c, double *lds_s,
                        char *lds_dyn, int lane, int wave) {
    typedef typename std::conditional<GEN, WideFmt, FastFmt>::type F;
    constexpr int P = fit_points<GEN, R, K, AD, LN>();
    constexpr int JAC = (K == 0) ? 0 : (AD == CO_AD_REVERSE ? 2 : 1);
    constexpr int KC = FitStatic<GEN>::KC;
    const int Kr = GEN ? e.K : K;   // the expression's K (wave-uniform)
    char *my_lds = lds_dyn + (size_t)wave * fa.wave_bytes;
    const bool lead = wave == 0;     // the wavefront that writes shared state
    double *jt = (double *)my_lds;   // matrix sums: the slice's augmented rows first
    // then the K x K Cholesky factor and rhs (the general kernel's solve
    // reuses the rows' bytes: it runs between passes; reverse AD puts both
    // in the tape's bytes)
    if constexpr (GEN) {
        my_lds += kGenJtBytes;
    } else if constexpr (matrix_sums<K, AD>() && !sums_over_tape<K, AD>()) {
        // columns K+1.. of every row stay zero for the whole fit
#pragma unroll
        for (int j = 0; j < kJtStride; ++j) jt[lane * kJtStride + j] = 0.0;
        my_lds += kJtBytes + (size_t)K * (K + 1) * sizeof(double);
    }
    WaveLds<R, P> wl;
    wl.x = (R *)my_lds;
    wl.slot = wl.x + (size_t)fa.D * P * kLanes;
    wl.tape = wl.slot + (size_t)fa.slots * P * kLanes;
    if constexpr (!GEN && sums_over_tape<K, AD>()) jt = (double *)wl.tape;
    double *lds_l = GEN ? jt : jt + kLanes * kJtStride;
    PassArgs pa;
    pa.prog = (ProgPtr)(fa.prog + e.prog_off);
    pa.n = e.n;
    pa.X = fa.X;
    pa.y = fa.Y + (fa.shared_y ? (size_t)0 : (size_t)e.y_row * fa.N);
    pa.N = fa.N;
    pa.D = fa.D;
    pa.parts = fa.parts;
    pa.pwaves = fa.pwaves;
    pa.wave = wave;
    pa.part = (double *)(lds_dyn + (size_t)fa.pwaves * fa.wave_bytes);
    pa.jt = jt;
    pa.split = 0;
    pa.part_stride = 0;

    double *c_cur = lds_c, *c_try = lds_c + KC;
    double *s_cur = lds_s, *s_try = lds_s + FitStatic<GEN>::SW;
    double *sv = fa.state ? fa.state + (size_t)e.y_row * fa.state_stride : nullptr;
    double loss, loss_init, lambda;
    int st, it;
    if (!fa.resume) {
        if (lead && lane < Kr) c_cur[lane] = fa.C0[e.c_off + lane];
        block_sync(fa.pwaves);
        if constexpr (GEN) {
            if (Kr == 0) data_pass<0, R, 1, 0, F>(pa, wl, c_cur, s_cur, lane);
            else data_pass_gen<R, JAC, F>(pa, wl, c_cur, s_cur, lane, Kr);
        } else {
            data_pass<K, R, P, JAC, F>(pa, wl, c_cur, s_cur, lane);
        }
        loss = uni(0.5 * s_cur[0]);
        loss_init = loss;
        st = (Kr == 0) ? ST_K0 : (loss_ok(fa, loss) ? ST_RUN : ST_NAN);
        lambda = fa.lambda0;
        it = 0;
    } else {
        // an expression that finished in an earlier launch has nothing to do
        const double sst = uni(sv[3]);
        if (sst == kStateDone) return;
        if (lead) {
            if (lane < Kr) c_cur[lane] = fa.C[e.c_off + lane];
            for (int j = lane; j < sums_width(Kr); j += kLanes) s_cur[j] = sv[kStateSums + j];
        }
        loss = uni(sv[0]);
        loss_init = uni(sv[1]);
        lambda = uni(sv[2]);
        st = (int)sst;
        it = (int)uni(sv[4]);
        block_sync(fa.pwaves);
    }
    if constexpr (K > 0) {
        while (uni(st) == ST_RUN && it < fa.it_end) {
            ++it;
            double delta[GEN ? 1 : K];
            bool solved;
            if constexpr (GEN)
                solved = fa.damp == CO_DAMP_RELATIVE
                             ? damped_solve_rt<true>(s_cur, lambda, 0, Kr, lds_l, lane)
                             : damped_solve_rt<false>(s_cur, lambda, fa.damp, Kr, lds_l, lane);
            else if constexpr (matrix_sums<K, AD>())
                solved = fa.damp == CO_DAMP_RELATIVE
                             ? damped_solve_lds<K, true>(s_cur, lambda, 0, delta, lds_l, lane)
                             : damped_solve_lds<K, false>(s_cur, lambda, fa.damp, delta, lds_l,
                                                          lane);
            else
                solved = fa.damp == CO_DAMP_RELATIVE
                             ? damped_solve<K, true>(s_cur, lambda, 0, delta)
                             : damped_solve<K, false>(s_cur, lambda, fa.damp, delta);
            if (!solved) {
                lambda = lambda * 10.0;
                if (lambda > 1e12) st = ST_CHOL;
                continue;
            }
            // every wavefront is done reading c_try (the norm below) before
            // the lead overwrites it
            if (fa.pwaves > 1) __syncthreads();
            double dn2 = 0.0, cn2 = 0.0;
            if constexpr (GEN) {
                // the solution sits in the rows' bytes, which the pass
                // overwrites: the step norms are formed before it
                const double *db = lds_l + Kr * Kr;
                if (lead && lane < Kr) {
                    const double v = c_cur[lane] + db[lane];
                    c_try[lane] = fa.f32_range ? (double)(float)v : v;
                }
                block_sync(fa.pwaves);
                for (int j = 0; j < Kr; ++j) {
                    dn2 = fma(db[j], db[j], dn2);
                    cn2 = fma(c_try[j], c_try[j], cn2);
                }
            } else {
                if (lead && lane < K) {
#pragma unroll
                    for (int j = 0; j < K; ++j) {
                        if (j == lane) {
                            const double v = c_cur[j] + delta[j];
                            c_try[j] = fa.f32_range ? (double)(float)v : v;
                        }
                    }
                }
                block_sync(fa.pwaves);
            }
            if (fa.f32_range) {
                // trial constants are held in fp32, as the reference's are; one
                // beyond the fp32 range makes its trial loss non-finite
                // (batch_lm_ad.cu:437-443): no pass needed
                int over = 0;
                for (int j = 0; j < Kr; ++j) over |= !isfinite(c_try[j]) ? 1 : 0;
                if (uni(over)) {
                    st = ST_NAN;
                    continue;
                }
            }
            if constexpr (GEN) {
                data_pass_gen<R, JAC, F>(pa, wl, c_try, s_try, lane, Kr);
            } else {
                data_pass<K, R, P, JAC, F>(pa, wl, c_try, s_try, lane);
#pragma unroll
                for (int j = 0; j < K; ++j) {
                    dn2 = fma(delta[j], delta[j], dn2);
                    cn2 = fma(c_try[j], c_try[j], cn2);
                }
            }
            const double loss_try = uni(0.5 * s_try[0]);
            if (!loss_ok(fa, loss_try)) { st = ST_NAN; continue; }
            const double dn = ::sqrt(dn2), cn = ::sqrt(cn2);
            const bool small = dn < fa.xtol * (cn + fa.xtol);
            bool accept, conv;
            if (fa.lm_order == CO_ORDER_CONVERGE_FIRST) {
                // FD variant (co_lib.cu:457-473): a small step converges
                // whatever the loss; otherwise only a strict decrease
                conv = small;
                accept = small || loss_try < loss;
            } else {
                // AD variant (batch_lm_ad.cu:456-473): improvement first
                accept = loss_try <= loss;
                conv = accept && small;
            }
            if (accept) {
                double *t = c_cur; c_cur = c_try; c_try = t;
                t = s_cur; s_cur = s_try; s_try = t;
                loss = loss_try;
            }
            if (conv) {
                st = ST_CONV;
            } else if (accept) {
                lambda = lambda * 0.1;
                if (lambda < 1e-12) lambda = 1e-12;
            } else {
                lambda = lambda * 10.0;
                if (lambda > 1e12) st = ST_NAN;
            }
        }
    }
    if (st == ST_RUN && it < fa.max_iter) {
        // paused at the end of this launch's segment: save the loop state
        if (lead) {
            if (lane < Kr) fa.C[e.c_off + lane] = c_cur[lane];
            for (int j = lane; j < sums_width(Kr); j += kLanes) sv[kStateSums + j] = s_cur[j];
            if (lane == 0) {
                sv[0] = loss;
                sv[1] = loss_init;
                sv[2] = lambda;
                sv[3] = (double)st;
                sv[4] = (double)it;
            }
        }
        return;
    }
    double lf = loss, li = loss_init;
    if constexpr (sizeof(R) == 4) {
        // fp64 losses at the delivered point and at the start; the fp64
        // value pass reuses the same LDS bytes per row and lane (half the
        // points of the fp32 passes). A lane sums its points in the same
        // ascending order at any number of points per pass.
        constexpr int AP = fit_audit_points<GEN, R, K, AD, LN>();
        constexpr int KA = GEN ? 0 : K;
        WaveLds<double, AP> w64;
        w64.x = (double *)my_lds;
        w64.slot = w64.x + (size_t)fa.D * AP * kLanes;
        w64.tape = w64.slot + (size_t)fa.slots * AP * kLanes;
        data_pass<KA, double, AP, 0, F>(pa, w64, c_cur, s_try, lane);
        lf = uni(0.5 * s_try[0]);
        if (fa.pwaves > 1) __syncthreads();
        if (lead && lane < Kr) c_try[lane] = fa.C0[e.c_off + lane];
        block_sync(fa.pwaves);
        data_pass<KA, double, AP, 0, F>(pa, w64, c_try, s_try, lane);
        li = uni(0.5 * s_try[0]);
    }
    bool revert = false;
    if (fa.guard && Kr > 0) revert = !isfinite(lf) || (isfinite(li) && lf > li);
    if (revert) {
        if (st == ST_CONV) st = ST_RUN;
        lf = li;
    }
    if (!lead) return;
    if (lane < Kr) fa.C[e.c_off + lane] = revert ? fa.C0[e.c_off + lane] : c_cur[lane];
    if (lane == 0) {
        // ST_RUN -> STATUS_MAXITER, ST_CONV -> STATUS_CONVERGED, the rest keep their code
        fa.status[e.y_row] = (st <= ST_CONV) ? (1 - st) : st;
        if (sv) sv[3] = kStateDone;
        fa.loss_init[e.y_row] = li;
        fa.loss_final[e.y_row] = lf;
        fa.iters[e.y_row] = it;
    }
}

// One kernel per (K, precision, AD mode): each K gets its own register
// allocation, so small-K expressions are not held to the occupancy of K = 16.
// Minimum waves per SIMD the register allocation must allow, per K (fp64
// forward / everything else); 2 caps a kernel at 256 VGPRs.
#ifndef CUSR_W64_TABLE
#define CUSR_W64_TABLE 1, 1, 1, 2, 2, 2, 2, 2, 2, 1, 1, 1, 1, 1, 1, 1, 1
#endif
// fp64 reverse AD, the fit kernels (N below the split path's): no cap except
// K = 9 (256 VGPRs with 23 spilled beats 300 at one wave per SIMD; from K = 10
// the spills grow to 76 and more)
#ifndef CUSR_WREV64_TABLE
#define CUSR_WREV64_TABLE 1, 1, 1, 1, 1, 1, 1, 1, 1, 2, 1, 1, 1, 1, 1, 1, 1
#endif
#ifndef CUSR_W64_LARGE_N_TABLE
#define CUSR_W64_LARGE_N_TABLE 1, 3, 3, 3, 3, 3, 3, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1
#endif
#ifndef CUSR_WAVES_OTHER
#define CUSR_WAVES_OTHER 1
#endif
constexpr int kW64[CO_FAST_MAX_K + 1] = {CUSR_W64_TABLE};
constexpr int kW64LargeN[CO_FAST_MAX_K + 1] = {CUSR_W64_LARGE_N_TABLE};
constexpr int kWRev64[CO_FAST_MAX_K + 1] = {CUSR_WREV64_TABLE};
template <typename R, int K, int AD, int LN = 0>
constexpr int waves_per_eu() {
    return sizeof(R) == 8 ? (AD == CO_AD_FORWARD ? (LN ? kW64LargeN[K] : kW64[K]) : kWRev64[K])
                          : CUSR_WAVES_OTHER;
}
// fp64 reverse AD on the split path (the pass kernels: one wavefront per
// workgroup, one point per lane): two waves per SIMD from K = 9 to 14, where
// one wavefront per SIMD issued its SALU and VALU back to back (C3 127.4 ->
// 116.7 ms); K = 15, 16 keep their 358 and 390 VGPRs (at 256 they spill
// heavily: C3 126.6 ms with two waves for K = 9..16).
#ifndef CUSR_WREV64_SPLIT_TABLE
#define CUSR_WREV64_SPLIT_TABLE 1, 1, 1, 1, 1, 1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 1, 1
#endif
constexpr int kWRev64Split[CO_FAST_MAX_K + 1] = {CUSR_WREV64_SPLIT_TABLE};
template <typename R, int K, int AD, int LN = 0>
constexpr int pass_waves_per_eu() {
    return (sizeof(R) == 8 && AD == CO_AD_REVERSE) ? kWRev64Split[K]
                                                   : waves_per_eu<R, K, AD, LN>();
}
// True when the large-N tables give (R, K, AD) another kernel (only those
// get an LN = 1 instance).
template <typename R, int K, int AD>
constexpr bool large_n_variant() {
    return points_per_pass<R, K, AD, 1>() != points_per_pass<R, K, AD, 0>() ||
           waves_per_eu<R, K, AD, 1>() != waves_per_eu<R, K, AD, 0>();
}
template <int K, typename R, int AD, int LN = 0>
__global__ void __launch_bounds__(kLanes * CO_MAX_PARTITIONS, (waves_per_eu<R, K, AD, LN>()))
lm_fit_kernel(FitArgs fa) {
    __shared__ double lds_c[2 * FitStatic<false>::KC];
    __shared__ double lds_s[2 * FitStatic<false>::SW];
    extern __shared__ char lds_dyn[];
    const ExprDesc e = fa.desc[blockIdx.x];
    const int lane = (int)threadIdx.x & (kLanes - 1);
    const int wave = uni((int)threadIdx.x >> 6);
    fit_one<K, R, AD, LN>(fa, e, lds_c, lds_s, lds_dyn, lane, wave);
}

// The general kernel: runtime K <= CO_MAX_K, wide programs, one point per
// lane; tangents / gradients in 32 fixed registers, sums on the matrix unit.
#ifndef CUSR_WAVES_GEN
#define CUSR_WAVES_GEN 2
#endif
template <typename R, int AD>
__global__ void __launch_bounds__(kLanes * CO_MAX_PARTITIONS, CUSR_WAVES_GEN)
lm_fit_gen_kernel(FitArgs fa) {
    __shared__ double lds_c[2 * FitStatic<true>::KC];
    __shared__ double lds_s[2 * FitStatic<true>::SW];
    extern __shared__ char lds_dyn[];
    const ExprDesc e = fa.desc[blockIdx.x];
    const int lane = (int)threadIdx.x & (kLanes - 1);
    const int wave = uni((int)threadIdx.x >> 6);
    fit_one<kGenK, R, AD, 0, true>(fa, e, lds_c, lds_s, lds_dyn, lane, wave);
}

// Static LDS bytes of a fit kernel family (kept out of the dynamic budget).
constexpr size_t fit_static_lds(bool gen) {
    return gen ? (2 * FitStatic<true>::KC + 2 * FitStatic<true>::SW) * sizeof(double)
               : (2 * FitStatic<false>::KC + 2 * FitStatic<false>::SW) * sizeof(double);
}

// Dynamic LDS bytes one wavefront of a fit launch needs (the mixed-precision
// fp64 audit pass reuses the same bytes at audit_points per lane).
template <typename R, int K, int AD, int LN = 0>
constexpr size_t fit_lds_bytes_t(int D, int slots, int tape) {
    const size_t row = (size_t)points_per_pass<R, K, AD, LN>() * kLanes * sizeof(R);
    const size_t mx = matrix_sums<K, AD>() ? kJtBytes + (size_t)K * (K + 1) * sizeof(double) : 0;
    const size_t t = sums_over_tape<K, AD>() && mx > (size_t)tape * row ? mx : (size_t)tape * row;
    const size_t a = (size_t)(D + slots) * row + t;
    const size_t b = (size_t)(D + slots) * audit_points<R, K, AD, LN>() * kLanes * sizeof(double);
    return (sums_over_tape<K, AD>() ? 0 : mx) + (a > b ? a : b);
}

// ... of a general-kernel launch (one point per lane; the fp64 audit at one)
template <typename R>
constexpr size_t fit_lds_bytes_gen(int D, int slots, int tape) {
    const size_t a = (size_t)(D + slots + tape) * kLanes * sizeof(R);
    const size_t b = (size_t)(D + slots) * kLanes * sizeof(double);
    return kGenJtBytes + (a > b ? a : b);
}

// Launch the fit kernel of one bin (k <= CO_FAST_MAX_K: the fast kernel of
// K = k; CO_GENERAL_BIN: the general kernel) for one (precision, AD mode).
hipError_t launch_fit_f64_fwd(int bin, unsigned grid, size_t lds, hipStream_t s, const FitArgs &fa);
hipError_t launch_fit_f64_rev(int bin, unsigned grid, size_t lds, hipStream_t s, const FitArgs &fa);
hipError_t launch_fit_f32_fwd(int bin, unsigned grid, size_t lds, hipStream_t s, const FitArgs &fa);
hipError_t launch_fit_f32_rev(int bin, unsigned grid, size_t lds, hipStream_t s, const FitArgs &fa);

// ------------------------------------------------------ plain evaluation

struct EvalArgs {
    const uint64_t *prog;
    const ExprDesc *desc;
    const double *X;   // [D][N]
    const double *C;   // [total_c]
    double *Yout;      // [M][N]
    int N, D;
};

template <typename R, typename F>
__global__ void __launch_bounds__(kLanes) eval_kernel(EvalArgs ea) {
    constexpr int P = 1;
    __shared__ double cs[CO_MAX_K];
    extern __shared__ char lds_dyn[];
    const int lane = threadIdx.x;
    const ExprDesc e = ea.desc[blockIdx.x];
    if (lane < e.K) cs[lane] = ea.C[e.c_off + lane];
    WaveLds<R, P> w;
    w.x = (R *)lds_dyn;
    w.slot = w.x + (size_t)ea.D * kLanes;
    w.tape = w.slot;
    wave_sync_lds();
    const ProgPtr prog = (ProgPtr)(ea.prog + e.prog_off);
    const int batches = (ea.N + kLanes - 1) / kLanes;
    for (int bt = 0; bt < batches; ++bt) {
        const int i = lane + kLanes * bt;
        const bool valid = i < ea.N;
        for (int v = 0; v < ea.D; ++v)
            lds_at<R, P>(w.x, v, 0, lane) = valid ? (R)ea.X[(size_t)v * ea.N + i] : R(0);
        R accv[1], T[1];
        forward_pass<0, R, P, 0, F>(prog, e.n, w, cs, lane, accv, T);
        if (valid) ea.Yout[(size_t)e.y_row * ea.N + i] = (double)accv[0];
    }
}

}  // namespace cusr
