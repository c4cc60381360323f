// lm_split.h -- the split path: one expression's passes spread over many
// workgroups.
//
// With more than CO_MAX_PARTITIONS point partitions (co_partitions_for: from
// CO_SPLIT_MIN_N points, and for reverse AD from 2,048 to 16,383 points; or
// CoOptions.partitions), each partition of a pass
// is a workgroup of its own: lm_pass_kernel runs one wavefront over the
// granules g = part, part + G, ... (the partition rule of data_pass) and
// writes the partition's sums to HBM; lm_step_kernel, one wavefront per
// expression, adds the G partition sums in partition order (the order of
// data_pass's in-workgroup combine and of the CPU oracle) and runs one step of
// the LM loop of fit_one: accept/reject, the lambda update, then the solves up
// to the next trial point, which the next pass evaluates. The host launches
// (pass, step) pairs 1 + max_iter times (+2 fp64 audit passes for mixed
// precision); an expression with nothing pending returns at once. Every
// decision and every sum is the one fit_one makes, so results equal the
// oracle's with the same partitions. Reference: one host loop over all trees
// per iteration (cusr/kernel/batch_lm_ad.cu:350-495); there the trees' passes
// are single-warp loops over N (lm_core.cuh:123-124).
#pragma once

#include "lm_device.h"

namespace cusr {

// Loop state of an expression on the split path (a row of FitArgs.state,
// indexed by y_row): the LM scalars, then c_cur, c_try and the sums at c_cur.
enum {
    kSpLoss = 0, kSpLossInit, kSpLambda, kSpStatus, kSpIter, kSpPending, kSpDn, kSpCn,
    kSpLf, kSpCCur = 16, kSpCTry = kSpCCur + CO_MAX_K, kSpSums = kSpCTry + CO_MAX_K
};
constexpr int kSplitStride = kSpSums + 576;   // >= sums_width(CO_MAX_K) = 561
// pending pass of an expression
enum { SP_NONE = 0, SP_INIT = 1, SP_TRIAL = 2, SP_AUDIT_CUR = 3, SP_AUDIT_INIT = 4 };

#ifdef CUSR_SPLIT_STEP_KERNELS
// Start of a split fit: c_try = c_init, a pass at it pending.
__global__ void __launch_bounds__(kLanes) lm_split_init_kernel(FitArgs fa) {
    const ExprDesc e = fa.desc[blockIdx.x];
    const int lane = threadIdx.x;
    double *sv = fa.state + (size_t)e.y_row * fa.state_stride;
    if (lane < e.K) sv[kSpCTry + lane] = fa.C0[e.c_off + lane];
    if (lane == 0) {
        sv[kSpPending] = (double)SP_INIT;
        sv[kSpStatus] = (double)ST_RUN;
        sv[kSpIter] = 0.0;
        sv[kSpLambda] = fa.lambda0;
    }
}

#endif  // CUSR_SPLIT_STEP_KERNELS

// One partition of one pending pass: workgroup b is partition b mod G of the
// launch's expression b / G. SP_INIT and SP_TRIAL are Jacobian passes at
// c_try (value only for K = 0); the audits are fp64 value passes at c_cur and
// c_init.
template <int K, typename R, int AD, int LN, bool GEN>
__global__ void __launch_bounds__(kLanes, (GEN ? CUSR_WAVES_GEN : pass_waves_per_eu<R, (GEN ? 0 : K), AD, LN>()))
lm_pass_kernel(FitArgs fa) {
    typedef typename std::conditional<GEN, WideFmt, FastFmt>::type F;
    constexpr int KC = FitStatic<GEN>::KC;
    constexpr int P = fit_points<GEN, R, K, AD, LN>();
    constexpr int AP = fit_audit_points<GEN, R, K, AD, LN>();
    constexpr int JAC = (K == 0) ? 0 : (AD == CO_AD_REVERSE ? 2 : 1);
    __shared__ double cs[KC];
    extern __shared__ char lds_dyn[];
    const int G = fa.parts;
    const int idx = uni((int)blockIdx.x / G);
    const int part = uni((int)blockIdx.x - idx * G);
    const int lane = (int)threadIdx.x;
    const ExprDesc e = fa.desc[idx];
    const double *sv = fa.state + (size_t)e.y_row * fa.state_stride;
    const int kind = (int)uni(sv[kSpPending]);
    if (kind == SP_NONE) return;
    const int Kr = GEN ? e.K : K;
    const double *src = kind == SP_AUDIT_INIT ? fa.C0 + e.c_off
                        : (kind == SP_AUDIT_CUR ? sv + kSpCCur : sv + kSpCTry);
    if (lane < Kr) cs[lane] = src[lane];
    wave_sync_lds();
    char *my_lds = lds_dyn;
    double *jt = (double *)my_lds;
    if constexpr (GEN) {
        my_lds += kGenJtBytes;
    } else if constexpr (sums_over_tape<K, AD>()) {
        // the rows go to the Jacobian pass's tape bytes (x and slot rows first)
        jt = (double *)(my_lds + (size_t)(fa.D + fa.slots) * P * kLanes * sizeof(R));
    } else if constexpr (matrix_sums<K, AD>()) {
#pragma unroll
        for (int j = 0; j < kJtStride; ++j) jt[lane * kJtStride + j] = 0.0;
        my_lds += kJtBytes + (size_t)K * (K + 1) * sizeof(double);
    }
    PassArgs pa;
    pa.prog = (ProgPtr)(fa.prog + e.prog_off);
    pa.n = e.n;
    pa.X = fa.X;
    pa.y = fa.Y + (fa.shared_y ? (size_t)0 : (size_t)e.y_row * fa.N);
    pa.N = fa.N;
    pa.D = fa.D;
    pa.parts = G;
    pa.pwaves = G;      // this workgroup's wavefront sums partition `part` only
    pa.wave = part;
    pa.part = fa.psum + (size_t)idx * G * fa.psum_width;
    pa.jt = jt;
    pa.split = 1;
    pa.part_stride = fa.psum_width;
    if (kind == SP_INIT || kind == SP_TRIAL) {
        WaveLds<R, P> wl;
        wl.x = (R *)my_lds;
        wl.slot = wl.x + (size_t)fa.D * P * kLanes;
        wl.tape = wl.slot + (size_t)fa.slots * P * kLanes;
        if constexpr (GEN) {
            if (Kr == 0) data_pass<0, R, 1, 0, F>(pa, wl, cs, nullptr, lane);
            else data_pass_gen<R, JAC, F>(pa, wl, cs, nullptr, lane, Kr);
        } else {
            data_pass<K, R, P, JAC, F>(pa, wl, cs, nullptr, lane);
        }
    } else {
        constexpr int KA = GEN ? 0 : K;
        WaveLds<double, AP> w64;
        w64.x = (double *)my_lds;
        w64.slot = w64.x + (size_t)fa.D * AP * kLanes;
        w64.tape = w64.slot + (size_t)fa.slots * AP * kLanes;
        data_pass<KA, double, AP, 0, F>(pa, w64, cs, nullptr, lane);
    }
}

#ifdef CUSR_SPLIT_STEP_KERNELS
// One LM step of one expression (a wavefront): the G partition sums of its
// pending pass added in partition order, then fit_one's decisions. The state
// row is worked on in LDS and written back.
// KS > 0: every expression of the launch has K = KS (a fast kernel's bin), and
// the solve is damped_solve<KS>, unrolled in registers; KS = 0: the runtime-K
// solve in LDS (the general bin). Both give the same bits; the unrolled one has
// no chain of LDS round trips (C3's step launches: the solves of K <= 16).
template <int KS>
__global__ void __launch_bounds__(kLanes) lm_step_kernel(FitArgs fa, int mixed) {
    __shared__ double s_new[sums_width(CO_MAX_K)];
    __shared__ double s_cur[sums_width(CO_MAX_K)];
    __shared__ double c_cur[CO_MAX_K], c_try[CO_MAX_K];
    __shared__ double L[CO_MAX_K * CO_MAX_K + CO_MAX_K];
    const int idx = blockIdx.x;
    const int lane = (int)threadIdx.x;
    const ExprDesc e = fa.desc[idx];
    double *sv = fa.state + (size_t)e.y_row * fa.state_stride;
    const int kind = (int)uni(sv[kSpPending]);
    if (kind == SP_NONE) return;
    const int K = KS > 0 ? KS : e.K;
    const int G = fa.parts;
    const bool audit = kind == SP_AUDIT_CUR || kind == SP_AUDIT_INIT;
    const int W = (audit || K == 0) ? 1 : sums_width(K);
    const double *ps = fa.psum + (size_t)idx * G * fa.psum_width;
    for (int q = lane; q < W; q += kLanes) {
        double v = ps[q];
        for (int g = 1; g < G; ++g) v = v + ps[(size_t)g * fa.psum_width + q];
        s_new[q] = v;
    }
    if (lane < K) {
        c_cur[lane] = sv[kSpCCur + lane];
        c_try[lane] = sv[kSpCTry + lane];
    }
    if (kind == SP_TRIAL)
        for (int q = lane; q < W; q += kLanes) s_cur[q] = sv[kSpSums + q];
    wave_sync_lds();
    const double half = uni(0.5 * s_new[0]);
    int st = (int)uni(sv[kSpStatus]);
    int it = (int)uni(sv[kSpIter]);
    double lambda = uni(sv[kSpLambda]);
    double loss = uni(sv[kSpLoss]);
    double loss_init = uni(sv[kSpLossInit]);
    if (kind == SP_AUDIT_CUR) {
        if (lane == 0) {
            sv[kSpLf] = half;
            sv[kSpPending] = (double)SP_AUDIT_INIT;
        }
        return;
    }
    double lf = loss, li = loss_init;
    if (kind == SP_AUDIT_INIT) {
        lf = uni(sv[kSpLf]);
        li = half;
    } else {
        if (kind == SP_INIT) {
            if (lane < K) c_cur[lane] = c_try[lane];
            for (int q = lane; q < W; q += kLanes) s_cur[q] = s_new[q];
            loss = half;
            loss_init = half;
            st = (K == 0) ? ST_K0 : (loss_ok(fa, loss) ? ST_RUN : ST_NAN);
            lambda = fa.lambda0;
            it = 0;
        } else if (!loss_ok(fa, half)) {
            st = ST_NAN;
        } else {
            const double loss_try = half;
            const double dn = uni(sv[kSpDn]), cn = uni(sv[kSpCn]);
            const bool small = dn < fa.xtol * (cn + fa.xtol);
            bool accept, conv;
            if (fa.lm_order == CO_ORDER_CONVERGE_FIRST) {
                // FD variant (co_lib.cu:457-473)
                conv = small;
                accept = small || loss_try < loss;
            } else {
                // AD variant (batch_lm_ad.cu:456-473)
                accept = loss_try <= loss;
                conv = accept && small;
            }
            if (accept) {
                if (lane < K) c_cur[lane] = c_try[lane];
                for (int q = lane; q < W; q += kLanes) s_cur[q] = s_new[q];
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
        wave_sync_lds();
        // solves up to the next trial point (fit_one's loop head)
        int pending = SP_NONE;
        double dn = 0.0, cn = 0.0;
        while (st == ST_RUN && it < fa.max_iter) {
            ++it;
            bool solved;
            if constexpr (KS > 0) {
                double delta[KS];
                solved = fa.damp == CO_DAMP_RELATIVE
                             ? damped_solve<KS, true>(s_cur, lambda, 0, delta)
                             : damped_solve<KS, false>(s_cur, lambda, fa.damp, delta);
                if (solved && lane == 0) {
#pragma unroll
                    for (int j = 0; j < KS; ++j) L[KS * KS + j] = delta[j];
                }
                wave_sync_lds();
            } else {
                solved = fa.damp == CO_DAMP_RELATIVE
                             ? damped_solve_rt<true>(s_cur, lambda, 0, K, L, lane)
                             : damped_solve_rt<false>(s_cur, lambda, fa.damp, K, L, lane);
            }
            if (!solved) {
                lambda = lambda * 10.0;
                if (lambda > 1e12) st = ST_CHOL;
                continue;
            }
            const double *db = L + K * K;
            if (lane < K) {
                const double v = c_cur[lane] + db[lane];
                c_try[lane] = fa.f32_range ? (double)(float)v : v;
            }
            wave_sync_lds();
            double dn2 = 0.0, cn2 = 0.0;
            int over = 0;
            for (int j = 0; j < K; ++j) {
                dn2 = fma(db[j], db[j], dn2);
                cn2 = fma(c_try[j], c_try[j], cn2);
                over |= !isfinite(c_try[j]) ? 1 : 0;
            }
            if (fa.f32_range && uni(over)) {
                st = ST_NAN;
                continue;
            }
            dn = ::sqrt(dn2);
            cn = ::sqrt(cn2);
            pending = SP_TRIAL;
            break;
        }
        if (pending == SP_NONE && mixed) pending = SP_AUDIT_CUR;
        if (pending != SP_NONE) {
            // save the loop state for the next pass
            if (lane < K) {
                sv[kSpCCur + lane] = c_cur[lane];
                sv[kSpCTry + lane] = c_try[lane];
            }
            for (int q = lane; q < W; q += kLanes) sv[kSpSums + q] = s_cur[q];
            if (lane == 0) {
                sv[kSpDn] = dn;
                sv[kSpCn] = cn;
                sv[kSpLoss] = loss;
                sv[kSpLossInit] = loss_init;
                sv[kSpLambda] = lambda;
                sv[kSpStatus] = (double)st;
                sv[kSpIter] = (double)it;
                sv[kSpPending] = (double)pending;
            }
            return;
        }
        lf = loss;
        li = loss_init;
    }
    // the outputs (fit_one's end): fp64 guard, status map
    bool revert = false;
    if (fa.guard && K > 0) revert = !isfinite(lf) || (isfinite(li) && lf > li);
    if (revert) {
        if (st == ST_CONV) st = ST_RUN;
        lf = li;
    }
    if (lane < K) fa.C[e.c_off + lane] = revert ? fa.C0[e.c_off + lane] : c_cur[lane];
    if (lane == 0) {
        fa.status[e.y_row] = (st <= ST_CONV) ? (1 - st) : st;
        fa.loss_init[e.y_row] = li;
        fa.loss_final[e.y_row] = lf;
        fa.iters[e.y_row] = it;
        sv[kSpPending] = (double)SP_NONE;
    }
}
#endif  // CUSR_SPLIT_STEP_KERNELS

// Launch the pass kernel of one bin (as launch_fit_*) for one (precision, AD mode).
hipError_t launch_pass_f64_fwd(int bin, unsigned grid, size_t lds, hipStream_t s, const FitArgs &fa);
hipError_t launch_pass_f64_rev(int bin, unsigned grid, size_t lds, hipStream_t s, const FitArgs &fa);
hipError_t launch_pass_f32_fwd(int bin, unsigned grid, size_t lds, hipStream_t s, const FitArgs &fa);
hipError_t launch_pass_f32_rev(int bin, unsigned grid, size_t lds, hipStream_t s, const FitArgs &fa);

}  // namespace cusr
