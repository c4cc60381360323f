/* cusr_co.h -- C ABI of the MI355X batched Levenberg-Marquardt constant fitter.
 *
 * Drop-in for the reference in-process CO library (cusr/kernel/co_lib.h:45-71):
 * the four symbols co_init / co_optimize / co_last_split / co_teardown keep
 * their names, argument meaning, return codes and ownership rules, so the
 * reference ctypes loader (cusr/kernel/co_inproc.py:101-215) binds this
 * library unchanged. Everything else below is an extension with no
 * counterpart in the reference and says so.
 *
 * Threading: a handle is not re-entrant; one handle per (device, process)
 * is the intended use, serialised by the caller (the Python loader holds a
 * lock). Every call selects the handle's device first.
 */
#ifndef CUSR_CO_H
#define CUSR_CO_H

#include <stdint.h>
#include "pop_format.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes (cusr/kernel/co_lib.h:27-41, plus CO_ERR_PROGRAM and
 * CO_ERR_DATA). */
#define CO_OK 0
#define CO_ERR_BOUNDS 2      /* K_max, max_stack or n_vars beyond the bounds below, or
                                LDS rows beyond the device's LDS */
#define CO_ERR_CUDA (-1)     /* HIP runtime error */
#define CO_ERR_SUM_C (-2)    /* sum(K) != header.total_c */
#define CO_ERR_SUM_NODES (-3) /* sum(n_nodes) != header.total_nodes */
#define CO_ERR_NULLARG (-4)  /* null pointer or bad argument */
#define CO_ERR_OOM (-5)      /* device allocation failed */
#define CO_ERR_PROGRAM (-6)  /* malformed expression: unknown op id, bad node type,
                                stack under/overflow, bad const rank or var index.
                                Extension: the reference silently evaluates unknown
                                ops to 0 (cusr/kernel/lm_core.cuh:82,100). */
#define CO_ERR_DATA (-7)     /* co_optimize_data: no data set uploaded, or the header's
                                N / n_vars differ from the uploaded one;
                                co_data_upload_device: a pointer that is not
                                device memory of the handle's device, or an
                                extent that runs past its allocation */

/* Bounds of this build. K and the value stack are the reference's
 * (MAX_K = 32, MAX_STACK = 64, cusr/kernel/ad_interp.cuh:34-39, checked on the
 * header like cusr/kernel/co_lib.cu:211-212 and again per expression); the
 * reference has no bound on n_vars or on nodes per expression. Populations
 * beyond them get CO_ERR_BOUNDS before anything is copied to the device, and
 * so does a launch whose per-wavefront LDS rows (inputs, spill slots, reverse
 * tape) exceed the device's LDS. */
#define CO_MAX_K 32
#define CO_MAX_STACK 64
#define CO_MAX_VARS 255

/* Two kernel families fit an expression. The fast kernels, one instance per
 * K (0..CO_FAST_MAX_K), take expressions with K <= CO_FAST_MAX_K, a value
 * stack <= CO_FAST_MAX_STACK and <= CO_FAST_MAX_NODES nodes, in populations
 * with n_vars <= CO_FAST_MAX_VARS; the general kernel (runtime K, one point
 * per lane, matrix-instruction sums) takes every other expression. The
 * choice is a function of the expression and n_vars only, and part of the
 * arithmetic order: the general kernel forms every sum of a Jacobian pass
 * (r^2, J^T r and J^T J) as one fused multiply-add chain per entry over the
 * points in ascending order (see CO_SUMS_MATRIX_MIN_K), whatever K. */
#define CO_FAST_MAX_K 16
#define CO_FAST_MAX_STACK 16
#define CO_FAST_MAX_VARS 8
#define CO_FAST_MAX_NODES 255
static inline int co_fast_path(int K, int stack_depth, int n_nodes, int n_vars) {
    return K <= CO_FAST_MAX_K && stack_depth <= CO_FAST_MAX_STACK &&
           n_nodes <= CO_FAST_MAX_NODES && n_vars <= CO_FAST_MAX_VARS;
}

/* Launches of one fit: the K bins 0..CO_FAST_MAX_K of the fast kernels, then
 * the general kernel's bin (index CO_GENERAL_BIN). */
#define CO_GENERAL_BIN (CO_FAST_MAX_K + 1)
#define CO_BINS (CO_FAST_MAX_K + 2)

/* Jacobian mode and arithmetic of a fit (extension). */
#define CO_AD_FORWARD 0
#define CO_AD_REVERSE 1
#define CO_PREC_FP64 0   /* fp64 interpreter, Jacobian, reductions and solve */
#define CO_PREC_MIXED 1  /* fp32 interpreter and Jacobian, fp64 JtJ/Jtr/loss and solve */

/* Options of co_optimize_ex (extension; no counterpart in the reference,
 * whose knobs are compile-time flags, cusr/kernel/Makefile:9-88).
 * struct_size must be sizeof(CoOptions); co_options_default fills defaults:
 * forward AD, fp64, max_iter 50, lambda0 1e-3, xtol 1e-6, guard on
 * (the reference values, cusr/kernel/batch_lm_ad.cu:301-316). */
typedef struct CoOptions {
    int32_t struct_size;
    int32_t ad_mode;    /* CO_AD_FORWARD / CO_AD_REVERSE */
    int32_t precision;  /* CO_PREC_FP64 / CO_PREC_MIXED */
    int32_t max_iter;
    double lambda0;
    double xtol;
    int32_t fp64_guard; /* 1: deliver c_init where the fp64 loss at c_final is
                           non-finite or worse (cusr/kernel/lm_core.cuh:299-351) */
    int32_t partitions; /* point partitions per expression (a power of two up to
                           CO_MAX_SPLIT; 0: co_partitions_for). Part of
                           the arithmetic order: the sums of each partition are
                           formed separately and added in partition order. Up
                           to CO_MAX_PARTITIONS the wavefronts of one
                           workgroup sum them; beyond, each partition is a
                           workgroup of its own (the split path) */
    int32_t lm_order;   /* CO_ORDER_IMPROVE_FIRST (the AD variant,
                           cusr/kernel/batch_lm_ad.cu:456-473) or
                           CO_ORDER_CONVERGE_FIRST (the FD variant: a small step
                           converges, otherwise a strict decrease is accepted,
                           cusr/kernel/co_lib.cu:457-473) */
    int32_t tail_iter;  /* active-set compaction: after this many iterations
                           the expressions still running continue in a second
                           launch with tail_partitions partitions, one
                           wavefront per partition, while finished ones exit
                           at once.
                           0: co_tail_iter_for; -1: one launch, no tail */
    int32_t tail_partitions; /* partitions of the tail (1, 2 or 4; 0: 4) */
    int32_t f32_range;  /* 1: constants held in fp32 and losses in its range,
                           as in the reference's fp32 fit: each trial point is
                           rounded to fp32 (so the delivered constants are
                           exactly representable and loss_final is the fp64
                           loss at them); a trial constant or loss that is
                           +-inf in fp32 (or a start loss so) counts as a
                           non-finite trial, FAIL_NAN with the last accepted
                           constants kept (cusr/kernel/batch_lm_ad.cu:437-443).
                           co_optimize and the CLI on float32 files set it;
                           default 0 */
    int32_t damping;    /* the damped solve's variant (cusr/kernel/batch_lm_ad.cu:
                           149-172, chosen there by -DTRUST_REGION / -DPIVOT_FLOOR):
                           CO_DAMP_RELATIVE (default): A_jj (1 + lambda), a
                           pivot <= 0 fails the step;
                           CO_DAMP_TRUST_REGION (the reference's batch_lm_ad_tr,
                           cusr/kernel/Makefile:57-63): A_jj + lambda, a pivot
                           <= 0 is replaced by lambda; the reference starts
                           that variant at lambda 1e-4 (batch_lm_ad.cu:301-306),
                           which the caller sets in lambda0;
                           CO_DAMP_PIVOT_FLOOR: A_jj (1 + lambda), a pivot
                           below CO_PIVOT_FLOOR_EPS is raised to it */
    int32_t reserved;
} CoOptions;

#define CO_ORDER_IMPROVE_FIRST 0
#define CO_ORDER_CONVERGE_FIRST 1

#define CO_DAMP_RELATIVE 0
#define CO_DAMP_TRUST_REGION 1
#define CO_DAMP_PIVOT_FLOOR 2
/* the reference's PIVOT_FLOOR_EPS, the fp32 constant 1e-9f
 * (cusr/kernel/batch_lm_ad.cu:80-82), held exactly in fp64 */
#define CO_PIVOT_FLOOR_EPS ((double)1e-9f)
#define CO_TRUST_REGION_LAMBDA0 ((double)1e-4f)

/* Point partitions of an expression with N points when CoOptions.partitions
 * is 0: 64-point granule g belongs to partition g mod G, each partition is
 * summed by its own wavefront, so long expressions use several wavefronts.
 * A function of N only, so an expression fits the same alone or in any
 * population. Measured on MI355X: two partitions from N = 512 shorten the
 * slowest expressions of a K bin, which set its duration (C2 -11 %, C3
 * -20 %, C5 even), and give a bin of few expressions twice the wavefronts (a
 * GP generation of 4,000 expressions at N = 1,000, whose fast K bins hold
 * 150-500 expressions each: 103.5 -> 76.4 ms per fit); four pay off only for
 * long expressions (C2 +27 %). From
 * CO_SPLIT_MIN_N points an expression's passes spread over G = N / 4,096
 * (rounded down to a power of two, 16 to CO_MAX_SPLIT) workgroups, whose
 * partition sums meet in HBM and are added in partition order by a step
 * kernel that runs the LM update (the split path): the waves of many
 * workgroups hide the loads of long passes, and a population of a few long
 * expressions still fills the GPU (C4, N = 100,000: 16 partitions, 266 ->
 * 189 ms per fit against four wavefronts of one workgroup). */
#define CO_MAX_PARTITIONS 4
#define CO_MAX_SPLIT 256
#define CO_SPLIT_MIN_N 65536
static inline int co_partitions_for_n(int N) {
    if (N >= CO_SPLIT_MIN_N) {
        int g = 8;
        while (g < CO_MAX_SPLIT && (long)g * 2 * 4096 <= (long)N) g *= 2;
        return g;
    }
    return N >= 16384 ? 4 : (N >= 512 ? 2 : 1);
}

/* Point partitions when CoOptions.partitions is 0, by N and the AD mode.
 * Reverse AD from 2,048 to 16,383 points takes the split path with 8
 * partitions: its passes hold a tape and an adjoint sweep per point, so a
 * wavefront's pass is long and the split path's eight workgroups per
 * expression hide its loads where two wavefronts of one workgroup do not
 * (C3, N = 2,048, K 4-16, measured on MI355X: 136.5 -> 126.4 ms per fit;
 * 16 partitions 130.0, 32 140.2). Forward AD keeps co_partitions_for_n (C2
 * with 8 split partitions: 11.6 -> 23.5 ms). */
static inline int co_partitions_for(int N, int ad_mode) {
    if (ad_mode == CO_AD_REVERSE && N >= 2048 && N < 16384) return 8;
    return co_partitions_for_n(N);
}

/* The partitions options o give for N points (0 if o->partitions is not a
 * power of two up to CO_MAX_SPLIT). */
static inline int co_partitions_resolve(const CoOptions *o, int N) {
    const int g = o->partitions ? o->partitions : co_partitions_for(N, o->ad_mode);
    return (g >= 1 && g <= CO_MAX_SPLIT && (g & (g - 1)) == 0) ? g : 0;
}

/* Iterations before the tail when CoOptions.tail_iter is 0, CO_TAIL_ITER_DEFAULT
 * (0: no tail). The tail targets the spread of iteration counts (a few
 * expressions run to max_iter while most stop early) by giving the ones still
 * running more wavefronts. Measured on MI355X it does not pay on C1, C2, C3
 * or C5: the concurrent K bins keep the machine busy until the end, and the
 * extra partition reductions cost more than the shorter tail saves; so it is
 * off by default and kept as an option. A function of the expression's size
 * only, and part of the arithmetic order: passes of iterations after
 * tail_iter, and the final fp64 audit of an expression that finishes after
 * it, sum with the tail's partitions. */
#ifndef CO_TAIL_ITER_DEFAULT
#define CO_TAIL_ITER_DEFAULT 0
#endif
static inline int co_tail_iter_for(int N, int max_iter) {
    if (CO_TAIL_ITER_DEFAULT <= 0 || co_partitions_for_n(N) >= CO_MAX_PARTITIONS || N < 256)
        return 0;
    return CO_TAIL_ITER_DEFAULT < max_iter ? CO_TAIL_ITER_DEFAULT : 0;
}

/* The tail options o give for N points: returns the iterations before the
 * tail (0: no tail) and sets *tail_parts to its partitions. The split path
 * (more than CO_MAX_PARTITIONS partitions) has no tail: its step kernel
 * already runs iteration by iteration. */
static inline int co_tail_resolve(const CoOptions *o, int N, int *tail_parts) {
    *tail_parts = o->tail_partitions ? o->tail_partitions : CO_MAX_PARTITIONS;
    if (co_partitions_resolve(o, N) > CO_MAX_PARTITIONS) return 0;
    const int t = o->tail_iter < 0 ? 0
                  : (o->tail_iter > 0 ? o->tail_iter : co_tail_iter_for(N, o->max_iter));
    return (t > 0 && t < o->max_iter) ? t : 0;
}

/* Forward-AD fits of expressions with K >= CO_SUMS_MATRIX_MIN_K, and
 * reverse-AD fits with K >= CO_SUMS_MATRIX_MIN_K_REV, form their sums with
 * the fp64 matrix instruction (v_mfma_f64_16x16x4): the augmented Jacobian
 * rows [J | r] of a partition's points are multiplied into one 16 x 16
 * accumulator, which adds the products of each entry with one fused
 * multiply-add per point in ascending point order (no per-lane split, no
 * butterfly). For K = 16 the r column does not fit: r^2 and J^T r then keep
 * the per-lane order. Part of the arithmetic order, so the CPU oracle
 * follows the same rule. (Below the thresholds the per-lane sums are
 * faster. In reverse mode the staged rows share the LDS of the tape, which
 * the reverse sweep has consumed by then, so they cost no LDS, and they free
 * the registers of the per-lane sums: from K = 12 the reverse-AD pass kernels
 * need 106-110 VGPRs instead of the 257-322 the per-lane sums took, which
 * spilled at two waves per SIMD; measured on MI355X, C3 from K = 11, 13 and
 * 15 within noise of each other.) */
#ifndef CO_SUMS_MATRIX_MIN_K
#define CO_SUMS_MATRIX_MIN_K 13
#endif
#ifndef CO_SUMS_MATRIX_MIN_K_REV
#define CO_SUMS_MATRIX_MIN_K_REV 12
#endif

/* --- reference ABI (cusr/kernel/co_lib.h:45-71) ------------------------ */

/* Select device_id, create its context once and return an opaque handle. */
int co_init(int device_id, void **handle_out);

/* Fit one population; fp32 inputs and outputs (cusr/kernel/co_lib.h:55-61).
 * Inputs are host pointers read during the call. Outputs are caller-allocated
 * and sized to the current header: c_final_out[total_c], status_out[M_prob],
 * loss_init_out / loss_final_out [M_prob] (both may be NULL). The fit itself
 * runs in fp64 with forward AD, with constants and losses held to the fp32
 * range (CoOptions.f32_range); outputs go through co_narrow_fp32. */
int co_optimize(void *handle, const PopHeader *header,
                const int32_t *nt, const float *nv, const int32_t *ci,
                const TreeMeta *metas,
                const float *c_init, const float *xs, const float *ym,
                int max_iter,
                float *c_final_out, int32_t *status_out,
                float *loss_init_out, float *loss_final_out);

/* Wall-clock split of the last co_optimize / co_optimize_ex call on this
 * process: setup (entry to loop start: checks, plan, uploads) and loop
 * (device fit until results are back on the host). A population of 16,384
 * or more expressions is decoded, uploaded and launched in ranges, the host
 * decoding a range while the device fits the ones before: setup then ends at
 * the first range's launch. Returns 0 and fills
 * both (the reference returns 1 and -1.0 unless built with -DPROFILE,
 * cusr/kernel/co_lib.cu:531-541; this build always records). */
int co_last_split(double *setup_ms_out, double *loop_ms_out);

/* Free device and host state of a handle. Safe on NULL. */
void co_teardown(void *handle);

/* --- extensions (no counterpart in the reference) ------------------------ */

/* Fill *opt with the defaults listed above. */
void co_options_default(CoOptions *opt);

/* Fit with fp64 constants, data and outputs, for parity runs at fp64
 * tolerance (the fp32 carrier of co_optimize cannot hold 1e-9 loss parity).
 * xs is row-major [N][n_vars] like pop.bin; ym is [M_prob][N].
 * iters_out [M_prob] (may be NULL) receives the LM iterations each
 * expression ran. loss_* may be NULL. */
int co_optimize_ex(void *handle, const CoOptions *opt, const PopHeader *header,
                   const int32_t *nt, const float *nv, const int32_t *ci,
                   const TreeMeta *metas,
                   const double *c, const double *xs, const double *ym,
                   double *c_final_out, int32_t *status_out,
                   double *loss_init_out, double *loss_final_out,
                   int32_t *iters_out);

/* Evaluate every expression at every point: y_out[m*N + i] = f_m(x_i; c_m)
 * (counterpart of eval_kernel_batched, cusr/kernel/lm_core.cuh:108-125).
 * precision: CO_PREC_FP64 or CO_PREC_MIXED (fp32 interpreter). */
int co_eval_ex(void *handle, const PopHeader *header,
               const int32_t *nt, const float *nv, const int32_t *ci,
               const TreeMeta *metas, const double *c, const double *xs,
               int precision, double *y_out);

/* Decode and upload a population (fp64 inputs as in co_optimize_ex) into the
 * handle's device buffers, where it stays resident for co_fit_resident until
 * the next upload, co_optimize* or co_eval_ex call on the handle. Returns the
 * codes of co_optimize. */
int co_upload_ex(void *handle, const PopHeader *header,
                 const int32_t *nt, const float *nv, const int32_t *ci,
                 const TreeMeta *metas,
                 const double *c, const double *xs, const double *ym);

/* Fit the resident population from its uploaded starting constants. Output
 * pointers (all may be NULL; results then stay on the device) are as in
 * co_optimize_ex. CO_ERR_NULLARG when nothing is resident. */
int co_fit_resident(void *handle, const CoOptions *opt,
                    double *c_final_out, int32_t *status_out,
                    double *loss_init_out, double *loss_final_out,
                    int32_t *iters_out);

/* co_fit_resident without device allocation. No counterpart in the
 * reference: for callers that cannot allocate device memory (code under graph
 * capture, tight serving loops, harnesses that forbid it). Fits the resident
 * population exactly as co_fit_resident does (same kernels, same results),
 * with the fit's scratch -- the loop state of tail segments and of the split
 * path, and the split path's partition sums -- in a fixed device array of
 * CO_STATIC_SCRATCH_BYTES that each GPU holds from co_init until the process
 * ends, instead of handle buffers. A fit needing more gets CO_ERR_BOUNDS
 * before anything is launched. Every call on one GPU shares that GPU's array,
 * which keeps the last call's contents (each value a fit reads there it has
 * written first): calls that overlap on one GPU race. */
#define CO_STATIC_SCRATCH_BYTES (64u << 20)
int co_fit_resident_static(void *handle, const CoOptions *opt,
                           double *c_final_out, int32_t *status_out,
                           double *loss_init_out, double *loss_final_out,
                           int32_t *iters_out);

/* Upload one data set, xs [N][n_vars] row-major and one target y [N], into
 * buffers of the handle reserved for it. It stays on the device across calls
 * until the next co_data_upload or co_teardown; the other entry points do not
 * touch it. No counterpart in the reference: its GP bridge re-sends X and a
 * y tiled to every expression with each population
 * (cusr/demonstrator/kernel_bridge.py:200-206). Returns 0, CO_ERR_NULLARG
 * (N < 0, n_vars outside 0..CO_MAX_VARS, null pointers with N > 0),
 * CO_ERR_OOM or CO_ERR_CUDA. */
int co_data_upload(void *handle, int N, int n_vars, const double *xs, const double *y);

/* co_data_upload from device memory: xs_dev (N * n_vars fp64, row-major) and
 * y_dev (N fp64) are device pointers on the handle's device, such as the data
 * of torch CUDA tensors. They are copied device to device (X transposed on the
 * device), so the data set never crosses PCIe. Before reading them the call
 * waits for all work the process has queued on the device
 * (hipDeviceSynchronize), so data written by a kernel still queued on any of
 * the caller's streams is complete when it is read; the library does not keep
 * the pointers. No counterpart in the reference: it is
 * the data-residency half of the zero-copy entry its in-process plan
 * describes as the end state (docs/kernel/INPROCESS_CO_PLAN.md:69-75).
 * Returns as co_data_upload, and CO_ERR_DATA when a pointer is not device
 * memory of the handle's device or its N * n_vars (N) doubles run past the end
 * of the allocation it points into; then nothing is copied and the previous
 * data set stays. */
int co_data_upload_device(void *handle, int N, int n_vars, const double *xs_dev,
                          const double *y_dev);

/* co_optimize_ex against the uploaded data set: every expression fits its
 * target y; only the programs and c go to the device. header->N and
 * header->n_vars must equal the data set's (else CO_ERR_DATA, before any
 * copy); ym flags in the header are ignored. The population stays resident
 * for co_fit_resident. Other codes and outputs as co_optimize_ex. */
int co_optimize_data(void *handle, const CoOptions *opt, const PopHeader *header,
                     const int32_t *nt, const float *nv, const int32_t *ci,
                     const TreeMeta *metas, const double *c,
                     double *c_final_out, int32_t *status_out,
                     double *loss_init_out, double *loss_final_out,
                     int32_t *iters_out);

/* co_optimize_data with the constants and the results in device memory of the
 * caller (torch CUDA tensors): c_dev (total_c doubles) is read and
 * c_final_dev, status_dev and the optional loss_init_dev, loss_final_dev,
 * iters_dev are written device to device; the call returns when they are
 * complete. Only the programs (nt, nv, ci, metas) come from host memory,
 * decoded there. Before it reads c_dev or writes an output, the call waits for
 * all work the process has queued on the device (hipDeviceSynchronize): a
 * producer of c_dev, or a reader of the output buffers, still queued on any
 * of the caller's streams finishes first, so no stream ordering is left to
 * the caller. No counterpart in the reference: it is the device-I/O step of
 * the zero-copy in-process route its plan names as the end state
 * (docs/kernel/INPROCESS_CO_PLAN.md:69-75), for GP loops that keep their
 * populations' constants on the GPU. A given pointer that is not device
 * memory of the handle's device, or whose extent runs past its allocation,
 * returns CO_ERR_DATA before anything is copied; other codes as
 * co_optimize_data. */
int co_optimize_data_device(void *handle, const CoOptions *opt, const PopHeader *header,
                            const int32_t *nt, const float *nv, const int32_t *ci,
                            const TreeMeta *metas, const double *c_dev,
                            double *c_final_dev, int32_t *status_dev,
                            double *loss_init_dev, double *loss_final_dev,
                            int32_t *iters_dev);

/* Device time of the last fit on the handle, from HIP events recorded on the
 * handle's stream before the first and after the last fit kernel. */
int co_last_kernel_ms(void *handle, double *fit_ms_out);

/* Per-launch device time of the last fit: bin_ms_out[k] (CO_BINS entries)
 * is the duration of the fit launches of bin k (k <= CO_FAST_MAX_K: the fast
 * kernel of K = k; CO_GENERAL_BIN: the general kernel), from HIP events
 * recorded around them on the stream they ran on; -1 for bins with no
 * expressions. No counterpart in the reference (measurement only). */
int co_last_bin_ms(void *handle, double *bin_ms_out);

/* Host-only narrowing of an fp64 fit's results to the fp32 carrier of
 * co_optimize (extension; co_optimize and the CLI's float32 blobs use it).
 * Writes c_out[total_c], loss_init_out / loss_final_out [M_prob]; status[M_prob]
 * is updated in place. The reference fits in fp32, so a constant it commits
 * is representable there; an fp64 fit can leave a finite constant or loss
 * beyond FLT_MAX. Such an expression (K > 0, a finite fp64 constant or final
 * loss that is +-inf in fp32) is treated as the fp64 guard treats a
 * non-finite loss (cusr/kernel/lm_core.cuh:299-351): its c_init is delivered,
 * loss_final_out = loss_init_out, and CONVERGED becomes MAXITER. No device
 * needed. Returns the number of expressions so treated (>= 0), or
 * CO_ERR_NULLARG / CO_ERR_PROGRAM (metas beyond total_c). */
int co_narrow_fp32(const PopHeader *header, const TreeMeta *metas, const double *c_init,
                   const double *c_final, const double *loss_init, const double *loss_final,
                   int32_t *status, float *c_out, float *loss_init_out, float *loss_final_out);

/* Host-only decode of a population, no device needed: runs every check
 * co_optimize runs before touching the device and returns its code
 * (0, 2, -2, -3, -4, -6). When it returns 0 and the pointers are non-NULL:
 *   program_out[2*total_nodes] the device programs: expression m's
 *                             instructions in the order the device executes
 *                             them (last node first) from word
 *                             program_off_out[m], one 64-bit word each for the
 *                             fast kernels, two for the general kernel;
 *   order_out[M_prob]         expressions grouped by K ascending (stable);
 *   bin_start_out[CO_MAX_K+2] start of each K bin in order_out, with
 *                             bin_start_out[CO_MAX_K+1] == M_prob;
 *   stack_out[M_prob]         value-stack depth each expression needs;
 *   program_off_out[M_prob]   first word of expression m's program;
 *   route_out[M_prob]         1 where the general kernel fits expression m
 *                             (co_fast_path false), else 0. */
int co_decode(const PopHeader *header,
              const int32_t *nt, const float *nv, const int32_t *ci,
              const TreeMeta *metas,
              uint64_t *program_out, int32_t *order_out,
              int32_t *bin_start_out, int32_t *stack_out,
              int32_t *program_off_out, int32_t *route_out);

#ifdef __cplusplus
}
#endif

#endif /* CUSR_CO_H */
