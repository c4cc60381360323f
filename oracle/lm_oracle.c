/* lm_oracle.c -- CPU restatement of the reference batched-LM path, in fp64.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the HIP path is compared
 * against; nothing in the product (cusr_amd/) links, loads or calls it. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
 *
 * It restates, one expression at a time and one point at a time:
 *   - pop.bin checks          cusr/kernel/loader.c:58-68, popio.py:59-72,87-91
 *   - the stack interpreter   cusr/kernel/lm_core.cuh:58-106 (fp64 like :216-270)
 *   - forward-mode AD         cusr/kernel/ad_interp.cuh:58-233
 *   - reverse-mode AD         cusr/kernel/revad_interp.cuh:45-157
 *   - JtJ / Jtr / loss        cusr/kernel/lm_core.cuh:127-177
 *   - damped Cholesky solve   cusr/kernel/batch_lm_ad.cu:134-192
 *   - LM accept/reject loop   cusr/kernel/batch_lm_ad.cu:295-495
 *   - fp64 boundary audit     cusr/kernel/lm_core.cuh:299-351
 * with these fixed choices, which the device path follows too:
 *   - fp64 throughout (CO_PREC_MIXED: fp32 interpreter and Jacobian, fp64
 *     residual, sums and solve); fused multiply-adds only where fma() is
 *     written, so compile with -ffp-contract=off;
 *   - forward AD carries one tangent per constant; because constants are
 *     ranked in prefix order, every subtree owns a contiguous rank range and
 *     an operator scales its left range by dOut/dLeft and its right range by
 *     dOut/dRight (select-to-zero for max/min/comparisons and flat branches);
 *   - sums over points: point i goes to lane i % 64, each lane sums its points
 *     in ascending order starting from 0.0, then lanes combine pairwise with
 *     strides 32, 16, 8, 4, 2, 1 (p[l] + p[l ^ s]);
 *   - lambda, xtol and the norms are fp64.
 * Elementary functions come from include/cusr_math.h on both sides (its
 * accuracy against the C library is pinned by tests/test_math.py); +, -, *, /,
 * sqrt and fma are IEEE correctly rounded on both sides.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/cusr_co.h"
#include "../include/cusr_math.h"


#define ORC_LANES 64
/* exp(20) rounded to double / float: the clamp value of OP_CEXP */
#define CEXP_CAP64 485165195.4097903
#define CEXP_CAP32 485165184.0f
#define ORC_MAXK 64
#define ORC_MAXD 256   /* variables per point */

/* ------------------------------------------------------------------ decode */

static int is_unary(int f) {
    switch (f) {
    case OP_SIN: case OP_COS: case OP_TAN: case OP_SINH: case OP_COSH: case OP_TANH:
    case OP_LOG: case OP_LOOSE_LOG: case OP_EXP: case OP_INV: case OP_LOOSE_INV:
    case OP_NEG: case OP_ABS: case OP_SQRT: case OP_LOOSE_SQRT:
    case OP_CEXP: case OP_SQUARE: case OP_PLOG:
        return 1;
    default:
        return 0;
    }
}

static int is_binary(int f) {
    switch (f) {
    case OP_ADD: case OP_SUB: case OP_MUL: case OP_DIV: case OP_LOOSE_DIV:
    case OP_POW: case OP_LOOSE_POW: case OP_MAX: case OP_MIN:
    case OP_LT: case OP_GT: case OP_LE: case OP_GE: case OP_PDIV:
        return 1;
    default:
        return 0;
    }
}

/* Validate one expression; return its stack depth or a negative CO_ERR code.
 * Follows the stack simulation of popio._sim_stack_depth (popio.py:59-72) and
 * the prefix-order rank rule of popio.build_pop (popio.py:87-91). */
static int orc_check_tree(const int32_t *nt, const float *nv, const int32_t *ci,
                          int n, int K, int D) {
    if (n <= 0) return CO_ERR_PROGRAM;
    int sp = 0, depth = 0, rank = 0;
    for (int i = 0; i < n; i++) {          /* prefix scan: ranks must be 0..K-1 */
        if (nt[i] == NODE_CONST) {
            if (ci[i] != rank) return CO_ERR_PROGRAM;
            rank++;
        }
    }
    if (rank != K) return CO_ERR_PROGRAM;
    for (int i = n - 1; i >= 0; i--) {
        int t = nt[i];
        float v = nv[i];
        if (t == NODE_VAR) {
            if (!(v >= 0.0f) || v != (float)(int)v || (int)v >= D) return CO_ERR_PROGRAM;
            sp++;
        } else if (t == NODE_CONST) {
            sp++;
        } else if (t == NODE_UFUNC) {
            if (v != (float)(int)v || !is_unary((int)v)) return CO_ERR_PROGRAM;
            if (sp < 1) return CO_ERR_PROGRAM;
        } else if (t == NODE_BFUNC) {
            if (v != (float)(int)v || !is_binary((int)v)) return CO_ERR_PROGRAM;
            if (sp < 2) return CO_ERR_PROGRAM;
            sp--;
        } else {
            return CO_ERR_PROGRAM;
        }
        if (sp > depth) depth = sp;
    }
    if (sp != 1) return CO_ERR_PROGRAM;
    return depth;
}

/* Header/array consistency, loader.c:58-68 order: sums first. */
int orc_check_pop(const PopHeader *h, const int32_t *nt, const float *nv,
                  const int32_t *ci, const TreeMeta *metas, int32_t *stack_out) {
    if (!h || !metas || (h->total_nodes > 0 && (!nt || !nv || !ci))) return CO_ERR_NULLARG;
    if (h->M_prob < 0 || h->N < 0 || h->n_vars < 0) return CO_ERR_NULLARG;
    long ks = 0, ns = 0;
    for (int m = 0; m < h->M_prob; m++) { ks += metas[m].K; ns += metas[m].n_nodes; }
    if (ks != h->total_c) return CO_ERR_SUM_C;
    if (ns != h->total_nodes) return CO_ERR_SUM_NODES;
    for (int m = 0; m < h->M_prob; m++) {
        const TreeMeta *t = &metas[m];
        if (t->node_offset < 0 || t->n_nodes < 0 ||
            (long)t->node_offset + t->n_nodes > h->total_nodes ||
            t->c_offset < 0 || t->K < 0 || (long)t->c_offset + t->K > h->total_c)
            return CO_ERR_PROGRAM;
        int d = orc_check_tree(nt + t->node_offset, nv + t->node_offset,
                               ci + t->node_offset, t->n_nodes, t->K, h->n_vars);
        if (d < 0) return d;
        if (stack_out) stack_out[m] = d;
    }
    return CO_OK;
}

/* ------------------------------------------------------------ operator table */

/* Value and local partials of one operator (fp64). mode: 0 multiply the
 * operand tangents by the partial, 1 select (keep if partial != 0 else 0).
 * want_d2 is 0 when the right operand has no constants (POW then skips
 * log(l), as ad_interp.cuh:188-200 does when the exponent tangent is 0). */
static double op_u64(int f, double a, double *d, int *mode) {
    double r;
    *mode = 0;
    switch (f) {
    case OP_SIN: cm_sincos(a, &r, d); break;
    case OP_COS: { double sn; cm_sincos(a, &sn, &r); *d = -sn; break; }
    case OP_TAN: r = cm_tan(a); *d = 1.0 + r * r; break;
    case OP_SINH: r = cm_sinh(a); *d = cm_cosh(a); break;
    case OP_COSH: r = cm_cosh(a); *d = cm_sinh(a); break;
    case OP_TANH: r = cm_tanh(a); *d = 1.0 - r * r; break;
    case OP_LOG: r = cm_log(a); *d = 1.0 / a; break;
    case OP_LOOSE_LOG: r = cm_log(fabs(a)); *d = 1.0 / a; break;
    case OP_EXP: r = cm_exp(a); *d = r; break;
    case OP_INV: case OP_LOOSE_INV: r = 1.0 / a; *d = -(r * r); break;
    case OP_NEG: r = -a; *d = -1.0; break;
    case OP_ABS: r = fabs(a); *d = (a > 0.0) ? 1.0 : ((a < 0.0) ? -1.0 : 0.0); break;
    case OP_SQRT: r = sqrt(a); *d = 1.0 / (2.0 * r); break;
    case OP_LOOSE_SQRT:
        r = sqrt(fabs(a));
        *d = (a > 0.0) ? 1.0 / (2.0 * r) : ((a < 0.0) ? -1.0 / (2.0 * r) : 0.0);
        break;
    case OP_CEXP:
        if (a > 20.0) { r = CEXP_CAP64; *d = 0.0; *mode = 1; }
        else { r = cm_exp(a); *d = r; }
        break;
    case OP_SQUARE: r = a * a; *d = a + a; break;
    case OP_PLOG: {
        double t = fabs(a) + 1e-9;
        r = cm_log(t);
        *d = (a > 0.0) ? 1.0 / t : ((a < 0.0) ? -1.0 / t : 0.0);
        break;
    }
    default: r = 0.0; *d = 0.0; break;
    }
    return r;
}

static double op_b64(int f, double l, double rv, int want_d2, double *d1, double *d2,
                     int *mode) {
    double o;
    *mode = 0;
    switch (f) {
    case OP_ADD: o = l + rv; *d1 = 1.0; *d2 = 1.0; break;
    case OP_SUB: o = l - rv; *d1 = 1.0; *d2 = -1.0; break;
    case OP_MUL: o = l * rv; *d1 = rv; *d2 = l; break;
    /* d(l/r)/dr = -(l/r) * (1/r): one division for the value, one for 1/r */
    case OP_DIV: case OP_LOOSE_DIV: o = l / rv; *d1 = 1.0 / rv; *d2 = -(o * *d1); break;
    case OP_PDIV:
        if (fabs(rv) < 1e-9) { o = 1.0; *d1 = 0.0; *d2 = 0.0; *mode = 1; }
        else { o = l / rv; *d1 = 1.0 / rv; *d2 = -(o * *d1); }
        break;
    case OP_POW:
        o = cm_pow(l, rv);
        *d1 = rv * cm_pow(l, rv - 1.0);
        *d2 = want_d2 ? o * cm_log(l) : 0.0;
        break;
    case OP_LOOSE_POW: {
        double al = fabs(l);
        double s = (l > 0.0) ? 1.0 : ((l < 0.0) ? -1.0 : 0.0);
        o = cm_pow(al, rv);
        *d1 = s * (rv * cm_pow(al, rv - 1.0));
        *d2 = want_d2 ? o * cm_log(al) : 0.0;
        break;
    }
    case OP_MAX: o = fmax(l, rv); *d1 = (l >= rv) ? 1.0 : 0.0; *d2 = (l >= rv) ? 0.0 : 1.0;
        *mode = 1; break;
    case OP_MIN: o = fmin(l, rv); *d1 = (l <= rv) ? 1.0 : 0.0; *d2 = (l <= rv) ? 0.0 : 1.0;
        *mode = 1; break;
    case OP_LT: o = (l < rv) ? 1.0 : 0.0; *d1 = 0.0; *d2 = 0.0; *mode = 1; break;
    case OP_GT: o = (l > rv) ? 1.0 : 0.0; *d1 = 0.0; *d2 = 0.0; *mode = 1; break;
    case OP_LE: o = (l <= rv) ? 1.0 : 0.0; *d1 = 0.0; *d2 = 0.0; *mode = 1; break;
    case OP_GE: o = (l >= rv) ? 1.0 : 0.0; *d1 = 0.0; *d2 = 0.0; *mode = 1; break;
    default: o = 0.0; *d1 = 0.0; *d2 = 0.0; break;
    }
    return o;
}

/* fp32 counterparts (CO_PREC_MIXED), C library float functions. */
static float op_u32(int f, float a, float *d, int *mode) {
    float r;
    *mode = 0;
    switch (f) {
    case OP_SIN: cm_sincosf(a, &r, d); break;
    case OP_COS: { float sn; cm_sincosf(a, &sn, &r); *d = -sn; break; }
    case OP_TAN: r = cm_tanf(a); *d = 1.0f + r * r; break;
    case OP_SINH: r = cm_sinhf(a); *d = cm_coshf(a); break;
    case OP_COSH: r = cm_coshf(a); *d = cm_sinhf(a); break;
    case OP_TANH: r = cm_tanhf(a); *d = 1.0f - r * r; break;
    case OP_LOG: r = cm_logf(a); *d = 1.0f / a; break;
    case OP_LOOSE_LOG: r = cm_logf(fabsf(a)); *d = 1.0f / a; break;
    case OP_EXP: r = cm_expf(a); *d = r; break;
    case OP_INV: case OP_LOOSE_INV: r = 1.0f / a; *d = -(r * r); break;
    case OP_NEG: r = -a; *d = -1.0f; break;
    case OP_ABS: r = fabsf(a); *d = (a > 0.0f) ? 1.0f : ((a < 0.0f) ? -1.0f : 0.0f); break;
    case OP_SQRT: r = sqrtf(a); *d = 1.0f / (2.0f * r); break;
    case OP_LOOSE_SQRT:
        r = sqrtf(fabsf(a));
        *d = (a > 0.0f) ? 1.0f / (2.0f * r) : ((a < 0.0f) ? -1.0f / (2.0f * r) : 0.0f);
        break;
    case OP_CEXP:
        if (a > 20.0f) { r = CEXP_CAP32; *d = 0.0f; *mode = 1; }
        else { r = cm_expf(a); *d = r; }
        break;
    case OP_SQUARE: r = a * a; *d = a + a; break;
    case OP_PLOG: {
        float t = fabsf(a) + 1e-9f;
        r = cm_logf(t);
        *d = (a > 0.0f) ? 1.0f / t : ((a < 0.0f) ? -1.0f / t : 0.0f);
        break;
    }
    default: r = 0.0f; *d = 0.0f; break;
    }
    return r;
}

static float op_b32(int f, float l, float rv, int want_d2, float *d1, float *d2, int *mode) {
    float o;
    *mode = 0;
    switch (f) {
    case OP_ADD: o = l + rv; *d1 = 1.0f; *d2 = 1.0f; break;
    case OP_SUB: o = l - rv; *d1 = 1.0f; *d2 = -1.0f; break;
    case OP_MUL: o = l * rv; *d1 = rv; *d2 = l; break;
    case OP_DIV: case OP_LOOSE_DIV: o = l / rv; *d1 = 1.0f / rv; *d2 = -(o * *d1); break;
    case OP_PDIV:
        if (fabsf(rv) < 1e-9f) { o = 1.0f; *d1 = 0.0f; *d2 = 0.0f; *mode = 1; }
        else { o = l / rv; *d1 = 1.0f / rv; *d2 = -(o * *d1); }
        break;
    case OP_POW:
        o = cm_powf(l, rv);
        *d1 = rv * cm_powf(l, rv - 1.0f);
        *d2 = want_d2 ? o * cm_logf(l) : 0.0f;
        break;
    case OP_LOOSE_POW: {
        float al = fabsf(l);
        float s = (l > 0.0f) ? 1.0f : ((l < 0.0f) ? -1.0f : 0.0f);
        o = cm_powf(al, rv);
        *d1 = s * (rv * cm_powf(al, rv - 1.0f));
        *d2 = want_d2 ? o * cm_logf(al) : 0.0f;
        break;
    }
    case OP_MAX: o = fmaxf(l, rv); *d1 = (l >= rv) ? 1.0f : 0.0f; *d2 = (l >= rv) ? 0.0f : 1.0f;
        *mode = 1; break;
    case OP_MIN: o = fminf(l, rv); *d1 = (l <= rv) ? 1.0f : 0.0f; *d2 = (l <= rv) ? 0.0f : 1.0f;
        *mode = 1; break;
    case OP_LT: o = (l < rv) ? 1.0f : 0.0f; *d1 = 0.0f; *d2 = 0.0f; *mode = 1; break;
    case OP_GT: o = (l > rv) ? 1.0f : 0.0f; *d1 = 0.0f; *d2 = 0.0f; *mode = 1; break;
    case OP_LE: o = (l <= rv) ? 1.0f : 0.0f; *d1 = 0.0f; *d2 = 0.0f; *mode = 1; break;
    case OP_GE: o = (l >= rv) ? 1.0f : 0.0f; *d1 = 0.0f; *d2 = 0.0f; *mode = 1; break;
    default: o = 0.0f; *d1 = 0.0f; *d2 = 0.0f; break;
    }
    return o;
}

/* 0-annihilating product of the reverse sweep (revad_interp.cuh:45-47). */
static double safe_mul64(double a, double b) { return (a == 0.0 || b == 0.0) ? 0.0 : a * b; }
static float safe_mul32(float a, float b) { return (a == 0.0f || b == 0.0f) ? 0.0f : a * b; }

/* ----------------------------------------------------------- one point */

typedef struct {
    const int32_t *nt;
    const float *nv;
    const int32_t *ci;
    int n, K;
    int general;   /* fitted by the device's general kernel (co_fast_path false) */
    /* per-point scratch, n entries each (tree_init) */
    double *st, *t1, *t2, *sa;
    float *st32, *t132, *t232, *sa32;
    int *lo, *hi;
} Tree;

static int tree_init(Tree *t, const int32_t *nt, const float *nv, const int32_t *ci, int n,
                     int K, int general) {
    t->nt = nt; t->nv = nv; t->ci = ci; t->n = n; t->K = K; t->general = general;
    const size_t m = n > 0 ? (size_t)n : 1;
    char *b = (char *)malloc(m * (4 * sizeof(double) + 4 * sizeof(float) + 2 * sizeof(int)));
    if (!b) return CO_ERR_OOM;
    t->st = (double *)b; t->t1 = t->st + m; t->t2 = t->t1 + m; t->sa = t->t2 + m;
    t->st32 = (float *)(t->sa + m); t->t132 = t->st32 + m; t->t232 = t->t132 + m;
    t->sa32 = t->t232 + m;
    t->lo = (int *)(t->sa32 + m); t->hi = t->lo + m;
    return CO_OK;
}

static void tree_free(Tree *t) { free(t->st); t->st = NULL; }

/* Value and (optionally) gradient at one point, fp64.
 * jac: 0 none, 1 forward (range scaling), 2 reverse (tape + adjoint stack). */
static double point64(const Tree *t, const double *x, const double *c, int jac, double *g) {
    double *st = t->st, *tape1 = t->t1, *tape2 = t->t2;
    int *lo = t->lo, *hi = t->hi;
    int sp = 0;
    for (int i = t->n - 1; i >= 0; i--) {
        int ty = t->nt[i];
        int f = (int)t->nv[i];
        if (ty == NODE_VAR) {
            st[sp] = x[f]; lo[sp] = ORC_MAXK; hi[sp] = 0; sp++;
        } else if (ty == NODE_CONST) {
            int k = t->ci[i];
            st[sp] = c[k]; lo[sp] = k; hi[sp] = k + 1;
            if (jac == 1) g[k] = 1.0;
            sp++;
        } else if (ty == NODE_UFUNC) {
            double d; int mode;
            double a = st[sp - 1];
            double r = op_u64(f, a, &d, &mode);
            st[sp - 1] = r;
            if (jac == 1) {
                for (int j = lo[sp - 1]; j < hi[sp - 1]; j++)
                    g[j] = mode ? ((d != 0.0) ? g[j] : 0.0) : g[j] * d;
            } else if (jac == 2) {
                tape1[i] = d;
            }
        } else {
            double d1, d2; int mode;
            double l = st[sp - 1], rv = st[sp - 2];
            int want_d2 = (jac == 2) || (lo[sp - 2] < hi[sp - 2]);
            double o = op_b64(f, l, rv, want_d2, &d1, &d2, &mode);
            if (jac == 1) {
                for (int j = lo[sp - 1]; j < hi[sp - 1]; j++)
                    g[j] = mode ? ((d1 != 0.0) ? g[j] : 0.0) : g[j] * d1;
                for (int j = lo[sp - 2]; j < hi[sp - 2]; j++)
                    g[j] = mode ? ((d2 != 0.0) ? g[j] : 0.0) : g[j] * d2;
            } else if (jac == 2) {
                tape1[i] = d1; tape2[i] = d2;
            }
            int nlo = lo[sp - 1] < lo[sp - 2] ? lo[sp - 1] : lo[sp - 2];
            int nhi = hi[sp - 1] > hi[sp - 2] ? hi[sp - 1] : hi[sp - 2];
            sp -= 2;
            st[sp] = o; lo[sp] = nlo; hi[sp] = nhi; sp++;
        }
    }
    if (jac == 2) {
        /* backward sweep in prefix order, revad_interp.cuh:131-156 */
        double *sa = t->sa;
        int asp = 0;
        for (int k = 0; k < t->K; k++) g[k] = 0.0;
        sa[asp++] = 1.0;
        for (int i = 0; i < t->n; i++) {
            int ty = t->nt[i];
            double adj = sa[--asp];
            if (ty == NODE_CONST) {
                g[t->ci[i]] = g[t->ci[i]] + adj;
            } else if (ty == NODE_UFUNC) {
                sa[asp++] = safe_mul64(adj, tape1[i]);
            } else if (ty == NODE_BFUNC) {
                sa[asp++] = safe_mul64(adj, tape2[i]);
                sa[asp++] = safe_mul64(adj, tape1[i]);
            }
        }
    }
    return st[0];
}

static float point32(const Tree *t, const double *x, const double *c, int jac, float *g) {
    float *st = t->st32, *tape1 = t->t132, *tape2 = t->t232;
    int *lo = t->lo, *hi = t->hi;
    int sp = 0;
    for (int i = t->n - 1; i >= 0; i--) {
        int ty = t->nt[i];
        int f = (int)t->nv[i];
        if (ty == NODE_VAR) {
            st[sp] = (float)x[f]; lo[sp] = ORC_MAXK; hi[sp] = 0; sp++;
        } else if (ty == NODE_CONST) {
            int k = t->ci[i];
            st[sp] = (float)c[k]; lo[sp] = k; hi[sp] = k + 1;
            if (jac == 1) g[k] = 1.0f;
            sp++;
        } else if (ty == NODE_UFUNC) {
            float d; int mode;
            float r = op_u32(f, st[sp - 1], &d, &mode);
            st[sp - 1] = r;
            if (jac == 1) {
                for (int j = lo[sp - 1]; j < hi[sp - 1]; j++)
                    g[j] = mode ? ((d != 0.0f) ? g[j] : 0.0f) : g[j] * d;
            } else if (jac == 2) {
                tape1[i] = d;
            }
        } else {
            float d1, d2; int mode;
            float l = st[sp - 1], rv = st[sp - 2];
            int want_d2 = (jac == 2) || (lo[sp - 2] < hi[sp - 2]);
            float o = op_b32(f, l, rv, want_d2, &d1, &d2, &mode);
            if (jac == 1) {
                for (int j = lo[sp - 1]; j < hi[sp - 1]; j++)
                    g[j] = mode ? ((d1 != 0.0f) ? g[j] : 0.0f) : g[j] * d1;
                for (int j = lo[sp - 2]; j < hi[sp - 2]; j++)
                    g[j] = mode ? ((d2 != 0.0f) ? g[j] : 0.0f) : g[j] * d2;
            } else if (jac == 2) {
                tape1[i] = d1; tape2[i] = d2;
            }
            int nlo = lo[sp - 1] < lo[sp - 2] ? lo[sp - 1] : lo[sp - 2];
            int nhi = hi[sp - 1] > hi[sp - 2] ? hi[sp - 1] : hi[sp - 2];
            sp -= 2;
            st[sp] = o; lo[sp] = nlo; hi[sp] = nhi; sp++;
        }
    }
    if (jac == 2) {
        float *sa = t->sa32;
        int asp = 0;
        for (int k = 0; k < t->K; k++) g[k] = 0.0f;
        sa[asp++] = 1.0f;
        for (int i = 0; i < t->n; i++) {
            int ty = t->nt[i];
            float adj = sa[--asp];
            if (ty == NODE_CONST) {
                g[t->ci[i]] = g[t->ci[i]] + adj;
            } else if (ty == NODE_UFUNC) {
                sa[asp++] = safe_mul32(adj, tape1[i]);
            } else if (ty == NODE_BFUNC) {
                sa[asp++] = safe_mul32(adj, tape2[i]);
                sa[asp++] = safe_mul32(adj, tape1[i]);
            }
        }
    }
    return st[0];
}

/* --------------------------------------------------------- one data pass */

typedef struct {
    double loss;              /* 0.5 * sum r^2 */
    double jtj[ORC_MAXK * ORC_MAXK]; /* upper triangle, row-major jtj[a*K+b], a <= b */
    double jtr[ORC_MAXK];
} PassOut;

/* One pass in the device's order (cusr_amd/csrc/lm_device.h data_pass and
 * data_pass_gen): 64-point granule g belongs to partition g mod G; the
 * partitions' sums are added in order 0, 1, ..., G-1 at the end. Within a
 * partition:
 *   - value-only passes, and Jacobian passes of the fast kernels with smaller
 *     K: point i goes to lane i mod 64, which sums its points
 *     in ascending order from 0.0 with fma; the lanes combine with strides
 *     32..1;
 *   - Jacobian passes of the fast kernels in forward AD with
 *     K >= CO_SUMS_MATRIX_MIN_K, or in reverse AD with
 *     K >= CO_SUMS_MATRIX_MIN_K_REV: every entry of [J | r]^T [J | r] is one fma
 *     chain over the partition's points in ascending order (the matrix
 *     instruction's order); for K = 16, r^2 and J^T r keep the lane order;
 *   - Jacobian passes of the general kernel (either AD mode, any K): every
 *     entry of [J | r]^T [J | r], r^2 and J^T r included, is one such chain. */
static void orc_pass(const Tree *t, int N, int D, const double *xs, const double *y,
                     const double *c, int prec, int jac, int G, PassOut *out) {
    int K = t->K;
    int nq = K * (K + 1) / 2;
    int width = 1 + K + nq;
    const int mx = jac != 0 && (t->general || (jac == 1 && K >= CO_SUMS_MATRIX_MIN_K) ||
                                (jac == 2 && K >= CO_SUMS_MATRIX_MIN_K_REV));
    const int full = t->general || K < 16;  /* r is a column of the product */
    const int ncol = full ? K + 1 : 16;     /* columns of the matrix product */
    const int lane_w = mx ? (full ? 0 : 1 + K) : width;
    double *acc = (double *)calloc((size_t)G * ORC_LANES * (lane_w ? lane_w : 1), sizeof(double));
    double *gm = mx ? (double *)calloc((size_t)G * ncol * ncol, sizeof(double)) : NULL;
    double g64[ORC_MAXK];
    float g32[ORC_MAXK];
    double x[ORC_MAXD], aug[ORC_MAXK + 1];
    for (int i = 0; i < N; i++) {
        int part = (i / ORC_LANES) % G;
        double *a = acc + ((size_t)part * ORC_LANES + (size_t)(i % ORC_LANES)) * (lane_w ? lane_w : 1);
        for (int k = 0; k < D; k++) x[k] = xs[(size_t)i * D + k];
        double f;
        if (prec == CO_PREC_FP64) {
            f = point64(t, x, c, jac, g64);
        } else {
            f = (double)point32(t, x, c, jac, g32);
            if (jac)
                for (int k = 0; k < K; k++) g64[k] = (double)g32[k];
        }
        double r = f - y[i];
        if (mx) {
            for (int k = 0; k < K; k++) aug[k] = g64[k];
            if (full) aug[K] = r;
            double *gp = gm + (size_t)part * ncol * ncol;
            for (int i1 = 0; i1 < ncol; i1++)
                for (int i2 = 0; i2 < ncol; i2++)
                    gp[i1 * ncol + i2] = fma(aug[i1], aug[i2], gp[i1 * ncol + i2]);
            if (!full) {
                a[0] = fma(r, r, a[0]);
                for (int j = 0; j < K; j++) a[1 + j] = fma(g64[j], r, a[1 + j]);
            }
            continue;
        }
        a[0] = fma(r, r, a[0]);
        if (jac) {
            for (int j = 0; j < K; j++) a[1 + j] = fma(g64[j], r, a[1 + j]);
            int q = 1 + K;
            for (int j1 = 0; j1 < K; j1++)
                for (int j2 = j1; j2 < K; j2++, q++) a[q] = fma(g64[j1], g64[j2], a[q]);
        }
    }
    /* per partition: lane butterfly (lane sums), then the sums vector */
    double *sums = (double *)calloc((size_t)G * width, sizeof(double));
    for (int part = 0; part < G; part++) {
        double *ps = sums + (size_t)part * width;
        if (lane_w) {
            double *pacc = acc + (size_t)part * ORC_LANES * lane_w;
            for (int s = ORC_LANES / 2; s >= 1; s >>= 1) {
                /* every lane becomes p[l] + p[l^s]; lanes l and l^s hold the same value */
                for (int l = 0; l < ORC_LANES; l++) {
                    if (l & s) continue;
                    double *pa = pacc + (size_t)l * lane_w, *pb = pacc + (size_t)(l ^ s) * lane_w;
                    for (int w = 0; w < lane_w; w++) { double v = pa[w] + pb[w]; pa[w] = v; pb[w] = v; }
                }
            }
            for (int w = 0; w < lane_w; w++) ps[w] = pacc[w];
        }
        if (mx) {
            const double *gp = gm + (size_t)part * ncol * ncol;
            if (full) {
                ps[0] = gp[K * ncol + K];
                for (int j = 0; j < K; j++) ps[1 + j] = gp[j * ncol + K];
            }
            int q = 1 + K;
            for (int j1 = 0; j1 < K; j1++)
                for (int j2 = j1; j2 < K; j2++, q++) ps[q] = gp[j1 * ncol + j2];
        }
    }
    /* partition sums added in partition order */
    for (int part = 1; part < G; part++) {
        const double *pp = sums + (size_t)part * width;
        for (int w = 0; w < width; w++) sums[w] = sums[w] + pp[w];
    }
    out->loss = 0.5 * sums[0];
    if (jac) {
        for (int j = 0; j < K; j++) out->jtr[j] = sums[1 + j];
        int q = 1 + K;
        for (int j1 = 0; j1 < K; j1++)
            for (int j2 = j1; j2 < K; j2++, q++) out->jtj[j1 * K + j2] = sums[q];
    }
    free(sums);
    free(gm);
    free(acc);
}

/* Partitions of an N-point expression under options o. */
static int orc_partitions(const CoOptions *o, int N) {
    return co_partitions_resolve(o, N);
}

/* ------------------------------------------------------------- the solve */

/* Damped Cholesky solve (batch_lm_ad.cu:149-191): A = JtJ, b = -Jtr, under
 * the damping variant of batch_lm_ad.cu:152-172 (its -DTRUST_REGION and
 * -DPIVOT_FLOOR builds): CO_DAMP_RELATIVE A_jj *= (1 + lambda) and a pivot
 * s <= 0 fails the step; CO_DAMP_TRUST_REGION A_jj += lambda and a pivot
 * s <= 0 is replaced by lambda; CO_DAMP_PIVOT_FLOOR A_jj *= (1 + lambda) and a
 * pivot below CO_PIVOT_FLOOR_EPS is raised to it.
 * Returns 0 and delta, or -1. */
static int orc_solve(int K, const double *jtj, const double *jtr, double lambda, int damp,
                     double *delta) {
    double L[ORC_MAXK * ORC_MAXK];
    double b[ORC_MAXK];
    for (int i = 0; i < K; i++) {
        b[i] = -jtr[i];
        for (int j = 0; j <= i; j++) L[i * K + j] = jtj[j * K + i];
        if (damp == CO_DAMP_TRUST_REGION) L[i * K + i] = L[i * K + i] + lambda;
        else L[i * K + i] = L[i * K + i] * (1.0 + lambda);
    }
    for (int j = 0; j < K; j++) {
        double s = L[j * K + j];
        for (int k = 0; k < j; k++) s = fma(-L[j * K + k], L[j * K + k], s);
        if (damp == CO_DAMP_TRUST_REGION) {
            if (s <= 0.0) s = lambda;
        } else if (damp == CO_DAMP_PIVOT_FLOOR) {
            if (s < CO_PIVOT_FLOOR_EPS) s = CO_PIVOT_FLOOR_EPS;
        } else if (s <= 0.0) {
            return -1;
        }
        double dj = sqrt(s);
        L[j * K + j] = dj;
        for (int i = j + 1; i < K; i++) {
            double t = L[i * K + j];
            for (int k = 0; k < j; k++) t = fma(-L[i * K + k], L[j * K + k], t);
            L[i * K + j] = t / dj;
        }
    }
    for (int i = 0; i < K; i++) {
        double s = b[i];
        for (int k = 0; k < i; k++) s = fma(-L[i * K + k], b[k], s);
        b[i] = s / L[i * K + i];
    }
    for (int i = K - 1; i >= 0; i--) {
        double s = b[i];
        for (int k = i + 1; k < K; k++) s = fma(-L[k * K + i], b[k], s);
        b[i] = s / L[i * K + i];
    }
    for (int i = 0; i < K; i++) delta[i] = b[i];
    return 0;
}

/* ------------------------------------------------------------ the LM fit */

void orc_options_default(CoOptions *o) {
    memset(o, 0, sizeof(*o));
    o->struct_size = (int32_t)sizeof(CoOptions);
    o->ad_mode = CO_AD_FORWARD;
    o->precision = CO_PREC_FP64;
    o->max_iter = 50;
    o->lambda0 = 1e-3;
    o->xtol = 1e-6;
    o->fp64_guard = 1;
}

/* A loss the fit may go on from: finite, and with f32_range finite in fp32
 * too (the reference accumulates it in fp32). */
static int orc_finite(const CoOptions *o, double loss) {
    return isfinite(loss) && (!o->f32_range || isfinite((float)loss));
}

/* One expression (batch_lm_ad.cu:295-495 restricted to tree m, with the
 * Jacobian evaluated at every accepted point and reused after a reject). */
static void orc_fit_one(const CoOptions *o, const Tree *t, int N, int D, const double *xs,
                        const double *y, const double *c0, double *c_out, int32_t *status,
                        double *loss_init, double *loss_final, int32_t *iters) {
    int K = t->K;
    int jac = (o->ad_mode == CO_AD_REVERSE) ? 2 : 1;
    double c[ORC_MAXK] = {0}, ct[ORC_MAXK], delta[ORC_MAXK];
    PassOut *cur = (PassOut *)malloc(sizeof(PassOut));
    PassOut *tri = (PassOut *)malloc(sizeof(PassOut));
    for (int k = 0; k < K; k++) c[k] = c0[k];
    int st = 0; /* 0 running, 1 conv, 2 nan, 3 K0, 4 chol */
    int it = 0;
    /* partitions: G1 up to iteration T1, then the tail's G2 (cusr_co.h
     * co_tail_resolve); T1 == 0 keeps G1 throughout */
    const int G1 = orc_partitions(o, N);
    int G2 = G1;
    const int T1 = co_tail_resolve(o, N, &G2);
    int G = G1;
    orc_pass(t, N, D, xs, y, c, o->precision, K > 0 ? jac : 0, G, cur);
    double li = cur->loss;
    if (K == 0) st = 3;
    else if (!orc_finite(o, cur->loss)) st = 2;
    double lambda = o->lambda0;
    while (st == 0 && it < o->max_iter) {
        it++;
        G = (T1 && it > T1) ? G2 : G1;
        if (orc_solve(K, cur->jtj, cur->jtr, lambda, o->damping, delta) != 0) {
            lambda = lambda * 10.0;
            if (lambda > 1e12) st = 4;
            continue;
        }
        for (int k = 0; k < K; k++) ct[k] = c[k] + delta[k];
        if (o->f32_range) {
            /* trial constants held in fp32 like the reference's; one the fp32
             * fit cannot hold makes its trial loss non-finite there
             * (batch_lm_ad.cu:437-443); no pass needed */
            int over = 0;
            for (int k = 0; k < K; k++) {
                ct[k] = (double)(float)ct[k];
                over |= !isfinite(ct[k]);
            }
            if (over) { st = 2; continue; }
        }
        orc_pass(t, N, D, xs, y, ct, o->precision, jac, G, tri);
        if (!orc_finite(o, tri->loss)) { st = 2; continue; }
        double dn2 = 0.0, cn2 = 0.0;
        for (int k = 0; k < K; k++) {
            dn2 = fma(delta[k], delta[k], dn2);
            cn2 = fma(ct[k], ct[k], cn2);
        }
        double dn = sqrt(dn2), cn = sqrt(cn2);
        const int small = dn < o->xtol * (cn + o->xtol);
        int accept, conv;
        if (o->lm_order == CO_ORDER_CONVERGE_FIRST) {
            /* FD variant (co_lib.cu:457-473): a small step converges whatever
             * the loss; otherwise only a strict decrease is accepted */
            conv = small;
            accept = small || tri->loss < cur->loss;
        } else {
            /* AD variant (batch_lm_ad.cu:456-473): improvement first */
            accept = tri->loss <= cur->loss;
            conv = accept && small;
        }
        if (accept) {
            for (int k = 0; k < K; k++) c[k] = ct[k];
            PassOut *sw = cur; cur = tri; tri = sw;
        }
        if (conv) {
            st = 1;
        } else if (accept) {
            lambda = lambda * 0.1;
            if (lambda < 1e-12) lambda = 1e-12;
        } else {
            lambda = lambda * 10.0;
            if (lambda > 1e12) st = 2;
        }
    }
    double lf = cur->loss;
    if (o->precision != CO_PREC_FP64) {
        /* fp64 losses at the delivered point and at the start */
        PassOut *p = tri;
        orc_pass(t, N, D, xs, y, c, CO_PREC_FP64, 0, G, p);
        lf = p->loss;
        orc_pass(t, N, D, xs, y, c0, CO_PREC_FP64, 0, G, p);
        li = p->loss;
    }
    if (o->fp64_guard && K > 0) {
        if (!isfinite(lf) || (isfinite(li) && lf > li)) {
            for (int k = 0; k < K; k++) c[k] = c0[k];
            if (st == 1) st = 0;
            lf = li;
        }
    }
    for (int k = 0; k < K; k++) c_out[k] = c[k];
    static const int32_t map[5] = {STATUS_MAXITER, STATUS_CONVERGED, STATUS_FAIL_NAN,
                                   STATUS_K0_SKIP, STATUS_FAIL_CHOLESKY};
    *status = map[st];
    *loss_init = li;
    *loss_final = lf;
    *iters = it;
    free(cur);
    free(tri);
}

/* Checks a population and sets up expression m's tree and its kernel family
 * (co_fast_path on K, stack depth, nodes and n_vars, as the device decode
 * routes it). */
static int *orc_depths(const PopHeader *h, const int32_t *nt, const float *nv,
                       const int32_t *ci, const TreeMeta *metas, int *rc) {
    int *depth = (int *)malloc(sizeof(int) * (h && h->M_prob > 0 ? (size_t)h->M_prob : 1));
    if (!depth) { *rc = CO_ERR_OOM; return NULL; }
    *rc = orc_check_pop(h, nt, nv, ci, metas, depth);
    if (*rc == CO_OK && h->n_vars > ORC_MAXD) *rc = CO_ERR_BOUNDS;
    for (int m = 0; *rc == CO_OK && m < h->M_prob; m++)
        if (metas[m].K > CO_MAX_K || depth[m] > CO_MAX_STACK) *rc = CO_ERR_BOUNDS;
    if (*rc != CO_OK) { free(depth); return NULL; }
    return depth;
}

static int orc_tree(const PopHeader *h, const int32_t *nt, const float *nv, const int32_t *ci,
                    const TreeMeta *metas, const int *depth, int m, Tree *t) {
    const TreeMeta *mt = &metas[m];
    const int general = !co_fast_path(mt->K, depth[m], mt->n_nodes, h->n_vars);
    return tree_init(t, nt + mt->node_offset, nv + mt->node_offset, ci + mt->node_offset,
                     mt->n_nodes, mt->K, general);
}

/* Whole-population fit; same arguments as co_optimize_ex minus the handle. */
int orc_fit(const CoOptions *o, const PopHeader *h, const int32_t *nt, const float *nv,
            const int32_t *ci, const TreeMeta *metas, const double *c_init,
            const double *xs, const double *ym, double *c_final, int32_t *status,
            double *loss_init, double *loss_final, int32_t *iters) {
    int rc;
    if (co_partitions_resolve(o, h->N) == 0) return CO_ERR_NULLARG;
    int *depth = orc_depths(h, nt, nv, ci, metas, &rc);
    if (!depth) return rc;
    for (int m = 0; m < h->M_prob; m++) {
        const TreeMeta *mt = &metas[m];
        Tree t;
        if ((rc = orc_tree(h, nt, nv, ci, metas, depth, m, &t)) != CO_OK) break;
        double li, lf;
        int32_t st, itn;
        const double *yrow = (pop_flags(h) & POP_FLAG_SHARED_Y) ? ym : ym + (size_t)m * h->N;
        orc_fit_one(o, &t, h->N, h->n_vars, xs, yrow, c_init + mt->c_offset,
                    c_final + mt->c_offset, &st, &li, &lf, &itn);
        tree_free(&t);
        status[m] = st;
        if (loss_init) loss_init[m] = li;
        if (loss_final) loss_final[m] = lf;
        if (iters) iters[m] = itn;
    }
    free(depth);
    return rc;
}

/* Values y[m*N+i] (prec CO_PREC_FP64 or CO_PREC_MIXED). */
int orc_eval(const PopHeader *h, const int32_t *nt, const float *nv, const int32_t *ci,
             const TreeMeta *metas, const double *c, const double *xs, int prec,
             double *y) {
    int rc;
    int *depth = orc_depths(h, nt, nv, ci, metas, &rc);
    if (!depth) return rc;
    double x[ORC_MAXD];
    for (int m = 0; m < h->M_prob; m++) {
        const TreeMeta *mt = &metas[m];
        Tree t;
        if ((rc = orc_tree(h, nt, nv, ci, metas, depth, m, &t)) != CO_OK) break;
        for (int i = 0; i < h->N; i++) {
            for (int k = 0; k < h->n_vars; k++) x[k] = xs[(size_t)i * h->n_vars + k];
            y[(size_t)m * h->N + i] = (prec == CO_PREC_FP64)
                ? point64(&t, x, c + mt->c_offset, 0, NULL)
                : (double)point32(&t, x, c + mt->c_offset, 0, NULL);
        }
        tree_free(&t);
    }
    free(depth);
    return rc;
}

/* Jacobian rows J[(m*N + i)*K_max + j] (fp64), ad_mode 0 forward / 1 reverse. */
int orc_jacobian(const PopHeader *h, const int32_t *nt, const float *nv, const int32_t *ci,
                 const TreeMeta *metas, const double *c, const double *xs, int ad_mode,
                 double *J) {
    int rc;
    int *depth = orc_depths(h, nt, nv, ci, metas, &rc);
    if (!depth) return rc;
    double x[ORC_MAXD], g[ORC_MAXK];
    int KM = h->K_max;
    for (int m = 0; m < h->M_prob; m++) {
        const TreeMeta *mt = &metas[m];
        if (mt->K > KM) { rc = CO_ERR_BOUNDS; break; }
        Tree t;
        if ((rc = orc_tree(h, nt, nv, ci, metas, depth, m, &t)) != CO_OK) break;
        for (int i = 0; i < h->N; i++) {
            for (int k = 0; k < h->n_vars; k++) x[k] = xs[(size_t)i * h->n_vars + k];
            if (mt->K > 0) point64(&t, x, c + mt->c_offset, ad_mode == CO_AD_REVERSE ? 2 : 1, g);
            for (int j = 0; j < KM; j++)
                J[((size_t)m * h->N + i) * KM + j] = (j < mt->K) ? g[j] : 0.0;
        }
        tree_free(&t);
    }
    free(depth);
    return rc;
}

/* The damped solve alone, for tests against a textbook Cholesky. */
int orc_solve_api(int K, const double *jtj_upper, const double *jtr, double lambda,
                  int damping, double *delta) {
    if (K < 1 || K > ORC_MAXK) return CO_ERR_BOUNDS;
    return orc_solve(K, jtj_upper, jtr, lambda, damping, delta);
}

/* The canonical pass alone: loss, Jtr and the JtJ upper triangle of one
 * expression at c (tests use it to pin the reduction order). */
int orc_pass_api(const PopHeader *h, const int32_t *nt, const float *nv, const int32_t *ci,
                 const TreeMeta *metas, int m, const double *c, const double *xs,
                 const double *y, int prec, int ad_mode, int partitions, double *loss,
                 double *jtj, double *jtr) {
    int rc;
    int *depth = orc_depths(h, nt, nv, ci, metas, &rc);
    if (!depth) return rc;
    if (m < 0 || m >= h->M_prob) { free(depth); return CO_ERR_NULLARG; }
    const TreeMeta *mt = &metas[m];
    Tree t;
    rc = orc_tree(h, nt, nv, ci, metas, depth, m, &t);
    free(depth);
    if (rc != CO_OK) return rc;
    PassOut *p = (PassOut *)malloc(sizeof(PassOut));
    const int G = partitions ? partitions : co_partitions_for(h->N, ad_mode);
    orc_pass(&t, h->N, h->n_vars, xs, y, c, prec, mt->K > 0 ? (ad_mode ? 2 : 1) : 0, G, p);
    *loss = p->loss;
    for (int j = 0; j < mt->K; j++) {
        jtr[j] = p->jtr[j];
        for (int k = 0; k < mt->K; k++)
            jtj[j * mt->K + k] = (j <= k) ? p->jtj[j * mt->K + k] : p->jtj[k * mt->K + j];
    }
    free(p);
    tree_free(&t);
    return CO_OK;
}

/* Elementary functions of include/cusr_math.h over arrays, for the accuracy
 * tests against the C library. fn: 0 exp, 1 log, 2 sin, 3 cos, 4 tan, 5 sinh,
 * 6 cosh, 7 tanh, 8 pow(x, y); +16 for the fp32 versions (inputs rounded to
 * float, results widened). */
int orc_math(int fn, int n, const double *x, const double *y, double *out) {
    for (int i = 0; i < n; i++) {
        double a = x[i], b = y ? y[i] : 0.0;
        float af = (float)a, bf = (float)b;
        double r;
        switch (fn) {
        case 0: r = cm_exp(a); break;
        case 1: r = cm_log(a); break;
        case 2: r = cm_sin(a); break;
        case 3: r = cm_cos(a); break;
        case 4: r = cm_tan(a); break;
        case 5: r = cm_sinh(a); break;
        case 6: r = cm_cosh(a); break;
        case 7: r = cm_tanh(a); break;
        case 8: r = cm_pow(a, b); break;
        case 16: r = cm_expf(af); break;
        case 17: r = cm_logf(af); break;
        case 18: r = cm_sinf(af); break;
        case 19: r = cm_cosf(af); break;
        case 20: r = cm_tanf(af); break;
        case 21: r = cm_sinhf(af); break;
        case 22: r = cm_coshf(af); break;
        case 23: r = cm_tanhf(af); break;
        case 24: r = cm_powf(af, bf); break;
        default: return CO_ERR_NULLARG;
        }
        out[i] = r;
    }
    return CO_OK;
}
