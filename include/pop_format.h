/* pop_format.h -- on-disk / in-memory layout of a pop.bin v1 population.
 *
 * Byte-compatible with the reference format (cusr/kernel/pop_format.h:6-51):
 * a 64-byte header of 16 little-endian int32, then the arrays
 *
 *   nt     int32  [total_nodes]   node type (NODE_VAR/CONST/UFUNC/BFUNC)
 *   nv     float32[total_nodes]   VAR -> input index, FUNC -> op id, CONST -> 0
 *   ci     int32  [total_nodes]   CONST -> local rank 0..K-1 in prefix order, else -1
 *   metas  TreeMeta[M_prob]       (node_offset, n_nodes, c_offset, K)
 *   c_init float32[total_c]
 *   xs     float32[N * n_vars]    row-major, xs[i*n_vars + k]
 *   ym     float32[M_prob * N]    per-expression targets, ym[m*N + i]
 *
 * Each expression is stored in prefix order; it is evaluated from its last
 * node to its first with a value stack, and a binary node [op, L, R] computes
 * L op R where L is the operand popped first (cusr/kernel/lm_core.cuh:85-87).
 */
#ifndef CUSR_POP_FORMAT_H
#define CUSR_POP_FORMAT_H

#include <stdint.h>

#define POP_MAGIC   0x4D4C344D /* "M4LM" read as a little-endian uint32 */
#define POP_VERSION 1

/* pop.bin v2 (extension; v1 files are unchanged and still read): version 2
 * and reserved[0] holds flags.
 *   POP_FLAG_F64       c_init, xs and ym are stored as float64
 *   POP_FLAG_SHARED_Y  ym holds one row [N] that every expression fits (the
 *                      GP case, where the reference tiles one target M
 *                      times, cusr/demonstrator/kernel_bridge.py:202)
 * The library honours POP_FLAG_SHARED_Y in every entry point that takes ym
 * (ym then points at N values); the array precision of an entry point is set
 * by the entry point itself (co_optimize fp32, co_optimize_ex fp64). */
#define POP_VERSION_2 2
#define POP_FLAG_F64 1
#define POP_FLAG_SHARED_Y 2

typedef struct PopHeader {
    int32_t magic;       /* POP_MAGIC */
    int32_t version;     /* POP_VERSION */
    int32_t M_prob;      /* number of expressions */
    int32_t total_nodes; /* sum of n_nodes */
    int32_t total_c;     /* sum of K */
    int32_t N;           /* data points */
    int32_t n_vars;      /* input variables D */
    int32_t K_max;       /* max K over expressions */
    int32_t max_stack;   /* max value-stack depth over expressions */
    int32_t reserved[7];
} PopHeader;

typedef struct TreeMeta {
    int32_t node_offset;
    int32_t n_nodes;
    int32_t c_offset;
    int32_t K;
} TreeMeta;

/* Flags of a header: reserved[0] of a v2 header; a v1 header has none. */
static inline int32_t pop_flags(const PopHeader *h) {
    return h->version == POP_VERSION_2 ? h->reserved[0] : 0;
}

#ifdef __cplusplus
static_assert(sizeof(PopHeader) == 64, "PopHeader must be 64 bytes");
static_assert(sizeof(TreeMeta) == 16, "TreeMeta must be 16 bytes");
#endif

/* Node types (cusr/kernel/ad_interp.cuh:21). Ternary nodes are rejected. */
enum {
    NODE_VAR = 0,
    NODE_CONST = 1,
    NODE_UFUNC = 2,
    NODE_BFUNC = 3,
    NODE_TFUNC = 4
};

/* Function ids. 1..28 follow the EvoGP numbering used by the reference
 * (cusr/kernel/ad_interp.cuh:24-31, cusr/benchmark/interp.py:18-29); the
 * LOOSE_* forms take the numpy-oracle meaning (interp.py:32-49).
 * 32..35 are the protected/clamped operators of the benchmark op set; they
 * have no counterpart in the reference and are defined here:
 *   OP_PDIV   l/r, or 1 when |r| < 1e-9 (both partials 0 on that branch)
 *   OP_CEXP   exp(min(a, 20)); derivative exp(a) for a <= 20, else 0
 *   OP_SQUARE a*a; derivative a+a
 *   OP_PLOG   log(|a| + 1e-9); derivative sign(a)/(|a| + 1e-9), sign(0) = 0
 * OP_LOOSE_SQRT is sqrt(|a|) with derivative sign(a)/(2 sqrt|a|), 0 at a = 0.
 * Any other id is rejected when a population is decoded. */
enum {
    OP_ADD = 1, OP_SUB = 2, OP_MUL = 3, OP_DIV = 4, OP_LOOSE_DIV = 5,
    OP_POW = 6, OP_LOOSE_POW = 7, OP_MAX = 8, OP_MIN = 9,
    OP_LT = 10, OP_GT = 11, OP_LE = 12, OP_GE = 13,
    OP_SIN = 14, OP_COS = 15, OP_TAN = 16,
    OP_SINH = 17, OP_COSH = 18, OP_TANH = 19,
    OP_LOG = 20, OP_LOOSE_LOG = 21, OP_EXP = 22,
    OP_INV = 23, OP_LOOSE_INV = 24, OP_NEG = 25, OP_ABS = 26,
    OP_SQRT = 27, OP_LOOSE_SQRT = 28,
    OP_PDIV = 32, OP_CEXP = 33, OP_SQUARE = 34, OP_PLOG = 35
};

/* Per-expression status codes (cusr/kernel/lm_core.cuh:46-56). */
enum {
    STATUS_CONVERGED = 0,
    STATUS_MAXITER = 1,
    STATUS_FAIL_NAN = 2,
    STATUS_K0_SKIP = 3,
    STATUS_FAIL_CHOLESKY = 4
};

#endif /* CUSR_POP_FORMAT_H */
