// program.cpp -- population checks and decode into device programs.
//
// Check order follows co_optimize (cusr/kernel/co_lib.cu:208-220): device
// bounds on the header, then the sum checks of cusr/kernel/loader.c:58-68,
// then per-expression validation, all before any device memory is touched.
// The per-expression checks go further than the reference, which trusts its
// input: every node type, operator id, variable index, constant rank and stack
// move is validated, so the device interpreter never indexes out of bounds.
#include <string.h>

#include <vector>

#include "program.h"

namespace cusr {

static bool unary_op(int f) {
    switch (f) {
    case OP_SIN: case OP_COS: case OP_TAN: case OP_SINH: case OP_COSH: case OP_TANH:
    case OP_LOG: case OP_LOOSE_LOG: case OP_EXP: case OP_INV: case OP_LOOSE_INV:
    case OP_NEG: case OP_ABS: case OP_SQRT: case OP_LOOSE_SQRT:
    case OP_CEXP: case OP_SQUARE: case OP_PLOG:
        return true;
    default:
        return false;
    }
}

static bool binary_op(int f) {
    switch (f) {
    case OP_ADD: case OP_SUB: case OP_MUL: case OP_DIV: case OP_LOOSE_DIV:
    case OP_POW: case OP_LOOSE_POW: case OP_MAX: case OP_MIN:
    case OP_LT: case OP_GT: case OP_LE: case OP_GE: case OP_PDIV:
        return true;
    default:
        return false;
    }
}

// Integral node value in [0, limit) or -1.
static int node_int(float v, int limit) {
    if (!(v >= 0.0f) || v >= (float)limit) return -1;
    int i = (int)v;
    return ((float)i == v) ? i : -1;
}

struct TreeScratch {
    std::vector<int> size, left, cc, stk;
};

// Decode one expression (n nodes at nt/nv/ci) into out[0..n) in execution
// order. Returns CO_OK, CO_ERR_BOUNDS or CO_ERR_PROGRAM.
static int decode_tree(const int32_t *nt, const float *nv, const int32_t *ci, int n, int K,
                       int D, uint64_t *out, int *stack_depth, int *tape_slots,
                       TreeScratch &s) {
    if (n <= 0) return CO_ERR_PROGRAM;
    if (n > CO_MAX_NODES) return CO_ERR_BOUNDS;
    s.size.assign(n, 0);
    s.left.assign(n, 0);
    s.cc.assign(n + 1, 0);
    s.stk.clear();
    // prefix pass: constant ranks must be 0..K-1 in prefix order
    for (int i = 0; i < n; i++) {
        s.cc[i + 1] = s.cc[i] + (nt[i] == NODE_CONST ? 1 : 0);
        if (nt[i] == NODE_CONST && ci[i] != s.cc[i]) return CO_ERR_PROGRAM;
    }
    if (s.cc[n] != K) return CO_ERR_PROGRAM;
    // execution pass (last node first): stack simulation and subtree sizes
    int depth = 0;
    for (int i = n - 1; i >= 0; i--) {
        int t = nt[i];
        if (t == NODE_VAR) {
            if (node_int(nv[i], D) < 0) return CO_ERR_PROGRAM;
            s.stk.push_back(1);
            s.size[i] = 1;
        } else if (t == NODE_CONST) {
            s.stk.push_back(1);
            s.size[i] = 1;
        } else if (t == NODE_UFUNC) {
            if (!unary_op(node_int(nv[i], 64))) return CO_ERR_PROGRAM;
            if (s.stk.empty()) return CO_ERR_PROGRAM;
            s.size[i] = s.stk.back() + 1;
            s.stk.back() = s.size[i];
        } else if (t == NODE_BFUNC) {
            if (!binary_op(node_int(nv[i], 64))) return CO_ERR_PROGRAM;
            if (s.stk.size() < 2) return CO_ERR_PROGRAM;
            int sl = s.stk.back();   // left operand = top of stack
            s.stk.pop_back();
            int sr = s.stk.back();
            s.left[i] = sl;
            s.size[i] = sl + sr + 1;
            s.stk.back() = s.size[i];
        } else {
            return CO_ERR_PROGRAM;
        }
        if ((int)s.stk.size() > depth) depth = (int)s.stk.size();
    }
    if (s.stk.size() != 1) return CO_ERR_PROGRAM;
    if (depth > CO_MAX_STACK) return CO_ERR_BOUNDS;
    // second execution pass: emit instructions with stack depth and tape slots
    int sp = 0, tape = 0;
    for (int i = n - 1, pc = 0; i >= 0; i--, pc++) {
        int t = nt[i];
        uint64_t w = (uint64_t)(t & 3) << 8;
        w |= (uint64_t)sp << 24;
        if (t == NODE_VAR) {
            w |= (uint64_t)node_int(nv[i], D) << 16;
            sp++;
        } else if (t == NODE_CONST) {
            w |= (uint64_t)ci[i] << 16;
            sp++;
        } else {
            int f = (int)nv[i];
            int lo = s.cc[i + 1];
            int hi = s.cc[i + s.size[i]];
            int mid = (t == NODE_BFUNC) ? s.cc[i + 1 + s.left[i]] : hi;
            w |= (uint64_t)f;
            w |= (uint64_t)lo << 32 | (uint64_t)mid << 37 | (uint64_t)hi << 42;
            w |= (uint64_t)tape << 47;
            tape += (t == NODE_BFUNC) ? 2 : 1;
            if (t == NODE_BFUNC) sp--;
        }
        out[pc] = w;
    }
    if (tape > 255) return CO_ERR_BOUNDS;
    // reverse sweep (prefix order): adjoint source and adjoint-stack depth
    int asp = 0;
    for (int i = 0; i < n; i++) {
        uint64_t &w = out[n - 1 - i];
        int apop = (i > 0 && (nt[i - 1] == NODE_VAR || nt[i - 1] == NODE_CONST)) ? 1 : 0;
        if (apop && asp == 0) return CO_ERR_PROGRAM;
        w |= (uint64_t)asp << 55 | (uint64_t)apop << 61;
        asp -= apop;
        if (nt[i] == NODE_BFUNC) asp++;
        if (asp > CO_MAX_STACK) return CO_ERR_BOUNDS;
    }
    if (asp != 0) return CO_ERR_PROGRAM;
    *stack_depth = depth;
    *tape_slots = tape;
    return CO_OK;
}

int decode_population(const PopHeader *h, const int32_t *nt, const float *nv,
                      const int32_t *ci, const TreeMeta *metas, uint64_t *prog,
                      int32_t *order, int32_t *bin_start, ExprDesc *descs,
                      int32_t *stack, Plan *plan) {
    if (!h || !metas) return CO_ERR_NULLARG;
    if (h->total_nodes > 0 && (!nt || !nv || !ci)) return CO_ERR_NULLARG;
    if (h->M_prob < 0 || h->N < 0 || h->n_vars < 0 || h->total_nodes < 0 || h->total_c < 0)
        return CO_ERR_NULLARG;
    if (h->K_max > CO_MAX_K || h->max_stack > CO_MAX_STACK || h->n_vars > CO_MAX_VARS)
        return CO_ERR_BOUNDS;
    int M = h->M_prob;
    long ksum = 0, nsum = 0;
    for (int m = 0; m < M; m++) { ksum += metas[m].K; nsum += metas[m].n_nodes; }
    if (ksum != (long)h->total_c) return CO_ERR_SUM_C;
    if (nsum != (long)h->total_nodes) return CO_ERR_SUM_NODES;

    TreeScratch s;
    int max_tape = 0, max_n = 0;
    std::vector<int> count(CO_MAX_K + 1, 0);
    std::vector<int32_t> depth(M), tapes(M), poff(M);
    // programs are laid out expression after expression (prefix sum of
    // n_nodes), which equals node_offset for well-formed populations and
    // keeps overlapping metas from aliasing each other's instructions
    int64_t run = 0;
    for (int m = 0; m < M; m++) {
        const TreeMeta &t = metas[m];
        if (t.K < 0 || t.n_nodes < 0 || t.node_offset < 0 || t.c_offset < 0 ||
            (long)t.node_offset + t.n_nodes > (long)h->total_nodes ||
            (long)t.c_offset + t.K > (long)h->total_c)
            return CO_ERR_PROGRAM;
        if (t.K > CO_MAX_K) return CO_ERR_BOUNDS;
        poff[m] = (int32_t)run;
        int rc = decode_tree(nt + t.node_offset, nv + t.node_offset, ci + t.node_offset,
                             t.n_nodes, t.K, h->n_vars, prog + run, &depth[m],
                             &tapes[m], s);
        if (rc != CO_OK) return rc;
        run += t.n_nodes;
        if (tapes[m] > max_tape) max_tape = tapes[m];
        if (t.n_nodes > max_n) max_n = t.n_nodes;
        count[t.K]++;
    }
    // stable K bins, ascending
    std::vector<int32_t> start(CO_MAX_K + 2, 0);
    for (int k = 0; k <= CO_MAX_K; k++) start[k + 1] = start[k] + count[k];
    std::vector<int32_t> fill(start.begin(), start.end() - 1);
    std::vector<int32_t> ord(M);
    for (int m = 0; m < M; m++) ord[fill[metas[m].K]++] = m;
    if (order) memcpy(order, ord.data(), sizeof(int32_t) * M);
    if (bin_start) memcpy(bin_start, start.data(), sizeof(int32_t) * (CO_MAX_K + 2));
    if (stack) memcpy(stack, depth.data(), sizeof(int32_t) * M);
    if (descs) {
        // launch position p runs expression ord[M-1-p]: largest K first, so the
        // longest-running workgroups start earliest
        for (int p = 0; p < M; p++) {
            int m = ord[M - 1 - p];
            ExprDesc &d = descs[p];
            d.prog_off = poff[m];
            d.n = metas[m].n_nodes;
            d.c_off = metas[m].c_offset;
            d.K = metas[m].K;
            d.y_row = m;
            d.tape = tapes[m];
            d.stack = depth[m];
            d.pad = 0;
        }
    }
    if (plan) {
        plan->M = M;
        plan->N = h->N;
        plan->D = h->n_vars;
        plan->total_nodes = h->total_nodes;
        plan->total_c = h->total_c;
        plan->max_tape = max_tape;
        plan->max_n = max_n;
    }
    return CO_OK;
}

}  // namespace cusr
