// program.cpp -- population checks and decode into device programs.
//
// Check order follows co_optimize (cusr/kernel/co_lib.cu:208-220): device
// bounds on the header, then the sum checks of cusr/kernel/loader.c:58-68,
// then per-expression validation, all before any device memory is touched.
// The per-expression checks go further than the reference, which trusts its
// input: every node type, operator id, variable index, constant rank and stack
// move is validated, so the device interpreter never indexes out of bounds.
#include <string.h>

#include <algorithm>
#include <functional>
#include <thread>
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

// Relative device cost of one instruction per interpreter pass (VALU
// instructions per 64 lanes x 4 points, measured with SQ_INSTS_VALU on
// single-operator expressions); only the launch order within a K bin uses it.
static int op_cost(int f) {
    switch (f) {
    case OP_ADD: case OP_SUB: return 12;
    case OP_MUL: return 23;
    case OP_SQUARE: return 83;
    case OP_DIV: case OP_LOOSE_DIV: case OP_PDIV: case OP_SQRT: case OP_LOOSE_SQRT: return 224;
    case OP_EXP: case OP_CEXP: return 284;
    case OP_SIN: case OP_COS: return 333;
    case OP_LOG: case OP_LOOSE_LOG: case OP_PLOG: return 391;
    case OP_TAN: case OP_POW: case OP_LOOSE_POW: return 450;
    default: return 100;
    }
}

// Forward-AD and reverse-AD flags of an instruction: flat-branch select
// rule, which of its rank ranges get scaled (ADD's partials and SUB's left
// one are exactly 1; the identity has no partial to apply), and which partials
// keep a reverse-AD tape slot (read, and not exactly +-1).
struct Ins {
    int fid, bin, ak, ai, bk, bi, toslot, di, lo, mid, hi, tape;
    bool sel, sa, sb, ta, tb;
};

static void set_flags(Ins &w) {
    const int f = w.fid;
    w.sel = f == OP_MAX || f == OP_MIN || f == OP_LT || f == OP_GT || f == OP_LE || f == OP_GE ||
            f == OP_PDIV || f == OP_CEXP;
    const bool unit_a = w.bin ? (f == OP_ADD || f == OP_SUB) : (f == OP_IDENT);
    const bool unit_b = !w.bin || f == OP_ADD;
    w.sa = !unit_a && w.mid > w.lo;
    w.sb = !unit_b && w.hi > w.mid;
}

// program.h bit layouts
static uint64_t encode_fast(const Ins &w) {
    uint64_t x = (uint64_t)w.fid | (uint64_t)w.bin << 6;
    x |= (uint64_t)w.ak << 7 | (uint64_t)(w.ai & 15) << 9;
    x |= (uint64_t)w.bk << 13 | (uint64_t)(w.bi & 15) << 15;
    x |= (uint64_t)w.toslot << 19 | (uint64_t)(w.di & 15) << 20;
    x |= (uint64_t)w.lo << 24 | (uint64_t)w.mid << 29 | (uint64_t)w.hi << 34;
    x |= (uint64_t)w.tape << 39;
    x |= (uint64_t)w.sel << 47 | (uint64_t)w.sa << 48 | (uint64_t)w.sb << 49;
    x |= (uint64_t)w.ta << 50 | (uint64_t)w.tb << 51;
    return x;
}

static void encode_wide(const Ins &w, uint64_t *out) {
    uint64_t a = (uint64_t)w.fid | (uint64_t)w.bin << 6;
    a |= (uint64_t)w.ak << 7 | (uint64_t)(w.ai & 255) << 9;
    a |= (uint64_t)w.bk << 17 | (uint64_t)(w.bi & 255) << 19;
    a |= (uint64_t)w.toslot << 27 | (uint64_t)(w.di & 255) << 28;
    a |= (uint64_t)w.sel << 36 | (uint64_t)w.sa << 37 | (uint64_t)w.sb << 38;
    a |= (uint64_t)w.ta << 39 | (uint64_t)w.tb << 40;
    uint64_t b = (uint64_t)w.lo | (uint64_t)w.mid << 8 | (uint64_t)w.hi << 16;
    b |= (uint64_t)(uint32_t)w.tape << 24;
    out[0] = a;
    out[1] = b;
}

// Integral node value in [0, limit) or -1.
static int node_int(float v, int limit) {
    if (!(v >= 0.0f) || v >= (float)limit) return -1;
    int i = (int)v;
    return ((float)i == v) ? i : -1;
}

struct Operand {
    int kind;      // OPD_*
    int idx;       // var / const rank / slot
    int producer;  // instruction that produced an ACC value, else -1
};

struct Visit {
    int node;   // subtree root (prefix index)
    int stage;  // 0: nothing evaluated, 1: first operand done, 2: both done
};

struct TreeScratch {
    std::vector<int> size, left, cc, need;
    std::vector<int> depth_stack;
    std::vector<Operand> res;
    std::vector<Visit> work;
    std::vector<Ins> ins;
};

// Validate one expression (n nodes, K constants, D variables): node types,
// operator ids, variable indices, prefix-order constant ranks and stack moves.
// Returns CO_OK, CO_ERR_BOUNDS (value stack beyond CO_MAX_STACK) or
// CO_ERR_PROGRAM, and its value-stack depth. Fills s.size / s.left / s.cc for
// the emission.
static int check_tree(const int32_t *nt, const float *nv, const int32_t *ci, int n, int K,
                      int D, int *stack_depth, TreeScratch &s) {
    if (n <= 0) return CO_ERR_PROGRAM;
    s.size.assign(n, 0);
    s.left.assign(n, 0);
    s.cc.assign(n + 1, 0);
    // prefix pass: constant ranks must be 0..K-1 in prefix order
    for (int i = 0; i < n; i++) {
        s.cc[i + 1] = s.cc[i] + (nt[i] == NODE_CONST ? 1 : 0);
        if (nt[i] == NODE_CONST && ci[i] != s.cc[i]) return CO_ERR_PROGRAM;
    }
    if (s.cc[n] != K) return CO_ERR_PROGRAM;
    // execution pass (last node first): validation, stack depth, subtree sizes
    s.depth_stack.clear();
    int depth = 0;
    for (int i = n - 1; i >= 0; i--) {
        const int t = nt[i];
        if (t == NODE_VAR) {
            if (node_int(nv[i], D) < 0) return CO_ERR_PROGRAM;
            s.depth_stack.push_back(1);
            s.size[i] = 1;
        } else if (t == NODE_CONST) {
            s.depth_stack.push_back(1);
            s.size[i] = 1;
        } else if (t == NODE_UFUNC) {
            if (!unary_op(node_int(nv[i], 64))) return CO_ERR_PROGRAM;
            if (s.depth_stack.empty()) return CO_ERR_PROGRAM;
            s.size[i] = s.depth_stack.back() + 1;
            s.depth_stack.back() = s.size[i];
        } else if (t == NODE_BFUNC) {
            if (!binary_op(node_int(nv[i], 64))) return CO_ERR_PROGRAM;
            if (s.depth_stack.size() < 2) return CO_ERR_PROGRAM;
            const int sl = s.depth_stack.back();  // left operand = top of stack
            s.depth_stack.pop_back();
            const int sr = s.depth_stack.back();
            s.left[i] = sl;
            s.size[i] = sl + sr + 1;
            s.depth_stack.back() = s.size[i];
        } else {
            return CO_ERR_PROGRAM;
        }
        if ((int)s.depth_stack.size() > depth) depth = (int)s.depth_stack.size();
    }
    if (s.depth_stack.size() != 1) return CO_ERR_PROGRAM;
    *stack_depth = depth;
    if (depth > CO_MAX_STACK) return CO_ERR_BOUNDS;
    return CO_OK;
}

// Emit the instructions of a checked expression into s.ins in execution
// order. max_slots: slots the target format can address. Returns CO_OK,
// CO_ERR_BOUNDS or CO_ERR_PROGRAM; sets the tape and spill-slot counts.
//
// Operands are evaluated in Sethi-Ullman order: when both operands of a binary
// operator need instructions, the one whose subtree needs more spill slots runs
// first (the right one on a tie, as the reference's last-node-first order
// does) and its value waits in a slot while the other runs. A subtree's value
// and its constants' tangents and adjoints do not depend on which sibling runs
// first, and the order keeps the slot count at the minimum (at most
// log2(nodes + 1)), which is what sizes each wavefront's LDS.
static int emit_tree(const int32_t *nt, const float *nv, const int32_t *ci, int n, int D,
                     int max_slots_fmt, int *tape_slots, int *slots_used, TreeScratch &s) {
    s.ins.clear();
    auto leaf = [&](int i) { return nt[i] == NODE_VAR || nt[i] == NODE_CONST; };
    // need[i]: spill slots the subtree at node i needs in this order (children
    // follow their parent in prefix order, so a descending pass sees them first)
    s.need.assign(n, 0);
    for (int i = n - 1; i >= 0; i--) {
        if (nt[i] == NODE_UFUNC) {
            s.need[i] = s.need[i + 1];
        } else if (nt[i] == NODE_BFUNC) {
            const int l = i + 1, r = i + 1 + s.left[i];
            const int nl = s.need[l], nr = s.need[r];
            const int hi = nl > nr ? nl : nr;
            s.need[i] = (!leaf(l) && !leaf(r) && nl == nr) ? nl + 1 : hi;
        }
    }
    s.res.assign(n, Operand{OPD_ACC, 0, -1});
    s.work.clear();
    s.work.push_back({0, 0});
    int tape = 0, live_slots = 0, max_slots = 0;
    while (!s.work.empty()) {
        const int i = s.work.back().node, stage = s.work.back().stage;
        const int t = nt[i];
        if (t == NODE_VAR || t == NODE_CONST) {
            s.res[i] = t == NODE_VAR ? Operand{OPD_VAR, node_int(nv[i], D), -1}
                                     : Operand{OPD_CONST, ci[i], -1};
            s.work.pop_back();
            continue;
        }
        const bool bin = (t == NODE_BFUNC);
        const int l = i + 1, r = bin ? i + 1 + s.left[i] : -1;
        const bool both = bin && !leaf(l) && !leaf(r);
        const int first = (!bin || (both && s.need[l] > s.need[r])) ? l : r;
        const int second = !bin ? -1 : (first == l ? r : l);
        if (stage == 0) {
            s.work.back().stage = 1;
            s.work.push_back({first, 0});
            continue;
        }
        if (stage == 1 && bin) {
            s.work.back().stage = 2;
            if (both) {
                // the first operand's value waits in the next free slot
                if (live_slots >= max_slots_fmt) return CO_ERR_BOUNDS;
                const int slot = live_slots++;
                if (live_slots > max_slots) max_slots = live_slots;
                Operand &o = s.res[first];
                if (o.kind != OPD_ACC || o.producer < 0) return CO_ERR_PROGRAM;
                s.ins[o.producer].toslot = 1;
                s.ins[o.producer].di = slot;
                o = {OPD_SLOT, slot, -1};
            }
            s.work.push_back({second, 0});
            continue;
        }
        s.work.pop_back();
        const Operand a = s.res[l];
        const Operand b = bin ? s.res[r] : Operand{OPD_ACC, 0, -1};
        // spill slots are used last in, first out
        if (a.kind == OPD_SLOT) {
            if (a.idx != live_slots - 1) return CO_ERR_PROGRAM;
            live_slots--;
        }
        if (bin && b.kind == OPD_SLOT) {
            if (b.idx != live_slots - 1) return CO_ERR_PROGRAM;
            live_slots--;
        }
        Ins w = {};
        w.fid = (int)nv[i];
        w.bin = bin ? 1 : 0;
        w.ak = a.kind;
        w.ai = a.idx;
        if (bin) {
            w.bk = b.kind;
            w.bi = b.idx;
        }
        w.lo = s.cc[i + 1];
        w.hi = s.cc[i + s.size[i]];
        w.mid = bin ? s.cc[i + 1 + s.left[i]] : w.hi;
        w.tape = tape;
        set_flags(w);
        // reverse-AD tape slots only for partials that are read and not exactly +-1
        const bool unit = bin && (w.fid == OP_ADD || w.fid == OP_SUB);
        w.ta = a.kind != OPD_VAR && !unit;
        w.tb = bin && b.kind != OPD_VAR && !unit;
        tape += (w.ta ? 1 : 0) + (w.tb ? 1 : 0);
        s.res[i] = {OPD_ACC, 0, (int)s.ins.size()};
        s.ins.push_back(w);
    }
    if (s.ins.empty()) {
        // the expression is one leaf: its value is the identity of that leaf
        const Operand a = s.res[0];
        Ins w = {};
        w.fid = OP_IDENT;
        w.ak = a.kind;
        w.ai = a.idx;
        w.lo = s.cc[0];
        w.mid = w.hi = s.cc[n];
        w.tape = tape;     // the identity's partial is +1: no tape slot
        set_flags(w);
        s.ins.push_back(w);
    }
    if (live_slots != 0) return CO_ERR_PROGRAM;
    *tape_slots = tape;
    *slots_used = max_slots;
    return CO_OK;
}

// Runs fn(m0, m1) over contiguous chunks of [0, M) on up to nthreads host
// threads (fewer threads than chunks when the system refuses more: the chunks
// already started finish, then fn runs over everything on this thread).
template <typename Fn, typename Redo>
static void chunked(int M, int nthreads, const Fn &fn, const Redo &redo) {
    bool done = false;
    if (nthreads > 1) {
        std::vector<std::thread> pool;
        const int chunk = (M + nthreads - 1) / nthreads;
        try {
            // chunks 1.. on new threads, chunk 0 on this one
            for (int i = 1; i < nthreads; i++) {
                const int m0 = i * chunk, m1 = std::min(M, m0 + chunk);
                if (m0 < m1) pool.emplace_back(std::cref(fn), m0, m1);
            }
            done = true;
        } catch (...) {
            // no more threads
        }
        if (done) fn(0, std::min(M, chunk));
        for (std::thread &th : pool) th.join();
    }
    if (!done) redo(0, M);
}

int decode_population(const PopHeader *h, const int32_t *nt, const float *nv,
                      const int32_t *ci, const TreeMeta *metas, uint64_t *prog,
                      int32_t *order, int32_t *bin_start, ExprDesc *descs,
                      int32_t *stack, int32_t *n_ins, int32_t *prog_off, int32_t *route,
                      Plan *plan) {
    if (!h || !metas) return CO_ERR_NULLARG;
    if (h->total_nodes > 0 && (!nt || !nv || !ci)) return CO_ERR_NULLARG;
    if (h->M_prob < 0 || h->N < 0 || h->n_vars < 0 || h->total_nodes < 0 || h->total_c < 0)
        return CO_ERR_NULLARG;
    if (h->K_max > CO_MAX_K || h->max_stack > CO_MAX_STACK || h->n_vars > CO_MAX_VARS)
        return CO_ERR_BOUNDS;
    const int M = h->M_prob, D = h->n_vars;
    long ksum = 0, nsum = 0;
    for (int m = 0; m < M; m++) { ksum += metas[m].K; nsum += metas[m].n_nodes; }
    if (ksum != (long)h->total_c) return CO_ERR_SUM_C;
    if (nsum != (long)h->total_nodes) return CO_ERR_SUM_NODES;

    std::vector<uint64_t> tmp;
    if (!prog) {
        tmp.assign(h->total_nodes > 0 ? 2 * (size_t)h->total_nodes : 1, 0);
        prog = tmp.data();
    }
    for (int m = 0; m < M; m++) {
        const TreeMeta &t = metas[m];
        if (t.K < 0 || t.n_nodes < 0 || t.node_offset < 0 || t.c_offset < 0 ||
            (long)t.node_offset + t.n_nodes > (long)h->total_nodes ||
            (long)t.c_offset + t.K > (long)h->total_c)
            return CO_ERR_PROGRAM;
        if (t.K > CO_MAX_K) return CO_ERR_BOUNDS;
    }
    std::vector<int32_t> depth(M, 0), tapes(M, 0), poff(M), nins(M, 0), slots(M, 0);
    std::vector<int32_t> rcs(M, CO_OK), gen(M, 0);
    std::vector<int64_t> cost(descs ? M : 0);
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const int nthreads = (int)std::min<int64_t>(std::min(16u, hw), nsum / 65536 + 1);
    // phase 1: every expression's stack depth and so its kernel, by a count
    // over the node types (the depth check_tree finds for a valid tree); the
    // full check runs in phase 2, which still ends before anything is used
    auto depth_range = [&](int m0, int m1) {
        for (int m = m0; m < m1; m++) {
            const TreeMeta &t = metas[m];
            const int32_t *tnt = nt + t.node_offset;
            int sp = 0, dmax = 0;
            for (int i = t.n_nodes - 1; i >= 0; i--) {
                if (tnt[i] == NODE_BFUNC) sp -= 1;          // two operands in, one out
                else if (tnt[i] != NODE_UFUNC) sp += 1;     // a leaf
                if (sp > dmax) dmax = sp;
            }
            depth[m] = dmax;
            gen[m] = co_fast_path(t.K, depth[m], t.n_nodes, D) ? 0 : 1;
        }
    };
    chunked(M, nthreads, depth_range, depth_range);
    // programs are laid out expression after expression: n_nodes words in the
    // fast format, 2 * n_nodes in the wide one (node_offset order would let
    // overlapping metas alias each other's instructions)
    int64_t run = 0;
    int n_gen = 0;
    for (int m = 0; m < M; m++) {
        poff[m] = (int32_t)run;
        run += (int64_t)metas[m].n_nodes * (gen[m] ? 2 : 1);
        n_gen += gen[m];
    }
    // phase 2: emit and encode (expressions decode independently; C5's 1.7 M
    // nodes take 32 ms on one thread)
    auto emit_range = [&](int m0, int m1) {
        TreeScratch s;
        for (int m = m0; m < m1; m++) {
            const TreeMeta &t = metas[m];
            const int32_t *tnt = nt + t.node_offset;
            const float *tnv = nv + t.node_offset;
            const int32_t *tci = ci + t.node_offset;
            uint64_t *out = prog + poff[m];
            const int words = t.n_nodes * (gen[m] ? 2 : 1);
            if (words > 0) memset(out, 0, sizeof(uint64_t) * words);
            int dd = 0;
            rcs[m] = check_tree(tnt, tnv, tci, t.n_nodes, t.K, D, &dd, s);
            if (rcs[m] == CO_OK && dd != depth[m]) rcs[m] = CO_ERR_PROGRAM;   // never, for a valid tree
            if (rcs[m] == CO_OK)
                rcs[m] = emit_tree(tnt, tnv, tci, t.n_nodes, D, gen[m] ? kMaxSlotsWide : kMaxSlots,
                                   &tapes[m], &slots[m], s);
            if (rcs[m] != CO_OK) return;
            nins[m] = (int32_t)s.ins.size();
            if (!gen[m] && tapes[m] > 255) {   // 8-bit tape field (n <= 255 keeps it below)
                rcs[m] = CO_ERR_BOUNDS;
                return;
            }
            int64_t c = 229;
            for (int i = 0; i < nins[m]; i++) {
                if (gen[m]) encode_wide(s.ins[i], out + 2 * i);
                else out[i] = encode_fast(s.ins[i]);
                c += op_cost(s.ins[i].fid);
            }
            if (descs) cost[m] = c;
        }
    };
    auto emit_all = [&](int m0, int m1) {
        std::fill(rcs.begin(), rcs.end(), CO_OK);
        emit_range(m0, m1);
    };
    chunked(M, nthreads, emit_range, emit_all);
    int max_tape = 0, max_n = 0, max_slots = 0;
    std::vector<int> count(CO_MAX_K + 1, 0);
    for (int m = 0; m < M; m++) {
        if (rcs[m] != CO_OK) return rcs[m];
        if (tapes[m] > max_tape) max_tape = tapes[m];
        if (nins[m] > max_n) max_n = nins[m];
        if (slots[m] > max_slots) max_slots = slots[m];
        count[metas[m].K]++;
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
    if (n_ins) memcpy(n_ins, nins.data(), sizeof(int32_t) * M);
    if (prog_off) memcpy(prog_off, poff.data(), sizeof(int32_t) * M);
    if (route) memcpy(route, gen.data(), sizeof(int32_t) * M);
    if (descs) {
        // launch positions: the general kernel's bin first, then the fast K
        // bins, largest K first; within a bin by K descending (the general
        // bin) and the costliest programs first (fixed per-pass cost plus
        // op_cost of each instruction), so the longest-running workgroups
        // start earliest and a bin ends on cheap ones. Three stable counting
        // sorts over reversed ord: by cost descending (clamped to
        // kCostBuckets), by K descending, by kernel (general first); ties keep
        // the order of ord reversed
        constexpr int kCostBuckets = 1 << 15;
        std::vector<int32_t> a(M), launch(M);
        for (int p = 0; p < M; p++) a[p] = ord[M - 1 - p];
        std::vector<int32_t> next(kCostBuckets + 1, 0);
        auto bucket = [&](int32_t m) {
            const int64_t c = cost[m] < kCostBuckets - 1 ? cost[m] : kCostBuckets - 1;
            return (int)(kCostBuckets - 1 - c);
        };
        for (int p = 0; p < M; p++) next[bucket(a[p]) + 1]++;
        for (int i = 0; i < kCostBuckets; i++) next[i + 1] += next[i];
        for (int p = 0; p < M; p++) launch[next[bucket(a[p])]++] = a[p];
        std::vector<int32_t> knext(CO_MAX_K + 2, 0);
        for (int p = 0; p < M; p++) knext[CO_MAX_K - metas[launch[p]].K + 1]++;
        for (int i = 0; i <= CO_MAX_K; i++) knext[i + 1] += knext[i];
        for (int p = 0; p < M; p++) a[knext[CO_MAX_K - metas[launch[p]].K]++] = launch[p];
        int gpos = 0, fpos = n_gen;
        for (int p = 0; p < M; p++) launch[gen[a[p]] ? gpos++ : fpos++] = a[p];
        for (int p = 0; p < M; p++) {
            const int m = launch[p];
            ExprDesc &d = descs[p];
            d.prog_off = poff[m];
            d.n = nins[m];
            d.c_off = metas[m].c_offset;
            d.K = metas[m].K;
            d.y_row = m;
            d.tape = tapes[m];
            d.slots = slots[m];
            d.gen = gen[m];
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
        plan->max_slots = max_slots;
        plan->words = run;
        plan->n_gen = n_gen;
    }
    return CO_OK;
}

}  // namespace cusr
