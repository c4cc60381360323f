// program.cpp -- population checks and decode into device programs.
//
// Check order follows co_optimize (cusr/kernel/co_lib.cu:208-220): device
// bounds on the header, then the sum checks of cusr/kernel/loader.c:58-68,
// then per-expression validation, all before any device memory is touched.
// The per-expression checks go further than the reference, which trusts its
// input: every node type, operator id, variable index, constant rank and stack
// move is validated, so the device interpreter never indexes out of bounds.
#include <string.h>

#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <functional>
#include <mutex>
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

// Per-thread working arrays, grown to the largest expression seen and not
// cleared between expressions (every entry read is written first).
struct TreeScratch {
    std::vector<int> size, left, cc, need, depth_stack;
    std::vector<Operand> res;
    std::vector<Visit> work;
    void reserve(int n) {
        if ((int)size.size() >= n + 1) return;
        size.resize(n + 1);
        left.resize(n + 1);
        cc.resize(n + 1);
        need.resize(n + 1);
        depth_stack.resize(n + 1);
        res.resize(n + 1);
        work.resize(n + 1);
    }
};

static inline bool is_leaf(int t) { return t == NODE_VAR || t == NODE_CONST; }

// Validate one expression (n nodes, K constants, D variables): node types,
// operator ids, variable indices, prefix-order constant ranks and stack moves.
// Returns CO_OK, CO_ERR_BOUNDS (value stack beyond CO_MAX_STACK) or
// CO_ERR_PROGRAM, and its value-stack depth. Fills s.size / s.left / s.cc and
// s.need (the spill slots of each subtree in the emission's order) for the
// emission.
static int check_tree(const int32_t *nt, const float *nv, const int32_t *ci, int n, int K,
                      int D, int *stack_depth, TreeScratch &s) {
    if (n <= 0) return CO_ERR_PROGRAM;
    s.reserve(n);
    int *size = s.size.data(), *left = s.left.data(), *cc = s.cc.data(), *need = s.need.data();
    int *st = s.depth_stack.data();
    // prefix pass: constant ranks must be 0..K-1 in prefix order
    cc[0] = 0;
    for (int i = 0; i < n; i++) {
        const int c = nt[i] == NODE_CONST;
        if (c && ci[i] != cc[i]) return CO_ERR_PROGRAM;
        cc[i + 1] = cc[i] + c;
    }
    if (cc[n] != K) return CO_ERR_PROGRAM;
    // execution pass (last node first): validation, stack depth, subtree sizes;
    // the stack holds subtree roots (a subtree's size is known when it is pushed)
    int sp = 0, depth = 0;
    for (int i = n - 1; i >= 0; i--) {
        const int t = nt[i];
        if (t == NODE_VAR || t == NODE_CONST) {
            if (t == NODE_VAR && node_int(nv[i], D) < 0) return CO_ERR_PROGRAM;
            size[i] = 1;
            need[i] = 0;
            st[sp++] = i;
        } else if (t == NODE_UFUNC) {
            if (!unary_op(node_int(nv[i], 64))) return CO_ERR_PROGRAM;
            if (sp < 1) return CO_ERR_PROGRAM;
            const int c = st[sp - 1];
            size[i] = size[c] + 1;
            need[i] = need[c];
            st[sp - 1] = i;
        } else if (t == NODE_BFUNC) {
            if (!binary_op(node_int(nv[i], 64))) return CO_ERR_PROGRAM;
            if (sp < 2) return CO_ERR_PROGRAM;
            const int l = st[sp - 1], r = st[sp - 2];   // left operand = top of stack
            --sp;
            left[i] = size[l];
            size[i] = size[l] + size[r] + 1;
            // the operand that needs more slots runs first; two that both need
            // instructions hold one value in a slot while the other runs
            const int nl = need[l], nr = need[r];
            const int hi = nl > nr ? nl : nr;
            need[i] = (!is_leaf(nt[l]) && !is_leaf(nt[r]) && nl == nr) ? nl + 1 : hi;
            st[sp - 1] = i;
        } else {
            return CO_ERR_PROGRAM;
        }
        if (sp > depth) depth = sp;
    }
    if (sp != 1) return CO_ERR_PROGRAM;
    *stack_depth = depth;
    if (depth > CO_MAX_STACK) return CO_ERR_BOUNDS;
    return CO_OK;
}

// An instruction's word(s) in out (fast: one word, wide: two), and the later
// mark that sends its result to slot di.
static inline void put_ins(uint64_t *out, bool wide, int k, Ins &w) {
    set_flags(w);
    if (wide) encode_wide(w, out + 2 * k);
    else out[k] = encode_fast(w);
}
static inline void put_spill(uint64_t *out, bool wide, int k, int di) {
    if (wide) out[2 * k] |= (uint64_t)1 << 27 | (uint64_t)(di & 255) << 28;
    else out[k] |= (uint64_t)1 << 19 | (uint64_t)(di & 15) << 20;
}

// Emit the instructions of a checked expression, encoded, into out in
// execution order (out holds zeros on entry). max_slots: slots the target
// format can address. Returns CO_OK, CO_ERR_BOUNDS or CO_ERR_PROGRAM; sets the
// instruction count, the tape and spill-slot counts and the cost estimate.
//
// Operands are evaluated in Sethi-Ullman order: when both operands of a binary
// operator need instructions, the one whose subtree needs more spill slots runs
// first (the right one on a tie, as the reference's last-node-first order
// does) and its value waits in a slot while the other runs. A subtree's value
// and its constants' tangents and adjoints do not depend on which sibling runs
// first, and the order keeps the slot count at the minimum (at most
// log2(nodes + 1)), which is what sizes each wavefront's LDS.
static int emit_tree(const int32_t *nt, const float *nv, const int32_t *ci, int n, int D,
                     bool wide, int max_slots_fmt, uint64_t *out, int *n_ins, int *tape_slots,
                     int *slots_used, int64_t *cost, TreeScratch &s) {
    const int *left = s.left.data(), *cc = s.cc.data(), *need = s.need.data(),
              *size = s.size.data();
    Operand *res = s.res.data();
    Visit *work = s.work.data();
    auto leaf_opd = [&](int i) -> Operand {
        return nt[i] == NODE_VAR ? Operand{OPD_VAR, node_int(nv[i], D), -1}
                                 : Operand{OPD_CONST, ci[i], -1};
    };
    int k = 0, tape = 0, live_slots = 0, max_slots = 0;
    int64_t c = 229;   // fixed per-pass cost, then op_cost of each instruction
    if (is_leaf(nt[0])) {
        // the expression is one leaf: its value is the identity of that leaf
        const Operand a = leaf_opd(0);
        Ins w = {};
        w.fid = OP_IDENT;
        w.ak = a.kind;
        w.ai = a.idx;
        w.lo = cc[0];
        w.mid = w.hi = cc[n];
        w.tape = tape;     // the identity's partial is +1: no tape slot
        put_ins(out, wide, k++, w);
        c += op_cost(OP_IDENT);
    } else {
        int sp = 0;
        work[sp++] = {0, 0};
        while (sp > 0) {
            Visit &fr = work[sp - 1];
            const int i = fr.node;
            const bool bin = nt[i] == NODE_BFUNC;
            const int l = i + 1, r = bin ? i + 1 + left[i] : -1;
            const bool both = bin && !is_leaf(nt[l]) && !is_leaf(nt[r]);
            const int first = (!bin || (both && need[l] > need[r])) ? l : r;
            const int second = !bin ? -1 : (first == l ? r : l);
            if (fr.stage == 0) {
                fr.stage = 1;
                if (!is_leaf(nt[first])) {
                    work[sp++] = {first, 0};
                    continue;
                }
                res[first] = leaf_opd(first);
            }
            if (fr.stage == 1 && bin) {
                fr.stage = 2;
                if (both) {
                    // the first operand's value waits in the next free slot
                    if (live_slots >= max_slots_fmt) return CO_ERR_BOUNDS;
                    const int slot = live_slots++;
                    if (live_slots > max_slots) max_slots = live_slots;
                    Operand &o = res[first];
                    if (o.kind != OPD_ACC || o.producer < 0) return CO_ERR_PROGRAM;
                    put_spill(out, wide, o.producer, slot);
                    o = {OPD_SLOT, slot, -1};
                }
                if (!is_leaf(nt[second])) {
                    work[sp++] = {second, 0};
                    continue;
                }
                res[second] = leaf_opd(second);
            }
            --sp;
            const Operand a = res[l];
            const Operand b = bin ? res[r] : Operand{OPD_ACC, 0, -1};
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
            w.lo = cc[i + 1];
            w.hi = cc[i + size[i]];
            w.mid = bin ? cc[i + 1 + left[i]] : w.hi;
            w.tape = tape;
            // reverse-AD tape slots only for partials that are read and not exactly +-1
            const bool unit = bin && (w.fid == OP_ADD || w.fid == OP_SUB);
            w.ta = a.kind != OPD_VAR && !unit;
            w.tb = bin && b.kind != OPD_VAR && !unit;
            tape += (w.ta ? 1 : 0) + (w.tb ? 1 : 0);
            c += op_cost(w.fid);
            res[i] = {OPD_ACC, 0, k};
            put_ins(out, wide, k++, w);
        }
    }
    if (live_slots != 0) return CO_ERR_PROGRAM;
    *n_ins = k;
    *tape_slots = tape;
    *slots_used = max_slots;
    *cost = c;
    return CO_OK;
}

// Worker threads for the decode, started on first use and kept for the
// process: a decode phase hands its chunks to them instead of starting threads
// (starting 15 threads twice per decode cost about 1.5 ms of C5's 6 ms). One
// job at a time; a caller that finds the pool busy, or runs in a process
// forked after the pool started, does its chunks itself.
class DecodePool {
  public:
    static DecodePool &get() {
        static DecodePool pool;
        return pool;
    }
    // fn(i) for every i in [0, n) on the workers and this thread; false (and
    // nothing run) when the pool cannot take the job
    bool run(int n, const std::function<void(int)> &fn) {
        if (workers_.empty() || getpid() != pid_) return false;
        std::unique_lock<std::mutex> job(job_mu_, std::try_to_lock);
        if (!job.owns_lock()) return false;
        {
            std::lock_guard<std::mutex> g(mu_);
            fn_ = &fn;
            n_ = n;
            next_.store(0);
            busy_ = (int)workers_.size();
            ++gen_;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> g(mu_);
        done_cv_.wait(g, [&] { return busy_ == 0; });
        fn_ = nullptr;
        return true;
    }

  private:
    DecodePool() : pid_(getpid()) {
        const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
        const int n = (int)std::min(15u, hw - 1);
        try {
            for (int i = 0; i < n; i++) workers_.emplace_back([this] { loop(); });
        } catch (...) {
            // fewer workers than asked: the ones started serve
        }
    }
    ~DecodePool() {
        {
            std::lock_guard<std::mutex> g(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (std::thread &t : workers_) t.join();
    }
    void work() {
        for (int i = next_.fetch_add(1); i < n_; i = next_.fetch_add(1)) (*fn_)(i);
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> g(mu_);
                cv_.wait(g, [&] { return stop_ || gen_ != seen; });
                if (stop_) return;
                seen = gen_;
            }
            work();
            std::lock_guard<std::mutex> g(mu_);
            if (--busy_ == 0) done_cv_.notify_one();
        }
    }
    std::vector<std::thread> workers_;
    std::mutex job_mu_, mu_;
    std::condition_variable cv_, done_cv_;
    const std::function<void(int)> *fn_ = nullptr;
    int n_ = 0, busy_ = 0;
    std::atomic<int> next_{0};
    uint64_t gen_ = 0;
    bool stop_ = false;
    const pid_t pid_;
};

// Runs fn(m0, m1) over nthreads contiguous chunks of [0, M) on the decode
// pool and this thread; without the pool, redo(0, M) runs on this thread.
template <typename Fn, typename Redo>
static void chunked(int M, int nthreads, const Fn &fn, const Redo &redo) {
    if (nthreads > 1 && M > 0) {
        const int chunk = (M + nthreads - 1) / nthreads;
        const int n = (M + chunk - 1) / chunk;
        const std::function<void(int)> job = [&](int i) {
            fn(i * chunk, std::min(M, (i + 1) * chunk));
        };
        if (DecodePool::get().run(n, job)) return;
    }
    redo(0, M);
}

int check_header(const PopHeader *h, const int32_t *nt, const float *nv, const int32_t *ci,
                 const TreeMeta *metas) {
    if (!h || !metas) return CO_ERR_NULLARG;
    if (h->total_nodes > 0 && (!nt || !nv || !ci)) return CO_ERR_NULLARG;
    if (h->M_prob < 0 || h->N < 0 || h->n_vars < 0 || h->total_nodes < 0 || h->total_c < 0)
        return CO_ERR_NULLARG;
    if (h->K_max > CO_MAX_K || h->max_stack > CO_MAX_STACK || h->n_vars > CO_MAX_VARS)
        return CO_ERR_BOUNDS;
    long ksum = 0, nsum = 0;
    for (int m = 0; m < h->M_prob; m++) { ksum += metas[m].K; nsum += metas[m].n_nodes; }
    if (ksum != (long)h->total_c) return CO_ERR_SUM_C;
    if (nsum != (long)h->total_nodes) return CO_ERR_SUM_NODES;
    return CO_OK;
}

// Decode the M expressions at metas (rows row_base.. of the population whose
// header h is checked): programs into prog (word 0 of this range at word
// word_base of the device program buffer), descriptors in launch order.
static int decode_core(const PopHeader *h, const int32_t *nt, const float *nv,
                       const int32_t *ci, const TreeMeta *metas, int M, int row_base,
                       int64_t word_base, uint64_t *prog, int32_t *order, int32_t *bin_start,
                       ExprDesc *descs, int32_t *stack, int32_t *n_ins, int32_t *prog_off,
                       int32_t *route, Plan *plan, int64_t nodes_per_thread) {
    const int D = h->n_vars;
    long nsum = 0;
    for (int m = 0; m < M; m++) nsum += metas[m].n_nodes;
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
    const int nthreads = (int)std::min<int64_t>(std::min(16u, hw), nsum / nodes_per_thread + 1);
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
            int64_t c = 0;
            int ni = 0;
            if (rcs[m] == CO_OK)
                rcs[m] = emit_tree(tnt, tnv, tci, t.n_nodes, D, gen[m] != 0,
                                   gen[m] ? kMaxSlotsWide : kMaxSlots, out, &ni, &tapes[m],
                                   &slots[m], &c, s);
            if (rcs[m] != CO_OK) return;
            nins[m] = ni;
            if (!gen[m] && tapes[m] > 255) {   // 8-bit tape field (n <= 255 keeps it below)
                rcs[m] = CO_ERR_BOUNDS;
                return;
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
            d.prog_off = (int32_t)(word_base + poff[m]);
            d.n = nins[m];
            d.c_off = metas[m].c_offset;
            d.K = metas[m].K;
            d.y_row = row_base + m;
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

int decode_population(const PopHeader *h, const int32_t *nt, const float *nv,
                      const int32_t *ci, const TreeMeta *metas, uint64_t *prog,
                      int32_t *order, int32_t *bin_start, ExprDesc *descs,
                      int32_t *stack, int32_t *n_ins, int32_t *prog_off, int32_t *route,
                      Plan *plan) {
    const int rc = check_header(h, nt, nv, ci, metas);
    if (rc != CO_OK) return rc;
    std::vector<uint64_t> tmp;
    if (!prog) {
        tmp.assign(h->total_nodes > 0 ? 2 * (size_t)h->total_nodes : 1, 0);
        prog = tmp.data();
    }
    return decode_core(h, nt, nv, ci, metas, h->M_prob, 0, 0, prog, order, bin_start, descs,
                       stack, n_ins, prog_off, route, plan, 65536);
}

int decode_range(const PopHeader *h, const int32_t *nt, const float *nv, const int32_t *ci,
                 const TreeMeta *metas, int m0, int m1, int64_t word_base, uint64_t *prog,
                 ExprDesc *descs, Plan *plan) {
    // a range is decoded while the device fits the ones before it: more
    // threads per node than a whole population gets
    return decode_core(h, nt, nv, ci, metas + m0, m1 - m0, m0, word_base, prog + word_base,
                       nullptr, nullptr, descs + m0, nullptr, nullptr, nullptr, nullptr, plan,
                       16384);
}

}  // namespace cusr
