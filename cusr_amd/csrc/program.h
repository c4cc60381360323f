// program.h -- decoded expression programs shared by the host planner and
// the device interpreter.
//
// An expression (pop.bin nt/nv/ci, cusr/kernel/pop_format.h:6-16, prefix
// order) is a tree the reference evaluates last node first
// (cusr/kernel/lm_core.cuh:67), right operand before left. Here each operator
// runs after its operands, and when both operands need instructions the one
// whose subtree needs more spill slots runs first (Sethi-Ullman order; the
// right one on a tie): values, tangents and adjoints do not depend on which
// sibling runs first, and the spill slots (the LDS a wavefront reserves) stay
// at the tree's minimum. The decoded program is a list of operator
// instructions over three kinds of operand:
//   ACC   the running value, i.e. the result of the previous instruction;
//   SLOT  a spill slot holding the operand computed first while the other
//         operand's instructions run (slots are used last-in first-out);
//   VAR / CONST  a leaf, folded into the instruction that consumes it.
// Leaves therefore cost no instruction; an expression that is a single leaf
// becomes one OP_IDENT instruction.
//
// One 64-bit instruction per operator node, in execution order:
//   bits  0..5   fid     operator id (include/pop_format.h), OP_IDENT = 63
//   bit   6      binary
//   bits  7..8   a_kind  left / only operand: OPD_ACC, OPD_VAR, OPD_CONST, OPD_SLOT
//   bits  9..12  a_idx   variable index, constant rank or slot
//   bits 13..14  b_kind  right operand (binary only)
//   bits 15..18  b_idx
//   bit  19      to_slot result goes to slot d_idx instead of ACC
//   bits 20..23  d_idx
//   bits 24..28  lo      constant ranks of the left / only operand: [lo, mid)
//   bits 29..33  mid     constant ranks of the right operand: [mid, hi)
//   bits 34..38  hi      (unary: mid == hi)
//   bits 39..46  tape    first reverse-AD tape slot of this instruction
//   bit  47      sel     the partials have flat branches: where a point's
//                        partial is a structural zero its tangents become 0
//   bit  48      scale_a forward AD scales ranks [lo, mid) by the partial of
//                        the left / only operand (set when that range is
//                        non-empty and the partial is not exactly 1)
//   bit  49      scale_b forward AD scales ranks [mid, hi) by the right partial
//   bit  50      tape_a  reverse AD keeps the left / only partial in tape slot
//                        `tape`; without it the partial is never read (a
//                        variable operand) or exactly +1 (ADD, SUB's left)
//   bit  51      tape_b  the right partial is kept, in slot tape + tape_a;
//                        without it it is never read or exactly +1 (ADD) / -1
//                        (SUB)
// Constants are ranked in prefix order (cusr/benchmark/popio.py:87-91), so the
// constants of a subtree form one contiguous rank range; forward AD scales
// only those ranks.
//
// The general kernel (expressions outside co_fast_path: K up to 32, a value
// stack up to 64, any number of nodes, up to 255 variables) reads the same
// fields from two 64-bit words per instruction, wide enough for its ranges:
//   word 0: bits  0..5   fid         bit 6 binary
//           bits  7..8   a_kind      bits  9..16 a_idx
//           bits 17..18  b_kind      bits 19..26 b_idx
//           bit  27      to_slot     bits 28..35 d_idx
//           bits 36..40  sel, scale_a, scale_b, tape_a, tape_b
//   word 1: bits  0..7   lo          bits  8..15 mid      bits 16..23 hi
//           bits 24..55  tape
#pragma once

#include <stdint.h>

#include "../../include/cusr_co.h"

namespace cusr {

enum { OPD_ACC = 0, OPD_VAR = 1, OPD_CONST = 2, OPD_SLOT = 3 };
constexpr int OP_IDENT = 63;
constexpr int kMaxSlots = 16;                    // fast format (4-bit slot index)
constexpr int kMaxSlotsWide = CO_MAX_STACK;      // wide format

struct ExprDesc {          // one per expression, device-resident
    int32_t prog_off;      // first program word
    int32_t n;             // instructions
    int32_t c_off;         // constants offset
    int32_t K;             // constants
    int32_t y_row;         // row of ym / output index (original expression index)
    int32_t tape;          // reverse-mode tape slots
    int32_t slots;         // spill slots
    int32_t gen;           // 1: wide program, general kernel
};

static inline __host__ __device__ int ins_fid(uint64_t w) { return (int)(w & 63u); }
static inline __host__ __device__ int ins_binary(uint64_t w) { return (int)((w >> 6) & 1u); }
static inline __host__ __device__ int ins_akind(uint64_t w) { return (int)((w >> 7) & 3u); }
static inline __host__ __device__ int ins_aidx(uint64_t w) { return (int)((w >> 9) & 15u); }
static inline __host__ __device__ int ins_bkind(uint64_t w) { return (int)((w >> 13) & 3u); }
static inline __host__ __device__ int ins_bidx(uint64_t w) { return (int)((w >> 15) & 15u); }
static inline __host__ __device__ int ins_toslot(uint64_t w) { return (int)((w >> 19) & 1u); }
static inline __host__ __device__ int ins_didx(uint64_t w) { return (int)((w >> 20) & 15u); }
static inline __host__ __device__ int ins_lo(uint64_t w) { return (int)((w >> 24) & 31u); }
static inline __host__ __device__ int ins_mid(uint64_t w) { return (int)((w >> 29) & 31u); }
// fields above bit 31 are read from the high half alone: a 64-bit mask test
// costs the device an extra scalar compare per field
static inline __host__ __device__ uint32_t ins_w1(uint64_t w) { return (uint32_t)(w >> 32); }
static inline __host__ __device__ int ins_hi(uint64_t w) { return (int)((ins_w1(w) >> 2) & 31u); }
static inline __host__ __device__ int ins_tape(uint64_t w) { return (int)((ins_w1(w) >> 7) & 255u); }
static inline __host__ __device__ int ins_sel(uint64_t w) { return (int)((ins_w1(w) >> 15) & 1u); }
static inline __host__ __device__ int ins_scale_a(uint64_t w) { return (int)((ins_w1(w) >> 16) & 1u); }
static inline __host__ __device__ int ins_scale_b(uint64_t w) { return (int)((ins_w1(w) >> 17) & 1u); }
static inline __host__ __device__ int ins_tape_a(uint64_t w) { return (int)((ins_w1(w) >> 18) & 1u); }
static inline __host__ __device__ int ins_tape_b(uint64_t w) { return (int)((ins_w1(w) >> 19) & 1u); }

// wide-format fields (word 0 a, word 1 b)
struct Wide {
    uint64_t a, b;
};
static inline __host__ __device__ int wins_fid(uint64_t a) { return (int)(a & 63u); }
static inline __host__ __device__ int wins_binary(uint64_t a) { return (int)((a >> 6) & 1u); }
static inline __host__ __device__ int wins_akind(uint64_t a) { return (int)((a >> 7) & 3u); }
static inline __host__ __device__ int wins_aidx(uint64_t a) { return (int)((a >> 9) & 255u); }
static inline __host__ __device__ int wins_bkind(uint64_t a) { return (int)((a >> 17) & 3u); }
static inline __host__ __device__ int wins_bidx(uint64_t a) { return (int)((a >> 19) & 255u); }
static inline __host__ __device__ int wins_toslot(uint64_t a) { return (int)((a >> 27) & 1u); }
static inline __host__ __device__ int wins_didx(uint64_t a) { return (int)((a >> 28) & 255u); }
static inline __host__ __device__ int wins_sel(uint64_t a) { return (int)((ins_w1(a) >> 4) & 1u); }
static inline __host__ __device__ int wins_scale_a(uint64_t a) { return (int)((ins_w1(a) >> 5) & 1u); }
static inline __host__ __device__ int wins_scale_b(uint64_t a) { return (int)((ins_w1(a) >> 6) & 1u); }
static inline __host__ __device__ int wins_tape_a(uint64_t a) { return (int)((ins_w1(a) >> 7) & 1u); }
static inline __host__ __device__ int wins_tape_b(uint64_t a) { return (int)((ins_w1(a) >> 8) & 1u); }
static inline __host__ __device__ int wins_lo(uint64_t b) { return (int)(b & 255u); }
static inline __host__ __device__ int wins_mid(uint64_t b) { return (int)((b >> 8) & 255u); }
static inline __host__ __device__ int wins_hi(uint64_t b) { return (int)((b >> 16) & 255u); }
static inline __host__ __device__ int wins_tape(uint64_t b) { return (int)((b >> 24) & 0xffffffffu); }

struct Plan {
    int32_t M, N, D, total_nodes, total_c;
    int32_t max_tape, max_n, max_slots;
    int64_t words;         // program words (fast: 1 per instruction, wide: 2)
    int32_t n_gen;         // expressions of the general kernel
};

// Check a population and decode it. Returns a CO_* code. On success fills
// prog[2 * total_nodes] (expression m's program starts at word prog_off[m]:
// programs are laid out expression after expression, n_nodes words for the
// fast format and 2 * n_nodes for the wide one; words past its instructions
// are 0), order[M] (stable K bins, ascending), bin_start[CO_MAX_K+2],
// descs[M] (by launch position: the general kernel's bin first, then the fast
// K bins, largest K first), stack[M] (value-stack depth, by expression),
// n_ins[M] (instructions per expression), prog_off[M], route[M] (1: general
// kernel). Any output pointer may be null.
int decode_population(const PopHeader *h, const int32_t *nt, const float *nv,
                      const int32_t *ci, const TreeMeta *metas, uint64_t *prog,
                      int32_t *order, int32_t *bin_start, ExprDesc *descs,
                      int32_t *stack, int32_t *n_ins, int32_t *prog_off, int32_t *route,
                      Plan *plan);

// The header-level checks decode_population makes first: null inputs, device
// bounds on K_max / max_stack / n_vars, and the sums of K and of n_nodes.
int check_header(const PopHeader *h, const int32_t *nt, const float *nv, const int32_t *ci,
                 const TreeMeta *metas);

// Decode expressions [m0, m1) of a population whose header passed
// check_header, for an upload that decodes a population in pieces: their
// programs go to prog from word word_base on (the range's layout as
// decode_population's, its descriptors' prog_off counting from word 0 of
// prog), their descriptors to descs[m0..m1) in launch order within the range
// (y_row the population row). plan describes the range (M, words, slots,
// tape); the same per-expression checks and error codes as decode_population.
int decode_range(const PopHeader *h, const int32_t *nt, const float *nv, const int32_t *ci,
                 const TreeMeta *metas, int m0, int m1, int64_t word_base, uint64_t *prog,
                 ExprDesc *descs, Plan *plan);

}  // namespace cusr
