// program.h -- decoded expression programs shared by the host planner and
// the device interpreter.
//
// Each pop.bin node (nt, nv, ci; cusr/kernel/pop_format.h:6-16) becomes one
// 64-bit instruction. Instructions are stored in execution order, i.e. the
// last prefix node first (the evaluation order of cusr/kernel/lm_core.cuh:67),
// and carry everything the interpreter would otherwise track at run time:
//
//   bits  0..7   fid    operator id (NODE_UFUNC / NODE_BFUNC), else 0
//   bits  8..9   kind   NODE_VAR / NODE_CONST / NODE_UFUNC / NODE_BFUNC
//   bits 16..23  arg    variable index (VAR) or constant rank (CONST)
//   bits 24..31  sp     value-stack depth before the instruction
//   bits 32..36  lo     first constant rank of the (left) operand subtree
//   bits 37..41  mid    end of the left range = start of the right range
//   bits 42..46  hi     end of the operand ranks (unary: [lo, hi))
//   bits 47..54  tape   first tape slot of the node's local partials
//   bits 55..60  asp    adjoint-stack depth before the node, reverse sweep
//   bit  61      apop   the node's adjoint comes from the adjoint stack
//                       (it is a right child), not from the running value
//
// Constants are ranked in prefix order (cusr/benchmark/popio.py:87-91), so the
// constants of any subtree form one contiguous rank range; forward AD uses
// that to scale only the ranks an operator can touch.
#pragma once

#include <stdint.h>

#include "../../include/cusr_co.h"

namespace cusr {

struct ExprDesc {          // one per expression, device-resident
    int32_t prog_off;      // first instruction
    int32_t n;             // instructions
    int32_t c_off;         // constants offset
    int32_t K;             // constants
    int32_t y_row;         // row of ym / output index (original expression index)
    int32_t tape;          // reverse-mode tape slots
    int32_t stack;         // value-stack depth
    int32_t pad;
};

static inline __host__ __device__ int ins_fid(uint64_t w) { return (int)(w & 0xffu); }
static inline __host__ __device__ int ins_kind(uint64_t w) { return (int)((w >> 8) & 3u); }
static inline __host__ __device__ int ins_arg(uint64_t w) { return (int)((w >> 16) & 0xffu); }
static inline __host__ __device__ int ins_sp(uint64_t w) { return (int)((w >> 24) & 0xffu); }
static inline __host__ __device__ int ins_lo(uint64_t w) { return (int)((w >> 32) & 31u); }
static inline __host__ __device__ int ins_mid(uint64_t w) { return (int)((w >> 37) & 31u); }
static inline __host__ __device__ int ins_hi(uint64_t w) { return (int)((w >> 42) & 31u); }
static inline __host__ __device__ int ins_tape(uint64_t w) { return (int)((w >> 47) & 0xffu); }
static inline __host__ __device__ int ins_asp(uint64_t w) { return (int)((w >> 55) & 63u); }
static inline __host__ __device__ int ins_apop(uint64_t w) { return (int)((w >> 61) & 1u); }

struct Plan {
    int32_t M, N, D, total_nodes, total_c;
    int32_t max_tape, max_n;
};

// Check a population and decode it. Returns a CO_* code. On success fills
// prog[total_nodes], order[M] (K-ascending stable bins), bin_start[CO_MAX_K+2],
// descs[M] (indexed by launch position), stack[M] (indexed by expression).
int decode_population(const PopHeader *h, const int32_t *nt, const float *nv,
                      const int32_t *ci, const TreeMeta *metas, uint64_t *prog,
                      int32_t *order, int32_t *bin_start, ExprDesc *descs,
                      int32_t *stack, Plan *plan);

}  // namespace cusr
