// co_lib.hip -- C ABI of the MI355X batched LM fitter (include/cusr_co.h).
//
// Mirrors the reference in-process library (cusr/kernel/co_lib.cu:113-568):
// a persistent per-device context whose device buffers grow by byte capacity
// and never shrink (co_lib.cu:16-24,113-153), every call re-seeded from its own
// inputs (co_lib.cu:284-305), outputs written to caller buffers sized by the
// current header, errors returned as codes and never exit(). Unlike the
// reference, the whole LM loop is one kernel launch; the host only plans,
// uploads, launches once and reads the results back.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include <cmath>
#include <mutex>
#include <new>
#include <vector>

#include "lm_device.h"
#define CUSR_SPLIT_STEP_KERNELS
#include "lm_split.h"
#include "program.h"

namespace cusr {

// ------------------------------------------------------ layout kernels

// xs row-major [N][D] (f32 or f64) -> X column-major [D][N] f64
template <typename T>
__global__ void transpose_x_kernel(const T *xs, double *X, int N, int D) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (size_t)N * D) return;
    const size_t i = t / D, v = t % D;
    X[v * N + i] = (double)xs[t];
}

__global__ void widen_kernel(const float *src, double *dst, size_t n) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < n) dst[t] = (double)src[t];
}

// The scratch of co_fit_resident_static: a fixed array in device memory, one
// copy per GPU the library runs on, held until the process ends. In host code
// the name is a stand-in, not a device address: every use goes through the
// per-device address hipGetSymbolAddress gives at co_init.
static __device__ __align__(256) unsigned char scratch[CO_STATIC_SCRATCH_BYTES];

}  // namespace cusr

using namespace cusr;

// LM ordering of co_optimize and of co_options_default: the library named
// libcusr_co_fd.so is built with the FD variant's ordering, libcusr_co_ad.so
// with the AD variant's (the reference's two variants, co_lib.cu:3-7).
#ifndef CUSR_DEFAULT_ORDER
#define CUSR_DEFAULT_ORDER CO_ORDER_IMPROVE_FIRST
#endif

namespace {

double now_ms() {
    timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec * 1e3 + t.tv_nsec / 1e6;
}

double g_setup_ms = -1.0, g_loop_ms = -1.0;

struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
};

// Page-locked host staging for the decoded programs (hipHostMalloc), grown
// with 25 % headroom and never shrunk. Copies to the device from it run at
// DMA speed; from pageable memory the runtime stages them through buffers of
// its own (C5: 9.5 ms of setup per round, most of it those copies).
template <typename T>
struct HostBuf {
    T *p = nullptr;
    size_t cap = 0;   // elements
    T *data() { return p; }
    T &operator[](size_t i) { return p[i]; }
    const T &operator[](size_t i) const { return p[i]; }
};

// K bins run concurrently on the handle's stream and kExtraStreams more. HIP maps
// each stream of a process to one of GPU_MAX_HW_QUEUES (4) hardware queues,
// and two streams that share a queue run one after the other: a fifth stream
// was measured sharing a queue and serialising its bins behind another's
// (C2: 20.5 ms, the sum of the two streams' bins). So four streams in all.
constexpr int kExtraStreams = 3;
constexpr int kStreams = kExtraStreams + 1;
constexpr int kMaxRanges = 2;   // launch ranges of one fit (the upload pipeline's two)

// launchers per (precision, AD mode) come from fit_kernels.hip, each variant
// in its own translation unit so the four compile in parallel

// Device memory of a fit beyond its inputs and outputs: the loop state of
// paused (tail) or split fits, then the split path's partition sums. Either
// the handle's buffer, grown as needed, or a fixed region that is never grown
// (the static array of co_fit_resident_static).
struct Scratch {
    void *p = nullptr;
    size_t cap = 0;
    bool fixed = false;
};

// Per-device address of the static scratch array (hipGetSymbolAddress with
// the device current), resolved once per device at co_init.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

struct Ctx {
    int device = -1;
    hipStream_t stream = nullptr;
    hipStream_t lanes[kExtraStreams] = {};
    hipEvent_t ev_start = nullptr;
    hipEvent_t ev_done[kExtraStreams] = {};
    hipEvent_t ev_t0 = nullptr, ev_t1 = nullptr;  // timing pair around the fit launches
    // per bin and launch range (a pipelined co_optimize launches each bin once
    // per range): a bin's time is the sum of its launches' durations
    hipEvent_t ev_b0[kMaxRanges][CO_BINS] = {}, ev_b1[kMaxRanges][CO_BINS] = {};
    bool bin_launched[kMaxRanges][CO_BINS] = {};
    Plan plan = {};
    bool resident = false;
    std::vector<int> ranges;   // launch-order ranges of the resident descriptors: [r[i], r[i+1])
    hipStream_t copy_stream = nullptr;   // uploads of a pipelined co_optimize
    bool shared_y = false;   // the resident y is one row for every expression
    bool on_data = false;    // the resident population fits the uploaded data set
    bool dev_io = false;     // co_optimize_data_device: constants in, results out in device memory
    int data_N = -1, data_D = 0;  // shape of the uploaded data set (-1: none)
    double last_kernel_ms = -1.0;
    double last_bin_ms[CO_BINS] = {};
    size_t lds_per_block = 0;  // LDS one workgroup may use on this device
    DevBuf prog, desc, X, Y, C0, C, status, li, lf, iters, stage;
    DevBuf data_X, data_Y;   // co_data_upload: X [D][N] column-major, y [N]
    DevBuf state;            // scratch of tail and split fits (run_fit)
    void *static_scratch = nullptr;   // this device's address of `scratch`
    HostBuf<uint64_t> h_prog;
    HostBuf<ExprDesc> h_desc;
    HostBuf<char> h_stage;   // page-locked copies of small host inputs (upload_data)
    HostBuf<char> h_back;    // page-locked landing of small results (FitRun::finish)
    std::vector<double> h_c, h_li, h_lf, h_c0;   // co_optimize: fp64 results, c_init
    std::vector<float> h_li32, h_lf32;
};

#define CO_HIP(call)                                                                    \
    do {                                                                                \
        hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess) {                                                         \
            fprintf(stderr, "[cusr_co] HIP error %s at %s:%d\n", hipGetErrorString(e_), \
                    __FILE__, __LINE__);                                                \
            return CO_ERR_CUDA;                                                         \
        }                                                                               \
    } while (0)

int grow(DevBuf &b, size_t bytes) {
    if (bytes == 0) bytes = 256;
    if (bytes <= b.cap) return CO_OK;
    if (b.p) (void)hipFree(b.p);
    b.p = nullptr;
    b.cap = 0;
    hipError_t e = hipMalloc(&b.p, bytes);
    if (e != hipSuccess) {
        fprintf(stderr, "[cusr_co] hipMalloc(%zu) failed: %s\n", bytes, hipGetErrorString(e));
        b.p = nullptr;
        return (e == hipErrorOutOfMemory) ? CO_ERR_OOM : CO_ERR_CUDA;
    }
    b.cap = bytes;
    return CO_OK;
}

#define CO_GROW(buf, bytes)                   \
    do {                                      \
        int r_ = grow((buf), (bytes));        \
        if (r_ != CO_OK) return r_;           \
    } while (0)

template <typename T>
int grow_host(HostBuf<T> &b, size_t n) {
    if (n == 0) n = 1;
    if (n <= b.cap) return CO_OK;
    if (b.p) (void)hipHostFree(b.p);
    b.p = nullptr;
    b.cap = 0;
    const size_t want = n + n / 4;
    void *q = nullptr;
    hipError_t e = hipHostMalloc(&q, want * sizeof(T), hipHostMallocDefault);
    if (e != hipSuccess) {
        fprintf(stderr, "[cusr_co] hipHostMalloc(%zu) failed: %s\n", want * sizeof(T),
                hipGetErrorString(e));
        return (e == hipErrorOutOfMemory) ? CO_ERR_OOM : CO_ERR_CUDA;
    }
    b.p = (T *)q;
    b.cap = want;
    return CO_OK;
}

#define CO_GROW_HOST(buf, n)                  \
    do {                                      \
        int r_ = grow_host((buf), (n));       \
        if (r_ != CO_OK) return r_;           \
    } while (0)

template <typename T>
T *ptr(DevBuf &b) { return (T *)b.p; }

unsigned blocks_for(size_t n, unsigned t) { return (unsigned)((n + t - 1) / t); }

// dynamic LDS a workgroup of a fit kernel family may use: the device's LDS
// per workgroup less the family's static arrays (constants and pass sums)
size_t max_dyn_lds(const Ctx *ctx, bool gen) {
    const size_t st = fit_static_lds(gen);
    return ctx->lds_per_block > st ? ctx->lds_per_block - st : 0;
}

// the launcher's choice of instance (fit_kernels.hip): the large-N one from
// kLargeN points where its tables differ
template <typename R, int AD>
size_t lds_for_k(int K, int N, int D, int slots, int tape) {
    switch (K) {
#define CUSR_LDS_CASE(k)                                                        \
    case k:                                                                     \
        return (large_n_variant<R, k, AD>() && N >= kLargeN)                    \
                   ? fit_lds_bytes_t<R, k, AD, 1>(D, slots, tape)               \
                   : fit_lds_bytes_t<R, k, AD, 0>(D, slots, tape);
    CUSR_LDS_CASE(0) CUSR_LDS_CASE(1) CUSR_LDS_CASE(2) CUSR_LDS_CASE(3) CUSR_LDS_CASE(4)
    CUSR_LDS_CASE(5) CUSR_LDS_CASE(6) CUSR_LDS_CASE(7) CUSR_LDS_CASE(8) CUSR_LDS_CASE(9)
    CUSR_LDS_CASE(10) CUSR_LDS_CASE(11) CUSR_LDS_CASE(12) CUSR_LDS_CASE(13)
    CUSR_LDS_CASE(14) CUSR_LDS_CASE(15) CUSR_LDS_CASE(16)
#undef CUSR_LDS_CASE
    default: return 0;
    }
}

size_t fit_lds_bytes(bool mixed, bool rev, int K, int N, int D, int slots, int tape) {
    if (K == CO_GENERAL_BIN)
        return mixed ? fit_lds_bytes_gen<float>(D, slots, tape)
                     : fit_lds_bytes_gen<double>(D, slots, tape);
    if (mixed)
        return rev ? lds_for_k<float, CO_AD_REVERSE>(K, N, D, slots, tape)
                   : lds_for_k<float, CO_AD_FORWARD>(K, N, D, slots, tape);
    return rev ? lds_for_k<double, CO_AD_REVERSE>(K, N, D, slots, tape)
               : lds_for_k<double, CO_AD_FORWARD>(K, N, D, slots, tape);
}

// Device buffers of a population of M expressions with `words` program words.
int grow_buffers(Ctx *ctx, const PopHeader *h, size_t words, bool in32, bool on_data,
                 bool shared_y) {
    const int M = h->M_prob, N = h->N, D = h->n_vars, C = h->total_c;
    const size_t nX = on_data ? 0 : (size_t)N * D;
    const size_t nY = on_data ? 0 : shared_y ? (size_t)N : (size_t)M * N;
    const size_t esz = in32 ? 4 : 8;
    // the program words and constants vary from population to population: a
    // quarter of headroom, so a slightly larger next population (a GP
    // round's) does not free and allocate again (about 1 ms of a C5 round
    // when it did)
    if (sizeof(uint64_t) * words > ctx->prog.cap)
        CO_GROW(ctx->prog, sizeof(uint64_t) * (words + words / 4));
    CO_GROW(ctx->desc, sizeof(ExprDesc) * M);
    CO_GROW(ctx->X, sizeof(double) * nX);
    CO_GROW(ctx->Y, sizeof(double) * nY);
    const size_t Ch = (size_t)C + (size_t)C / 4;
    if (sizeof(double) * C > ctx->C0.cap) CO_GROW(ctx->C0, sizeof(double) * Ch);
    if (sizeof(double) * C > ctx->C.cap) CO_GROW(ctx->C, sizeof(double) * Ch);
    CO_GROW(ctx->status, sizeof(int32_t) * M);
    CO_GROW(ctx->li, sizeof(double) * M);
    CO_GROW(ctx->lf, sizeof(double) * M);
    CO_GROW(ctx->iters, sizeof(int32_t) * M);
    size_t stage = esz * nX;
    if (in32 && esz * nY > stage) stage = esz * nY;
    if (in32 && esz * C > stage) stage = esz * C;
    if (stage > ctx->stage.cap) CO_GROW(ctx->stage, stage + stage / 4);
    return CO_OK;
}

// Queue the copies of the data (X, y) and c_init on stream s (fp32 host
// inputs are widened on the device). With on_data only c_init goes over.
// Host inputs up to this many bytes in all are first copied into page-locked
// staging, so their copies to the device run as DMA without holding the host
// (from pageable memory the runtime stages each copy itself, and the host
// waits: C5, 1.1 MB of constants per round, 0.85 ms before the first range's
// decode could start). Larger inputs (a target per expression) go directly.
constexpr size_t kPinnedStageMax = 16u << 20;

int upload_data(Ctx *ctx, const PopHeader *h, const void *c, const void *xs, const void *ym,
                bool in32, bool on_data, bool shared_y, hipStream_t s) {
    const int M = h->M_prob, N = h->N, D = h->n_vars, C = h->total_c;
    const size_t nX = on_data ? 0 : (size_t)N * D;
    const size_t nY = on_data ? 0 : shared_y ? (size_t)N : (size_t)M * N;
    const size_t esz = in32 ? 4 : 8;
    const auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t bX = esz * nX, bY = esz * nY, bC = ctx->dev_io ? 0 : esz * (size_t)C;
    if (bX + bY + bC > 0 && up(bX) + up(bY) + up(bC) <= kPinnedStageMax) {
        // the previous call's copies from the staging have finished before
        // it is written again
        CO_HIP(hipStreamSynchronize(s));
        CO_GROW_HOST(ctx->h_stage, up(bX) + up(bY) + up(bC));
        char *q = ctx->h_stage.data();
        if (bX) { memcpy(q, xs, bX); xs = q; q += up(bX); }
        if (bY) { memcpy(q, ym, bY); ym = q; q += up(bY); }
        if (bC) { memcpy(q, c, bC); c = q; }
    }
    // xs: row-major host array -> column-major fp64 on the device
    if (nX) {
        CO_HIP(hipMemcpyAsync(ctx->stage.p, xs, esz * nX, hipMemcpyHostToDevice, s));
        if (in32)
            transpose_x_kernel<float><<<blocks_for(nX, 256), 256, 0, s>>>(
                ptr<float>(ctx->stage), ptr<double>(ctx->X), N, D);
        else
            transpose_x_kernel<double><<<blocks_for(nX, 256), 256, 0, s>>>(
                ptr<double>(ctx->stage), ptr<double>(ctx->X), N, D);
        CO_HIP(hipGetLastError());
    }
    if (in32) {
        if (nY) {
            CO_HIP(hipMemcpyAsync(ctx->stage.p, ym, 4 * nY, hipMemcpyHostToDevice, s));
            widen_kernel<<<blocks_for(nY, 256), 256, 0, s>>>(ptr<float>(ctx->stage),
                                                            ptr<double>(ctx->Y), nY);
            CO_HIP(hipGetLastError());
        }
        if (C) {
            CO_HIP(hipMemcpyAsync(ctx->stage.p, c, 4 * (size_t)C, hipMemcpyHostToDevice, s));
            widen_kernel<<<blocks_for(C, 256), 256, 0, s>>>(ptr<float>(ctx->stage),
                                                           ptr<double>(ctx->C0), C);
            CO_HIP(hipGetLastError());
        }
    } else {
        if (nY) CO_HIP(hipMemcpyAsync(ctx->Y.p, ym, 8 * nY, hipMemcpyHostToDevice, s));
        if (C)
            CO_HIP(hipMemcpyAsync(ctx->C0.p, c, 8 * (size_t)C,
                                  ctx->dev_io ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                                  s));
    }
    return CO_OK;
}

// Check, decode and upload one population into the context (fp32 or fp64
// host inputs); the population stays resident until the next upload.
// With on_data, xs and ym are unused: the population fits the data set of
// co_data_upload, whose shape must match the header's.
int upload_population(Ctx *ctx, const PopHeader *h, const int32_t *nt, const float *nv,
                      const int32_t *ci, const TreeMeta *metas, const void *c, const void *xs,
                      const void *ym, bool in32, bool on_data = false) {
    CO_HIP(hipSetDevice(ctx->device));
    ctx->resident = false;
    const int M = h->M_prob;
    CO_GROW_HOST(ctx->h_prog, h->total_nodes > 0 ? 2 * (size_t)h->total_nodes : 1);
    CO_GROW_HOST(ctx->h_desc, M > 0 ? (size_t)M : 1);
    int rc = decode_population(h, nt, nv, ci, metas, ctx->h_prog.data(), nullptr, nullptr,
                               ctx->h_desc.data(), nullptr, nullptr, nullptr, nullptr,
                               &ctx->plan);
    if (rc != CO_OK) return rc;
    if (on_data && (ctx->data_N < 0 || h->N != ctx->data_N || h->n_vars != ctx->data_D))
        return CO_ERR_DATA;
    ctx->on_data = on_data;
    ctx->ranges.assign({0, M});
    if (M == 0) {
        ctx->resident = true;
        return CO_OK;
    }
    const bool shared_y = on_data || (pop_flags(h) & POP_FLAG_SHARED_Y) != 0;
    const size_t words = (size_t)ctx->plan.words;
    rc = grow_buffers(ctx, h, words, in32, on_data, shared_y);
    if (rc != CO_OK) return rc;
    hipStream_t s = ctx->stream;
    if (words)
        CO_HIP(hipMemcpyAsync(ctx->prog.p, ctx->h_prog.data(), sizeof(uint64_t) * words,
                              hipMemcpyHostToDevice, s));
    CO_HIP(hipMemcpyAsync(ctx->desc.p, ctx->h_desc.data(), sizeof(ExprDesc) * M,
                          hipMemcpyHostToDevice, s));
    rc = upload_data(ctx, h, c, xs, ym, in32, on_data, shared_y, s);
    if (rc != CO_OK) return rc;
    CO_HIP(hipStreamSynchronize(s));
    ctx->shared_y = shared_y;
    ctx->resident = true;
    return CO_OK;
}

// One launch of a fit: its bin, workgroups, LDS and stream (planned before
// anything is launched, so a launch that cannot fit is refused up front).
struct LaunchPlan {
    int bin, pos, cnt, slots, tape, kmax, stream;
    size_t wave_bytes;
    int pwaves[2];
    size_t lds[2];
};

typedef hipError_t (*Launcher)(int, unsigned, size_t, hipStream_t, const FitArgs &);

// The launches of one fit, planned and issued range by range. The
// descriptors of a range are in launch order (decode_population /
// decode_range): a population decoded in several ranges has its bins planned
// range by range.

// The split path's step launch for a bin: the fast bins (K = 1..CO_FAST_MAX_K,
// every expression of that K) take the instance whose solve is unrolled for
// their K, the general bin and K = 0 the runtime-K one.
template <int KS>
static void launch_step_k(unsigned n, hipStream_t s, const FitArgs &fa, int mixed) {
    lm_step_kernel<KS><<<n, kLanes, 0, s>>>(fa, mixed);
}
static void launch_step(int bin, unsigned n, hipStream_t s, const FitArgs &fa, int mixed) {
    static_assert(CO_FAST_MAX_K == 16, "one step instance per fast K");
    switch (bin) {
    case 1: launch_step_k<1>(n, s, fa, mixed); break;
    case 2: launch_step_k<2>(n, s, fa, mixed); break;
    case 3: launch_step_k<3>(n, s, fa, mixed); break;
    case 4: launch_step_k<4>(n, s, fa, mixed); break;
    case 5: launch_step_k<5>(n, s, fa, mixed); break;
    case 6: launch_step_k<6>(n, s, fa, mixed); break;
    case 7: launch_step_k<7>(n, s, fa, mixed); break;
    case 8: launch_step_k<8>(n, s, fa, mixed); break;
    case 9: launch_step_k<9>(n, s, fa, mixed); break;
    case 10: launch_step_k<10>(n, s, fa, mixed); break;
    case 11: launch_step_k<11>(n, s, fa, mixed); break;
    case 12: launch_step_k<12>(n, s, fa, mixed); break;
    case 13: launch_step_k<13>(n, s, fa, mixed); break;
    case 14: launch_step_k<14>(n, s, fa, mixed); break;
    case 15: launch_step_k<15>(n, s, fa, mixed); break;
    case 16: launch_step_k<16>(n, s, fa, mixed); break;
    default: launch_step_k<0>(n, s, fa, mixed); break;
    }
}

struct FitRun {
    struct Segment {
        int parts, it_end, resume;
    };
    Ctx *ctx = nullptr;
    CoOptions opt = {};
    FitArgs fa = {};
    bool rev = false, mixed = false, split = false, started = false;
    int parts = 0, nseg = 1, pwidth = 0;
    Segment seg[2] = {};
    bool lane_used[kExtraStreams] = {};
    int range = 0;   // ranges issued so far
    Launcher launch = nullptr, launch_pass = nullptr;

    // Option checks and the fit's arguments (ctx->plan holds N, D, M, C).
    int begin(Ctx *c, const CoOptions &o) {
        ctx = c;
        opt = o;
        if (opt.ad_mode != CO_AD_FORWARD && opt.ad_mode != CO_AD_REVERSE) return CO_ERR_NULLARG;
        if (opt.precision != CO_PREC_FP64 && opt.precision != CO_PREC_MIXED)
            return CO_ERR_NULLARG;
        if (opt.max_iter < 0) return CO_ERR_NULLARG;
        if (opt.lm_order != CO_ORDER_IMPROVE_FIRST && opt.lm_order != CO_ORDER_CONVERGE_FIRST)
            return CO_ERR_NULLARG;
        if (opt.damping < CO_DAMP_RELATIVE || opt.damping > CO_DAMP_PIVOT_FLOOR)
            return CO_ERR_NULLARG;
        if (opt.tail_iter < -1 || (opt.tail_partitions != 0 && opt.tail_partitions != 1 &&
                                   opt.tail_partitions != 2 && opt.tail_partitions != 4))
            return CO_ERR_NULLARG;
        CO_HIP(hipSetDevice(ctx->device));
        const Plan &plan = ctx->plan;
        ctx->last_kernel_ms = 0.0;
        for (int k = 0; k < CO_BINS; ++k) {
            for (int r = 0; r < kMaxRanges; ++r) ctx->bin_launched[r][k] = false;
            ctx->last_bin_ms[k] = -1.0;
        }
        parts = co_partitions_resolve(&opt, plan.N);
        if (parts == 0) return CO_ERR_NULLARG;
        split = parts > CO_MAX_PARTITIONS;
        fa.prog = ptr<uint64_t>(ctx->prog);
        fa.desc = ptr<ExprDesc>(ctx->desc);
        fa.X = ptr<double>(ctx->on_data ? ctx->data_X : ctx->X);
        fa.Y = ptr<double>(ctx->on_data ? ctx->data_Y : ctx->Y);
        fa.C0 = ptr<double>(ctx->C0);
        fa.C = ptr<double>(ctx->C);
        fa.status = ptr<int32_t>(ctx->status);
        fa.loss_init = ptr<double>(ctx->li);
        fa.loss_final = ptr<double>(ctx->lf);
        fa.iters = ptr<int32_t>(ctx->iters);
        fa.N = plan.N;
        fa.D = plan.D;
        fa.max_iter = opt.max_iter;
        fa.guard = opt.fp64_guard ? 1 : 0;
        fa.shared_y = ctx->shared_y ? 1 : 0;
        fa.f32_range = opt.f32_range ? 1 : 0;
        fa.lm_order = opt.lm_order;
        fa.damp = opt.damping;
        fa.lambda0 = opt.lambda0;
        fa.xtol = opt.xtol;
        fa.psum = nullptr;
        fa.psum_width = 0;
        fa.state = nullptr;
        fa.state_stride = 0;
        rev = opt.ad_mode == CO_AD_REVERSE;
        mixed = opt.precision == CO_PREC_MIXED;
        // segments of the iteration loop: all expressions up to tail_it, then the
        // ones still running with tail_parts partitions (one launch each per bin)
        int tail_parts = parts;
        const int tail_it = co_tail_resolve(&opt, plan.N, &tail_parts);
        seg[0] = {parts, opt.max_iter, 0};
        nseg = 1;
        if (tail_it > 0) {
            seg[0].it_end = tail_it;
            seg[1] = {tail_parts, opt.max_iter, 1};
            nseg = 2;
        }
        launch = mixed ? (rev ? launch_fit_f32_rev : launch_fit_f32_fwd)
                       : (rev ? launch_fit_f64_rev : launch_fit_f64_fwd);
        launch_pass = mixed ? (rev ? launch_pass_f32_rev : launch_pass_f32_fwd)
                            : (rev ? launch_pass_f64_rev : launch_pass_f64_fwd);
        return CO_OK;
    }

    // The bins of descriptors [p0, p1) in launch order: the general kernel's
    // bin, then the fast K bins, largest K first. The streams are dealt
    // round-robin in that order (stream kExtraStreams is the handle's own).
    // The kernel launched first on a stream takes the machine first and so
    // ends first, so each stream's next bin is the next largest; this beats
    // balancing estimated costs over the streams (C2 12.15 -> 11.66 ms, C4
    // 173 -> 170 ms, C3 139.7 -> 137.8 ms on an MI355X). A general bin of at
    // least a sixteenth of the range's expressions is the exception: one
    // wavefront per expression at one point per lane, it outlasts any fast bin
    // many times over, so it gets stream 0 to itself and the fast bins are
    // dealt over the other three (a GP-generation population, a fifth of it
    // general: the fast bins dealt behind it on stream 0 had waited for it,
    // 74.6 ms per fit against the general bin's 45 ms).
    int plan_range(int p0, int p1, LaunchPlan *lp, int *nl_out, int *kmax_out) const {
        const Plan &plan = ctx->plan;
        int nl = 0, kmax = 0, pos = p0;
        bool gen_alone = false;
        for (int i = 0; i < CO_BINS; ++i) {
            const int bin = i == 0 ? CO_GENERAL_BIN : CO_FAST_MAX_K - (i - 1);
            const bool gen = bin == CO_GENERAL_BIN;
            LaunchPlan b = {};
            b.bin = bin;
            b.pos = pos;
            while (pos < p1 && (gen ? ctx->h_desc[pos].gen != 0
                                    : (!ctx->h_desc[pos].gen && ctx->h_desc[pos].K == bin))) {
                const ExprDesc &d = ctx->h_desc[pos];
                if (d.slots > b.slots) b.slots = d.slots;
                if (d.tape > b.tape) b.tape = d.tape;
                if (d.K > b.kmax) b.kmax = d.K;
                ++b.cnt;
                ++pos;
            }
            if (b.cnt == 0) continue;
            if (!rev) b.tape = 0;
            if (b.kmax > kmax) kmax = b.kmax;
            if (gen) gen_alone = (long)b.cnt * 16 >= (long)(p1 - p0) && b.cnt < p1 - p0;
            b.stream = !gen_alone ? nl % kStreams : (gen ? 0 : 1 + (nl - 1) % (kStreams - 1));
            // per-wavefront areas, then the partition sums; fewer wavefronts per
            // workgroup (each summing several partitions) when LDS is short. The
            // split path's pass workgroups are one wavefront with no partition
            // sums in LDS.
            b.wave_bytes =
                (fit_lds_bytes(mixed, rev, bin, plan.N, plan.D, b.slots, b.tape) + 15) &
                ~(size_t)15;
            const size_t cap = max_dyn_lds(ctx, gen);
            const int ks = gen ? b.kmax : bin;
            for (int g = 0; g < (b.kmax == 0 || split ? 1 : nseg); ++g) {
                const int sp = split ? 1 : seg[g].parts;
                const size_t part_bytes = sp > 1 ? (size_t)sp * sums_width(ks) * 8 : 0;
                int pw = sp;
                while (pw > 1 && pw * b.wave_bytes + part_bytes > cap) pw /= 2;
                b.pwaves[g] = pw;
                b.lds[g] = pw * b.wave_bytes + part_bytes;
                if (b.lds[g] > cap) return CO_ERR_BOUNDS;   // before any launch
            }
            lp[nl++] = b;
        }
        if (pos != p1) return CO_ERR_PROGRAM;   // descriptors out of launch order: never
        *nl_out = nl;
        *kmax_out = kmax;
        return CO_OK;
    }

    // Scratch of the whole fit: loop-state rows by expression, then the split
    // path's partition sums by launch position (null sc: the handle's buffer,
    // grown as needed; a fixed region that is too small refuses the fit).
    int set_scratch(int kmax, const Scratch *sc) {
        const int M = ctx->plan.M;
        int tail_parts = parts;
        const int tail_it = co_tail_resolve(&opt, ctx->plan.N, &tail_parts);
        const int stride = split ? kSplitStride : state_stride_for(kmax);
        pwidth = sums_width(kmax);
        const size_t state_bytes =
            (split || tail_it > 0) ? (((sizeof(double) * stride * (size_t)M) + 255) & ~(size_t)255)
                                   : 0;
        const size_t psum_bytes = split ? sizeof(double) * (size_t)parts * pwidth * M : 0;
        Scratch own;
        if (!sc) {
            if (state_bytes + psum_bytes) CO_GROW(ctx->state, state_bytes + psum_bytes);
            own.p = ctx->state.p;
            own.cap = ctx->state.cap;
            sc = &own;
        } else if (state_bytes + psum_bytes > sc->cap) {
            return CO_ERR_BOUNDS;   // a fixed region is never grown
        }
        fa.state = state_bytes ? (double *)sc->p : nullptr;
        fa.state_stride = stride;
        if (split) {
            fa.psum = (double *)((char *)sc->p + state_bytes);
            fa.psum_width = pwidth;
        }
        return CO_OK;
    }

    // After the first launch an error must not return with work still running
    // on the streams: they are joined first.
    int join_all() {
        for (int i = 0; i < kExtraStreams; ++i)
            if (lane_used[i]) (void)hipStreamSynchronize(ctx->lanes[i]);
        (void)hipStreamSynchronize(ctx->stream);
        return CO_OK;
    }
    int fail(hipError_t e, int line) {
        fprintf(stderr, "[cusr_co] HIP error %s at %s:%d\n", hipGetErrorString(e), __FILE__,
                line);
        join_all();
        return CO_ERR_CUDA;
    }

#define CO_LAUNCH_HIP(call)                              \
    do {                                                 \
        hipError_t e_ = (call);                          \
        if (e_ != hipSuccess) return fail(e_, __LINE__); \
    } while (0)

    // Issue the planned launches of one range (its inputs already on the device).
    int issue(const LaunchPlan *lp, int nl) {
        const hipStream_t s = ctx->stream;
        const int M = ctx->plan.M;
        if (range >= kMaxRanges) return CO_ERR_BOUNDS;   // never: at most kMaxRanges ranges
        if (!started) {
            CO_LAUNCH_HIP(hipEventRecord(ctx->ev_t0, s));
            if (split) {
                // every expression starts with a pass at c_init pending
                FitArgs fi = fa;
                lm_split_init_kernel<<<M, kLanes, 0, s>>>(fi);
                CO_LAUNCH_HIP(hipGetLastError());
            }
            CO_LAUNCH_HIP(hipEventRecord(ctx->ev_start, s));
            started = true;
        }
        // the split path's (pass, step) rounds: the pass at c_init, one per
        // iteration, two fp64 audit passes for mixed precision
        const int rounds = 1 + opt.max_iter + (mixed ? 2 : 0);
        for (int i = 0; i < nl; ++i) {
            const LaunchPlan &b = lp[i];
            hipStream_t ks = b.stream < kExtraStreams ? ctx->lanes[b.stream] : s;
            if (b.stream < kExtraStreams && !lane_used[b.stream]) {
                lane_used[b.stream] = true;
                CO_LAUNCH_HIP(hipStreamWaitEvent(ks, ctx->ev_start, 0));
            }
            CO_LAUNCH_HIP(hipEventRecord(ctx->ev_b0[range][b.bin], ks));
            if (split) {
                FitArgs fk = fa;
                fk.desc = fa.desc + b.pos;
                fk.psum = fa.psum + (size_t)b.pos * parts * pwidth;
                fk.slots = b.slots;
                fk.tape = b.tape;
                fk.parts = parts;
                fk.pwaves = 1;
                fk.wave_bytes = (int)b.wave_bytes;
                fk.it_end = opt.max_iter;
                fk.resume = 0;
                for (int r = 0; r < rounds; ++r) {
                    CO_LAUNCH_HIP(launch_pass(b.bin, (unsigned)b.cnt * parts, b.lds[0], ks, fk));
                    launch_step(b.bin, (unsigned)b.cnt, ks, fk, mixed ? 1 : 0);
                    CO_LAUNCH_HIP(hipGetLastError());
                }
            } else {
                // K = 0 expressions have no iterations, so no tail either
                for (int g = 0; g < (b.kmax == 0 ? 1 : nseg); ++g) {
                    FitArgs fk = fa;
                    fk.desc = fa.desc + b.pos;
                    fk.slots = b.slots;
                    fk.tape = b.tape;
                    fk.parts = seg[g].parts;
                    fk.pwaves = b.pwaves[g];
                    fk.wave_bytes = (int)b.wave_bytes;
                    fk.it_end = seg[g].it_end;
                    fk.resume = seg[g].resume;
                    CO_LAUNCH_HIP(launch(b.bin, (unsigned)b.cnt, b.lds[g], ks, fk));
                }
            }
            CO_LAUNCH_HIP(hipEventRecord(ctx->ev_b1[range][b.bin], ks));
            ctx->bin_launched[range][b.bin] = true;
        }
        ++range;
        return CO_OK;
    }

    // Join the streams, copy results to the host pointers that are non-null
    // (results otherwise stay on the device) and record the timings. Returns
    // after the device work and copies are complete.
    int finish(double *c_out, int32_t *status_out, double *li_out, double *lf_out,
               int32_t *iters_out) {
        const hipStream_t s = ctx->stream;
        const int M = ctx->plan.M, C = ctx->plan.total_c;
        for (int i = 0; i < kExtraStreams; ++i) {
            if (!lane_used[i]) continue;
            CO_LAUNCH_HIP(hipEventRecord(ctx->ev_done[i], ctx->lanes[i]));
            CO_LAUNCH_HIP(hipStreamWaitEvent(s, ctx->ev_done[i], 0));
        }
        CO_LAUNCH_HIP(hipEventRecord(ctx->ev_t1, s));
        // co_optimize_data_device: the outputs are device memory of the caller
        const hipMemcpyKind k = ctx->dev_io ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost;
        struct Out {
            void *dst;
            const void *src;
            size_t bytes;
        } outs[5] = {{c_out, ctx->C.p, c_out ? 8 * (size_t)C : 0},
                     {status_out, ctx->status.p, status_out ? 4 * (size_t)M : 0},
                     {li_out, ctx->li.p, li_out ? 8 * (size_t)M : 0},
                     {lf_out, ctx->lf.p, lf_out ? 8 * (size_t)M : 0},
                     {iters_out, ctx->iters.p, iters_out ? 4 * (size_t)M : 0}};
        const auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
        size_t total = 0;
        for (const Out &o : outs) total += up(o.bytes);
        if (!ctx->dev_io && total > 0 && total <= kPinnedStageMax) {
            // small results land in page-locked memory (DMA) and are copied
            // out on the host, as small inputs go in (upload_data)
            CO_GROW_HOST(ctx->h_back, total);
            size_t off = 0;
            for (const Out &o : outs) {
                if (o.bytes)
                    CO_HIP(hipMemcpyAsync(ctx->h_back.data() + off, o.src, o.bytes,
                                          hipMemcpyDeviceToHost, s));
                off += up(o.bytes);
            }
            CO_HIP(hipStreamSynchronize(s));
            off = 0;
            for (const Out &o : outs) {
                if (o.bytes) memcpy(o.dst, ctx->h_back.data() + off, o.bytes);
                off += up(o.bytes);
            }
        } else {
            for (const Out &o : outs)
                if (o.bytes) CO_HIP(hipMemcpyAsync(o.dst, o.src, o.bytes, k, s));
            CO_HIP(hipStreamSynchronize(s));
        }
        float ms = 0.0f;
        CO_HIP(hipEventElapsedTime(&ms, ctx->ev_t0, ctx->ev_t1));
        ctx->last_kernel_ms = ms;
        for (int k = 0; k < CO_BINS; ++k) {
            double sum = -1.0;
            for (int r = 0; r < kMaxRanges; ++r) {
                if (!ctx->bin_launched[r][k]) continue;
                CO_HIP(hipEventElapsedTime(&ms, ctx->ev_b0[r][k], ctx->ev_b1[r][k]));
                sum = (sum < 0.0 ? 0.0 : sum) + ms;
            }
            ctx->last_bin_ms[k] = sum;
        }
        return CO_OK;
    }
#undef CO_LAUNCH_HIP
};

// Fit the resident population; copy results to the host pointers that are
// non-null (c_out and status_out too may be null: results then stay on the
// device). sc: where the fit's scratch goes (null: the handle's buffer, grown
// as needed; a fixed region is never grown, and a fit that needs more is
// refused with CO_ERR_BOUNDS before anything is launched). Every range's
// launches are planned before the first is issued. Returns after the device
// work and copies are complete.
int run_fit(Ctx *ctx, const CoOptions &opt, double *c_out, int32_t *status_out, double *li_out,
            double *lf_out, int32_t *iters_out, const Scratch *sc = nullptr) {
    if (!ctx->resident) return CO_ERR_NULLARG;
    FitRun fr;
    int rc = fr.begin(ctx, opt);
    if (rc != CO_OK) return rc;
    if (ctx->plan.M == 0) return CO_OK;
    const int nr = (int)ctx->ranges.size() - 1;
    std::vector<LaunchPlan> lp((size_t)nr * CO_BINS);
    std::vector<int> nl(nr, 0);
    int kmax = 0;
    for (int r = 0; r < nr; ++r) {
        int km = 0;
        rc = fr.plan_range(ctx->ranges[r], ctx->ranges[r + 1], lp.data() + (size_t)r * CO_BINS,
                           &nl[r], &km);
        if (rc != CO_OK) return rc;
        if (km > kmax) kmax = km;
    }
    rc = fr.set_scratch(kmax, sc);
    if (rc != CO_OK) return rc;
    for (int r = 0; r < nr; ++r) {
        rc = fr.issue(lp.data() + (size_t)r * CO_BINS, nl[r]);
        if (rc != CO_OK) return rc;
    }
    return fr.finish(c_out, status_out, li_out, lf_out, iters_out);
}

// A population uploaded from host buffers of at least 2 kPipeMinRange
// expressions is decoded, uploaded and launched in two ranges: the first, an
// eighth of the population (at least kPipeMinRange expressions), is decoded
// alone, and while the device fits it the host decodes the rest. (The host
// decode of C5's 65,536 expressions, 1.7 M nodes, takes about 5 ms of a 41 ms
// round. Measured on an MI355X, C5 rounds: one piece 41.1 ms, two ranges
// 38.1 ms, three growing ranges 38.2 ms, four equal ranges 38.6 ms, eight
// 40.5 ms: each range's bins are launches of their own, and more of them
// lengthen the fit's tail.)
constexpr int kPipeMinRange = 8192;

// Ranges a co_optimize of this population is decoded in (1: one piece).
int pipe_ranges(const CoOptions &opt, const PopHeader *h) {
    if (!h || h->M_prob < 2 * kPipeMinRange) return 1;
    const int parts = co_partitions_resolve(&opt, h->N);
    int tail_parts = parts;
    // the split path and the tail segments size their scratch over the whole
    // population: those fits take the one-piece path
    if (parts == 0 || parts > CO_MAX_PARTITIONS || co_tail_resolve(&opt, h->N, &tail_parts) > 0)
        return 1;
    return 2;
}

// End of range j of the nr ranges of M expressions.
int range_end(int M, int j, int nr) {
    if (j + 1 >= nr) return M;
    return M / 8 > kPipeMinRange ? M / 8 : kPipeMinRange;
}

// co_optimize in ranges: X, y and c_init go over first, then each range is
// decoded, copied (on the handle's copy stream, waited for by the host) and
// launched while the host decodes the next. Same checks, results and
// error codes as upload_population + run_fit; a range that fails to decode
// after earlier ones were launched returns its code once they are done, with
// no output written. setup_ms: host time to the first launch.
int fit_pipelined(Ctx *ctx, const CoOptions &opt, const PopHeader *h, const int32_t *nt,
                  const float *nv, const int32_t *ci, const TreeMeta *metas, const void *c,
                  const void *xs, const void *ym, bool in32, double *c_out, int32_t *status_out,
                  double *li_out, double *lf_out, int32_t *iters_out, bool on_data, int nr,
                  double t0, double *setup_ms) {
    CO_HIP(hipSetDevice(ctx->device));
    ctx->resident = false;
    int rc = check_header(h, nt, nv, ci, metas);
    if (rc != CO_OK) return rc;
    if (on_data && (ctx->data_N < 0 || h->N != ctx->data_N || h->n_vars != ctx->data_D))
        return CO_ERR_DATA;
    const int M = h->M_prob;
    const bool shared_y = on_data || (pop_flags(h) & POP_FLAG_SHARED_Y) != 0;
    CO_GROW_HOST(ctx->h_prog, h->total_nodes > 0 ? 2 * (size_t)h->total_nodes : 1);
    CO_GROW_HOST(ctx->h_desc, (size_t)M);
    rc = grow_buffers(ctx, h, h->total_nodes > 0 ? 2 * (size_t)h->total_nodes : 1, in32, on_data,
                      shared_y);
    if (rc != CO_OK) return rc;
    ctx->on_data = on_data;
    ctx->shared_y = shared_y;
    Plan &pl = ctx->plan;
    pl = Plan{};
    pl.M = M;
    pl.N = h->N;
    pl.D = h->n_vars;
    pl.total_nodes = h->total_nodes;
    pl.total_c = h->total_c;
    FitRun fr;
#ifdef CUSR_EXP_TIMING
    const double u0 = now_ms();
#endif
    rc = fr.begin(ctx, opt);
    if (rc != CO_OK) return rc;
    const hipStream_t cs = ctx->copy_stream;
#ifdef CUSR_EXP_TIMING
    const double u1 = now_ms();
#endif
    rc = upload_data(ctx, h, c, xs, ym, in32, on_data, shared_y, cs);
    if (rc != CO_OK) {
        (void)hipStreamSynchronize(cs);
        return rc;
    }
#ifdef CUSR_EXP_TIMING
    fprintf(stderr, "[pipe] checks+grow %.2f begin %.2f upload %.2f ms\n", u0 - t0, u1 - u0,
            now_ms() - u1);
#endif
    ctx->ranges.assign(1, 0);
    int64_t wb = 0;
    for (int j = 0; j < nr; ++j) {
        const int m0 = j == 0 ? 0 : range_end(M, j - 1, nr), m1 = range_end(M, j, nr);
        Plan rp = {};
#ifdef CUSR_EXP_TIMING
        const double q0 = now_ms();
#endif
        rc = decode_range(h, nt, nv, ci, metas, m0, m1, wb, ctx->h_prog.data(),
                          ctx->h_desc.data(), &rp);
#ifdef CUSR_EXP_TIMING
        const double q1 = now_ms();
#endif
        LaunchPlan lp[CO_BINS];
        int nl = 0, km = 0;
        if (rc == CO_OK) rc = fr.plan_range(m0, m1, lp, &nl, &km);
        hipError_t e = hipSuccess;
        if (rc == CO_OK && rp.words)
            e = hipMemcpyAsync((char *)ctx->prog.p + sizeof(uint64_t) * wb, ctx->h_prog.data() + wb,
                               sizeof(uint64_t) * rp.words, hipMemcpyHostToDevice, cs);
        if (rc == CO_OK && e == hipSuccess)
            e = hipMemcpyAsync((char *)ctx->desc.p + sizeof(ExprDesc) * m0, ctx->h_desc.data() + m0,
                               sizeof(ExprDesc) * (m1 - m0), hipMemcpyHostToDevice, cs);
        // the host waits for the range's copies (tens of microseconds): an event
        // the streams waited on would be signalled through a hardware queue
        // that a fitting stream shares, after that stream's earlier kernels
        if (rc == CO_OK && e == hipSuccess) e = hipStreamSynchronize(cs);
        if (e != hipSuccess) {
            fprintf(stderr, "[cusr_co] HIP error %s at %s:%d\n", hipGetErrorString(e), __FILE__,
                    __LINE__);
            rc = CO_ERR_CUDA;
        }
        if (rc != CO_OK) {
            fr.join_all();
            (void)hipStreamSynchronize(cs);
            return rc;
        }
#ifdef CUSR_EXP_TIMING
        const double q2 = now_ms();
#endif
        rc = fr.issue(lp, nl);
#ifdef CUSR_EXP_TIMING
        fprintf(stderr, "[pipe] range %d at %.2f: decode %.2f copies %.2f issue %.2f ms\n", j,
                q0 - t0, q1 - q0, q2 - q1, now_ms() - q2);
#endif
        if (rc != CO_OK) {
            (void)hipStreamSynchronize(cs);
            return rc;
        }
        if (j == 0) *setup_ms = now_ms() - t0;
        wb += rp.words;
        pl.n_gen += rp.n_gen;
        if (rp.max_tape > pl.max_tape) pl.max_tape = rp.max_tape;
        if (rp.max_n > pl.max_n) pl.max_n = rp.max_n;
        if (rp.max_slots > pl.max_slots) pl.max_slots = rp.max_slots;
        ctx->ranges.push_back(m1);
    }
    pl.words = wb;
    rc = fr.finish(c_out, status_out, li_out, lf_out, iters_out);
    CO_HIP(hipStreamSynchronize(cs));
    if (rc == CO_OK) ctx->resident = true;
    return rc;
}

// Shared body of co_optimize / co_optimize_ex: upload, fit, read back.
int fit_common(Ctx *ctx, const CoOptions &opt, const PopHeader *h, const int32_t *nt,
               const float *nv, const int32_t *ci, const TreeMeta *metas, const void *c,
               const void *xs, const void *ym, bool in32, double *c_out, int32_t *status_out,
               double *li_out, double *lf_out, int32_t *iters_out, bool on_data = false) {
    const double t0 = now_ms();
    if (opt.ad_mode != CO_AD_FORWARD && opt.ad_mode != CO_AD_REVERSE) return CO_ERR_NULLARG;
    if (opt.precision != CO_PREC_FP64 && opt.precision != CO_PREC_MIXED) return CO_ERR_NULLARG;
    if (opt.max_iter < 0) return CO_ERR_NULLARG;
    if (opt.lm_order != CO_ORDER_IMPROVE_FIRST && opt.lm_order != CO_ORDER_CONVERGE_FIRST)
        return CO_ERR_NULLARG;
    if (opt.damping < CO_DAMP_RELATIVE || opt.damping > CO_DAMP_PIVOT_FLOOR)
        return CO_ERR_NULLARG;
    const int nr = pipe_ranges(opt, h);
    if (nr > 1) {
        double setup = 0.0;
        const int rc = fit_pipelined(ctx, opt, h, nt, nv, ci, metas, c, xs, ym, in32, c_out,
                                     status_out, li_out, lf_out, iters_out, on_data, nr, t0,
                                     &setup);
        g_setup_ms = setup;
        g_loop_ms = now_ms() - t0 - setup;
        return rc;
    }
    int rc = upload_population(ctx, h, nt, nv, ci, metas, c, xs, ym, in32, on_data);
    if (rc != CO_OK) return rc;
    const double t1 = now_ms();
    rc = run_fit(ctx, opt, c_out, status_out, li_out, lf_out, iters_out);
    g_setup_ms = t1 - t0;
    g_loop_ms = now_ms() - t1;
    return rc;
}

}  // namespace

extern "C" void co_options_default(CoOptions *o) {
    if (!o) return;
    memset(o, 0, sizeof(*o));
    o->struct_size = (int32_t)sizeof(CoOptions);
    o->ad_mode = CO_AD_FORWARD;
    o->precision = CO_PREC_FP64;
    o->max_iter = 50;
    o->lambda0 = 1e-3;
    o->xtol = 1e-6;
    o->fp64_guard = 1;
    o->lm_order = CUSR_DEFAULT_ORDER;
    o->tail_iter = 0;         // co_tail_iter_for
    o->tail_partitions = 0;   // CO_MAX_PARTITIONS
}

extern "C" int co_init(int device_id, void **handle_out) {
    if (!handle_out) return CO_ERR_NULLARG;
    *handle_out = nullptr;
    CO_HIP(hipSetDevice(device_id));
    CO_HIP(hipFree(nullptr));  // create the device context now, once
    Ctx *ctx = new (std::nothrow) Ctx();
    if (!ctx) return CO_ERR_OOM;
    ctx->device = device_id;
    {
        // this device's address of the static scratch array, once per device
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (device_id >= 0 && device_id < kMaxDevices) {
            if (!g_scratch_ptr[device_id]) {
                void *p = nullptr;
                const hipError_t es = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
                if (es != hipSuccess) {
                    fprintf(stderr, "[cusr_co] hipGetSymbolAddress(scratch): %s\n",
                            hipGetErrorString(es));
                    delete ctx;
                    return CO_ERR_CUDA;
                }
                g_scratch_ptr[device_id] = p;
            }
            ctx->static_scratch = g_scratch_ptr[device_id];
        }
    }
    int lds_per_block = 0;
    hipError_t e = hipDeviceGetAttribute(&lds_per_block, hipDeviceAttributeMaxSharedMemoryPerBlock,
                                         device_id);
    if (e == hipSuccess)
        ctx->lds_per_block = lds_per_block > 0 ? (size_t)lds_per_block : 0;
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    for (int i = 0; i < kExtraStreams && e == hipSuccess; ++i)
        e = hipStreamCreateWithFlags(&ctx->lanes[i], hipStreamNonBlocking);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->copy_stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->ev_start, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreate(&ctx->ev_t0);
    if (e == hipSuccess) e = hipEventCreate(&ctx->ev_t1);
    for (int k = 0; k < CO_BINS && e == hipSuccess; ++k) {
        for (int r = 0; r < kMaxRanges && e == hipSuccess; ++r) {
            e = hipEventCreate(&ctx->ev_b0[r][k]);
            if (e == hipSuccess) e = hipEventCreate(&ctx->ev_b1[r][k]);
        }
    }
    for (int i = 0; i < kExtraStreams && e == hipSuccess; ++i)
        e = hipEventCreateWithFlags(&ctx->ev_done[i], hipEventDisableTiming);
    if (e != hipSuccess) {
        fprintf(stderr, "[cusr_co] stream/event create: %s\n", hipGetErrorString(e));
        co_teardown(ctx);
        return CO_ERR_CUDA;
    }
    *handle_out = ctx;
    return CO_OK;
}

extern "C" int co_optimize(void *handle, const PopHeader *h, const int32_t *nt, const float *nv,
                           const int32_t *ci, const TreeMeta *metas, const float *c_init,
                           const float *xs, const float *ym, int max_iter, float *c_final_out,
                           int32_t *status_out, float *loss_init_out, float *loss_final_out) {
    if (!handle || !h || !nt || !nv || !ci || !metas || !c_init || !xs || !ym || !c_final_out ||
        !status_out)
        return CO_ERR_NULLARG;
    Ctx *ctx = (Ctx *)handle;
    CoOptions opt;
    co_options_default(&opt);
    opt.max_iter = max_iter;
    opt.f32_range = 1;   // the reference fits in fp32: no constant beyond its range
    const int M = h->M_prob > 0 ? h->M_prob : 0;
    const int C = h->total_c > 0 ? h->total_c : 0;
    ctx->h_c.resize(C > 0 ? C : 1);
    ctx->h_li.resize(M > 0 ? M : 1);
    ctx->h_lf.resize(M > 0 ? M : 1);
    int rc = fit_common(ctx, opt, h, nt, nv, ci, metas, c_init, xs, ym, true, ctx->h_c.data(),
                        status_out, ctx->h_li.data(), ctx->h_lf.data(), nullptr);
    if (rc != CO_OK) return rc;
    ctx->h_c0.resize(C > 0 ? C : 1);
    for (int j = 0; j < C; j++) ctx->h_c0[j] = c_init[j];
    ctx->h_li32.resize(M > 0 ? M : 1);
    ctx->h_lf32.resize(M > 0 ? M : 1);
    rc = co_narrow_fp32(h, metas, ctx->h_c0.data(), ctx->h_c.data(), ctx->h_li.data(),
                        ctx->h_lf.data(), status_out, c_final_out, ctx->h_li32.data(),
                        ctx->h_lf32.data());
    if (rc < 0) return rc;
    for (int m = 0; m < M; m++) {
        if (loss_init_out) loss_init_out[m] = ctx->h_li32[m];
        if (loss_final_out) loss_final_out[m] = ctx->h_lf32[m];
    }
    return CO_OK;
}

extern "C" int co_narrow_fp32(const PopHeader *h, const TreeMeta *metas, const double *c_init,
                              const double *c_final, const double *loss_init,
                              const double *loss_final, int32_t *status, float *c_out,
                              float *loss_init_out, float *loss_final_out) {
    if (!h || h->M_prob < 0 || h->total_c < 0) return CO_ERR_NULLARG;
    const int M = h->M_prob, C = h->total_c;
    if ((M > 0 && (!metas || !loss_init || !loss_final || !status || !loss_init_out ||
                   !loss_final_out)) ||
        (C > 0 && (!c_init || !c_final || !c_out)))
        return CO_ERR_NULLARG;
    for (int m = 0; m < M; m++) {
        const TreeMeta &t = metas[m];
        if (t.K < 0 || t.c_offset < 0 || (long)t.c_offset + t.K > (long)C) return CO_ERR_PROGRAM;
    }
    for (int j = 0; j < C; j++) c_out[j] = (float)c_final[j];
    int demoted = 0;
    for (int m = 0; m < M; m++) {
        const TreeMeta &t = metas[m];
        const float lf = (float)loss_final[m];
        loss_init_out[m] = (float)loss_init[m];
        loss_final_out[m] = lf;
        if (t.K == 0) continue;
        // a value the fp64 fit left finite that the fp32 carrier cannot hold
        bool lost = std::isfinite(loss_final[m]) && !std::isfinite(lf);
        for (int j = 0; j < t.K && !lost; j++) {
            const double v = c_final[t.c_offset + j];
            lost = std::isfinite(v) && !std::isfinite((float)v);
        }
        if (!lost) continue;
        // as the fp64 guard treats a non-finite loss (lm_core.cuh:299-351)
        for (int j = 0; j < t.K; j++) c_out[t.c_offset + j] = (float)c_init[t.c_offset + j];
        loss_final_out[m] = (float)loss_init[m];
        if (status[m] == STATUS_CONVERGED) status[m] = STATUS_MAXITER;
        ++demoted;
    }
    return demoted;
}

extern "C" int co_optimize_ex(void *handle, const CoOptions *opt, const PopHeader *h,
                              const int32_t *nt, const float *nv, const int32_t *ci,
                              const TreeMeta *metas, const double *c, const double *xs,
                              const double *ym, double *c_final_out, int32_t *status_out,
                              double *loss_init_out, double *loss_final_out,
                              int32_t *iters_out) {
    if (!handle || !opt || !h || !nt || !nv || !ci || !metas || !c || !xs || !ym ||
        !c_final_out || !status_out)
        return CO_ERR_NULLARG;
    if (opt->struct_size != (int32_t)sizeof(CoOptions)) return CO_ERR_NULLARG;
    return fit_common((Ctx *)handle, *opt, h, nt, nv, ci, metas, c, xs, ym, false, c_final_out,
                      status_out, loss_init_out, loss_final_out, iters_out);
}

extern "C" int co_data_upload(void *handle, int N, int n_vars, const double *xs,
                              const double *y) {
    if (!handle || N < 0 || n_vars < 0 || n_vars > CO_MAX_VARS) return CO_ERR_NULLARG;
    if (N > 0 && (!y || (n_vars > 0 && !xs))) return CO_ERR_NULLARG;
    Ctx *ctx = (Ctx *)handle;
    CO_HIP(hipSetDevice(ctx->device));
    ctx->data_N = -1;   // no data set until this upload completes
    if (ctx->on_data) ctx->resident = false;
    const size_t nX = (size_t)N * n_vars;
    CO_GROW(ctx->data_X, sizeof(double) * nX);
    CO_GROW(ctx->data_Y, sizeof(double) * N);
    CO_GROW(ctx->stage, sizeof(double) * nX);
    hipStream_t s = ctx->stream;
    if (nX) {
        CO_HIP(hipMemcpyAsync(ctx->stage.p, xs, 8 * nX, hipMemcpyHostToDevice, s));
        transpose_x_kernel<double><<<blocks_for(nX, 256), 256, 0, s>>>(
            ptr<double>(ctx->stage), ptr<double>(ctx->data_X), N, n_vars);
        CO_HIP(hipGetLastError());
    }
    if (N) CO_HIP(hipMemcpyAsync(ctx->data_Y.p, y, 8 * (size_t)N, hipMemcpyHostToDevice, s));
    CO_HIP(hipStreamSynchronize(s));
    ctx->data_N = N;
    ctx->data_D = n_vars;
    return CO_OK;
}

// True when [p, p + bytes) is device memory of the handle's device, inside one
// allocation (a torch CUDA tensor's storage on that device, for instance).
static bool on_device(const void *p, size_t bytes, int device) {
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();   // a pageable host pointer is not an error to keep
        return false;
    }
    if (a.type != hipMemoryTypeDevice || a.device != device) return false;
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    const uintptr_t lo = (uintptr_t)base, at = (uintptr_t)p;
    return at >= lo && bytes <= size && at - lo <= size - bytes;
}

extern "C" int co_data_upload_device(void *handle, int N, int n_vars, const double *xs_dev,
                                     const double *y_dev) {
    if (!handle || N < 0 || n_vars < 0 || n_vars > CO_MAX_VARS) return CO_ERR_NULLARG;
    if (N > 0 && (!y_dev || (n_vars > 0 && !xs_dev))) return CO_ERR_NULLARG;
    Ctx *ctx = (Ctx *)handle;
    CO_HIP(hipSetDevice(ctx->device));
    // every pointer and extent checked before anything is copied
    if (N > 0 && (!on_device(y_dev, sizeof(double) * (size_t)N, ctx->device) ||
                  (n_vars > 0 && !on_device(xs_dev, sizeof(double) * (size_t)N * n_vars,
                                            ctx->device))))
        return CO_ERR_DATA;
    // the caller's producer of xs_dev / y_dev may still be queued on a stream
    // of its own: every stream of the process drains before the library's
    // non-blocking streams read that memory
    CO_HIP(hipDeviceSynchronize());
    ctx->data_N = -1;   // no data set until this upload completes
    if (ctx->on_data) ctx->resident = false;
    const size_t nX = (size_t)N * n_vars;
    CO_GROW(ctx->data_X, sizeof(double) * nX);
    CO_GROW(ctx->data_Y, sizeof(double) * N);
    hipStream_t s = ctx->stream;
    if (nX) {
        // row-major [N][D] straight from the caller's memory to column-major
        transpose_x_kernel<double><<<blocks_for(nX, 256), 256, 0, s>>>(
            xs_dev, ptr<double>(ctx->data_X), N, n_vars);
        CO_HIP(hipGetLastError());
    }
    if (N)
        CO_HIP(hipMemcpyAsync(ctx->data_Y.p, y_dev, 8 * (size_t)N, hipMemcpyDeviceToDevice, s));
    CO_HIP(hipStreamSynchronize(s));
    ctx->data_N = N;
    ctx->data_D = n_vars;
    return CO_OK;
}

extern "C" int co_optimize_data(void *handle, const CoOptions *opt, const PopHeader *h,
                                const int32_t *nt, const float *nv, const int32_t *ci,
                                const TreeMeta *metas, const double *c, double *c_final_out,
                                int32_t *status_out, double *loss_init_out,
                                double *loss_final_out, int32_t *iters_out) {
    if (!handle || !opt || !h || !nt || !nv || !ci || !metas || !c || !c_final_out ||
        !status_out)
        return CO_ERR_NULLARG;
    if (opt->struct_size != (int32_t)sizeof(CoOptions)) return CO_ERR_NULLARG;
    return fit_common((Ctx *)handle, *opt, h, nt, nv, ci, metas, c, nullptr, nullptr, false,
                      c_final_out, status_out, loss_init_out, loss_final_out, iters_out, true);
}

extern "C" int co_optimize_data_device(void *handle, const CoOptions *opt, const PopHeader *h,
                                       const int32_t *nt, const float *nv, const int32_t *ci,
                                       const TreeMeta *metas, const double *c_dev,
                                       double *c_final_dev, int32_t *status_dev,
                                       double *loss_init_dev, double *loss_final_dev,
                                       int32_t *iters_dev) {
    if (!handle || !opt || !h || !nt || !nv || !ci || !metas) return CO_ERR_NULLARG;
    if (opt->struct_size != (int32_t)sizeof(CoOptions)) return CO_ERR_NULLARG;
    Ctx *ctx = (Ctx *)handle;
    const int M = h->M_prob, C = h->total_c;
    if (M < 0 || C < 0) return CO_ERR_NULLARG;
    if ((C > 0 && (!c_dev || !c_final_dev)) || (M > 0 && !status_dev)) return CO_ERR_NULLARG;
    CO_HIP(hipSetDevice(ctx->device));
    // every pointer that is given must be device memory of this handle's
    // device covering its extent, checked before anything is copied
    const size_t cb = sizeof(double) * (size_t)C, mb = sizeof(double) * (size_t)M,
                 ib = sizeof(int32_t) * (size_t)M;
    if ((C > 0 && (!on_device(c_dev, cb, ctx->device) || !on_device(c_final_dev, cb, ctx->device))) ||
        (M > 0 && !on_device(status_dev, ib, ctx->device)) ||
        (M > 0 && loss_init_dev && !on_device(loss_init_dev, mb, ctx->device)) ||
        (M > 0 && loss_final_dev && !on_device(loss_final_dev, mb, ctx->device)) ||
        (M > 0 && iters_dev && !on_device(iters_dev, ib, ctx->device)))
        return CO_ERR_DATA;
    // c_dev's producer, and earlier users of the output buffers, may still be
    // queued on the caller's streams: they finish before the library's
    // non-blocking streams read or write that memory
    CO_HIP(hipDeviceSynchronize());
    ctx->dev_io = true;
    const int rc = fit_common(ctx, *opt, h, nt, nv, ci, metas, c_dev, nullptr, nullptr, false,
                              c_final_dev, status_dev, loss_init_dev, loss_final_dev, iters_dev,
                              true);
    ctx->dev_io = false;
    return rc;
}

extern "C" int co_eval_ex(void *handle, const PopHeader *h, const int32_t *nt, const float *nv,
                          const int32_t *ci, const TreeMeta *metas, const double *c,
                          const double *xs, int precision, double *y_out) {
    if (!handle || !h || !nt || !nv || !ci || !metas || !c || !xs || !y_out)
        return CO_ERR_NULLARG;
    if (precision != CO_PREC_FP64 && precision != CO_PREC_MIXED) return CO_ERR_NULLARG;
    Ctx *ctx = (Ctx *)handle;
    CO_HIP(hipSetDevice(ctx->device));
    ctx->resident = false;  // the evaluation reuses the population buffers
    const int M = h->M_prob;
    CO_GROW_HOST(ctx->h_prog, h->total_nodes > 0 ? 2 * (size_t)h->total_nodes : 1);
    CO_GROW_HOST(ctx->h_desc, M > 0 ? (size_t)M : 1);
    Plan plan = {};
    int rc = decode_population(h, nt, nv, ci, metas, ctx->h_prog.data(), nullptr, nullptr,
                               ctx->h_desc.data(), nullptr, nullptr, nullptr, nullptr, &plan);
    if (rc != CO_OK || M == 0) return rc;
    const int N = h->N, D = h->n_vars, C = h->total_c;
    const size_t nX = (size_t)N * D, nY = (size_t)M * N, words = (size_t)plan.words;
    // one workgroup per expression: inputs and spill slots of 64 points in LDS
    const size_t lds = (size_t)(D + plan.max_slots) * kLanes * (precision == CO_PREC_FP64 ? 8 : 4);
    if (lds + sizeof(double) * CO_MAX_K > ctx->lds_per_block) return CO_ERR_BOUNDS;
    CO_GROW(ctx->prog, sizeof(uint64_t) * words);
    CO_GROW(ctx->desc, sizeof(ExprDesc) * M);
    CO_GROW(ctx->X, sizeof(double) * nX);
    CO_GROW(ctx->Y, sizeof(double) * nY);
    CO_GROW(ctx->C0, sizeof(double) * C);
    CO_GROW(ctx->stage, sizeof(double) * nX);
    hipStream_t s = ctx->stream;
    if (words)
        CO_HIP(hipMemcpyAsync(ctx->prog.p, ctx->h_prog.data(), sizeof(uint64_t) * words,
                              hipMemcpyHostToDevice, s));
    CO_HIP(hipMemcpyAsync(ctx->desc.p, ctx->h_desc.data(), sizeof(ExprDesc) * M,
                          hipMemcpyHostToDevice, s));
    if (C) CO_HIP(hipMemcpyAsync(ctx->C0.p, c, 8 * (size_t)C, hipMemcpyHostToDevice, s));
    if (nX) {
        CO_HIP(hipMemcpyAsync(ctx->stage.p, xs, 8 * nX, hipMemcpyHostToDevice, s));
        transpose_x_kernel<double><<<blocks_for(nX, 256), 256, 0, s>>>(
            ptr<double>(ctx->stage), ptr<double>(ctx->X), N, D);
        CO_HIP(hipGetLastError());
    }
    EvalArgs ea;
    ea.prog = ptr<uint64_t>(ctx->prog);
    ea.X = ptr<double>(ctx->X);
    ea.C = ptr<double>(ctx->C0);
    ea.Yout = ptr<double>(ctx->Y);
    ea.N = N;
    ea.D = D;
    // descriptors in launch order: the wide programs first, then the fast ones
    const int ng = plan.n_gen, nf = M - plan.n_gen;
    ea.desc = ptr<ExprDesc>(ctx->desc);
    if (ng) {
        if (precision == CO_PREC_FP64)
            eval_kernel<double, WideFmt><<<ng, kLanes, lds, s>>>(ea);
        else
            eval_kernel<float, WideFmt><<<ng, kLanes, lds, s>>>(ea);
        CO_HIP(hipGetLastError());
    }
    ea.desc = ptr<ExprDesc>(ctx->desc) + ng;
    if (nf) {
        if (precision == CO_PREC_FP64)
            eval_kernel<double, FastFmt><<<nf, kLanes, lds, s>>>(ea);
        else
            eval_kernel<float, FastFmt><<<nf, kLanes, lds, s>>>(ea);
        CO_HIP(hipGetLastError());
    }
    if (nY) CO_HIP(hipMemcpyAsync(y_out, ctx->Y.p, 8 * nY, hipMemcpyDeviceToHost, s));
    CO_HIP(hipStreamSynchronize(s));
    return CO_OK;
}

extern "C" int co_decode(const PopHeader *h, const int32_t *nt, const float *nv,
                         const int32_t *ci, const TreeMeta *metas, uint64_t *program_out,
                         int32_t *order_out, int32_t *bin_start_out, int32_t *stack_out,
                         int32_t *program_off_out, int32_t *route_out) {
    if (!h) return CO_ERR_NULLARG;
    std::vector<uint64_t> tmp;
    uint64_t *prog = program_out;
    if (!prog) {
        tmp.resize(h->total_nodes > 0 ? 2 * (size_t)h->total_nodes : 1);
        prog = tmp.data();
    }
    return decode_population(h, nt, nv, ci, metas, prog, order_out, bin_start_out, nullptr,
                             stack_out, nullptr, program_off_out, route_out, nullptr);
}

extern "C" int co_upload_ex(void *handle, const PopHeader *h, const int32_t *nt,
                            const float *nv, const int32_t *ci, const TreeMeta *metas,
                            const double *c, const double *xs, const double *ym) {
    if (!handle || !h || !nt || !nv || !ci || !metas || !c || !xs || !ym) return CO_ERR_NULLARG;
    return upload_population((Ctx *)handle, h, nt, nv, ci, metas, c, xs, ym, false);
}

extern "C" int co_fit_resident(void *handle, const CoOptions *opt, double *c_final_out,
                               int32_t *status_out, double *loss_init_out,
                               double *loss_final_out, int32_t *iters_out) {
    if (!handle || !opt || opt->struct_size != (int32_t)sizeof(CoOptions)) return CO_ERR_NULLARG;
    const double t0 = now_ms();
    int rc = run_fit((Ctx *)handle, *opt, c_final_out, status_out, loss_init_out, loss_final_out,
                     iters_out);
    g_setup_ms = 0.0;
    g_loop_ms = now_ms() - t0;
    return rc;
}

extern "C" int co_fit_resident_static(void *handle, const CoOptions *opt, double *c_final_out,
                                      int32_t *status_out, double *loss_init_out,
                                      double *loss_final_out, int32_t *iters_out) {
    if (!handle || !opt || opt->struct_size != (int32_t)sizeof(CoOptions)) return CO_ERR_NULLARG;
    Ctx *ctx = (Ctx *)handle;
    if (!ctx->static_scratch) return CO_ERR_CUDA;   // device id beyond kMaxDevices
    Scratch sc;
    sc.p = ctx->static_scratch;
    sc.cap = CO_STATIC_SCRATCH_BYTES;
    sc.fixed = true;
    const double t0 = now_ms();
    int rc = run_fit(ctx, *opt, c_final_out, status_out, loss_init_out, loss_final_out,
                     iters_out, &sc);
    g_setup_ms = 0.0;
    g_loop_ms = now_ms() - t0;
    return rc;
}

extern "C" int co_last_kernel_ms(void *handle, double *fit_ms_out) {
    if (!handle || !fit_ms_out) return CO_ERR_NULLARG;
    *fit_ms_out = ((Ctx *)handle)->last_kernel_ms;
    return CO_OK;
}

extern "C" int co_last_bin_ms(void *handle, double *bin_ms_out) {
    if (!handle || !bin_ms_out) return CO_ERR_NULLARG;
    const Ctx *ctx = (const Ctx *)handle;
    for (int k = 0; k < CO_BINS; ++k) bin_ms_out[k] = ctx->last_bin_ms[k];
    return CO_OK;
}

extern "C" int co_last_split(double *setup_ms_out, double *loop_ms_out) {
    if (setup_ms_out) *setup_ms_out = g_setup_ms;
    if (loop_ms_out) *loop_ms_out = g_loop_ms;
    return 0;
}

extern "C" void co_teardown(void *handle) {
    if (!handle) return;
    Ctx *ctx = (Ctx *)handle;
    (void)hipSetDevice(ctx->device);
    DevBuf *bufs[] = {&ctx->prog, &ctx->desc, &ctx->X, &ctx->Y, &ctx->C0, &ctx->C,
                      &ctx->status, &ctx->li, &ctx->lf, &ctx->iters, &ctx->stage,
                      &ctx->data_X, &ctx->data_Y, &ctx->state};
    for (DevBuf *b : bufs)
        if (b->p) (void)hipFree(b->p);
    if (ctx->h_prog.p) (void)hipHostFree(ctx->h_prog.p);
    if (ctx->h_desc.p) (void)hipHostFree(ctx->h_desc.p);
    if (ctx->h_stage.p) (void)hipHostFree(ctx->h_stage.p);
    if (ctx->h_back.p) (void)hipHostFree(ctx->h_back.p);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    if (ctx->copy_stream) (void)hipStreamDestroy(ctx->copy_stream);
    for (int i = 0; i < kExtraStreams; ++i) {
        if (ctx->lanes[i]) (void)hipStreamDestroy(ctx->lanes[i]);
        if (ctx->ev_done[i]) (void)hipEventDestroy(ctx->ev_done[i]);
    }
    if (ctx->ev_start) (void)hipEventDestroy(ctx->ev_start);
    if (ctx->ev_t0) (void)hipEventDestroy(ctx->ev_t0);
    if (ctx->ev_t1) (void)hipEventDestroy(ctx->ev_t1);
    for (int k = 0; k < CO_BINS; ++k) {
        for (int r = 0; r < kMaxRanges; ++r) {
            if (ctx->ev_b0[r][k]) (void)hipEventDestroy(ctx->ev_b0[r][k]);
            if (ctx->ev_b1[r][k]) (void)hipEventDestroy(ctx->ev_b1[r][k]);
        }
    }
    delete ctx;
}
