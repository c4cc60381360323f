// batch_lm_main.cpp -- command-line front end with the reference CLI contract
// (cusr/kernel/batch_lm_ad.cu:196-551):
//
//   batch_lm_ad <pop.bin> [out_dir] [--max-iter N] [--quiet] [--rev] [--mixed]
//               [--trust-region | --pivot-floor] [--profile]
//
// Reads pop.bin v1 and the v2 extension (float64 payloads, shared target;
// include/pop_format.h).
// writes out_dir/{status.bin, c_final.bin, loss_init.bin, loss_final.bin}
// (int32 / float32 blobs, batch_lm_ad.cu:526-536) and prints the completion
// line the reference benchmark parses (cusr/benchmark/backends.py:745):
//   [batch-lm] 总耗时 <seconds> 秒 (<trees/s> trees/s, M_prob=<M>)
// Exit status: 0 ok, 1 load or device failure, 2 beyond device bounds.
// --rev / --mixed select reverse AD / mixed precision (extensions).
// --trust-region is the reference's batch_lm_ad_tr build (-DTRUST_REGION,
// cusr/kernel/Makefile:57-63): absolute damping A_jj + lambda from lambda 1e-4,
// a pivot <= 0 replaced by lambda; --pivot-floor its -DPIVOT_FLOOR ablation
// (relative damping, a pivot below 1e-9f raised to it).
// --profile prints one machine-readable line whatever --quiet says, with the
// fields of the reference's -DPROFILE build that a caller compares against
// (batch_lm_ad.cu:553-575): PROFILE_JSON {"M","N","load_ms","setup_ms",
// "loop_ms","total_ms","gpu_sum_ms"}; setup/loop are co_last_split's (upload
// and checks / device fit until the results are on the host), gpu_sum_ms the
// device time of the fit (co_last_kernel_ms).
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include <string>
#include <vector>

#include "../../include/cusr_co.h"

namespace {

struct Pop {
    PopHeader h;
    std::vector<int32_t> nt, ci;
    std::vector<float> nv;
    std::vector<double> c_init, xs, ym;   // promoted from float32 for v1 files
    std::vector<TreeMeta> metas;
};

// float32 (v1) or float64 (v2 with POP_FLAG_F64) payload array, as double
bool read_payload(FILE *f, std::vector<double> &dst, size_t count, bool f64, const char *what);

bool read_exact(FILE *f, void *dst, size_t bytes, const char *what) {
    if (bytes == 0) return true;
    if (fread(dst, 1, bytes, f) != bytes) {
        fprintf(stderr, "load_pop_bin: short read on %s\n", what);
        return false;
    }
    return true;
}

bool load_pop(const char *path, Pop &p) {
    FILE *f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "load_pop_bin: cannot open %s\n", path);
        return false;
    }
    bool ok = read_exact(f, &p.h, sizeof(p.h), "header");
    if (ok && p.h.magic != POP_MAGIC) {
        fprintf(stderr, "load_pop_bin: bad magic 0x%08x\n", (unsigned)p.h.magic);
        ok = false;
    }
    if (ok && p.h.version != POP_VERSION && p.h.version != POP_VERSION_2) {
        fprintf(stderr, "load_pop_bin: version %d is neither %d nor %d\n", p.h.version,
                POP_VERSION, POP_VERSION_2);
        ok = false;
    }
    const int flags = ok ? pop_flags(&p.h) : 0;
    if (ok && (flags & ~(POP_FLAG_F64 | POP_FLAG_SHARED_Y))) {
        fprintf(stderr, "load_pop_bin: unknown flags 0x%x\n", (unsigned)flags);
        ok = false;
    }
    if (ok && p.h.version == POP_VERSION) p.h.reserved[0] = 0;
    if (ok && (p.h.M_prob < 0 || p.h.total_nodes < 0 || p.h.total_c < 0 || p.h.N < 0 ||
               p.h.n_vars < 0)) {
        fprintf(stderr, "load_pop_bin: negative size in header\n");
        ok = false;
    }
    if (ok) {
        const size_t T = p.h.total_nodes, M = p.h.M_prob, C = p.h.total_c;
        const size_t N = p.h.N, D = p.h.n_vars;
        const bool f64 = flags & POP_FLAG_F64;
        const size_t rows = (flags & POP_FLAG_SHARED_Y) ? 1 : M;
        p.nt.resize(T); p.nv.resize(T); p.ci.resize(T); p.metas.resize(M);
        ok = read_exact(f, p.nt.data(), 4 * T, "nt") && read_exact(f, p.nv.data(), 4 * T, "nv") &&
             read_exact(f, p.ci.data(), 4 * T, "ci") &&
             read_exact(f, p.metas.data(), 16 * M, "metas") &&
             read_payload(f, p.c_init, C, f64, "c_init") &&
             read_payload(f, p.xs, N * D, f64, "xs") &&
             read_payload(f, p.ym, rows * N, f64, "ym");
    }
    fclose(f);
    return ok;
}

bool read_payload(FILE *f, std::vector<double> &dst, size_t count, bool f64, const char *what) {
    dst.resize(count);
    if (f64) return read_exact(f, dst.data(), 8 * count, what);
    std::vector<float> tmp(count);
    if (!read_exact(f, tmp.data(), 4 * count, what)) return false;
    for (size_t i = 0; i < count; i++) dst[i] = tmp[i];
    return true;
}

bool write_blob(const std::string &path, const void *buf, size_t bytes) {
    FILE *f = fopen(path.c_str(), "wb");
    if (!f) {
        fprintf(stderr, "cannot write %s\n", path.c_str());
        return false;
    }
    bool ok = fwrite(buf, 1, bytes, f) == bytes;
    fclose(f);
    return ok;
}

double seconds() {
    timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec + t.tv_nsec * 1e-9;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc < 2) {
        fprintf(stderr,
                "usage: %s <pop.bin> [out_dir] [--max-iter N] [--quiet] [--rev] [--mixed] "
                "[--trust-region | --pivot-floor] [--profile]\n",
                argv[0]);
        return 1;
    }
    const double t0 = seconds();
    const char *pop_path = argv[1];
    std::string out_dir;
    int max_iter = 50, quiet = 0, rev = 0, mixed = 0, profile = 0, damping = CO_DAMP_RELATIVE;
    for (int i = 2; i < argc; i++) {
        if (!strcmp(argv[i], "--max-iter") && i + 1 < argc) max_iter = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--quiet")) quiet = 1;
        else if (!strcmp(argv[i], "--rev")) rev = 1;
        else if (!strcmp(argv[i], "--mixed")) mixed = 1;
        else if (!strcmp(argv[i], "--profile")) profile = 1;
        else if (!strcmp(argv[i], "--trust-region")) damping = CO_DAMP_TRUST_REGION;
        else if (!strcmp(argv[i], "--pivot-floor")) damping = CO_DAMP_PIVOT_FLOOR;
        else if (argv[i][0] != '-') out_dir = argv[i];
    }
    if (out_dir.empty()) {
        const char *slash = strrchr(pop_path, '/');
        out_dir = slash ? std::string(pop_path, slash - pop_path) : std::string(".");
    }
    Pop p;
    if (!load_pop(pop_path, p)) {
        fprintf(stderr, "load failed.\n");
        return 1;
    }
    const double t_load = seconds();
    const PopHeader &h = p.h;
    if (!quiet)
        printf("[batch-lm] loaded %s: M_prob=%d total_nodes=%d total_c=%d N=%d n_vars=%d "
               "K_max=%d max_stack=%d\n",
               pop_path, h.M_prob, h.total_nodes, h.total_c, h.N, h.n_vars, h.K_max,
               h.max_stack);
    const int rc0 = co_decode(&h, p.nt.data(), p.nv.data(), p.ci.data(), p.metas.data(), nullptr,
                              nullptr, nullptr, nullptr, nullptr, nullptr);
    if (rc0 == CO_ERR_BOUNDS) {
        fprintf(stderr, "[batch-lm] population beyond device bounds (K<=%d, stack<=%d, "
                        "n_vars<=%d)\n", CO_MAX_K, CO_MAX_STACK, CO_MAX_VARS);
        return 2;
    }
    if (rc0 != CO_OK) {
        fprintf(stderr, "[batch-lm] invalid population (code %d)\n", rc0);
        return 1;
    }
    void *handle = nullptr;
    if (co_init(0, &handle) != CO_OK) {
        fprintf(stderr, "[batch-lm] device init failed\n");
        return 1;
    }
    const size_t M = h.M_prob, C = h.total_c;
    std::vector<double> cf(C > 0 ? C : 1), li(M > 0 ? M : 1), lf(M > 0 ? M : 1);
    std::vector<int32_t> status(M > 0 ? M : 1), iters(M > 0 ? M : 1);
    CoOptions opt;
    co_options_default(&opt);
    opt.max_iter = max_iter;
    opt.ad_mode = rev ? CO_AD_REVERSE : CO_AD_FORWARD;
    opt.precision = mixed ? CO_PREC_MIXED : CO_PREC_FP64;
    opt.damping = damping;
    if (damping == CO_DAMP_TRUST_REGION) opt.lambda0 = CO_TRUST_REGION_LAMBDA0;
    // a float32 (v1) population fits as the reference's fp32 fit does: no
    // constant beyond the fp32 range; a float64 (v2) one in full fp64
    opt.f32_range = (pop_flags(&h) & POP_FLAG_F64) ? 0 : 1;
    int rc = co_optimize_ex(handle, &opt, &h, p.nt.data(), p.nv.data(), p.ci.data(),
                            p.metas.data(), p.c_init.data(), p.xs.data(), p.ym.data(), cf.data(),
                            status.data(), li.data(), lf.data(), iters.data());
    double setup_ms = -1.0, loop_ms = -1.0, gpu_ms = -1.0;
    co_last_split(&setup_ms, &loop_ms);
    co_last_kernel_ms(handle, &gpu_ms);
    co_teardown(handle);
    if (rc != CO_OK) {
        fprintf(stderr, "[batch-lm] fit failed (code %d)\n", rc);
        return rc == CO_ERR_BOUNDS ? 2 : 1;
    }
    // float32 blobs: an expression whose fitted constants overflow fp32 gets
    // its c_init back, as co_optimize does
    std::vector<float> cf32(C > 0 ? C : 1), li32(M > 0 ? M : 1), lf32(M > 0 ? M : 1);
    rc = co_narrow_fp32(&h, p.metas.data(), p.c_init.data(), cf.data(), li.data(), lf.data(),
                        status.data(), cf32.data(), li32.data(), lf32.data());
    if (rc < 0) {
        fprintf(stderr, "[batch-lm] narrowing failed (code %d)\n", rc);
        return 1;
    }
    bool ok = write_blob(out_dir + "/status.bin", status.data(), 4 * M) &&
              write_blob(out_dir + "/c_final.bin", cf32.data(), 4 * C) &&
              write_blob(out_dir + "/loss_final.bin", lf32.data(), 4 * M) &&
              write_blob(out_dir + "/loss_init.bin", li32.data(), 4 * M);
    if (!ok) return 1;
    const double el = seconds() - t0;
    if (!quiet) {
        int cnt[5] = {0, 0, 0, 0, 0};
        for (size_t m = 0; m < M; m++)
            if (status[m] >= 0 && status[m] < 5) cnt[status[m]]++;
        printf("[batch-lm] 完成: converged=%d (%.1f%%)  maxiter=%d  fail_nan=%d  "
               "fail_cholesky=%d  k0_skip=%d  (M_prob=%d)\n",
               cnt[0], M ? 100.0 * cnt[0] / M : 0.0, cnt[1], cnt[2], cnt[4], cnt[3], h.M_prob);
        printf("[batch-lm] 总耗时 %.3f 秒 (%.0f trees/s, M_prob=%d)\n", el, M / el, h.M_prob);
    }
    if (profile)
        printf("PROFILE_JSON {\"M\":%d,\"N\":%d,\"load_ms\":%.4f,\"setup_ms\":%.4f,"
               "\"loop_ms\":%.4f,\"total_ms\":%.4f,\"gpu_sum_ms\":%.4f}\n",
               h.M_prob, h.N, 1e3 * (t_load - t0), setup_ms, loop_ms, 1e3 * el, gpu_ms);
    return 0;
}
