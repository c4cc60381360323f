// ref_ad_shim.cpp -- extern "C" entry points over the reference's own fp32
// interpreters (cusr/kernel/ad_interp.cuh:58-233, revad_interp.cuh:66-157),
// compiled host-only from the reference tree by oracle/Makefile. Test
// infrastructure: used only to pin the oracle's operator semantics.
#include <hip/hip_runtime.h>
#include "revad_interp.cuh"

extern "C" float ref_value(const int *nt, const float *nv, int n, const int *ci,
                           const float *x, const float *c) {
    return eval_tree_val_host(nt, nv, n, ci, x, c);
}

// Forward-mode gradient for all K columns, AD_W columns per pass like
// ad_jacobian_kernel (ad_interp.cuh:265-274).
extern "C" float ref_jvp(const int *nt, const float *nv, int n, const int *ci,
                         const float *x, const float *c, int K, float *grad) {
    float val = 0.0f, t[AD_W];
    for (int lo = 0; lo < K; lo += AD_W) {
        int W = (K - lo < AD_W) ? (K - lo) : AD_W;
        eval_tree_jvp_d(nt, nv, n, ci, x, c, lo, W, &val, t);
        for (int w = 0; w < W; w++) grad[lo + w] = t[w];
    }
    if (K == 0) val = eval_tree_val_host(nt, nv, n, ci, x, c);
    return val;
}

extern "C" void ref_vjp(const int *nt, const float *nv, int n, const int *ci,
                        const float *x, const float *c, int K, float *grad) {
    eval_tree_vjp_d(nt, nv, n, ci, x, c, K, grad);
}
