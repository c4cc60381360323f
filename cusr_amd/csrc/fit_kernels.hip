// fit_kernels.hip -- instantiates the fit kernels of one (precision, AD mode)
// variant: the fast kernels for K = 0..CO_FAST_MAX_K and the general kernel.
// Built four times with
//   -DCUSR_FIT_R=double|float -DCUSR_FIT_AD=0|1 -DCUSR_FIT_LAUNCH=<name>
//   -DCUSR_PASS_LAUNCH=<name>
// and the pass kernels of the split path (lm_split.h) for the same bins.
#include "lm_device.h"
#include "lm_split.h"

#if !defined(CUSR_FIT_R) || !defined(CUSR_FIT_AD) || !defined(CUSR_FIT_LAUNCH) || \
    !defined(CUSR_PASS_LAUNCH)
#error "fit_kernels.hip needs CUSR_FIT_R, CUSR_FIT_AD, CUSR_FIT_LAUNCH and CUSR_PASS_LAUNCH"
#endif

namespace cusr {

hipError_t CUSR_FIT_LAUNCH(int bin, unsigned grid, size_t lds, hipStream_t s, const FitArgs &fa) {
    if (fa.pwaves < 1 || fa.pwaves > CO_MAX_PARTITIONS || fa.parts % fa.pwaves != 0)
        return hipErrorInvalidValue;
    // a segment that can pause or resume needs the state buffer
    if (fa.it_end < 0 || fa.it_end > fa.max_iter ||
        ((fa.resume || fa.it_end < fa.max_iter) && !fa.state))
        return hipErrorInvalidValue;
    switch (bin) {
// the large-N instance where its tables differ (large_n_variant), chosen by N
#define CUSR_CASE(k)                                                                        \
    case k:                                                                                 \
        if constexpr (large_n_variant<CUSR_FIT_R, k, CUSR_FIT_AD>()) {                      \
            if (fa.N >= kLargeN) {                                                          \
                lm_fit_kernel<k, CUSR_FIT_R, CUSR_FIT_AD, 1>                                \
                    <<<grid, kLanes * fa.pwaves, lds, s>>>(fa);                             \
                break;                                                                      \
            }                                                                               \
        }                                                                                   \
        lm_fit_kernel<k, CUSR_FIT_R, CUSR_FIT_AD, 0><<<grid, kLanes * fa.pwaves, lds, s>>>(fa); \
        break;
        CUSR_CASE(0) CUSR_CASE(1) CUSR_CASE(2) CUSR_CASE(3) CUSR_CASE(4) CUSR_CASE(5)
        CUSR_CASE(6) CUSR_CASE(7) CUSR_CASE(8) CUSR_CASE(9) CUSR_CASE(10) CUSR_CASE(11)
        CUSR_CASE(12) CUSR_CASE(13) CUSR_CASE(14) CUSR_CASE(15) CUSR_CASE(16)
#undef CUSR_CASE
    case CO_GENERAL_BIN:
        lm_fit_gen_kernel<CUSR_FIT_R, CUSR_FIT_AD><<<grid, kLanes * fa.pwaves, lds, s>>>(fa);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t CUSR_PASS_LAUNCH(int bin, unsigned grid, size_t lds, hipStream_t s, const FitArgs &fa) {
    if (fa.parts < 1 || !fa.psum || !fa.state) return hipErrorInvalidValue;
    switch (bin) {
#define CUSR_CASE(k)                                                                        \
    case k:                                                                                 \
        if constexpr (large_n_variant<CUSR_FIT_R, k, CUSR_FIT_AD>()) {                      \
            if (fa.N >= kLargeN) {                                                          \
                lm_pass_kernel<k, CUSR_FIT_R, CUSR_FIT_AD, 1, false>                        \
                    <<<grid, kLanes, lds, s>>>(fa);                                         \
                break;                                                                      \
            }                                                                               \
        }                                                                                   \
        lm_pass_kernel<k, CUSR_FIT_R, CUSR_FIT_AD, 0, false><<<grid, kLanes, lds, s>>>(fa);  \
        break;
        CUSR_CASE(0) CUSR_CASE(1) CUSR_CASE(2) CUSR_CASE(3) CUSR_CASE(4) CUSR_CASE(5)
        CUSR_CASE(6) CUSR_CASE(7) CUSR_CASE(8) CUSR_CASE(9) CUSR_CASE(10) CUSR_CASE(11)
        CUSR_CASE(12) CUSR_CASE(13) CUSR_CASE(14) CUSR_CASE(15) CUSR_CASE(16)
#undef CUSR_CASE
    case CO_GENERAL_BIN:
        lm_pass_kernel<kGenK, CUSR_FIT_R, CUSR_FIT_AD, 0, true><<<grid, kLanes, lds, s>>>(fa);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace cusr
