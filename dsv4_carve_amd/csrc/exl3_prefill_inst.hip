// Instantiates the grouped-GEMM kernels of the routed-MoE prefill path for one
// bit width (EXL3_BITS, set by the build), or for two widths in one kernel
// (EXL3_BITS2 as well), every codebook, both directions.
#include "exl3_prefill.hpp"

#ifndef EXL3_BITS
#error "EXL3_BITS must be defined"
#endif

namespace exl3 {
namespace prefill {

#ifndef EXL3_BITS2
#define EXL3_BITS2 0
#endif

#if EXL3_BITS2 == 0
template <>
int launch_pf_gemm<EXL3_BITS>(const PfParams& P, int codebook, bool down, int blocks, hipStream_t stream) {
#else
int launch_pf_gemm_32(const PfParams& P, int codebook, bool down, int blocks, hipStream_t stream) {
    static_assert(EXL3_BITS == 3 && EXL3_BITS2 == 2, "the two-width unit is built for widths 3 and 2");
#endif
    constexpr int B = EXL3_BITS, B2 = EXL3_BITS2;
    // `blocks` workgroups of two waves (pf_gemm_grid)
    const unsigned grid = (unsigned)blocks;
    auto go = [&](auto cbc) {
        constexpr int C = decltype(cbc)::value;
        if (down)
            hipLaunchKernelGGL((pf_gemm_kernel<B, B2, C, true>), dim3(grid), dim3(2 * WAVE), 0, stream, P);
        else
            hipLaunchKernelGGL((pf_gemm_kernel<B, B2, C, false>), dim3(grid), dim3(2 * WAVE), 0, stream, P);
    };
    switch (codebook) {
        case CB_MCG: go(std::integral_constant<int, CB_MCG>{}); break;
        case CB_3INST: go(std::integral_constant<int, CB_3INST>{}); break;
        default: go(std::integral_constant<int, CB_MUL1>{}); break;
    }
    return check_launch();
}

}  // namespace prefill
}  // namespace exl3
