// Instantiates the dense kernels for one bit width (EXL3_BITS, set by the build).
#include "exl3_dense.hpp"

#ifndef EXL3_BITS
#error "EXL3_BITS must be defined (1..8)"
#endif

namespace exl3 {

template <>
int launch_dequant<EXL3_BITS>(const DequantArgs& a) {
    constexpr int B = EXL3_BITS;
    auto go = [&](auto cbc) {
        constexpr int C = decltype(cbc)::value;
        if (a.suh) {
            const int blocks = (a.k16 / 8) * (a.n16 / 8);
            hipLaunchKernelGGL((dequant_had_kernel<B, C>), dim3(blocks), dim3(64), 0, a.stream, a.trellis,
                               a.k16, a.n16, a.suh, a.svh, a.out);
        } else {
            const int tiles = a.k16 * a.n16;
            hipLaunchKernelGGL((dequant_raw_kernel<B, C>), dim3((tiles + 63) / 64), dim3(64), 0, a.stream,
                               a.trellis, a.k16, a.n16, a.out);
        }
    };
    switch (a.codebook) {
        case CB_MCG: go(std::integral_constant<int, CB_MCG>{}); break;
        case CB_3INST: go(std::integral_constant<int, CB_3INST>{}); break;
        default: go(std::integral_constant<int, CB_MUL1>{}); break;
    }
    return check_launch();
}

template <>
int launch_gemv<EXL3_BITS>(const GemvArgs& a) {
    constexpr int B = EXL3_BITS;
    auto go = [&](auto cbc) {
        constexpr int C = decltype(cbc)::value;
        if (a.plan.split_reduce)
            hipLaunchKernelGGL((gemv_kernel<B, C, true>), dim3(a.plan.n_cb * a.plan.n_kc), dim3(64), 0, a.stream,
                               a.x, a.trellis, a.suh, a.svh, a.out, a.out_kind, a.R, a.K, a.N, a.plan.nsteps,
                               a.plan.n_kc, a.counters, a.partials);
        else
            hipLaunchKernelGGL((gemv_kernel<B, C, false>), dim3(a.plan.n_cb * a.plan.n_kc), dim3(64), 0, a.stream,
                               a.x, a.trellis, a.suh, a.svh, a.out, a.out_kind, a.R, a.K, a.N, a.plan.nsteps,
                               a.plan.n_kc, a.counters, a.partials);
    };
    switch (a.codebook) {
        case CB_MCG: go(std::integral_constant<int, CB_MCG>{}); break;
        case CB_3INST: go(std::integral_constant<int, CB_3INST>{}); break;
        default: go(std::integral_constant<int, CB_MUL1>{}); break;
    }
    return check_launch();
}

template <>
int launch_gemv_fan<EXL3_BITS>(const FanParams& P, int codebook, int blocks, hipStream_t stream) {
    constexpr int B = EXL3_BITS;
    auto go = [&](auto cbc) {
        constexpr int C = decltype(cbc)::value;
        hipLaunchKernelGGL((gemv_fan_kernel<B, C>), dim3(blocks), dim3(64), 0, stream, P);
    };
    switch (codebook) {
        case CB_MCG: go(std::integral_constant<int, CB_MCG>{}); break;
        case CB_3INST: go(std::integral_constant<int, CB_3INST>{}); break;
        default: go(std::integral_constant<int, CB_MUL1>{}); break;
    }
    return check_launch();
}

}  // namespace exl3
