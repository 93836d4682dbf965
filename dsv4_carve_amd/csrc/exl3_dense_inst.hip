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
            if (a.nk)
                hipLaunchKernelGGL((dequant_had_kernel<B, C, true>), dim3(blocks), dim3(256), 0, a.stream, a.trellis,
                                   a.k16, a.n16, a.suh, a.svh, a.out);
            else
                hipLaunchKernelGGL((dequant_had_kernel<B, C, false>), dim3(blocks), dim3(256), 0, a.stream,
                                   a.trellis, a.k16, a.n16, a.suh, a.svh, a.out);
        } else {
            const int tiles = a.k16 * a.n16;
            if (a.nk)
                hipLaunchKernelGGL((dequant_raw_kernel<B, C, true>), dim3((tiles + 63) / 64), dim3(64), 0, a.stream,
                                   a.trellis, a.k16, a.n16, a.out);
            else
                hipLaunchKernelGGL((dequant_raw_kernel<B, C, false>), dim3((tiles + 63) / 64), dim3(64), 0,
                                   a.stream, a.trellis, a.k16, a.n16, a.out);
        }
    };
    switch (a.codebook) {
        case CB_MCG: go(std::integral_constant<int, CB_MCG>{}); break;
        case CB_3INST: go(std::integral_constant<int, CB_3INST>{}); break;
        default: go(std::integral_constant<int, CB_MUL1>{}); break;
    }
    return check_launch();
}

template <int B, int C, int W, int RB>
static void launch_gemv_w(const GemvArgs& a) {
    const dim3 grid(a.plan.n_cb * a.plan.n_kc), block(64 * W);
    if (a.plan.split_reduce)
        hipLaunchKernelGGL((gemv_kernel<B, C, W, RB, true>), grid, block, 0, a.stream, a.x, a.trellis, a.suh,
                           a.svh, a.out, a.out_kind, a.R, a.K, a.N, a.plan.nsteps, a.plan.n_kc, a.plan.xcd ? 1 : 0,
                           a.counters, a.partials);
    else
        hipLaunchKernelGGL((gemv_kernel<B, C, W, RB, false>), grid, block, 0, a.stream, a.x, a.trellis, a.suh,
                           a.svh, a.out, a.out_kind, a.R, a.K, a.N, a.plan.nsteps, a.plan.n_kc, a.plan.xcd ? 1 : 0,
                           a.counters, a.partials);
}

// Up to 16 rows: one MFMA row block, 1, 2 or 4 column groups; 17-32 rows:
// two row blocks, 2 or 4 column groups (the plan never picks 1 there).
template <>
int launch_gemv<EXL3_BITS>(const GemvArgs& a) {
    constexpr int B = EXL3_BITS;
    auto go = [&](auto cbc) {
        constexpr int C = decltype(cbc)::value;
        if (a.R > MAX_ROWS) {
            if (a.plan.waves == 4) launch_gemv_w<B, C, 4, 2>(a);
            else launch_gemv_w<B, C, 2, 2>(a);
        } else if (a.plan.waves == 4) launch_gemv_w<B, C, 4, 1>(a);
        else if (a.plan.waves == 2) launch_gemv_w<B, C, 2, 1>(a);
        else launch_gemv_w<B, C, 1, 1>(a);
    };
    switch (a.codebook) {
        case CB_MCG: go(std::integral_constant<int, CB_MCG>{}); break;
        case CB_3INST: go(std::integral_constant<int, CB_3INST>{}); break;
        default: go(std::integral_constant<int, CB_MUL1>{}); break;
    }
    return check_launch();
}

template <>
int launch_gemv_fan<EXL3_BITS>(const FanParams& P, int codebook, int waves, int blocks, hipStream_t stream) {
    constexpr int B = EXL3_BITS;
    auto go = [&](auto cbc) {
        constexpr int C = decltype(cbc)::value;
        const dim3 grid(blocks);
        if (P.R > MAX_ROWS) {
            if (waves == 4) hipLaunchKernelGGL((gemv_fan_kernel<B, C, 4, 2>), grid, dim3(256), 0, stream, P);
            else hipLaunchKernelGGL((gemv_fan_kernel<B, C, 2, 2>), grid, dim3(128), 0, stream, P);
        } else if (waves == 4) hipLaunchKernelGGL((gemv_fan_kernel<B, C, 4, 1>), grid, dim3(256), 0, stream, P);
        else if (waves == 2) hipLaunchKernelGGL((gemv_fan_kernel<B, C, 2, 1>), grid, dim3(128), 0, stream, P);
        else hipLaunchKernelGGL((gemv_fan_kernel<B, C, 1, 1>), grid, dim3(64), 0, stream, P);
    };
    switch (codebook) {
        case CB_MCG: go(std::integral_constant<int, CB_MCG>{}); break;
        case CB_3INST: go(std::integral_constant<int, CB_3INST>{}); break;
        default: go(std::integral_constant<int, CB_MUL1>{}); break;
    }
    return check_launch();
}

}  // namespace exl3
