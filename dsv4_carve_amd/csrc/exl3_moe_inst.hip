// Instantiates the routed-MoE kernel for one (bit-width mask, codebook) pair,
// set by the build: EXL3_MOE_MASK (bit b set = b-bit experts supported) and
// EXL3_MOE_CB (0 = 3INST, 1 = MCG, 2 = MUL1).
#include "exl3_moe.hpp"

#ifndef EXL3_MOE_MASK
#error "EXL3_MOE_MASK must be defined"
#endif
#ifndef EXL3_MOE_CB
#error "EXL3_MOE_CB must be defined"
#endif

namespace exl3 {
namespace moe {

template <>
int launch_moe<EXL3_MOE_MASK, EXL3_MOE_CB>(const Params& P, int waves, int lds_kb, hipStream_t stream) {
    hipLaunchKernelGGL((moe_kernel<EXL3_MOE_MASK, EXL3_MOE_CB>), dim3(waves), dim3(WAVE), (size_t)lds_kb * 1024,
                       stream, P);
    return check_launch();
}

template <>
int launch_phased<EXL3_MOE_MASK, EXL3_MOE_CB>(const Params& P, int lds_kb, hipStream_t stream) {
    const Layout& L = P.L;
    const size_t lds = (size_t)lds_kb * 1024;
    const int slots = P.m * P.topk;
    hipLaunchKernelGGL((moe_slot_gateup<EXL3_MOE_MASK, EXL3_MOE_CB>), dim3(slots * 2 * L.nI * L.SA), dim3(WAVE),
                       lds, stream, P);
    int rc = check_launch();
    if (rc) return rc;
    if (!P.fuse_act) {
        hipLaunchKernelGGL((moe_slot_act<0>), dim3(slots * L.nI), dim3(WAVE), 0, stream, P);
        if ((rc = check_launch())) return rc;
    }
    hipLaunchKernelGGL((moe_slot_down<EXL3_MOE_MASK, EXL3_MOE_CB>), dim3(slots * L.nH * L.SB), dim3(WAVE), lds,
                       stream, P);
    if ((rc = check_launch())) return rc;
    hipLaunchKernelGGL((moe_slot_finish<0>), dim3(L.nH * P.m), dim3(P.topk * WAVE), 0, stream, P);
    return check_launch();
}

template <>
int moe_waves_per_cu<EXL3_MOE_MASK, EXL3_MOE_CB>(int lds_kb) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, reinterpret_cast<const void*>(moe_kernel<EXL3_MOE_MASK, EXL3_MOE_CB>), WAVE,
            (size_t)lds_kb * 1024) != hipSuccess ||
        n < 1)
        n = 1;
    return n;
}

}  // namespace moe
}  // namespace exl3
