// Ceiling probes for the benchmark (not part of the decode path's ABI).
//
// 1. HBM read ceiling.
// Streams `bytes` of a device buffer once with 16-byte loads, eight in flight
// per lane, and folds them into one word per lane so no load is dead.  Timed
// by the caller on `stream`; with the buffer far larger than the 256 MB
// Infinity Cache and a flush between runs, the rate is the achievable cold
// read bandwidth that the decode kernels' weight streams are measured against
// (the role of recipe-lna/lna2/cold_read_bw.cu:23-153 on the reference's card).
//
// 2. Decode-rate ceiling.  The decode kernels' inner loop (exl3_gemv.hpp
// mma_tile: trellis windows, codebook, MFMA accumulate) run on tiles that stay
// in registers, with no memory traffic and no item overheads, at the decode
// kernels' residency (single-wave workgroups, two per SIMD).  Its rate in
// decoded weights per second bounds any launch built on that loop: a layer of
// W weights cannot finish in less than W / rate, whatever the memory system
// delivers.  The tile words are made opaque to the compiler every iteration,
// so each iteration decodes and multiplies all 256 weights of the lane's tile.
// Three modes split the loop's cost: the decode and the MFMAs together (the
// loop the kernels run), the decode alone (each decoded B operand is handed
// to an empty asm statement, which forces its computation and emits no
// instruction), and the MFMAs alone (the B operands are the tile words
// themselves, register moves at most).  A fourth runs the whole loop with the
// MFMA accumulators in the accumulation registers (AGPRs) instead of VGPRs,
// and a fifth sums each weight's two addends on the VALU so an MFMA takes
// eight weights per lane (half the MFMAs, no duplicated activations).
// The launch's block count sets the waves per SIMD.
//
// 3. Instruction issue rates.  One VALU instruction of the decode's kinds in a
// loop: eight independent chains per lane, 64 instructions per iteration, in
// four-wave workgroups (one wave per SIMD of a CU), so a launch of n * CUs
// workgroups puts n waves on each SIMD.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "exl3_gemv.hpp"
#include "exl3_prefill.hpp"

using exl3::u32x4_t;

constexpr int PROBE_THREADS = 256;
constexpr int PROBE_UNROLL = 8;

__global__ __launch_bounds__(PROBE_THREADS) void probe_read_kernel(const u32x4_t* __restrict__ buf, int64_t nvec,
                                                                   uint32_t* __restrict__ sink) {
    const int64_t tid = (int64_t)blockIdx.x * PROBE_THREADS + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * PROBE_THREADS;
    u32x4_t acc = {0u, 0u, 0u, 0u};
    int64_t i = tid;
    // whole rounds of PROBE_UNROLL loads per lane, every address in range
    for (; i + (PROBE_UNROLL - 1) * stride < nvec; i += PROBE_UNROLL * stride) {
        u32x4_t v[PROBE_UNROLL];
#pragma unroll
        for (int u = 0; u < PROBE_UNROLL; ++u) v[u] = __builtin_nontemporal_load(buf + i + u * stride);
#pragma unroll
        for (int u = 0; u < PROBE_UNROLL; ++u) acc ^= v[u];
    }
    for (; i < nvec; i += stride) acc ^= buf[i];
    sink[tid] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

enum ProbeMode : int {
    PROBE_FULL = 0, PROBE_DECODE_ONLY = 1, PROBE_MFMA_ONLY = 2, PROBE_FULL_AGPR = 3, PROBE_NO_DUP = 4
};

// The decode kernels' mma_tile with the decode or the MFMA taken out (MODE).
template <int BITS, int MODE>
__device__ __forceinline__ void probe_tile(const uint32_t* W, const exl3::half8_t (&A)[4], exl3::float4_t (&acc)[16]) {
    using namespace exl3;
    if constexpr (MODE == PROBE_FULL || MODE == PROBE_FULL_AGPR) {
        mma_tile<BITS, CB_MCG>(W, A, acc);
    } else if constexpr (MODE == PROBE_NO_DUP) {
        // Each weight's two fp16 addends summed on the VALU (one packed add per
        // two weights, after two byte permutes gather their low and high
        // addends), so one MFMA takes eight weights per lane instead of four:
        // half the MFMAs, A not duplicated (the probe reuses A[0..1] as the
        // eight distinct activations).
        typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
        static_for<16>([&](auto NI) {
            constexpr int n = decltype(NI)::value;
            static_for<2>([&](auto RI) {
                constexpr int r2 = decltype(RI)::value;
                u32x4_t b;
                static_for<4>([&](auto JI) {
                    constexpr int j = decltype(JI)::value;
                    constexpr int r = 2 * r2 + j / 2, q0 = 2 * (j & 1);
                    constexpr int T0 = 32 * (n & 7) + 8 * r + 4 * (n >> 3) + q0;
                    const uint32_t xa = decode_pair<BITS, CB_MCG, T0>(W);
                    const uint32_t xb = decode_pair<BITS, CB_MCG, T0 + 1>(W);
                    const h2_t lo = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(xb, xa, 0x01000504u));
                    const h2_t hi = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(xb, xa, 0x03020706u));
                    b[j] = __builtin_bit_cast(uint32_t, lo + hi);
                });
                acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[r2], __builtin_bit_cast(half8_t, b), acc[n], 0, 0, 0);
            });
        });
    } else {
        static_for<16>([&](auto NI) {
            constexpr int n = decltype(NI)::value;
            static_for<4>([&](auto RI) {
                constexpr int r = decltype(RI)::value;
                constexpr int T0 = 32 * (n & 7) + 8 * r + 4 * (n >> 3);
                u32x4_t b;
                if constexpr (MODE == PROBE_DECODE_ONLY) {
                    b[0] = decode_pair<BITS, CB_MCG, T0 + 0>(W);
                    b[1] = decode_pair<BITS, CB_MCG, T0 + 1>(W);
                    b[2] = decode_pair<BITS, CB_MCG, T0 + 2>(W);
                    b[3] = decode_pair<BITS, CB_MCG, T0 + 3>(W);
                    asm volatile("" : : "v"(b));
                } else {
                    constexpr int NW = 8 * BITS;
                    b[0] = W[(T0 + 0) % NW];
                    b[1] = W[(T0 + 1) % NW];
                    b[2] = W[(T0 + 2) % NW];
                    b[3] = W[(T0 + 3) % NW];
                    acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[r], __builtin_bit_cast(half8_t, b), acc[n],
                                                                    0, 0, 0);
                }
            });
        });
    }
}

template <int BITS, int MODE>
__global__ __launch_bounds__(64, 2) void probe_decode_kernel(const uint32_t* __restrict__ words, int iters,
                                                            float* __restrict__ sink, uint64_t* __restrict__ clk) {
    using namespace exl3;
    // PROBE_FULL_AGPR: an (empty) asm statement that clobbers an accumulation
    // register makes the compiler keep the MFMA accumulators there
    if constexpr (MODE == PROBE_FULL_AGPR) asm volatile("" ::: "a0");
    const int lane = threadIdx.x;
    uint32_t W[8 * BITS];
#pragma unroll
    for (int i = 0; i < 8 * BITS; ++i) W[i] = words[lane * 8 * BITS + i];
    half8_t A[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < 8; ++j) A[r][j] = (_Float16)((float)((lane + 3 * r + j) & 7) * 0.125f - 0.4375f);
    float4_t acc[16];
    zero_acc(acc);
    const uint64_t c0 = __builtin_amdgcn_s_memtime(), t0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 8 * BITS; ++i) asm volatile("" : "+v"(W[i]));
        probe_tile<BITS, MODE>(W, A, acc);
    }
    const uint64_t c1 = __builtin_amdgcn_s_memtime(), t1 = __builtin_amdgcn_s_memrealtime();
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) sum += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
    sink[blockIdx.x * 64 + lane] = sum;
    if (lane == 0) {
        clk[2 * blockIdx.x] = c1 - c0;
        clk[2 * blockIdx.x + 1] = t1 - t0;
    }
}

template <int BITS>
static int launch_probe_decode(int mode, int blocks, int iters, const uint32_t* words, float* sink, uint64_t* clk,
                               hipStream_t st) {
    switch (mode) {
        case PROBE_FULL:
            hipLaunchKernelGGL((probe_decode_kernel<BITS, PROBE_FULL>), dim3(blocks), dim3(64), 0, st, words, iters,
                               sink, clk);
            break;
        case PROBE_DECODE_ONLY:
            hipLaunchKernelGGL((probe_decode_kernel<BITS, PROBE_DECODE_ONLY>), dim3(blocks), dim3(64), 0, st, words,
                               iters, sink, clk);
            break;
        case PROBE_MFMA_ONLY:
            hipLaunchKernelGGL((probe_decode_kernel<BITS, PROBE_MFMA_ONLY>), dim3(blocks), dim3(64), 0, st, words,
                               iters, sink, clk);
            break;
        case PROBE_FULL_AGPR:
            hipLaunchKernelGGL((probe_decode_kernel<BITS, PROBE_FULL_AGPR>), dim3(blocks), dim3(64), 0, st, words,
                               iters, sink, clk);
            break;
        case PROBE_NO_DUP:
            hipLaunchKernelGGL((probe_decode_kernel<BITS, PROBE_NO_DUP>), dim3(blocks), dim3(64), 0, st, words,
                               iters, sink, clk);
            break;
        default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Wave-role probe: one workgroup per CU.  Modes 0-2 use eight waves (two per
// SIMD), modes 3-4 twelve (three per SIMD).  mode 0: every wave runs the
// decode loop (decode + MFMA); mode 1: waves 0-3 decode only and waves 4-7 run
// the MFMAs only; mode 2: even waves decode only and odd waves run the MFMAs
// only; mode 3: waves 0-7 decode only and waves 8-11 run the MFMAs of two
// iterations per iteration (two decoding waves and one multiplying wave per
// SIMD, the same work); mode 4: every one of the twelve waves runs the decode
// loop.  Each wave also records the SIMD it ran on (HW_ID bits 5:4), so which
// roles shared a SIMD is read back, not assumed.
constexpr int PROBE_ROLES_MAX_WAVES = 12;

template <int BITS>
__global__ __launch_bounds__(64 * PROBE_ROLES_MAX_WAVES, 1) void probe_roles_kernel(
    const uint32_t* __restrict__ words, int iters, int mode, float* __restrict__ sink, uint64_t* __restrict__ clk) {
    using namespace exl3;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    uint32_t W[8 * BITS];
#pragma unroll
    for (int i = 0; i < 8 * BITS; ++i) W[i] = words[lane * 8 * BITS + i];
    half8_t A[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < 8; ++j) A[r][j] = (_Float16)((float)((lane + 3 * r + j) & 7) * 0.125f - 0.4375f);
    float4_t acc[16];
    zero_acc(acc);
    const int role = (mode == 0 || mode == 4) ? PROBE_FULL
                   : mode == 1 ? (w < 4 ? PROBE_DECODE_ONLY : PROBE_MFMA_ONLY)
                   : mode == 2 ? ((w & 1) ? PROBE_MFMA_ONLY : PROBE_DECODE_ONLY)
                               : (w < 8 ? PROBE_DECODE_ONLY : PROBE_MFMA_ONLY);
    const int n_it = (mode == 3 && role == PROBE_MFMA_ONLY) ? 2 * iters : iters;
    auto loop = [&](auto M) {
        for (int it = 0; it < n_it; ++it) {
#pragma unroll
            for (int i = 0; i < 8 * BITS; ++i) asm volatile("" : "+v"(W[i]));
            probe_tile<BITS, decltype(M)::value>(W, A, acc);
        }
    };
    const uint64_t c0 = __builtin_amdgcn_s_memtime(), t0 = __builtin_amdgcn_s_memrealtime();
    if (role == PROBE_FULL) loop(std::integral_constant<int, PROBE_FULL>{});
    else if (role == PROBE_DECODE_ONLY) loop(std::integral_constant<int, PROBE_DECODE_ONLY>{});
    else loop(std::integral_constant<int, PROBE_MFMA_ONLY>{});
    const uint64_t c1 = __builtin_amdgcn_s_memtime(), t1 = __builtin_amdgcn_s_memrealtime();
    // HW_ID (hardware register 4), all 32 bits: SIMD_ID is bits 5:4
    const uint32_t hw = __builtin_amdgcn_s_getreg((31 << 11) | (0 << 6) | 4);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) sum += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
    sink[blockIdx.x * 64 * PROBE_ROLES_MAX_WAVES + threadIdx.x] = sum;
    if (lane == 0) {
        const size_t o = 3 * ((size_t)blockIdx.x * PROBE_ROLES_MAX_WAVES + w);
        clk[o] = c1 - c0;
        clk[o + 1] = t1 - t0;
        clk[o + 2] = (hw >> 4) & 3u;
    }
}

// Row-block probe: the grouped GEMM's inner loop with each decoded B operand
// applied to RB row blocks (16 rows each), the lane decoding the 16 / D
// columns n = D m + p of its tile (D = 1: all 16).  A lane whose tile words are
// rotated by p 32-element blocks (p * BITS words) finds those columns' windows
// at the positions of p = 0, so the positions stay compile-time for any p; the
// probe's words are opaque, so it decodes the p = 0 set.  MFMAs run in the
// (n & 7, r, n >> 3) order of the GEMM, row block 0's right after its B is
// decoded and row block b's (b > 0) on the previous B after the b-th of its
// four windows, so no two MFMAs are adjacent.  One A operand per k-group
// serves every row block (timing only).  Rates are per decoded weight.
template <int BITS, int RB, int D>
__device__ __forceinline__ void probe_rows_tile(const uint32_t* W, const exl3::half8_t (&A)[4],
                                                exl3::float4_t (&acc)[RB][16 / D]) {
    using namespace exl3;
    constexpr int NA = 8 / D;                    // values of n & 7 per lane
    half8_t Bprev;
    static_for<NA * 8>([&](auto II) {
        constexpr int i = decltype(II)::value;
        constexpr int n = D * (i / 8) + 8 * (i & 1), r = (i >> 1) & 3;
        constexpr int T0 = 32 * (n & 7) + 8 * r + 4 * (n >> 3);
        u32x4_t b;
        static_for<4>([&](auto QI) {
            constexpr int q = decltype(QI)::value;
            b[q] = decode_pair<BITS, CB_MCG, T0 + q>(W);
            if constexpr (i > 0 && q + 1 < RB && q < 3) {
                constexpr int np = D * ((i - 1) / 8) + 8 * ((i - 1) & 1), rp = ((i - 1) >> 1) & 3;
                acc[q + 1][np / D] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[rp], Bprev, acc[q + 1][np / D], 0, 0, 0);
            }
        });
        if constexpr (i > 0 && RB > 4) {
            constexpr int np = D * ((i - 1) / 8) + 8 * ((i - 1) & 1), rp = ((i - 1) >> 1) & 3;
            static_for<RB - 4>([&](auto BI) {
                constexpr int bb = 4 + decltype(BI)::value;
                acc[bb][np / D] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[rp], Bprev, acc[bb][np / D], 0, 0, 0);
            });
        }
        const half8_t B = __builtin_bit_cast(half8_t, b);
        acc[0][n / D] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[r], B, acc[0][n / D], 0, 0, 0);
        Bprev = B;
    });
    constexpr int nl = D * ((NA * 8 - 1) / 8) + 8, rl = 3;
    static_for<RB - 1>([&](auto BI) {
        constexpr int bb = 1 + decltype(BI)::value;
        acc[bb][nl / D] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[rl], Bprev, acc[bb][nl / D], 0, 0, 0);
    });
}

template <int BITS, int RB, int D>
__global__ __launch_bounds__(64, 2) void probe_rows_kernel(const uint32_t* __restrict__ words, int iters,
                                                          float* __restrict__ sink, uint64_t* __restrict__ clk) {
    using namespace exl3;
    const int lane = threadIdx.x;
    uint32_t W[8 * BITS];
#pragma unroll
    for (int i = 0; i < 8 * BITS; ++i) W[i] = words[lane * 8 * BITS + i];
    half8_t A[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < 8; ++j) A[r][j] = (_Float16)((float)((lane + 3 * r + j) & 7) * 0.125f - 0.4375f);
    float4_t acc[RB][16 / D];
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int i = 0; i < 16 / D; ++i) acc[b][i] = float4_t{0.f, 0.f, 0.f, 0.f};
    const uint64_t c0 = __builtin_amdgcn_s_memtime(), t0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 8 * BITS; ++i) asm volatile("" : "+v"(W[i]));
        probe_rows_tile<BITS, RB, D>(W, A, acc);
    }
    const uint64_t c1 = __builtin_amdgcn_s_memtime(), t1 = __builtin_amdgcn_s_memrealtime();
    float sum = 0.f;
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int i = 0; i < 16 / D; ++i) sum += acc[b][i][0] + acc[b][i][1] + acc[b][i][2] + acc[b][i][3];
    sink[blockIdx.x * 64 + lane] = sum;
    if (lane == 0) {
        clk[2 * blockIdx.x] = c1 - c0;
        clk[2 * blockIdx.x + 1] = t1 - t0;
    }
}

// (row blocks, column divisor) pairs of the row-block probe, by index
constexpr int PROBE_ROWS_CFG[][2] = {{1, 1}, {2, 1}, {2, 2}, {3, 2}, {4, 2}, {4, 4}, {6, 4}, {8, 4}};
constexpr int PROBE_ROWS_N = 8;

template <int BITS, int C>
static void launch_probe_rows(int blocks, int iters, const uint32_t* words, float* sink, uint64_t* clk,
                              hipStream_t st) {
    hipLaunchKernelGGL((probe_rows_kernel<BITS, PROBE_ROWS_CFG[C][0], PROBE_ROWS_CFG[C][1]>), dim3(blocks), dim3(64),
                       0, st, words, iters, sink, clk);
}
template <int BITS, int... C>
static void probe_rows_dispatch(int cfg, int blocks, int iters, const uint32_t* words, float* sink, uint64_t* clk,
                                hipStream_t st, std::integer_sequence<int, C...>) {
    ((cfg == C ? launch_probe_rows<BITS, C>(blocks, iters, words, sink, clk, st) : void()), ...);
}

// Grouped-GEMM step probe: the prefill kernels' own step functions
// (exl3_prefill.hpp mma_tile2 for a narrow tile of one or two 16-row blocks,
// mma_tile_wide for a wide tile's four) on tile words and raw A words held in
// registers and made opaque every iteration, so each iteration builds the A
// operands, decodes every window the step decodes and issues its MFMAs, with
// no memory traffic and no item overheads.  Rates are per decoded weight.
enum ProbeGemmStep : int { STEP_NARROW_1 = 0, STEP_NARROW_2 = 1, STEP_WIDE_4 = 2, STEP_WIDE_4_SUMMED = 3, STEP_KINDS = 4 };

// A wide step with each weight's two addends summed on the VALU (two byte
// permutes gather the low and the high addends of two weights, one packed f16
// add sums them), so an MFMA takes eight weights per lane: half the MFMAs,
// and the A operand of two k-groups is the lane's raw activation words (no
// duplication, no permutes).  Timing only: it rounds each weight to fp16 as
// the dequantized weight is, where the kernels' duplicated-A MFMA sums the
// addends exactly.
template <int BITS>
__device__ __forceinline__ void mma_tile_wide_summed(const uint32_t* W, const exl3::u32x4_t (&a)[4][2],
                                                     exl3::float4_t (&acc)[4][8]) {
    using namespace exl3;
    typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
    static_for<2>([&](auto RI) {
        constexpr int r2 = decltype(RI)::value;          // k-groups 2 r2, 2 r2 + 1
        __builtin_amdgcn_sched_barrier(0);
        half8_t Ar[4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            u32x4_t w;
            w[0] = a[rb][0][2 * r2]; w[1] = a[rb][1][2 * r2];
            w[2] = a[rb][0][2 * r2 + 1]; w[3] = a[rb][1][2 * r2 + 1];
            Ar[rb] = __builtin_bit_cast(half8_t, w);
        }
        static_for<8>([&](auto II) {
            constexpr int i = decltype(II)::value;
            constexpr int n = 2 * (i >> 1) + 8 * (i & 1), m = n / 2;
            u32x4_t b;
            static_for<4>([&](auto JI) {
                constexpr int j = decltype(JI)::value;
                constexpr int r = 2 * r2 + j / 2, q0 = 2 * (j & 1);
                constexpr int T0 = 32 * (n & 7) + 8 * r + 4 * (n >> 3) + q0;
                const uint32_t xa = decode_pair<BITS, CB_MCG, T0>(W);
                const uint32_t xb = decode_pair<BITS, CB_MCG, T0 + 1>(W);
                const h2_t lo = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(xb, xa, 0x01000504u));
                const h2_t hi = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(xb, xa, 0x03020706u));
                b[j] = __builtin_bit_cast(uint32_t, lo + hi);
            });
            const half8_t B = __builtin_bit_cast(half8_t, b);
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
                acc[rb][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ar[rb], B, acc[rb][m], 0, 0, 0);
        });
    });
}

template <int BITS, int KIND>
__global__ __launch_bounds__(64, 2) void probe_gemm_step_kernel(const uint32_t* __restrict__ words, int iters,
                                                               float* __restrict__ sink,
                                                               uint64_t* __restrict__ clk) {
    using namespace exl3;
    using namespace exl3::prefill;
    const int lane = threadIdx.x;
    uint32_t W[8 * BITS];
#pragma unroll
    for (int i = 0; i < 8 * BITS; ++i) W[i] = words[lane * 8 * BITS + i];
    constexpr bool WIDE = KIND == STEP_WIDE_4 || KIND == STEP_WIDE_4_SUMMED;
    constexpr int RB = WIDE ? 4 : 2;
    u32x4_t a[RB][2];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < 4; ++j) a[rb][h][j] = 0x3c003c00u ^ (uint32_t)(lane + 7 * rb + 3 * h + j);
    constexpr int NC = WIDE ? 8 : 16;
    float4_t acc[RB][NC];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < NC; ++i) acc[rb][i] = float4_t{0.f, 0.f, 0.f, 0.f};
    const uint64_t c0 = __builtin_amdgcn_s_memtime(), t0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 8 * BITS; ++i) asm volatile("" : "+v"(W[i]));
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) asm volatile("" : "+v"(a[rb][0]), "+v"(a[rb][1]));
        if constexpr (KIND == STEP_WIDE_4) {
            mma_tile_wide<BITS, CB_MCG>(W, a, acc);
        } else if constexpr (KIND == STEP_WIDE_4_SUMMED) {
            mma_tile_wide_summed<BITS>(W, a, acc);
        } else {
            const u32x4_t(&a2)[2][2] = reinterpret_cast<const u32x4_t(&)[2][2]>(a);
            float4_t(&acc2)[2][16] = reinterpret_cast<float4_t(&)[2][16]>(acc);
            mma_tile2<BITS, CB_MCG, KIND == STEP_NARROW_2>(W, a2, acc2);
        }
    }
    const uint64_t c1 = __builtin_amdgcn_s_memtime(), t1 = __builtin_amdgcn_s_memrealtime();
    float sum = 0.f;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < NC; ++i) sum += acc[rb][i][0] + acc[rb][i][1] + acc[rb][i][2] + acc[rb][i][3];
    sink[blockIdx.x * 64 + lane] = sum;
    if (lane == 0) {
        clk[2 * blockIdx.x] = c1 - c0;
        clk[2 * blockIdx.x + 1] = t1 - t0;
    }
}

template <int BITS>
static int launch_probe_gemm_step(int kind, int blocks, int iters, const uint32_t* words, float* sink, uint64_t* clk,
                                  hipStream_t st) {
    switch (kind) {
        case STEP_NARROW_1:
            hipLaunchKernelGGL((probe_gemm_step_kernel<BITS, STEP_NARROW_1>), dim3(blocks), dim3(64), 0, st, words,
                               iters, sink, clk);
            break;
        case STEP_NARROW_2:
            hipLaunchKernelGGL((probe_gemm_step_kernel<BITS, STEP_NARROW_2>), dim3(blocks), dim3(64), 0, st, words,
                               iters, sink, clk);
            break;
        case STEP_WIDE_4:
            hipLaunchKernelGGL((probe_gemm_step_kernel<BITS, STEP_WIDE_4>), dim3(blocks), dim3(64), 0, st, words,
                               iters, sink, clk);
            break;
        case STEP_WIDE_4_SUMMED:
            hipLaunchKernelGGL((probe_gemm_step_kernel<BITS, STEP_WIDE_4_SUMMED>), dim3(blocks), dim3(64), 0, st,
                               words, iters, sink, clk);
            break;
        default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// The instruction kinds of the issue-rate probe (exl3_probe_isa's `op`).
enum ProbeIsaOp : int {
    ISA_AND = 0, ISA_XOR, ISA_LSHRREV, ISA_BITOP3, ISA_MUL_LO_U16, ISA_ADD_U32,
    ISA_BFE, ISA_ALIGNBIT, ISA_PERM, ISA_MUL_LO_U32, ISA_LSHLREV, ISA_ADD3,
    // candidates for other decode sequences
    ISA_MAD_U32_U16, ISA_MAD_U32_U16_HI, ISA_PK_MAD_U16, ISA_PK_MUL_LO_U16, ISA_MAD_U16_HI,
    ISA_MUL_U32_U24, ISA_MUL_HI_U32_U24, ISA_MAD_U32_U24, ISA_MUL_HI_U32, ISA_LSHL_OR, ISA_AND_OR,
    ISA_BFI, ISA_ALIGNBYTE, ISA_XAD, ISA_OR3, ISA_LSHL_ADD, ISA_LSHRREV_V, ISA_LSHLREV_V,
    ISA_DOT2_U32_U16, ISA_PK_LSHRREV_B16, ISA_MUL_LO_U16_SDWA_HI, ISA_MUL_U32_U24_SDWA_W1,
    ISA_LSHRREV_SDWA, ISA_AND_SDWA_W0, ISA_PK_ADD_F16, ISA_ADD_F16, ISA_FMA_F32, ISA_CVT_F32_U32,
    // instruction sequences, one per call (the rate is per sequence)
    SEQ_MUL_AND, SEQ_MUL_AND2, SEQ_MUL_BITOP3, SEQ_BFE_MUL_BITOP3, SEQ_LSHR_AND_MUL_BITOP3,
    SEQ_LSHR_MUL_BITOP3, SEQ_AND_MUL_BITOP3, SEQ_PERM_AND, SEQ_BFE_MUL_BITOP3_IL,
    ISA_OPS
};

template <int OP>
__device__ __forceinline__ void isa_op(uint32_t& x, uint32_t k) {
    if constexpr (OP == ISA_AND) asm volatile("v_and_b32 %0, %0, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_XOR) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_LSHRREV) asm volatile("v_lshrrev_b32 %0, 3, %0" : "+v"(x));
    else if constexpr (OP == ISA_BITOP3) asm volatile("v_bitop3_b32 %0, %0, %1, %0 bitop3:0x6c" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_MUL_LO_U16) asm volatile("v_mul_lo_u16 %0, %0, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_ADD_U32) asm volatile("v_add_u32 %0, %0, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_BFE) asm volatile("v_bfe_u32 %0, %0, 3, 16" : "+v"(x));
    else if constexpr (OP == ISA_ALIGNBIT) asm volatile("v_alignbit_b32 %0, %0, %1, 16" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_PERM) asm volatile("v_perm_b32 %0, %0, %1, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_MUL_LO_U32) asm volatile("v_mul_lo_u32 %0, %0, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_LSHLREV) asm volatile("v_lshlrev_b32 %0, 3, %0" : "+v"(x));
    else if constexpr (OP == ISA_ADD3) asm volatile("v_add3_u32 %0, %0, %1, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_MAD_U32_U16) asm volatile("v_mad_u32_u16 %0, %0, %1, %0" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_MAD_U32_U16_HI)
        asm volatile("v_mad_u32_u16 %0, %0, %1, %0 op_sel:[1,0,0,0]" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_PK_MAD_U16) asm volatile("v_pk_mad_u16 %0, %0, %1, %0" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_PK_MUL_LO_U16) asm volatile("v_pk_mul_lo_u16 %0, %0, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_MAD_U16_HI)
        asm volatile("v_mad_u16 %0, %0, %1, %0 op_sel:[0,0,1,1]" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_MUL_U32_U24) asm volatile("v_mul_u32_u24 %0, %0, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_MUL_HI_U32_U24) asm volatile("v_mul_hi_u32_u24 %0, %0, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_MAD_U32_U24) asm volatile("v_mad_u32_u24 %0, %0, %1, %0" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_MUL_HI_U32) asm volatile("v_mul_hi_u32 %0, %0, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_LSHL_OR) asm volatile("v_lshl_or_b32 %0, %0, 3, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_AND_OR) asm volatile("v_and_or_b32 %0, %0, %1, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_BFI) asm volatile("v_bfi_b32 %0, %1, %0, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_ALIGNBYTE) asm volatile("v_alignbyte_b32 %0, %0, %1, 2" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_XAD) asm volatile("v_xad_u32 %0, %0, %1, %0" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_OR3) asm volatile("v_or3_b32 %0, %0, %1, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_LSHL_ADD) asm volatile("v_lshl_add_u32 %0, %0, 3, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_LSHRREV_V) asm volatile("v_lshrrev_b32 %0, %1, %0" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_LSHLREV_V) asm volatile("v_lshlrev_b32 %0, %1, %0" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_DOT2_U32_U16) asm volatile("v_dot2_u32_u16 %0, %0, %1, %0" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_PK_LSHRREV_B16) asm volatile("v_pk_lshrrev_b16 %0, 3, %0" : "+v"(x));
    else if constexpr (OP == ISA_MUL_LO_U16_SDWA_HI)
        asm volatile("v_mul_lo_u16_sdwa %0, %0, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 "
                     "src1_sel:WORD_0" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_MUL_U32_U24_SDWA_W1)
        asm volatile("v_mul_u32_u24_sdwa %0, %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1 "
                     "src1_sel:DWORD" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_LSHRREV_SDWA)
        asm volatile("v_lshrrev_b32_sdwa %0, %1, %0 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD "
                     "src1_sel:WORD_1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_AND_SDWA_W0)
        asm volatile("v_and_b32_sdwa %0, %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_0 "
                     "src1_sel:DWORD" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_PK_ADD_F16) asm volatile("v_pk_add_f16 %0, %0, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_ADD_F16) asm volatile("v_add_f16 %0, %0, %1" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_FMA_F32) asm volatile("v_fma_f32 %0, %0, %1, %0" : "+v"(x) : "v"(k));
    else if constexpr (OP == ISA_CVT_F32_U32) asm volatile("v_cvt_f32_u32 %0, %0" : "+v"(x));
    else static_assert(OP < SEQ_MUL_AND, "sequences run through isa_seq");
}

// One instruction sequence on each of eight independent chains, stage by
// stage (all eight chains' first instruction, then their second, ...), so a
// chain's next instruction issues eight instructions after its previous one.
#define EXL3_R8(F) F(0) F(1) F(2) F(3) F(4) F(5) F(6) F(7)
#define EXL3_MUL(i) "v_mul_lo_u32 %" #i ", %" #i ", %8\n\t"
#define EXL3_AND(i) "v_and_b32 %" #i ", %" #i ", %8\n\t"
#define EXL3_ANDC(i) "v_and_b32 %" #i ", 0xffff, %" #i "\n\t"
#define EXL3_XOR(i) "v_xor_b32 %" #i ", %" #i ", %8\n\t"
#define EXL3_BITOP3(i) "v_bitop3_b32 %" #i ", %" #i ", %8, %" #i " bitop3:0x6c\n\t"
#define EXL3_BFE(i) "v_bfe_u32 %" #i ", %" #i ", 3, 16\n\t"
#define EXL3_LSHR3(i) "v_lshrrev_b32 %" #i ", 3, %" #i "\n\t"
#define EXL3_LSHR16(i) "v_lshrrev_b32 %" #i ", 16, %" #i "\n\t"
#define EXL3_PERM(i) "v_perm_b32 %" #i ", %" #i ", %8, %8\n\t"
#define EXL3_SEQ_ASM(BODY)                                                                   \
    asm volatile(BODY : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), \
                 "+v"(x[6]), "+v"(x[7]) : "v"(k))

template <int OP>
__device__ __forceinline__ void isa_seq(uint32_t (&x)[8], uint32_t k) {
    if constexpr (OP == SEQ_MUL_AND) EXL3_SEQ_ASM(EXL3_R8(EXL3_MUL) EXL3_R8(EXL3_AND));
    else if constexpr (OP == SEQ_MUL_AND2) EXL3_SEQ_ASM(EXL3_R8(EXL3_MUL) EXL3_R8(EXL3_AND) EXL3_R8(EXL3_XOR));
    else if constexpr (OP == SEQ_MUL_BITOP3) EXL3_SEQ_ASM(EXL3_R8(EXL3_MUL) EXL3_R8(EXL3_BITOP3));
    else if constexpr (OP == SEQ_BFE_MUL_BITOP3)
        EXL3_SEQ_ASM(EXL3_R8(EXL3_BFE) EXL3_R8(EXL3_MUL) EXL3_R8(EXL3_BITOP3));
    else if constexpr (OP == SEQ_LSHR_AND_MUL_BITOP3)
        EXL3_SEQ_ASM(EXL3_R8(EXL3_LSHR3) EXL3_R8(EXL3_ANDC) EXL3_R8(EXL3_MUL) EXL3_R8(EXL3_BITOP3));
    else if constexpr (OP == SEQ_LSHR_MUL_BITOP3)
        EXL3_SEQ_ASM(EXL3_R8(EXL3_LSHR16) EXL3_R8(EXL3_MUL) EXL3_R8(EXL3_BITOP3));
    else if constexpr (OP == SEQ_AND_MUL_BITOP3)
        EXL3_SEQ_ASM(EXL3_R8(EXL3_ANDC) EXL3_R8(EXL3_MUL) EXL3_R8(EXL3_BITOP3));
    else if constexpr (OP == SEQ_PERM_AND) EXL3_SEQ_ASM(EXL3_R8(EXL3_PERM) EXL3_R8(EXL3_AND));
    else  // software-pipelined: round j extracts chain j, multiplies chain j-3, masks chain j-6
        EXL3_SEQ_ASM(EXL3_BFE(0) EXL3_MUL(5) EXL3_BITOP3(2) EXL3_BFE(1) EXL3_MUL(6) EXL3_BITOP3(3)
                     EXL3_BFE(2) EXL3_MUL(7) EXL3_BITOP3(4) EXL3_BFE(3) EXL3_MUL(0) EXL3_BITOP3(5)
                     EXL3_BFE(4) EXL3_MUL(1) EXL3_BITOP3(6) EXL3_BFE(5) EXL3_MUL(2) EXL3_BITOP3(7)
                     EXL3_BFE(6) EXL3_MUL(3) EXL3_BITOP3(0) EXL3_BFE(7) EXL3_MUL(4) EXL3_BITOP3(1));
}

template <int OP>
__global__ __launch_bounds__(256) void probe_isa_kernel(int iters, uint32_t* __restrict__ sink,
                                                        uint64_t* __restrict__ clk) {
    const int lane = threadIdx.x & 63, wave = (int)(blockIdx.x * 4 + threadIdx.x / 64);
    uint32_t x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = (uint32_t)lane * 2654435761u + (uint32_t)i;
    const uint32_t k = 0x8fff8fffu ^ (uint32_t)wave;
    const uint64_t c0 = __builtin_amdgcn_s_memtime(), t0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            if constexpr (OP >= SEQ_MUL_AND) {
                isa_seq<OP>(x, k);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) isa_op<OP>(x[i], k);
            }
        }
    }
    const uint64_t c1 = __builtin_amdgcn_s_memtime(), t1 = __builtin_amdgcn_s_memrealtime();
    uint32_t v = 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) v ^= x[i];
    sink[wave * 64 + lane] = v;
    if (lane == 0) {
        clk[2 * wave] = c1 - c0;
        clk[2 * wave + 1] = t1 - t0;
    }
}

template <int OP>
static void launch_isa(int blocks, int iters, uint32_t* sink, uint64_t* clk, hipStream_t st) {
    hipLaunchKernelGGL((probe_isa_kernel<OP>), dim3(blocks), dim3(256), 0, st, iters, sink, clk);
}

template <int... OPS>
static void isa_dispatch(int op, int blocks, int iters, uint32_t* sink, uint64_t* clk, hipStream_t st,
                         std::integer_sequence<int, OPS...>) {
    ((op == OPS ? launch_isa<OPS>(blocks, iters, sink, clk, st) : void()), ...);
}

// ---------------------------------------------------------------- cross-launch hand-off
//
// Does what one launch writes stay in the writing XCD's L2 for the next?
// probe_handoff_write: workgroup b writes 256 16-byte vectors at region b.
// probe_handoff_read: workgroup b reads region (b + shift) % blocks.
// Workgroups go to the XCDs in turn, so a shift that is a multiple of 8 reads
// data written on the reading workgroup's own XCD.
constexpr int HANDOFF_THREADS = 256;

__global__ __launch_bounds__(HANDOFF_THREADS) void probe_handoff_write(u32x4_t* buf, uint32_t salt) {
    const uint32_t i = blockIdx.x * HANDOFF_THREADS + threadIdx.x;
    buf[i] = u32x4_t{i + salt, 2u * i, 3u * i, 4u * i};
}

__global__ __launch_bounds__(HANDOFF_THREADS) void probe_handoff_read(const u32x4_t* buf, uint32_t* sink,
                                                                      int shift) {
    const uint32_t src = (blockIdx.x + (uint32_t)shift) % gridDim.x;
    const u32x4_t v = buf[src * HANDOFF_THREADS + threadIdx.x];
    sink[blockIdx.x * HANDOFF_THREADS + threadIdx.x] = v[0] ^ v[1] ^ v[2] ^ v[3];
}

extern "C" {

// Launches the probe over bytes (a multiple of 16) at buf; sink holds one
// uint32 per launched thread: blocks * 256.  Returns 0, or -1 on a bad
// argument or launch error.
int exl3_probe_read(const void* buf, int64_t bytes, uint32_t* sink, int blocks, void* stream) {
    if (!buf || !sink || bytes <= 0 || bytes % 16 || blocks < 1) return -1;
    hipLaunchKernelGGL(probe_read_kernel, dim3(blocks), dim3(PROBE_THREADS), 0, reinterpret_cast<hipStream_t>(stream),
                       reinterpret_cast<const u32x4_t*>(buf), bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int exl3_probe_threads(void) { return PROBE_THREADS; }

// `pairs` (write, read) launch pairs over `blocks` workgroups: buf holds
// blocks * 256 16-byte vectors, sink blocks * 256 uint32.  The read launch of
// each pair reads the region written `shift` workgroups on (0 <= shift).
int exl3_probe_handoff(void* buf, uint32_t* sink, int blocks, int shift, int pairs, void* stream) {
    if (!buf || !sink || blocks < 1 || shift < 0 || pairs < 1) return -1;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    for (int k = 0; k < pairs; ++k) {
        hipLaunchKernelGGL(probe_handoff_write, dim3(blocks), dim3(HANDOFF_THREADS), 0, st,
                           reinterpret_cast<u32x4_t*>(buf), (uint32_t)k);
        hipLaunchKernelGGL(probe_handoff_read, dim3(blocks), dim3(HANDOFF_THREADS), 0, st,
                           reinterpret_cast<const u32x4_t*>(buf), sink, shift);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Launches `blocks` single-wave workgroups of the decode-rate probe at `bits`
// (2, 3, 4 or 6; MCG codebook) in `mode` (0 decode + MFMA, 1 decode only, 2
// MFMA only, 3 decode + MFMA with the accumulators in AGPRs, 4 decode + the
// addends summed on the VALU + half the MFMAs), each covering 16384 weights per iteration for `iters`
// iterations.  words: 64 * 8 * bits uint32 of tile data (any values); sink:
// blocks * 64 floats; clk: 2 * blocks uint64 (per workgroup the shader clock
// cycles and the 100 MHz reference ticks of its loop, which give the clock the
// loop ran at).  Returns 0, or -1 on a bad argument or launch error.
int exl3_probe_decode_mode(int bits, int mode, int blocks, int iters, const uint32_t* words, float* sink,
                           uint64_t* clk, void* stream) {
    if (!words || !sink || !clk || blocks < 1 || iters < 1) return -1;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    switch (bits) {
        case 2: return launch_probe_decode<2>(mode, blocks, iters, words, sink, clk, st);
        case 3: return launch_probe_decode<3>(mode, blocks, iters, words, sink, clk, st);
        case 4: return launch_probe_decode<4>(mode, blocks, iters, words, sink, clk, st);
        case 6: return launch_probe_decode<6>(mode, blocks, iters, words, sink, clk, st);
        default: return -1;
    }
}

// Launches `blocks` workgroups of the wave-role probe at `bits` (2 or 3;
// MCG) in `mode` (0-2: eight waves; 0 every wave decode + MFMA, 1 waves 0-3
// decode only and 4-7 MFMA only, 2 even waves decode only and odd MFMA only;
// 3-4: twelve waves; 3 waves 0-7 decode only and 8-11 the MFMAs of two
// iterations per iteration, 4 every wave decode + MFMA), each wave covering
// 16384 weights per iteration for `iters` iterations.  words as
// exl3_probe_decode_mode; sink: blocks * 768 floats; clk: 3 * 12 * blocks
// uint64, per wave slot (12 per workgroup; eight-wave modes leave the last four
// unwritten) its loop's shader clock cycles, 100 MHz reference ticks and the
// SIMD (0-3) it ran on.  Returns 0, or -1 on a bad argument or launch error.
int exl3_probe_roles(int bits, int mode, int blocks, int iters, const uint32_t* words, float* sink, uint64_t* clk,
                     void* stream) {
    if (!words || !sink || !clk || blocks < 1 || iters < 1 || mode < 0 || mode > 4) return -1;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const dim3 threads(mode >= 3 ? 64 * PROBE_ROLES_MAX_WAVES : 512);
    if (bits == 2)
        hipLaunchKernelGGL(probe_roles_kernel<2>, dim3(blocks), threads, 0, st, words, iters, mode, sink, clk);
    else if (bits == 3)
        hipLaunchKernelGGL(probe_roles_kernel<3>, dim3(blocks), threads, 0, st, words, iters, mode, sink, clk);
    else
        return -1;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Instruction issue-rate probe: `blocks` four-wave workgroups, each wave
// running `iters` iterations of 64 instructions of kind `op` (ProbeIsaOp order:
// 0 v_and_b32 ... 11 v_add3_u32, then the candidates from 12 v_mad_u32_u16).
// sink: blocks * 256 uint32; clk: 2 * 4 * blocks uint64, per
// wave as exl3_probe_decode_mode's per workgroup.  Returns 0, or -1 on a bad
// argument or launch error.
int exl3_probe_isa(int op, int blocks, int iters, uint32_t* sink, uint64_t* clk, void* stream) {
    if (!sink || !clk || blocks < 1 || iters < 1 || op < 0 || op >= ISA_OPS) return -1;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    isa_dispatch(op, blocks, iters, sink, clk, st, std::make_integer_sequence<int, ISA_OPS>{});
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int exl3_probe_isa_ops(void) { return ISA_OPS; }

// Launches `blocks` single-wave workgroups of the row-block probe at `bits`
// (2 or 3; MCG) for configuration `cfg` (0-7: (row blocks, column divisor) =
// (1,1) (2,1) (2,2) (3,2) (4,2) (4,4) (6,4) (8,4)), each iteration decoding
// 64 * 256 / divisor weights; buffers and clocks as exl3_probe_decode_mode.
// Returns 0, or -1 on a bad argument or launch error.
int exl3_probe_rows(int bits, int cfg, int blocks, int iters, const uint32_t* words, float* sink, uint64_t* clk,
                    void* stream) {
    if (!words || !sink || !clk || blocks < 1 || iters < 1 || cfg < 0 || cfg >= PROBE_ROWS_N) return -1;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (bits == 2)
        probe_rows_dispatch<2>(cfg, blocks, iters, words, sink, clk, st, std::make_integer_sequence<int, PROBE_ROWS_N>{});
    else if (bits == 3)
        probe_rows_dispatch<3>(cfg, blocks, iters, words, sink, clk, st, std::make_integer_sequence<int, PROBE_ROWS_N>{});
    else
        return -1;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Launches `blocks` single-wave workgroups of the grouped-GEMM step probe at
// `bits` (2 or 3; MCG) for step `kind` (0 narrow tile, one row block; 1 narrow
// tile, two; 2 wide tile, four; 3 wide tile with the addends summed on the
// VALU), each iteration one step (16384 decoded weights narrow, 8192 wide);
// buffers and clocks as exl3_probe_decode_mode.
// Returns 0, or -1 on a bad argument or launch error.
int exl3_probe_gemm_step(int bits, int kind, int blocks, int iters, const uint32_t* words, float* sink,
                         uint64_t* clk, void* stream) {
    if (!words || !sink || !clk || blocks < 1 || iters < 1) return -1;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (bits == 2) return launch_probe_gemm_step<2>(kind, blocks, iters, words, sink, clk, st);
    if (bits == 3) return launch_probe_gemm_step<3>(kind, blocks, iters, words, sink, clk, st);
    return -1;
}

// The decode kernels' loop (mode 0) at `bits`.
int exl3_probe_decode(int bits, int blocks, int iters, const uint32_t* words, float* sink, uint64_t* clk,
                      void* stream) {
    return exl3_probe_decode_mode(bits, PROBE_FULL, blocks, iters, words, sink, clk, stream);
}

}  // extern "C"
