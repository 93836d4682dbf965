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
// themselves, register moves at most).  The launch's block count sets the
// waves per SIMD.
//
// 3. Instruction issue rates.  One VALU instruction of the decode's kinds in a
// loop: eight independent chains per lane, 64 instructions per iteration, in
// four-wave workgroups (one wave per SIMD of a CU), so a launch of n * CUs
// workgroups puts n waves on each SIMD.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "exl3_gemv.hpp"

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

enum ProbeMode : int { PROBE_FULL = 0, PROBE_DECODE_ONLY = 1, PROBE_MFMA_ONLY = 2 };

// The decode kernels' mma_tile with the decode or the MFMA taken out (MODE).
template <int BITS, int MODE>
__device__ __forceinline__ void probe_tile(const uint32_t* W, const exl3::half8_t (&A)[4], exl3::float4_t (&acc)[16]) {
    using namespace exl3;
    if constexpr (MODE == PROBE_FULL) {
        mma_tile<BITS, CB_MCG>(W, A, acc);
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
        default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// The instruction kinds of the issue-rate probe (exl3_probe_isa's `op`).
enum ProbeIsaOp : int {
    ISA_AND = 0, ISA_XOR, ISA_LSHRREV, ISA_BITOP3, ISA_MUL_LO_U16, ISA_ADD_U32,
    ISA_BFE, ISA_ALIGNBIT, ISA_PERM, ISA_MUL_LO_U32, ISA_LSHLREV, ISA_ADD3,
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
    else asm volatile("v_add3_u32 %0, %0, %1, %1" : "+v"(x) : "v"(k));
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
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int i = 0; i < 8; ++i) isa_op<OP>(x[i], k);
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

// Launches `blocks` single-wave workgroups of the decode-rate probe at `bits`
// (2, 3, 4 or 6; MCG codebook) in `mode` (0 decode + MFMA, 1 decode only, 2
// MFMA only), each covering 16384 weights per iteration for `iters`
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

// Instruction issue-rate probe: `blocks` four-wave workgroups, each wave
// running `iters` iterations of 64 instructions of kind `op` (0 v_and_b32, 1
// v_xor_b32, 2 v_lshrrev_b32, 3 v_bitop3_b32, 4 v_mul_lo_u16, 5 v_add_u32, 6
// v_bfe_u32, 7 v_alignbit_b32, 8 v_perm_b32, 9 v_mul_lo_u32, 10 v_lshlrev_b32,
// 11 v_add3_u32).  sink: blocks * 256 uint32; clk: 2 * 4 * blocks uint64, per
// wave as exl3_probe_decode_mode's per workgroup.  Returns 0, or -1 on a bad
// argument or launch error.
int exl3_probe_isa(int op, int blocks, int iters, uint32_t* sink, uint64_t* clk, void* stream) {
    if (!sink || !clk || blocks < 1 || iters < 1 || op < 0 || op >= ISA_OPS) return -1;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    switch (op) {
        case ISA_AND: launch_isa<ISA_AND>(blocks, iters, sink, clk, st); break;
        case ISA_XOR: launch_isa<ISA_XOR>(blocks, iters, sink, clk, st); break;
        case ISA_LSHRREV: launch_isa<ISA_LSHRREV>(blocks, iters, sink, clk, st); break;
        case ISA_BITOP3: launch_isa<ISA_BITOP3>(blocks, iters, sink, clk, st); break;
        case ISA_MUL_LO_U16: launch_isa<ISA_MUL_LO_U16>(blocks, iters, sink, clk, st); break;
        case ISA_ADD_U32: launch_isa<ISA_ADD_U32>(blocks, iters, sink, clk, st); break;
        case ISA_BFE: launch_isa<ISA_BFE>(blocks, iters, sink, clk, st); break;
        case ISA_ALIGNBIT: launch_isa<ISA_ALIGNBIT>(blocks, iters, sink, clk, st); break;
        case ISA_PERM: launch_isa<ISA_PERM>(blocks, iters, sink, clk, st); break;
        case ISA_MUL_LO_U32: launch_isa<ISA_MUL_LO_U32>(blocks, iters, sink, clk, st); break;
        case ISA_LSHLREV: launch_isa<ISA_LSHLREV>(blocks, iters, sink, clk, st); break;
        default: launch_isa<ISA_ADD3>(blocks, iters, sink, clk, st); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int exl3_probe_isa_ops(void) { return ISA_OPS; }

// The decode kernels' loop (mode 0) at `bits`.
int exl3_probe_decode(int bits, int blocks, int iters, const uint32_t* words, float* sink, uint64_t* clk,
                      void* stream) {
    return exl3_probe_decode_mode(bits, PROBE_FULL, blocks, iters, words, sink, clk, stream);
}

}  // extern "C"
