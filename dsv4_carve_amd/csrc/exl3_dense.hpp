// Dense EXL3 kernels for gfx950: trellis dequant (raw and Hadamard-folded) and
// the small-row GEMV/GEMM y = had_out(had_in(x) . Wq) * svh.  Templates only;
// exl3_dense_inst.hip instantiates them once per bit width.
#pragma once

#include "exl3_gemv.hpp"
#include "exl3_capi_util.hpp"

namespace exl3 {

// ---------------------------------------------------------------- dequant (raw)

// One lane per tile; writes the 16x16 fp16 block in row-major [K][N].
template <int BITS, int CB>
__global__ __launch_bounds__(64) void dequant_raw_kernel(const int16_t* __restrict__ trellis,
                                                         int k16, int n16, uint16_t* __restrict__ out) {
    const int tile = blockIdx.x * 64 + threadIdx.x;
    if (tile >= k16 * n16) return;
    const int kt = tile / n16, nt = tile - kt * n16;
    TileRegs<BITS> t;
    load_tile<BITS>(t, reinterpret_cast<const u32x4_t*>(trellis) + (size_t)tile * tile_vecs<BITS>());
    const uint32_t* W = t.words();
    const size_t N = (size_t)n16 * 16;
    static_for<16>([&](auto KI) {
        constexpr int k = decltype(KI)::value;
        u32x4_t row[2];
        static_for<8>([&](auto PI) {
            constexpr int p = decltype(PI)::value;
            const uint32_t lo = decode_half<BITS, CB, tile_t(k, 2 * p)>(W);
            const uint32_t hi = decode_half<BITS, CB, tile_t(k, 2 * p + 1)>(W);
            row[p >> 2][p & 3] = lo | (hi << 16);
        });
        u32x4_t* o = reinterpret_cast<u32x4_t*>(out + (size_t)(kt * 16 + k) * N + nt * 16);
        o[0] = row[0];
        o[1] = row[1];
    });
}

// ---------------------------------------------------------------- dequant (Hadamard folded)

// W = diag(suh) H Wq H diag(svh) / 128, one wave per 128x128 block, in the
// operation order of dequant_cpu (recipe-lna/lna2/bindings.cpp:80-99): row
// transforms (* 1/sqrt(128)), then column transforms, value = ((v*norm)*su)*sv.
constexpr int HB_LD = 129;   // padded LDS row (floats)

__device__ __forceinline__ void fwht128_regs(float (&v)[128]) {
    static_for<7>([&](auto SI) {
        constexpr int h = 1 << decltype(SI)::value;
        static_for<64>([&](auto JI) {
            constexpr int j = decltype(JI)::value;
            constexpr int i = (j / h) * 2 * h + (j % h);
            const float a = v[i], b = v[i + h];
            v[i] = a + b;
            v[i + h] = a - b;
        });
    });
}

template <int BITS, int CB>
__global__ __launch_bounds__(64) void dequant_had_kernel(const int16_t* __restrict__ trellis, int k16,
                                                         int n16, const uint16_t* __restrict__ suh,
                                                         const uint16_t* __restrict__ svh,
                                                         uint16_t* __restrict__ out) {
    __shared__ float mat[128 * HB_LD];
    const int lane = threadIdx.x;
    const int nbc = n16 / 8;
    const int br = blockIdx.x / nbc, bc = blockIdx.x - br * nbc;
    const size_t N = (size_t)n16 * 16;
    {
        const int kt = 8 * br + (lane >> 3), nt = 8 * bc + (lane & 7);
        TileRegs<BITS> t;
        load_tile<BITS>(t, reinterpret_cast<const u32x4_t*>(trellis) +
                               ((size_t)kt * n16 + nt) * tile_vecs<BITS>());
        const uint32_t* W = t.words();
        float* base = mat + (16 * (lane >> 3)) * HB_LD + 16 * (lane & 7);
        static_for<16>([&](auto KI) {
            constexpr int k = decltype(KI)::value;
            static_for<16>([&](auto NI) {
                constexpr int n = decltype(NI)::value;
                base[k * HB_LD + n] = f16_bits_to_f32(decode_half<BITS, CB, tile_t(k, n)>(W));
            });
        });
    }
    __syncthreads();
    for (int rr = lane; rr < 128; rr += 64) {
        float v[128];
#pragma unroll
        for (int c = 0; c < 128; ++c) v[c] = mat[rr * HB_LD + c];
        fwht128_regs(v);
#pragma unroll
        for (int c = 0; c < 128; ++c) mat[rr * HB_LD + c] = v[c] * HAD_NORM;
    }
    __syncthreads();
    for (int cc = lane; cc < 128; cc += 64) {
        float v[128];
#pragma unroll
        for (int r = 0; r < 128; ++r) v[r] = mat[r * HB_LD + cc];
        fwht128_regs(v);
        const float sv = f16_bits_to_f32(svh[128 * bc + cc]);
#pragma unroll
        for (int r = 0; r < 128; ++r) {
            float x = v[r] * HAD_NORM;
            x = x * f16_bits_to_f32(suh[128 * br + r]);
            x = x * sv;
            out[(size_t)(128 * br + r) * N + 128 * bc + cc] = f32_to_f16_bits(x);
        }
    }
}

// ---------------------------------------------------------------- dense GEMV

constexpr int GEMV_NSTEP_CAP = 8;   // k rows per item <= 512

struct GemvPlan {
    int nsteps;         // steps (64 k-rows) per item, even
    int n_kc;           // k-chunks
    int n_cb;           // 256-column blocks
    bool split_reduce;  // partial sums finished by gemv_reduce_kernel
};

inline GemvPlan gemv_plan(int64_t rows, int64_t k, int64_t n, int cus) {
    GemvPlan p;
    p.n_cb = (int)((n + COLS - 1) / COLS);
    const int ksteps = (int)(k / STEP_K);
    // Aim for >= ~4 waves per CU: small matrices need short k-chunks to spread
    // over 256 CUs (the partials are small next to the weights either way).
    int nsteps = GEMV_NSTEP_CAP;
    while (nsteps > 2 && (int64_t)p.n_cb * (ksteps / nsteps) < 4LL * cus) nsteps /= 2;
    while (ksteps % nsteps) nsteps /= 2;
    if (nsteps < 2) nsteps = 2;
    p.nsteps = nsteps;
    p.n_kc = ksteps / nsteps;
    // The last arriver of a 256-column block would sum rows * n_kc partial
    // vectors behind a device-scope counter; beyond a handful, a separate
    // reduction launch (one wave per column block and row) is shorter.
    p.split_reduce = (int64_t)(rows < MAX_ROWS ? rows : MAX_ROWS) * p.n_kc > 4;
    return p;
}

inline int64_t gemv_scratch_bytes(int64_t rows, int64_t k, int64_t n, int cus) {
    const GemvPlan p = gemv_plan(rows, k, n, cus);
    const int64_t ctr = align_up((int64_t)p.n_cb * 4, 256);
    return ctr + (int64_t)p.n_kc * (rows < 16 ? rows : 16) * n * 4;
}

// Partial sums of one (256-column block cb, k-chunk kc) item of
// y = had_in(x) . Wq for rows 0..R-1, stored as fp32 to
// partials[kc][row][N] (DEV: device-scope stores, read in the same launch;
// otherwise plain stores, read by a later launch).  xa: the block's LDS.
template <int BITS, int CB, bool DEV>
__device__ __forceinline__ void gemv_partials(const uint16_t* __restrict__ x, const int16_t* __restrict__ trellis,
                                              const uint16_t* __restrict__ suh, int R, int K, int N, int nsteps,
                                              int cb, int kc, float* __restrict__ partials, uint16_t* xa) {
    const int k0 = kc * nsteps * STEP_K;
    // weights for step 0 are in flight while the input rotation runs
    const u32x4_t* tp = tile_ptr<BITS>(trellis, N / 16, k0 / 16, cb * 16);
    TileRegs<BITS> first;
    rotate_rows_and_load<BITS>(x, K, k0, 0, suh + k0, R >= 32 ? ~0u : (1u << R) - 1u, xa, nsteps * STEP_K / 128,
                               GEMV_NSTEP_CAP, first, tp);
    __syncthreads();

    float4_t acc[16];
    mma_steps<BITS, CB, false>(first, tp, N / 16, nsteps, xa, GEMV_NSTEP_CAP, R, acc);

    const int cols = min(COLS, N - cb * COLS);
    store_partials<DEV>(acc, partials + (size_t)kc * R * N + cb * COLS, N, R, cols, reinterpret_cast<float*>(xa));
}

// SPLIT: store the partials and stop (gemv_reduce_kernel finishes them);
// otherwise the last arriver of each column block finishes it.
template <int BITS, int CB, bool SPLIT>
__global__ __launch_bounds__(64) void gemv_kernel(const uint16_t* __restrict__ x,
                                                  const int16_t* __restrict__ trellis,
                                                  const uint16_t* __restrict__ suh,
                                                  const uint16_t* __restrict__ svh, void* __restrict__ out,
                                                  int out_kind, int R, int K, int N, int nsteps, int n_kc,
                                                  int* __restrict__ counters, float* __restrict__ partials) {
    __shared__ uint16_t xa[MAX_ROWS * GEMV_NSTEP_CAP * STEP_K];
    const int lane = threadIdx.x;
    const int cb = blockIdx.x / n_kc, kc = blockIdx.x - cb * n_kc;
    gemv_partials<BITS, CB, !SPLIT>(x, trellis, suh, R, K, N, nsteps, cb, kc, partials, xa);
    if constexpr (SPLIT) return;
    publish_fence();
    int old = 0;
    if (lane == 0) old = atomicAdd(&counters[cb], 1);
    old = __shfl(old, 0, 64);
    if (old != n_kc - 1) return;

    // Last arriver: fixed-order split-K sum, output Hadamard, svh, store.
    const int col = cb * COLS + 128 * (lane >> 5) + 4 * (lane & 31);
    const bool ok = col < N;
    float sv[4] = {0.f, 0.f, 0.f, 0.f};
    if (ok)
        for (int e = 0; e < 4; ++e) sv[e] = f16_bits_to_f32(svh[col + e]);
    for (int m = 0; m < R; ++m) {
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        if (ok) {
            const float4_t t = sum_partials(partials + (size_t)m * N, (uint32_t)col * 4u, (size_t)R * N, n_kc);
            v[0] = t[0]; v[1] = t[1]; v[2] = t[2]; v[3] = t[3];
        }
        fwht128_x4(v);
        if (ok)
            for (int e = 0; e < 4; ++e) store_out(out, (size_t)m * N + col + e, out_kind, v[e] * HAD_NORM * sv[e]);
    }
    if (lane == 0) __hip_atomic_store(&counters[cb], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split-K finish of (256-column block cb, row m): the partials of chunks
// 0..n_kc-1 summed in chunk order (as the last-arriver path does), output
// Hadamard, svh, store.  Plain loads: a previous launch wrote the partials.
template <int BATCH>
__device__ __forceinline__ void gemv_reduce_block(const float* __restrict__ partials, const uint16_t* __restrict__ svh,
                                                  void* __restrict__ out, int out_kind, int R, int N, int n_kc,
                                                  int cb, int m) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int col = cb * COLS + 128 * (lane >> 5) + 4 * (lane & 31);
    const bool ok = col < N;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (ok) {
        const float* p = partials + (size_t)m * N + col;
        const size_t stride = (size_t)R * N;
        for (int k0 = 0; k0 < n_kc; k0 += BATCH) {
            float4_t t[BATCH];
#pragma unroll
            for (int j = 0; j < BATCH; ++j)
                t[j] = k0 + j < n_kc ? *reinterpret_cast<const float4_t*>(p + (size_t)(k0 + j) * stride)
                                     : float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < BATCH; ++j)
                if (k0 + j < n_kc)
                    for (int e = 0; e < 4; ++e) v[e] = v[e] + t[j][e];
        }
    }
    fwht128_x4(v);
    if (ok)
        for (int e = 0; e < 4; ++e)
            store_out(out, (size_t)m * N + col + e, out_kind, v[e] * HAD_NORM * f16_bits_to_f32(svh[col + e]));
}

// Split-K finish, one wave per (256-column block, row).  Runs after
// gemv_kernel<.., true> on the same stream.
template <int BATCH>
__global__ __launch_bounds__(64) void gemv_reduce_kernel(const float* __restrict__ partials,
                                                         const uint16_t* __restrict__ svh, void* __restrict__ out,
                                                         int out_kind, int R, int N, int n_kc) {
    const int cb = blockIdx.x / R, m = blockIdx.x - (blockIdx.x / R) * R;
    gemv_reduce_block<BATCH>(partials, svh, out, out_kind, R, N, n_kc, cb, m);
}

// ---------------------------------------------------------------- same-input fan
//
// Several matrices that read the same input x (same K, each with its own
// suh/svh, N, bit width and output): one launch of partial sums over all of
// them per bit width present, then one split-K finish launch over all of them.
// A matrix's items and sums are those of exl3_gemm at the fan's k-chunking.
// Reference counterpart: exl3_mgemm with a broadcast A (bszm_in == 1),
// recipe-lna/vllm_exl3_exl3.py.lna:546-613.

constexpr int MAX_FAN = 8;

struct FanParams {
    const uint16_t* x;
    int R, K, nsteps, n_kc, count, out_kind;
    const int16_t* trellis[MAX_FAN];
    const uint16_t* suh[MAX_FAN];
    const uint16_t* svh[MAX_FAN];
    void* out[MAX_FAN];
    float* partials[MAX_FAN];
    int N[MAX_FAN];
    int bits[MAX_FAN];
    int block0[MAX_FAN + 1];    // partial-sum items: member j owns [block0[j], block0[j+1])
    int rblock0[MAX_FAN + 1];   // finish items: member j owns [rblock0[j], rblock0[j+1])
};

__device__ __forceinline__ int fan_member(const int (&first)[MAX_FAN + 1], int count, int blk) {
    int j = 0;
    while (j + 1 < count && blk >= first[j + 1]) ++j;
    return j;
}

// Items of the members with bit width BITS; the other members' items return
// at once (one launch per width present).
template <int BITS, int CB>
__global__ __launch_bounds__(64) void gemv_fan_kernel(FanParams P) {
    __shared__ uint16_t xa[MAX_ROWS * GEMV_NSTEP_CAP * STEP_K];
    const int j = fan_member(P.block0, P.count, blockIdx.x);
    if (P.bits[j] != BITS) return;
    const int local = blockIdx.x - P.block0[j];
    const int cb = local / P.n_kc, kc = local - (local / P.n_kc) * P.n_kc;
    gemv_partials<BITS, CB, false>(P.x, P.trellis[j], P.suh[j], P.R, P.K, P.N[j], P.nsteps, cb, kc,
                                   P.partials[j], xa);
}

template <int BATCH>
__global__ __launch_bounds__(64) void gemv_fan_reduce_kernel(FanParams P) {
    const int j = fan_member(P.rblock0, P.count, blockIdx.x);
    const int local = blockIdx.x - P.rblock0[j];
    const int cb = local / P.R, m = local - (local / P.R) * P.R;
    gemv_reduce_block<BATCH>(P.partials[j], P.svh[j], P.out[j], P.out_kind, P.R, P.N[j], P.n_kc, cb, m);
}

// k-chunking of a fan: as gemv_plan, over the column blocks of every member.
inline GemvPlan gemv_fan_plan(int64_t k, int64_t total_cb, int cus) {
    GemvPlan p;
    p.n_cb = (int)total_cb;
    const int ksteps = (int)(k / STEP_K);
    int nsteps = GEMV_NSTEP_CAP;
    while (nsteps > 2 && total_cb * (ksteps / nsteps) < 4LL * cus) nsteps /= 2;
    while (ksteps % nsteps) nsteps /= 2;
    if (nsteps < 2) nsteps = 2;
    p.nsteps = nsteps;
    p.n_kc = ksteps / nsteps;
    p.split_reduce = true;
    return p;
}

// ---------------------------------------------------------------- per-bit-width launchers

struct DequantArgs {
    const int16_t* trellis; int k16, n16; int codebook;
    const uint16_t* suh; const uint16_t* svh; uint16_t* out; hipStream_t stream;
};
struct GemvArgs {
    const uint16_t* x; const int16_t* trellis; const uint16_t* suh; const uint16_t* svh;
    void* out; int out_kind; int R, K, N; GemvPlan plan; int codebook;
    int* counters; float* partials; hipStream_t stream;
};

// Defined in exl3_dense_inst.hip, one translation unit per BITS.
template <int BITS> int launch_dequant(const DequantArgs& a);
template <int BITS> int launch_gemv(const GemvArgs& a);
template <int BITS> int launch_gemv_fan(const FanParams& P, int codebook, int blocks, hipStream_t stream);

}  // namespace exl3
