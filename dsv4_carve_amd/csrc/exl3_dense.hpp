// Dense EXL3 kernels for gfx950: trellis dequant (raw and Hadamard-folded) and
// the small-row GEMV/GEMM y = had_out(had_in(x) . Wq) * svh.  Templates only;
// exl3_dense_inst.hip instantiates them once per bit width.
#pragma once

#include <stdlib.h>

#include "exl3_gemv.hpp"
#include "exl3_capi_util.hpp"

namespace exl3 {

// ---------------------------------------------------------------- dequant (raw)

// One lane per tile; writes the 16x16 fp16 block in row-major [K][N], or with
// NK in row-major [N][K] (the transposed operand, which hipBLASLt's fp16 GEMM
// reads faster).  With NK neighbouring lanes take tiles neighbouring along k,
// so each of a lane's 16 n-rows lands next to its neighbours' in memory.
template <int BITS, int CB, bool NK = false>
__global__ __launch_bounds__(64) void dequant_raw_kernel(const int16_t* __restrict__ trellis,
                                                         int k16, int n16, uint16_t* __restrict__ out) {
    const int tile = blockIdx.x * 64 + threadIdx.x;
    if (tile >= k16 * n16) return;
    int kt, nt;
    if constexpr (NK) {
        nt = tile / k16;
        kt = tile - nt * k16;
    } else {
        kt = tile / n16;
        nt = tile - kt * n16;
    }
    TileRegs<BITS> t;
    load_tile<BITS>(t, reinterpret_cast<const u32x4_t*>(trellis) + ((size_t)kt * n16 + nt) * tile_vecs<BITS>());
    const uint32_t* W = t.words();
    if constexpr (NK) {
        const size_t K = (size_t)k16 * 16;
        static_for<16>([&](auto NI) {
            constexpr int n = decltype(NI)::value;
            u32x4_t col[2];
            static_for<8>([&](auto PI) {
                constexpr int p = decltype(PI)::value;
                const uint32_t lo = decode_half<BITS, CB, tile_t(2 * p, n)>(W);
                const uint32_t hi = decode_half<BITS, CB, tile_t(2 * p + 1, n)>(W);
                col[p >> 2][p & 3] = lo | (hi << 16);
            });
            u32x4_t* o = reinterpret_cast<u32x4_t*>(out + (size_t)(nt * 16 + n) * K + kt * 16);
            o[0] = col[0];
            o[1] = col[1];
        });
    } else {
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
}

// ---------------------------------------------------------------- dequant (Hadamard folded)

// W = diag(suh) H Wq H diag(svh) / 128 in the operation order of dequant_cpu
// (recipe-lna/lna2/bindings.cpp:80-99): row transforms (* 1/sqrt(128)), then
// column transforms, value = ((v*norm)*su)*sv.  One workgroup of four waves
// per 128x128 block:
//   1. rows: lane l of every wave owns tile (l >> 3, l & 7) of the block and
//      wave w its tile rows 4w..4w+3.  A tile row's 16 values are decoded into
//      registers, transformed by butterflies h = 1..8 in registers and
//      h = 16, 32, 64 with the lanes of the same tile row (lane ^ 1, 2, 4),
//      normalised, and written to LDS as fp32.
//   2. columns: wave w owns columns 32w..32w+31, lanes l and l ^ 32 the upper
//      and lower 64 rows of column 32w + (l & 31): butterflies h = 1..32 in
//      registers, h = 64 across the two lanes, then norm, su, sv, fp16.
// The butterfly stages run in the order h = 1, 2, ..., 64 of the reference's
// scalar loop and every butterfly is a single fp32 add or subtract of the same
// two operands, so the result is bitwise the loop's.
//
// LDS position of block element (r, c), fp32, unpadded: 16-byte chunks are
// XOR-swizzled within each aligned group of 8 by the tile column (c >> 4) & 7,
// so the eight lanes of a tile row writing the same chunk of their own tiles,
// and 32 lanes reading 32 consecutive columns of one row, fall on distinct
// banks.
__device__ __forceinline__ int hb_pos(int r, int c) {
    return r * 128 + ((((c >> 2) ^ ((c >> 4) & 7)) << 2) | (c & 3));
}

// Phase 1 for tile rows K0..K0+3 of this lane's tile.
template <int BITS, int CB, int K0>
__device__ __forceinline__ void had_rows(const uint32_t* W, int kt, int nt, float* mat) {
    const float s1 = (nt & 1) ? -1.f : 1.f, s2 = (nt & 2) ? -1.f : 1.f, s4 = (nt & 4) ? -1.f : 1.f;
    static_for<4>([&](auto KI) {
        constexpr int k = K0 + decltype(KI)::value;
        float v[16];
        static_for<16>([&](auto NI) {
            constexpr int n = decltype(NI)::value;
            v[n] = f16_bits_to_f32(decode_half<BITS, CB, tile_t(k, n)>(W));
        });
#pragma unroll
        for (int h = 1; h < 16; h <<= 1)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = (j / h) * 2 * h + (j % h);
                const float a = v[i], b = v[i + h];
                v[i] = a + b;
                v[i + h] = a - b;
            }
#pragma unroll
        for (int n = 0; n < 16; ++n) v[n] = bfly(v[n], dpp_xor<1>(v[n]), s1);
#pragma unroll
        for (int n = 0; n < 16; ++n) v[n] = bfly(v[n], dpp_xor<2>(v[n]), s2);
#pragma unroll
        for (int n = 0; n < 16; ++n) v[n] = bfly(v[n], dpp_xor<4>(v[n]), s4);
        const int r = 16 * kt + k;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *reinterpret_cast<float4_t*>(mat + hb_pos(r, 16 * nt + 4 * q)) =
                float4_t{v[4 * q] * HAD_NORM, v[4 * q + 1] * HAD_NORM, v[4 * q + 2] * HAD_NORM,
                         v[4 * q + 3] * HAD_NORM};
    });
}

template <int BITS, int CB, bool NK = false>
__global__ __launch_bounds__(256) void dequant_had_kernel(const int16_t* __restrict__ trellis, int k16,
                                                          int n16, const uint16_t* __restrict__ suh,
                                                          const uint16_t* __restrict__ svh,
                                                          uint16_t* __restrict__ out) {
    __shared__ __align__(16) float mat[128 * 128];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int nbc = n16 / 8;
    const int br = blockIdx.x / nbc, bc = blockIdx.x - br * nbc;
    const size_t N = (size_t)n16 * 16;
    {
        const int kt = lane >> 3, nt = lane & 7;
        TileRegs<BITS> t;
        load_tile<BITS>(t, reinterpret_cast<const u32x4_t*>(trellis) +
                               ((size_t)(8 * br + kt) * n16 + 8 * bc + nt) * tile_vecs<BITS>());
        const uint32_t* W = t.words();
        switch (wave) {
            case 0: had_rows<BITS, CB, 0>(W, kt, nt, mat); break;
            case 1: had_rows<BITS, CB, 4>(W, kt, nt, mat); break;
            case 2: had_rows<BITS, CB, 8>(W, kt, nt, mat); break;
            default: had_rows<BITS, CB, 12>(W, kt, nt, mat); break;
        }
    }
    const int c = 32 * wave + (lane & 31), half = lane >> 5;
    // this lane's 64 row scales (128 contiguous bytes), requested before the barrier
    u32x4_t su4[8];
    const u32x4_t* sp = reinterpret_cast<const u32x4_t*>(suh + 128 * br + 64 * half);
#pragma unroll
    for (int i = 0; i < 8; ++i) su4[i] = sp[i];
    const float sv = f16_bits_to_f32(svh[128 * bc + c]);
    __syncthreads();
    float v[64];
#pragma unroll
    for (int j = 0; j < 64; ++j) v[j] = mat[hb_pos(64 * half + j, c)];
    __syncthreads();                               // mat is free: it becomes the fp16 output tile
#pragma unroll
    for (int h = 1; h < 64; h <<= 1)
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const int i = (j / h) * 2 * h + (j % h);
            const float a = v[i], b = v[i + h];
            v[i] = a + b;
            v[i + h] = a - b;
        }
    const uint32_t* su = reinterpret_cast<const uint32_t*>(su4);
    const float s32 = half ? -1.f : 1.f;
    if constexpr (NK) {
        // this lane's 64 values are consecutive along k in output row n = 128 bc + c
        uint32_t pk[32];
#pragma unroll
        for (int j = 0; j < 64; ++j) {
            float x = bfly(v[j], shfl_xor(v[j], 32), s32);
            x = x * HAD_NORM;
            x = x * f16_bits_to_f32((uint16_t)(su[j >> 1] >> (16 * (j & 1))));
            x = x * sv;
            const uint32_t h = f32_to_f16_bits(x);
            pk[j >> 1] = (j & 1) ? (pk[j >> 1] | (h << 16)) : h;
        }
        const size_t K = (size_t)k16 * 16;
        u32x4_t* o = reinterpret_cast<u32x4_t*>(out + (size_t)(128 * bc + c) * K + 128 * br + 64 * half);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = u32x4_t{pk[4 * i], pk[4 * i + 1], pk[4 * i + 2], pk[4 * i + 3]};
        return;
    }
    uint16_t* o16 = reinterpret_cast<uint16_t*>(mat);
#pragma unroll
    for (int j = 0; j < 64; ++j) {
        float x = bfly(v[j], shfl_xor(v[j], 32), s32);
        x = x * HAD_NORM;
        x = x * f16_bits_to_f32((uint16_t)(su[j >> 1] >> (16 * (j & 1))));
        x = x * sv;
        o16[(64 * half + j) * 128 + c] = f32_to_f16_bits(x);
    }
    __syncthreads();
    // 128 rows x 256 bytes, 16 bytes per lane and pass
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int id = i * 256 + (int)threadIdx.x, row = id >> 4, seg = id & 15;
        *reinterpret_cast<u32x4_t*>(out + (size_t)(128 * br + row) * N + 128 * bc + 8 * seg) =
            *reinterpret_cast<const u32x4_t*>(o16 + row * 128 + 8 * seg);
    }
}

// ---------------------------------------------------------------- row Hadamard (had_r_128)

// y[r][128b + i] = (H128 v / sqrt(128))[i] * scale * post[128b + i] for every
// 128-block b of every row r, v = x[r][128b ..]; with a pre scale v is
// half(half(x) * pre), the rounding of the GEMV path's input rotation.  Butterflies
// in fp32, h = 1, 2, ..., 64.  One wave per (row, two blocks): lanes 0-31 and
// 32-63 hold one block each, 4 consecutive elements per lane; a block past the
// row (odd block count) is computed from block 2p and not stored.
__device__ __forceinline__ void load4_kind(const void* p, int kind, size_t i, float (&v)[4], bool to_half) {
    if (kind == OUT_F32) {
        const float4_t f = *reinterpret_cast<const float4_t*>(reinterpret_cast<const float*>(p) + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = to_half ? f16_bits_to_f32(f32_to_f16_bits(f[e])) : f[e];
    } else {
        const uint2 u = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p) + i);
        const uint16_t h[4] = {(uint16_t)(u.x & 0xffffu), (uint16_t)(u.x >> 16), (uint16_t)(u.y & 0xffffu),
                               (uint16_t)(u.y >> 16)};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (kind == OUT_F16) v[e] = f16_bits_to_f32(h[e]);
            else v[e] = to_half ? f16_bits_to_f32(f32_to_f16_bits(bf16_to_f32(h[e]))) : bf16_to_f32(h[e]);
        }
    }
}

template <int DUMMY = 0>
__global__ __launch_bounds__(64) void had_rows_kernel(const void* x, int x_kind, void* y, int y_kind, int cols,
                                                      const uint16_t* pre, const uint16_t* post, float scale) {
    const int nb = cols / 128, npair = (nb + 1) / 2;
    const int r = blockIdx.x / npair, pb = blockIdx.x - r * npair;
    const int lane = threadIdx.x;
    int b = 2 * pb + (lane >> 5);
    const bool keep = b < nb;
    if (!keep) b = 2 * pb;
    const int c0 = 128 * b + 4 * (lane & 31);
    const size_t i0 = (size_t)r * cols + c0;
    float v[4];
    load4_kind(x, x_kind, i0, v, pre != nullptr);
    if (pre) {
        const uint2 u = *reinterpret_cast<const uint2*>(pre + c0);
        const uint16_t s[4] = {(uint16_t)(u.x & 0xffffu), (uint16_t)(u.x >> 16), (uint16_t)(u.y & 0xffffu),
                               (uint16_t)(u.y >> 16)};
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = f16_bits_to_f32(f32_to_f16_bits(v[e] * f16_bits_to_f32(s[e])));
    }
    fwht128_x4(v);
    float sv[4] = {1.f, 1.f, 1.f, 1.f};
    if (post) {
        const uint2 u = *reinterpret_cast<const uint2*>(post + c0);
        sv[0] = f16_bits_to_f32((uint16_t)(u.x & 0xffffu)); sv[1] = f16_bits_to_f32((uint16_t)(u.x >> 16));
        sv[2] = f16_bits_to_f32((uint16_t)(u.y & 0xffffu)); sv[3] = f16_bits_to_f32((uint16_t)(u.y >> 16));
    }
    if (!keep) return;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float o = v[e] * HAD_NORM;
        if (scale != 1.0f) o = o * scale;
        if (post) o = o * sv[e];
        store_out(y, i0 + e, y_kind, o);
    }
}

// ---------------------------------------------------------------- dense GEMV
//
// An item is (256-column block cb, k-chunk kc of `nsteps` 64-row steps) of
// y = had_in(x) . Wq for rows 0..R-1.  Its workgroup has W waves (1, 2 or 4):
// wave w accumulates the output columns n in [w*16/W, (w+1)*16/W) of each of
// the block's 16 n-tiles, so one step's decode is spread over W SIMDs with no
// cross-wave sum.  Every wave loads the whole tile (a lane's windows interleave
// the column groups); the repeats hit the CU's L1.  At few rows the call is
// latency-bound: the plan shortens items and splits columns until there is a
// wave per SIMD, so each wave decodes as little as possible.

constexpr int GEMV_NSTEP_CAP = 8;   // k rows per item <= 512
constexpr int GEMV_MAX_WAVES = 4;   // column groups per item
constexpr int GEMV_MAX_ROWS = 32;   // rows per call: one or two 16-row MFMA blocks share each decode

struct GemvPlan {
    int nsteps;         // steps (64 k-rows) per item
    int n_kc;           // k-chunks
    int n_cb;           // 256-column blocks
    int waves;          // waves per item (column groups), 1, 2 or 4
    bool split_reduce;  // partial sums finished by gemv_reduce_kernel
    bool xcd = false;   // items and finish keyed by column block (xcd_split)
};

// Rows of x per call of the kernels: up to 16 rows one MFMA row block, 17 and
// more two (32 rows).
inline int64_t gemv_block_rows(int64_t m) { return m > MAX_ROWS ? GEMV_MAX_ROWS : MAX_ROWS; }

// EXL3_GEMV_STEPS / EXL3_GEMV_WAVES override the plan's steps per item
// (1, 2, 4, 8; kept only if it divides the k steps) and waves per item
// (1, 2, 4); EXL3_GEMV_LAST_ARRIVER=1 finishes every call in the last
// arriving workgroup of each column block instead of a reduction launch.
// 0 or unset: the plan below.
inline int gemv_override(const char* name) {
    const char* v = getenv(name);
    const int x = v && *v ? atoi(v) : 0;
    return (x == 1 || x == 2 || x == 4 || x == 8) ? x : 0;
}

inline GemvPlan gemv_plan_cb(int64_t rows, int64_t k, int64_t total_cb, int cus) {
    static const int env_steps = gemv_override("EXL3_GEMV_STEPS");
    static const int env_waves = gemv_override("EXL3_GEMV_WAVES");
    static const bool env_last = gemv_override("EXL3_GEMV_LAST_ARRIVER") == 1;
    GemvPlan p;
    p.n_cb = (int)total_cb;
    const int ksteps = (int)(k / STEP_K);
    const int64_t r = rows < GEMV_MAX_ROWS ? rows : GEMV_MAX_ROWS;
    // Two waves per SIMD, with four column groups per item first: splitting
    // columns costs nothing but repeated (L1-hit) tile loads, while shorter
    // items cost fp32 partials (k-chunks x rows x 256 x 4 bytes per column
    // block) and finish loads.  Measured at 1, 16, 32 and 144 rows on
    // 4096x4096, 4096x1536, 1536x4096 and 4096x12288: four groups beat one
    // and two at every shape, 2-step items beat 1-step ones, and the items
    // this loop picks were the fastest or within 4% of them.
    const int64_t target = 8LL * cus;
    const int min_steps = 2;
    int nsteps = GEMV_NSTEP_CAP;
    while (nsteps > min_steps && total_cb * (ksteps / nsteps) * GEMV_MAX_WAVES < target) nsteps /= 2;
    if (env_steps && ksteps % env_steps == 0) nsteps = env_steps;
    while (ksteps % nsteps) nsteps /= 2;
    const int64_t items = total_cb * (ksteps / nsteps);
    int waves = GEMV_MAX_WAVES;
    while (waves > 1 && items * (waves / 2) >= target) waves /= 2;
    if (env_waves && env_waves <= GEMV_MAX_WAVES) waves = env_waves;
    if (r > MAX_ROWS && waves < 2) waves = 2;    // 32-row blocks are built for 2 and 4 groups
    p.nsteps = nsteps;
    p.n_kc = ksteps / nsteps;
    p.waves = waves;
    // The last arriver of a 256-column block would sum rows * n_kc partial
    // vectors behind a device-scope counter; beyond a handful, a separate
    // reduction launch is shorter.
    p.split_reduce = r * p.n_kc > 4 && !env_last;
    return p;
}

// The partial-sum items of a column block and that block's finish run on one
// XCD (xcd_split) when the column blocks (of a matrix, or of all members of a
// fan) are whole and a multiple of 8: 16 rows of 4096x4096 14.0 against 16.0
// us, the gain in the partial-sum launch.  EXL3_XCD_ORDER=0 turns it off (read
// at every call, so one process can compare both orders).
inline bool xcd_order_allowed() {
    const char* v = getenv("EXL3_XCD_ORDER");
    return !(v && *v && atoi(v) == 0);
}

inline GemvPlan gemv_plan(int64_t rows, int64_t k, int64_t n, int cus) {
    GemvPlan p = gemv_plan_cb(rows, k, (n + COLS - 1) / COLS, cus);
    p.xcd = xcd_order_allowed() && n % COLS == 0 && p.n_cb % N_XCD == 0;
    return p;
}

// Split-K partials of a matrix: [column block][row][k-chunk][256] fp32, so
// the finish of one (column block, row) reads its k-chunks from one
// contiguous range (strided reads of the same offset in every k-chunk all
// fell on a few memory channels).
inline int64_t gemv_partial_bytes(int64_t rows, int64_t n_cb, int64_t n_kc) {
    return n_cb * (rows < GEMV_MAX_ROWS ? rows : GEMV_MAX_ROWS) * n_kc * COLS * 4;
}
__device__ __forceinline__ size_t gemv_partial_off(int cb, int row, int kc, int R, int n_kc) {
    return ((size_t)(cb * R + row) * n_kc + kc) * COLS;
}

inline int64_t gemv_scratch_bytes(int64_t rows, int64_t k, int64_t n, int cus) {
    const GemvPlan p = gemv_plan(rows, k, n, cus);
    const int64_t ctr = align_up((int64_t)p.n_cb * 4, 256);
    return ctr + gemv_partial_bytes(rows, p.n_cb, p.n_kc);
}

// Input rotation of one item: rows 0..R-1, k in [k0, k0 + span), into the LDS
// A tile, by the item's W waves.  A job is (row, 128-block); for a 64-row
// item the block is rotated whole and its other half dropped.  A batch's
// loads are all issued before its arithmetic.
constexpr int ROT_BATCH = 16;

struct RotJobs {
    int kb0, nblk, jobs, span;
};
struct RotBatch {
    uint32_t x[ROT_BATCH], s[ROT_BATCH];
};

__device__ __forceinline__ RotJobs rot_jobs(int k0, int nsteps, int R) {
    RotJobs j;
    j.span = nsteps * STEP_K;
    j.kb0 = k0 & ~127;
    j.nblk = (k0 + j.span - j.kb0 + 127) >> 7;
    j.jobs = R * j.nblk;
    return j;
}

__device__ __forceinline__ void rot_load(const uint16_t* x, int K, const uint16_t* suh, const RotJobs& J, int j0,
                                         int stride, RotBatch& b) {
    const int lane = threadIdx.x & (WAVE - 1);
#pragma unroll
    for (int i = 0; i < ROT_BATCH; ++i) {
        const int j = j0 + i * stride;
        if (j < J.jobs) {
            const int m = j / J.nblk, blk = j - m * J.nblk;
            const int kk = J.kb0 + 128 * blk + 2 * lane;
            b.x[i] = *reinterpret_cast<const uint32_t*>(x + (size_t)m * K + kk);
            b.s[i] = *reinterpret_cast<const uint32_t*>(suh + kk);
        }
    }
}

__device__ __forceinline__ void rot_store(const RotJobs& J, int k0, int j0, int stride, const RotBatch& b,
                                          uint16_t* xa) {
    const int lane = threadIdx.x & (WAVE - 1);
#pragma unroll
    for (int i = 0; i < ROT_BATCH; ++i) {
        const int j = j0 + i * stride;
        if (j < J.jobs) {
            const int m = j / J.nblk, blk = j - m * J.nblk;
            const uint32_t h = had_in_pair(b.x[i], b.s[i], 0);
            const int kr = J.kb0 + 128 * blk + 2 * lane - k0;   // even: both halves in one step
            if (kr >= 0 && kr < J.span) {
                xa[xa_index(m, kr >> 6, GEMV_NSTEP_CAP, kr & 63)] = (uint16_t)(h & 0xffffu);
                xa[xa_index(m, kr >> 6, GEMV_NSTEP_CAP, (kr & 63) + 1)] = (uint16_t)(h >> 16);
            }
        }
    }
}

// Decodes output columns [N0, N0+NC) of each n-tile of the lane's tile and
// accumulates them into each of the RB 16-row blocks (acc[rb][j] = column
// N0 + j); the MFMA sequence per column and row block is the one mma_tile
// issues.
template <int BITS, int CB, int N0, int NC, int RB>
__device__ __forceinline__ void mma_tile_cols(const uint32_t* W, const half8_t (&A)[RB][4],
                                              float4_t (&acc)[RB][NC]) {
    static_for<NC>([&](auto JI) {
        constexpr int j = decltype(JI)::value;
        constexpr int n = N0 + j;
        static_for<4>([&](auto RI) {
            constexpr int r = decltype(RI)::value;
            constexpr int T0 = 32 * (n & 7) + 8 * r + 4 * (n >> 3);
            u32x4_t b;
            b[0] = decode_pair<BITS, CB, T0 + 0>(W);
            b[1] = decode_pair<BITS, CB, T0 + 1>(W);
            b[2] = decode_pair<BITS, CB, T0 + 2>(W);
            b[3] = decode_pair<BITS, CB, T0 + 3>(W);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
                acc[rb][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[rb][r], __builtin_bit_cast(half8_t, b),
                                                                     acc[rb][j], 0, 0, 0);
        });
    });
}

// The item's `nsteps` steps (any count >= 1) for columns [N0, N0+NC).  `first`
// holds step 0's tile (loaded by the caller); later tiles are loaded one step
// ahead.  The load two steps on sits behind a branch, unlike mma_steps: the
// short dense items then keep 2 waves per SIMD resident.
template <int BITS, int CB, int N0, int NC, int RB>
__device__ __forceinline__ void gemv_mma(TileRegs<BITS>& first, const u32x4_t* p, int n16, int nsteps, int R,
                                         const uint16_t* xa, float4_t (&acc)[RB][NC]) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int g = lane >> 4, c = lane & 15;
    const size_t step = (size_t)4 * n16 * tile_vecs<BITS>();
    // A rows >= R repeat row R-1 (a valid row, no branch): their outputs are never stored
    int arow[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) arow[rb] = min(16 * rb + c, R - 1);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < NC; ++i) acc[rb][i] = float4_t{0.f, 0.f, 0.f, 0.f};
    auto step_mma = [&](const TileRegs<BITS>& t, int si) {
        half8_t A[RB][4];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int r = 0; r < 4; ++r) A[rb][r] = a_operand(xa, arow[rb], si, GEMV_NSTEP_CAP, g, r);
        mma_tile_cols<BITS, CB, N0, NC, RB>(t.words(), A, acc);
    };
    TileRegs<BITS> second;
    int s = 0;
    for (; s + 1 < nsteps; s += 2) {
        load_tile<BITS>(second, p + (s + 1) * step);
        step_mma(first, s);
        if (s + 2 < nsteps) load_tile<BITS>(first, p + (s + 2) * step);
        step_mma(second, s + 1);
    }
    if (nsteps & 1) step_mma(first, s);
}

// One item by its W waves: fp32 partial sums of rows < R stored to the
// partials at gemv_partial_off(cb, row, kc) (DEV: device-scope stores, read in the same launch;
// otherwise plain stores, read by a later launch).  xa: the item's LDS.
template <int BITS, int CB, int W, int RB, bool DEV>
__device__ __forceinline__ void gemv_item(const uint16_t* __restrict__ x, const int16_t* __restrict__ trellis,
                                          const uint16_t* __restrict__ suh, int R, int K, int N, int nsteps, int cb,
                                          int kc, float* __restrict__ partials, uint16_t* xa) {
    constexpr int NC = 16 / W;
    const int lane = threadIdx.x & (WAVE - 1);
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / WAVE));
    const int k0 = kc * nsteps * STEP_K;
    const u32x4_t* tp = tile_ptr<BITS>(trellis, N / 16, k0 / 16, cb * 16);

    // first rotation batch's loads, then step 0's tile, then the rotation
    const RotJobs J = rot_jobs(k0, nsteps, R);
    RotBatch rb;
    rot_load(x, K, suh, J, w, W, rb);
    TileRegs<BITS> first;
    load_tile<BITS>(first, tp);
    rot_store(J, k0, w, W, rb, xa);
    for (int j0 = w + W * ROT_BATCH; j0 < J.jobs; j0 += W * ROT_BATCH) {
        rot_load(x, K, suh, J, j0, W, rb);
        rot_store(J, k0, j0, W, rb, xa);
    }
    __syncthreads();

    float4_t acc[RB][NC];
    if constexpr (W == 1) {
        gemv_mma<BITS, CB, 0, NC, RB>(first, tp, N / 16, nsteps, R, xa, acc);
    } else if constexpr (W == 2) {
        if (w == 0) gemv_mma<BITS, CB, 0, NC, RB>(first, tp, N / 16, nsteps, R, xa, acc);
        else gemv_mma<BITS, CB, NC, NC, RB>(first, tp, N / 16, nsteps, R, xa, acc);
    } else {
        static_assert(W == 4, "1, 2 or 4 waves per item");
        if (w == 0) gemv_mma<BITS, CB, 0, NC, RB>(first, tp, N / 16, nsteps, R, xa, acc);
        else if (w == 1) gemv_mma<BITS, CB, NC, NC, RB>(first, tp, N / 16, nsteps, R, xa, acc);
        else if (w == 2) gemv_mma<BITS, CB, 2 * NC, NC, RB>(first, tp, N / 16, nsteps, R, xa, acc);
        else gemv_mma<BITS, CB, 3 * NC, NC, RB>(first, tp, N / 16, nsteps, R, xa, acc);
    }

    // Transpose through LDS (the A tile is free once every wave is past its
    // MFMAs) so each store instruction writes one contiguous 1 KB row.
    __syncthreads();
    float* tbuf = reinterpret_cast<float*>(xa);
    {
        const int c = lane & 15, rg = lane >> 4;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * rb + 4 * rg + i;
                if (row < R) {
                    float4_t* t = reinterpret_cast<float4_t*>(tbuf + row * COLS + 16 * c + w * NC);
#pragma unroll
                    for (int q = 0; q < NC / 4; ++q)
                        t[q] = float4_t{acc[rb][4 * q][i], acc[rb][4 * q + 1][i], acc[rb][4 * q + 2][i],
                                        acc[rb][4 * q + 3][i]};
                }
            }
    }
    __syncthreads();
    const int cols = min(COLS, N - cb * COLS);
    const int n_kc = K / (nsteps * STEP_K);
    if (4 * lane < cols)
        for (int row = w; row < R; row += W) {
            const float4_t v = reinterpret_cast<const float4_t*>(tbuf + row * COLS)[lane];
            float* d = partials + gemv_partial_off(cb, row, kc, R, n_kc) + 4 * lane;
            if constexpr (DEV) st_dev4(d, v);
            else *reinterpret_cast<float4_t*>(d) = v;
        }
}

// SPLIT: store the partials and stop (gemv_reduce_kernel finishes them);
// otherwise the last arriver of each column block finishes it (wave 0).
template <int BITS, int CB, int W, int RB, bool SPLIT>
__global__ __launch_bounds__(64 * W) void gemv_kernel(const uint16_t* __restrict__ x,
                                                      const int16_t* __restrict__ trellis,
                                                      const uint16_t* __restrict__ suh,
                                                      const uint16_t* __restrict__ svh, void* __restrict__ out,
                                                      int out_kind, int R, int K, int N, int nsteps, int n_kc,
                                                      int xcd, int* __restrict__ counters,
                                                      float* __restrict__ partials) {
    __shared__ uint16_t xa[MAX_ROWS * RB * GEMV_NSTEP_CAP * STEP_K];
    int cb, kc;
    xcd_split(blockIdx.x, n_kc, xcd, cb, kc);      // group: column block
    gemv_item<BITS, CB, W, RB, !SPLIT>(x, trellis, suh, R, K, N, nsteps, cb, kc, partials, xa);
    if constexpr (SPLIT) return;
    publish_fence();
    __syncthreads();
    if (threadIdx.x >= WAVE) return;
    const int lane = threadIdx.x;
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
            const float4_t t = sum_partials(partials + gemv_partial_off(cb, m, 0, R, n_kc),
                                            (uint32_t)(col - cb * COLS) * 4u, (size_t)COLS, n_kc);
            v[0] = t[0]; v[1] = t[1]; v[2] = t[2]; v[3] = t[3];
        }
        fwht128_x4(v);
        if (ok)
            for (int e = 0; e < 4; ++e) store_out(out, (size_t)m * N + col + e, out_kind, v[e] * HAD_NORM * sv[e]);
    }
    if (lane == 0) __hip_atomic_store(&counters[cb], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split-K finish of (128-column block hb, row m): the partials of chunks
// 0..n_kc-1 summed in chunk order (as the last-arriver path does), output
// Hadamard, svh, store; two columns per lane, up to RED_BATCH loads in
// flight.  Plain loads: a previous launch wrote the partials.
constexpr int RED_BATCH = 64;

template <int BATCH>
__device__ __forceinline__ void gemv_reduce_block(const float* __restrict__ partials, const uint16_t* __restrict__ svh,
                                                  void* __restrict__ out, int out_kind, int R, int N, int n_kc,
                                                  int hb, int m) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int col = hb * 128 + 2 * lane;
    const uint32_t s2 = *reinterpret_cast<const uint32_t*>(svh + col);
    const int cb = hb >> 1;
    const float* p = partials + gemv_partial_off(cb, m, 0, R, n_kc) + (col - cb * COLS);
    const size_t stride = COLS;
    float v0 = 0.f, v1 = 0.f;
    for (int k0 = 0; k0 < n_kc; k0 += BATCH) {
        float2 t[BATCH];
#pragma unroll
        for (int j = 0; j < BATCH; ++j)
            if (k0 + j < n_kc) t[j] = *reinterpret_cast<const float2*>(p + (size_t)(k0 + j) * stride);
#pragma unroll
        for (int j = 0; j < BATCH; ++j)
            if (k0 + j < n_kc) {
                v0 = v0 + t[j].x;
                v1 = v1 + t[j].y;
            }
    }
    fwht128_x2(v0, v1);
    store_out(out, (size_t)m * N + col, out_kind, v0 * HAD_NORM * f16_bits_to_f32(s2 & 0xffffu));
    store_out(out, (size_t)m * N + col + 1, out_kind, v1 * HAD_NORM * f16_bits_to_f32(s2 >> 16));
}

// Split-K finish, one wave per (128-column block, row).  Runs after
// gemv_kernel<.., true> on the same stream.
template <int BATCH>
__global__ __launch_bounds__(64) void gemv_reduce_kernel(const float* __restrict__ partials,
                                                         const uint16_t* __restrict__ svh, void* __restrict__ out,
                                                         int out_kind, int R, int N, int n_kc, int xcd) {
    // group: the 256-column block (two 128-blocks) whose partials gemv_kernel wrote on this XCD
    int cb, j;
    xcd_split(blockIdx.x, 2 * R, xcd, cb, j);
    const int hi = j >= R ? 1 : 0;
    const int hb = 2 * cb + hi, m = j - hi * R;
    gemv_reduce_block<BATCH>(partials, svh, out, out_kind, R, N, n_kc, hb, m);
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
    int xcd;                    // items and finish keyed by the fan's column block (xcd_split)
    int block0[MAX_FAN + 1];    // partial-sum items: member j owns [block0[j], block0[j+1])
    int rblock0[MAX_FAN + 1];   // finish items (128 columns x row): member j owns [rblock0[j], rblock0[j+1])
};

__device__ __forceinline__ int fan_member(const int (&first)[MAX_FAN + 1], int count, int blk) {
    int j = 0;
    while (j + 1 < count && blk >= first[j + 1]) ++j;
    return j;
}

// Items of the members with bit width BITS; the other members' items return
// at once (one launch per width present).
template <int BITS, int CB, int W, int RB>
__global__ __launch_bounds__(64 * W) void gemv_fan_kernel(FanParams P) {
    __shared__ uint16_t xa[MAX_ROWS * RB * GEMV_NSTEP_CAP * STEP_K];
    // the members' column blocks in order are the fan's column blocks
    int g, jj;
    xcd_split(blockIdx.x, P.n_kc, P.xcd, g, jj);
    const int i = g * P.n_kc + jj;
    const int j = fan_member(P.block0, P.count, i);
    if (P.bits[j] != BITS) return;
    const int local = i - P.block0[j];
    const int cb = local / P.n_kc, kc = local - (local / P.n_kc) * P.n_kc;
    gemv_item<BITS, CB, W, RB, false>(P.x, P.trellis[j], P.suh[j], P.R, P.K, P.N[j], P.nsteps, cb, kc, P.partials[j], xa);
}

template <int BATCH>
__global__ __launch_bounds__(64) void gemv_fan_reduce_kernel(FanParams P) {
    int g, jj;
    xcd_split(blockIdx.x, 2 * P.R, P.xcd, g, jj);
    const int i = g * 2 * P.R + jj;
    const int j = fan_member(P.rblock0, P.count, i);
    const int local = i - P.rblock0[j];
    const int hb = local / P.R, m = local - (local / P.R) * P.R;
    gemv_reduce_block<BATCH>(P.partials[j], P.svh[j], P.out[j], P.out_kind, P.R, P.N[j], P.n_kc, hb, m);
}

// k-chunking of a fan: as gemv_plan, over the column blocks of every member;
// always finished by the reduction launch.
inline GemvPlan gemv_fan_plan(int64_t rows, int64_t k, int64_t total_cb, int cus) {
    GemvPlan p = gemv_plan_cb(rows, k, total_cb, cus);
    p.split_reduce = true;
    return p;
}

// ---------------------------------------------------------------- per-bit-width launchers

struct DequantArgs {
    const int16_t* trellis; int k16, n16; int codebook;
    const uint16_t* suh; const uint16_t* svh; uint16_t* out; hipStream_t stream;
    bool nk;                 // write [n][k] instead of [k][n]
};
struct GemvArgs {
    const uint16_t* x; const int16_t* trellis; const uint16_t* suh; const uint16_t* svh;
    void* out; int out_kind; int R, K, N; GemvPlan plan; int codebook;
    int* counters; float* partials; hipStream_t stream;
};

// Defined in exl3_dense_inst.hip, one translation unit per BITS.
template <int BITS> int launch_dequant(const DequantArgs& a);
template <int BITS> int launch_gemv(const GemvArgs& a);
template <int BITS> int launch_gemv_fan(const FanParams& P, int codebook, int waves, int blocks, hipStream_t stream);

}  // namespace exl3
