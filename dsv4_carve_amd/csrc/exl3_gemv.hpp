// Shared GEMV machinery: tile-per-lane trellis decode feeding
// v_mfma_f32_16x16x32_f16, plus the 128-point Hadamard rotations on wave64.
//
// One wave processes a "step" = 4 k-slices x 16 n-tiles = 64 tiles = 64x256
// weights.  Lane l owns tile (k-slice 4s + l/16, n-tile l%16).  For output
// column n of the tile and k-group r (k in 2r+{0,1,8,9}) the four windows are
// t = 32(n&7) + 8r + 4(n>>3) + q, q = 0..3 (consecutive, see the permutation in
// exl3_decode.hpp).  The MFMA's B operand for lane l is those four weights as
// (lo, hi) fp16 addend pairs -> 8 K-slots; the A operand for lane l (row l%16,
// same k-group of k-slice 4s + l/16) is the four matching activations, each
// duplicated.  One MFMA therefore consumes 256 weights: column n of sixteen
// n-tiles across four k-slices.  The MFMA k-slot <-> k assignment is a free
// permutation (a sum is order-free up to fp32 rounding), chosen so every
// window position is a compile-time constant.
//
// Reference counterparts: the small-R GEMV core recipe-lna/lna2/lna_gemv_core.cuh:63-240
// (register decode + m16n8k16 MMA with fp16 accumulate folded to fp32) and the
// in/out Hadamard recipe-lna/lna2/lna_moe_ticket.cu:119-144, 342-343.
#pragma once

#include "exl3_decode.hpp"

namespace exl3 {

constexpr int WAVE = 64;
constexpr int STEP_K = 64;          // k rows per step (4 k-slices)
constexpr int COLS = 256;           // output columns per item (16 n-tiles)
constexpr int MAX_ROWS = 16;        // MFMA M

// LDS layout of the A operand for one item: halves [16 rows][nsteps][4 g][4 r][4 q]
__device__ __forceinline__ int xa_index(int m, int s, int nsteps_cap, int kk /*0..63*/) {
    const int g = kk >> 4, k16 = kk & 15;
    const int r = (k16 & 7) >> 1, q = (k16 & 1) + 2 * (k16 >> 3);
    return ((m * nsteps_cap + s) * 4 + g) * 16 + r * 4 + q;
}

// Where the 16-bit window of element T comes from, for the decoders that read
// it from a register half (MUL1, and the dequant kernels' codebook_half): the
// low or high half of either a tile word (free) or one funnel shift.  When
// 16 % BITS == 0 two windows 16 bits apart share one funnel (high half = the
// earlier window).
template <int BITS, int T>
struct WinSel {
    static constexpr int NB = 256 * BITS;
    static constexpr int E0 = ((T + 1) * BITS) % NB;
    static constexpr int E = E0 == 0 ? NB : E0;
    static constexpr int I1 = (E - 1) >> 5;
    static constexpr int O = E - 32 * I1;
    static constexpr bool PAIRED = (16 % BITS == 0) && (O != 16) && (O != 32) &&
                                   (((T / (16 / BITS)) & 1) == 0);
    // PAIRED: take window (T + 16/BITS) mod 256's funnel and use its high half.
    static constexpr int SRC_T = PAIRED ? (T + 16 / BITS) % 256 : T;
    static constexpr bool HI = PAIRED || (O == 16);
};

template <int BITS, int T>
__device__ __forceinline__ uint32_t win_src(const uint32_t* W) {
    using S = WinSel<BITS, T>;
    if constexpr (!S::PAIRED && S::O == 16) return W[S::I1];
    else return win_lo<BITS, S::SRC_T>(W);
}

// The window of element T alone (bits above it cleared), for the codebooks
// that multiply it as a 32-bit integer: one field extract from one register.
// A window inside a word is extracted from that word (a mask or a shift when
// it is the word's low or high half).  A window straddling words I1-1 and I1
// lies inside the 32 stream bits centred on their boundary, the funnel
// (W[I1-1]:W[I1]) >> 16; that funnel is the same expression for every window
// crossing the boundary (about 16/BITS of them), so the compiler computes it
// once per boundary and each window costs one extract.  With the single
// 32-bit multiply that follows, this takes fewer issue cycles at every width
// than a funnel per pair of windows 16 bits apart feeding two 16-bit
// multiplies that read the window halves in place (measured at 2, 3 and 4
// bits).
template <int BITS, int T>
__device__ __forceinline__ uint32_t win16(const uint32_t* W) {
    using S = WinSel<BITS, T>;
    constexpr int NW = 8 * BITS;
    if constexpr (S::O >= 16) {
        return (W[S::I1] >> (32 - S::O)) & 0xffffu;
    } else {
        // window bits [32*I1 + O - 16, 32*I1 + O): bits [16 - O, 32 - O) of the funnel
        const uint32_t mid = __builtin_amdgcn_alignbit(W[(S::I1 + NW - 1) % NW], W[S::I1], 16);
        return (mid >> (16 - S::O)) & 0xffffu;
    }
}

// EXL3_NULL_DECODE=1 builds a timing-only library (libexl3_null.so): every
// decoded B operand is replaced by a word of the loaded tile (a register move
// at most), so its kernels keep the loads, MFMAs, stores and launches of the
// real ones without the decode.  Their outputs are meaningless; the product
// library is always built with 0.
#ifndef EXL3_NULL_DECODE
#define EXL3_NULL_DECODE 0
#endif

template <int BITS, int CB, int T>
__device__ __forceinline__ uint32_t decode_pair(const uint32_t* W) {
    if constexpr (EXL3_NULL_DECODE) return W[T % (8 * BITS)];
    else if constexpr (CB == CB_MUL1) return codebook_pair<CB, WinSel<BITS, T>::HI>(win_src<BITS, T>(W));
    else return codebook_word<CB>(win16<BITS, T>(W));
}
template <int BITS, int CB, int T>
__device__ __forceinline__ uint16_t decode_half(const uint32_t* W) {
    return codebook_half<CB, WinSel<BITS, T>::HI>(win_src<BITS, T>(W));
}

// ---------------------------------------------------------------- XCD-keyed item order
//
// A launch's workgroups go to the 8 XCDs in turn (workgroup b runs on XCD
// b % 8), and what a launch writes stays in that XCD's L2 for the launches
// after it, while a read from another XCD goes to memory: writing 8 MB and
// reading it back in the next launch took 4.9 us per pair from the writing
// XCDs and 8.3 us from the others.  A launch whose output the next launch
// reads can therefore order its items by a group key the reader shares: every
// item of group g runs on XCD g % 8, and so does the reader's item for g.
// Item j of group g is workgroup 8 (per_group (g / 8) + j) + g % 8, a
// bijection onto the same grid when the group count is a multiple of 8.
// The dense GEMV and its split-K finish use it (16 rows of 4096x4096: 14.0
// against 16.0 us); in the routed-MoE phased launches the same keys (gate/up
// by column block of I, down and finish by column block of H) measured the
// same as the slot-major order at 1-16 rows, so they keep that order.
constexpr int N_XCD = 8;

// Item (g, j) of workgroup b: with `on` (0 or 1) the XCD-keyed order above,
// otherwise g = b / per_group, j = b % per_group.  One division and no branch
// on `on`: a branch on a kernel argument makes the kernel wait for that
// argument before it requests the others.
__device__ __forceinline__ void xcd_split(int b, int per_group, int on, int& g, int& j) {
    const unsigned ub = (unsigned)b, t = ub / N_XCD, x = ub % N_XCD;
    const unsigned d = on ? t : ub;
    const unsigned q = d / (unsigned)per_group;
    g = (int)(on ? x + N_XCD * q : q);
    j = (int)(d - q * (unsigned)per_group);
}

// ---------------------------------------------------------------- tile loads

// Register buffer for one tile.  CAP (16-byte vectors) may exceed the 2*BITS a
// tile needs so kernels serving several widths share one buffer; only the
// first 2*BITS vectors are loaded and decoded.
template <int CAP>
struct TileBuf {
    u32x4_t v[CAP > 0 ? CAP : 1];       // CAP 0: the buffer of a skipped item, never loaded
    __device__ __forceinline__ const uint32_t* words() const {
        return reinterpret_cast<const uint32_t*>(v);
    }
};
template <int BITS>
using TileRegs = TileBuf<2 * BITS>;
template <int BITS>
constexpr int tile_vecs() { return 2 * BITS; }      // 32*BITS bytes per tile

// A lane's tile is 32*BITS contiguous bytes read as 16-byte pieces; the lanes
// of a k-slice read neighbouring tiles, so every piece instruction touches the
// same cache lines.  Default-policy loads keep those lines in L1 for the
// remaining pieces (non-temporal loads re-fetch them from L2 each time, which
// measured ~1.4x slower for the whole decode).
template <int BITS, int CAP>
__device__ __forceinline__ void load_tile(TileBuf<CAP>& t, const u32x4_t* p) {
    static_assert(CAP >= 2 * BITS, "tile buffer too small");
    gptr_t<u32x4_t> q = as_global(p);
#pragma unroll
    for (int i = 0; i < 2 * BITS; ++i) t.v[i] = q[i];
}

// ---------------------------------------------------------------- MFMA step

// Builds the duplicated A operand for k-group r of this lane from the LDS tile.
__device__ __forceinline__ half8_t a_operand(const uint16_t* xa, int m, int s, int nsteps_cap, int g, int r) {
    const uint2 v = *reinterpret_cast<const uint2*>(xa + ((m * nsteps_cap + s) * 4 + g) * 16 + r * 4);
    // one byte permute per register: (lo, lo) and (hi, hi) of each word
    u32x4_t d;
    d[0] = __builtin_amdgcn_perm(v.x, v.x, 0x01000100u);
    d[1] = __builtin_amdgcn_perm(v.x, v.x, 0x03020302u);
    d[2] = __builtin_amdgcn_perm(v.y, v.y, 0x01000100u);
    d[3] = __builtin_amdgcn_perm(v.y, v.y, 0x03020302u);
    return __builtin_bit_cast(half8_t, d);
}

__device__ __forceinline__ void zero_acc(float4_t (&acc)[16]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = float4_t{0.f, 0.f, 0.f, 0.f};
}

// Decodes all 256 weights of the lane's tile and accumulates 64 MFMAs into acc.
template <int BITS, int CB>
__device__ __forceinline__ void mma_tile(const uint32_t* W, const half8_t (&A)[4], float4_t (&acc)[16]) {
    static_for<16>([&](auto NI) {
        constexpr int n = decltype(NI)::value;
        static_for<4>([&](auto RI) {
            constexpr int r = decltype(RI)::value;
            constexpr int T0 = 32 * (n & 7) + 8 * r + 4 * (n >> 3);
            u32x4_t b;
            b[0] = decode_pair<BITS, CB, T0 + 0>(W);
            b[1] = decode_pair<BITS, CB, T0 + 1>(W);
            b[2] = decode_pair<BITS, CB, T0 + 2>(W);
            b[3] = decode_pair<BITS, CB, T0 + 3>(W);
            acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[r], __builtin_bit_cast(half8_t, b),
                                                            acc[n], 0, 0, 0);
        });
    });
}

// Address of this lane's tile for the first step of an item, and the stride
// between steps (in 16-byte vectors).
template <int BITS>
__device__ __forceinline__ const u32x4_t* tile_ptr(const int16_t* trellis, int n16, int ks0, int nt0) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int g = lane >> 4, c = lane & 15;
    const int nt = min(nt0 + c, n16 - 1);
    return reinterpret_cast<const u32x4_t*>(trellis) + ((size_t)(ks0 + g) * n16 + nt) * tile_vecs<BITS>();
}

// Runs `nsteps` (even) steps over k-slices [ks0, ks0 + 4*nsteps) for n-tiles
// [nt0, nt0+16).  `first` must already hold the step-0 tile (issued by the
// caller with load_tile(first, tile_ptr(...)) so the loads overlap whatever the
// caller does meanwhile).  xa: LDS A tile for this item (see xa_index).  Lanes
// whose n-tile is past the matrix decode a valid tile; their columns are dropped.
// AHEAD: the load two steps ahead is issued unconditionally (the last
// iteration reloads the last step, which L1/L2 still hold).  Behind a branch,
// the compiler's wait before the next step's decode has to cover both paths
// and waits for those loads as soon as they are issued; unconditional, they
// stay in flight, at the price of the registers that keeps live (the short
// dense chunks keep more waves resident without it).
template <int BITS, int CB, bool AHEAD, int CAP>
__device__ __forceinline__ void mma_steps(TileBuf<CAP>& first, const u32x4_t* p, int n16, int nsteps,
                                          const uint16_t* xa, int nsteps_cap, int R, float4_t (&acc)[16]) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int g = lane >> 4, c = lane & 15;
    const size_t step = (size_t)4 * n16 * tile_vecs<BITS>();
    // A rows >= R repeat row R-1 (a valid row, no branch): their outputs are never stored
    const int arow = min(c, R - 1);

#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = float4_t{0.f, 0.f, 0.f, 0.f};

    // nsteps is always even: two steps per iteration, ping-ponging the tile registers
    TileBuf<CAP> second;
    for (int s = 0; s < nsteps; s += 2) {
        load_tile<BITS>(second, p + (s + 1) * step);
        {
            half8_t A[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) A[r] = a_operand(xa, arow, s, nsteps_cap, g, r);
            mma_tile<BITS, CB>(first.words(), A, acc);
        }
        if constexpr (AHEAD) load_tile<BITS>(first, p + min(s + 2, nsteps - 1) * step);
        else if (s + 2 < nsteps) load_tile<BITS>(first, p + (s + 2) * step);
        {
            half8_t A[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) A[r] = a_operand(xa, arow, s + 1, nsteps_cap, g, r);
            mma_tile<BITS, CB>(second.words(), A, acc);
        }
    }
}

// ---------------------------------------------------------------- cross-wave data
//
// Data handed from one wave to another (split-K partials, the MoE down input
// and down output) moves with device-scope relaxed atomic stores and loads.
// On gfx950 those are sc1 accesses that write through / bypass the per-XCD L2,
// so they are coherent across XCDs without a full-L2 writeback + invalidate
// (__threadfence at device scope costs one of each per call, which dominated
// every item).  A producer orders its data before the counter or flag that
// publishes it with publish_fence(); a consumer reads only after it observed
// that counter or flag through a device-scope atomic.

__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16-byte device-scope store (one instruction; consecutive lanes should write
// consecutive 16-byte chunks so the write-through traffic is whole lines).
// The compiler inserts no wait states around an asm block, so the block
// carries its own: a store of more than 8 bytes still reads its data registers
// in the cycle after issue, and a VALU write to them right behind it (which
// the register allocator is free to schedule) would change what is stored.
// Its data must not come straight from MFMA accumulators (whose wait states
// the block cannot know); callers store LDS-loaded or VALU-computed values.
__device__ __forceinline__ void st_dev4(float* p, float4_t v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st_dev2(uint32_t* p, uint2 v) {
    asm volatile("global_store_dwordx2 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
// Completes this wave's outstanding memory operations (its device-scope data
// stores included) before anything that follows, e.g. the counter or flag
// update that hands the data to another wave.
__device__ __forceinline__ void publish_fence() {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
}

// 16-byte loads through a raw buffer resource.  With the sc1 policy they are
// coherent at device scope, like the sc1 stores above (data another wave of
// the same launch published); with the default policy (0) they are plain
// cached loads, for data an earlier launch wrote.  Unlike an asm block, the
// compiler tracks their completion itself, so a batch of any size is in
// flight at once and each value is waited for where it is used.  The base
// address must be uniform across the wave; the lane's offset goes in `voff`
// and a per-load offset in `soff` (bytes, below 2 GiB in total).
constexpr int CPOL_SC1 = 16;
constexpr int CPOL_PLAIN = 0;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}
template <int CPOL = CPOL_SC1>
__device__ __forceinline__ float4_t ld_dev4_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, CPOL));
}
// No memory access is moved across this point by the compiler (loads that
// read published data stay after the counter or flag that published it).
__device__ __forceinline__ void compiler_barrier() { asm volatile("" ::: "memory"); }

// Sums two independent sets of `count` fp32 partial vectors in index order:
// a[i * stride], b[i * stride] at byte offset `voff` (the lane's columns) from
// the uniform bases a and b.  Up to 32 loads (16 of each) are in flight.
template <int CPOL = CPOL_SC1>
__device__ __forceinline__ void sum_partials2(const float* a, const float* b, uint32_t voff, size_t stride,
                                              int count, float4_t& sa, float4_t& sb) {
    compiler_barrier();
    const __amdgpu_buffer_rsrc_t ra = dev_rsrc(a), rb = dev_rsrc(b);
    const uint32_t st = (uint32_t)(stride * sizeof(float));
    sa = float4_t{0.f, 0.f, 0.f, 0.f};
    sb = sa;
    for (int i0 = 0; i0 < count; i0 += 16) {
        float4_t va[16], vb[16];
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (i0 + j < count) {
                va[j] = ld_dev4_buf<CPOL>(ra, voff, (uint32_t)(i0 + j) * st);
                vb[j] = ld_dev4_buf<CPOL>(rb, voff, (uint32_t)(i0 + j) * st);
            }
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (i0 + j < count) {
                sa += va[j];
                sb += vb[j];
            }
    }
}

// Sums `count` fp32 partial vectors p[i * stride] at byte offset `voff` from
// the uniform base p, in index order, with up to 32 loads in flight.
template <int CPOL = CPOL_SC1>
__device__ __forceinline__ float4_t sum_partials(const float* p, uint32_t voff, size_t stride, int count) {
    compiler_barrier();
    const __amdgpu_buffer_rsrc_t r = dev_rsrc(p);
    const uint32_t st = (uint32_t)(stride * sizeof(float));
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    for (int i0 = 0; i0 < count; i0 += 32) {
        float4_t v[32];
#pragma unroll
        for (int j = 0; j < 32; ++j)
            if (i0 + j < count) v[j] = ld_dev4_buf<CPOL>(r, voff, (uint32_t)(i0 + j) * st);
#pragma unroll
        for (int j = 0; j < 32; ++j)
            if (i0 + j < count) acc += v[j];
    }
    return acc;
}

// ---------------------------------------------------------------- Hadamard (wave64)

// The value of lane (lane ^ M) within rows of 16 lanes, M = 1, 2, 4 or 8, by
// DPP moves (no LDS traffic): xor 1 and 2 are quad permutations, xor 4 a quad
// reversal (xor 3) followed by the half-row mirror (xor 7), xor 8 the row
// mirror (xor 15) followed by the half-row mirror.
template <int M>
__device__ __forceinline__ float dpp_xor(float v) {
    const int x = __builtin_bit_cast(int, v);
    if constexpr (M == 1) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));
    else if constexpr (M == 2) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));
    else if constexpr (M == 4) {
        const int r = __builtin_amdgcn_mov_dpp(x, 0x1B, 0xF, 0xF, false);
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(r, 0x141, 0xF, 0xF, false));
    } else {
        static_assert(M == 8, "xor 1, 2, 4 or 8");
        const int r = __builtin_amdgcn_mov_dpp(x, 0x140, 0xF, 0xF, false);
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(r, 0x141, 0xF, 0xF, false));
    }
}

// Cross-lane butterfly of an element pair (a in the lane without the bit,
// b in the lane with it): a + b and a - b, each one exactly rounded fp32
// operation, as fma(+-1, own, partner).
__device__ __forceinline__ float bfly(float own, float partner, float sgn) {
    return __builtin_fmaf(sgn, own, partner);
}


// In-place natural-order 128-point FWHT of a block held as 2 consecutive
// elements per lane (element 2l+e in lane l), fp32, same add/sub sequence per
// element as the scalar loop in orders/F1-ref/exl3_dequant.cuh:136-147.
__device__ __forceinline__ void fwht128_x2(float& v0, float& v1) {
    const int lane = threadIdx.x & (WAVE - 1);
    {
        const float a = v0, b = v1;
        v0 = a + b;
        v1 = a - b;
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const float p0 = shfl_xor(v0, m), p1 = shfl_xor(v1, m);
        const bool upper = (lane & m) != 0;
        v0 = upper ? p0 - v0 : v0 + p0;
        v1 = upper ? p1 - v1 : v1 + p1;
    }
}

// Same transform for four independent 128-blocks, 8 consecutive elements per
// lane: lanes 16 b .. 16 b + 15 hold block b (element 8 j + e in lane j of the
// 16).  Stages h = 1, 2, 4 run in registers, h = 8 .. 64 between lanes by DPP
// moves within each row of 16 lanes (no LDS traffic); every stage pairs the
// same elements with the same operands as fwht128_x2, so the results are
// bitwise the same.
__device__ __forceinline__ void fwht128_x8(float (&v)[8]) {
    const int c = threadIdx.x & 15;
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int a = (q / h) * 2 * h + (q % h);
            const float x0 = v[a], x1 = v[a + h];
            v[a] = x0 + x1;
            v[a + h] = x0 - x1;
        }
    const float s1 = (c & 1) ? -1.f : 1.f, s2 = (c & 2) ? -1.f : 1.f;
    const float s4 = (c & 4) ? -1.f : 1.f, s8 = (c & 8) ? -1.f : 1.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = bfly(v[e], dpp_xor<1>(v[e]), s1);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = bfly(v[e], dpp_xor<2>(v[e]), s2);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = bfly(v[e], dpp_xor<4>(v[e]), s4);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = bfly(v[e], dpp_xor<8>(v[e]), s8);
}

// Same transform for two independent 128-blocks, 4 consecutive elements per
// lane: lanes 0-31 hold block 0, lanes 32-63 block 1 (element 4j+e of the block
// in lane j of the half-wave).
__device__ __forceinline__ void fwht128_x4(float (&v)[4]) {
    const int lane = threadIdx.x & (WAVE - 1);
    {
        float a = v[0], b = v[1];
        v[0] = a + b; v[1] = a - b;
        a = v[2]; b = v[3];
        v[2] = a + b; v[3] = a - b;
        a = v[0]; b = v[2];
        v[0] = a + b; v[2] = a - b;
        a = v[1]; b = v[3];
        v[1] = a + b; v[3] = a - b;
    }
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) {
        const bool upper = (lane & m) != 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float p = shfl_xor(v[e], m);
            v[e] = upper ? p - v[e] : v[e] + p;
        }
    }
}

// Input rotation of `nblocks` (<= 4) consecutive 128-element blocks of one row
// into the LDS A tile: xh = half( H (half(x * suh)) / sqrt(128) ),
// lna_moe_ticket.cu:119-144.  All global loads are issued before any math.
// x_kind: 0 = fp16, 1 = bf16 (converted to fp16 with RNE first).
constexpr int HAD_MAX_BLOCKS = 4;

// The global loads of had_in_row, apart from its arithmetic: a caller issues
// them before a weight-tile prefetch, so that waiting for them (loads complete
// in issue order) does not also wait for the tile.
struct RowIn {
    uint32_t x[HAD_MAX_BLOCKS], s[HAD_MAX_BLOCKS];
};

__device__ __forceinline__ void had_in_load(const void* x, size_t x_off, const uint16_t* suh, int nblocks, RowIn& in) {
    const int lane = threadIdx.x & (WAVE - 1);
    gptr_t<uint32_t> xp = as_global(reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(x) + x_off) + lane);
    gptr_t<uint32_t> sp = as_global(reinterpret_cast<const uint32_t*>(suh) + lane);
#pragma unroll
    for (int b = 0; b < HAD_MAX_BLOCKS; ++b)
        if (b < nblocks) {
            in.x[b] = xp[64 * b];
            in.s[b] = sp[64 * b];
        }
}

// The lane's two rotated elements (2l, 2l+1) of one 128-block, packed as fp16
// in natural order, from its loaded input pair v2 (x_kind) and sign pair s2.
__device__ __forceinline__ uint32_t had_in_pair(uint32_t v2, uint32_t s2, int x_kind) {
    if (x_kind != 0)
        v2 = (uint32_t)f32_to_f16_bits(bf16_to_f32((uint16_t)(v2 & 0xffffu))) |
             ((uint32_t)f32_to_f16_bits(bf16_to_f32((uint16_t)(v2 >> 16))) << 16);
    float v0 = f16_bits_to_f32(f32_to_f16_bits(f16_bits_to_f32(v2 & 0xffffu) * f16_bits_to_f32(s2 & 0xffffu)));
    float v1 = f16_bits_to_f32(f32_to_f16_bits(f16_bits_to_f32(v2 >> 16) * f16_bits_to_f32(s2 >> 16)));
    fwht128_x2(v0, v1);
    return (uint32_t)f32_to_f16_bits(v0 * HAD_NORM) | ((uint32_t)f32_to_f16_bits(v1 * HAD_NORM) << 16);
}

__device__ __forceinline__ void had_in_store(const RowIn& in, int x_kind, uint16_t* xa, int m, int nblocks,
                                             int nsteps_cap) {
    const int lane = threadIdx.x & (WAVE - 1);
#pragma unroll
    for (int b = 0; b < HAD_MAX_BLOCKS; ++b) {
        if (b >= nblocks) break;
        uint32_t v2 = in.x[b];
        if (x_kind != 0)
            v2 = (uint32_t)f32_to_f16_bits(bf16_to_f32((uint16_t)(v2 & 0xffffu))) |
                 ((uint32_t)f32_to_f16_bits(bf16_to_f32((uint16_t)(v2 >> 16))) << 16);
        // half(x*suh): the fp32 product of two halves is exact, so one RNE cast = half mul
        float v0 = f16_bits_to_f32(f32_to_f16_bits(f16_bits_to_f32(v2 & 0xffffu) * f16_bits_to_f32(in.s[b] & 0xffffu)));
        float v1 = f16_bits_to_f32(f32_to_f16_bits(f16_bits_to_f32(v2 >> 16) * f16_bits_to_f32(in.s[b] >> 16)));
        fwht128_x2(v0, v1);
        const int k0 = 128 * b + 2 * lane;
        xa[xa_index(m, k0 >> 6, nsteps_cap, k0 & 63)] = f32_to_f16_bits(v0 * HAD_NORM);
        xa[xa_index(m, (k0 + 1) >> 6, nsteps_cap, (k0 + 1) & 63)] = f32_to_f16_bits(v1 * HAD_NORM);
    }
}

__device__ __forceinline__ void had_in_row(const void* x, size_t x_off, int x_kind, const uint16_t* suh,
                                           uint16_t* xa, int m, int nblocks, int nsteps_cap) {
    RowIn in;
    had_in_load(x, x_off, suh, nblocks, in);
    had_in_store(in, x_kind, xa, m, nblocks, nsteps_cap);
}

// Input rotation of the rows in `mask` (row r of the tile = the r-th set bit)
// with the step-0 weight tile loaded in between: the first IN_AHEAD rows'
// inputs are requested before the tile, the rest after it.
constexpr int IN_AHEAD = 2;

template <int BITS>
__device__ __forceinline__ void rotate_rows_and_load(const void* x, size_t row_stride, size_t k0, int x_kind,
                                                     const uint16_t* suh, uint32_t mask, uint16_t* xa, int nblocks,
                                                     int nsteps_cap, TileRegs<BITS>& first, const u32x4_t* tp) {
    const int R = __popc(mask);
    RowIn in[IN_AHEAD];
    uint32_t rest = mask;
#pragma unroll
    for (int i = 0; i < IN_AHEAD; ++i)
        if (i < R) {
            const int row = __ffs((int)rest) - 1;
            rest &= rest - 1u;
            had_in_load(x, (size_t)row * row_stride + k0, suh, nblocks, in[i]);
        }
    load_tile<BITS>(first, tp);
#pragma unroll
    for (int i = 0; i < IN_AHEAD; ++i)
        if (i < R) had_in_store(in[i], x_kind, xa, i, nblocks, nsteps_cap);
    for (int r = IN_AHEAD; r < R; ++r) {
        const int row = __ffs((int)rest) - 1;
        rest &= rest - 1u;
        had_in_row(x, (size_t)row * row_stride + k0, x_kind, suh, xa, r, nblocks, nsteps_cap);
    }
}

// Copies `nblocks` (<= 4) already-rotated fp16 blocks of one row, written by
// other waves, into the LDS A tile.
template <bool DEV = true>
__device__ __forceinline__ void copy_row_load(const uint16_t* src, int nblocks, uint32_t (&v)[HAD_MAX_BLOCKS]) {
    const int lane = threadIdx.x & (WAVE - 1);
    const uint32_t* sp = reinterpret_cast<const uint32_t*>(src) + lane;
#pragma unroll
    for (int b = 0; b < HAD_MAX_BLOCKS; ++b)
        if (b < nblocks) v[b] = DEV ? ld_dev(sp + 64 * b) : sp[64 * b];
}

__device__ __forceinline__ void copy_row_store(const uint32_t (&v)[HAD_MAX_BLOCKS], uint16_t* xa, int m, int nblocks,
                                               int nsteps_cap) {
    const int lane = threadIdx.x & (WAVE - 1);
#pragma unroll
    for (int b = 0; b < HAD_MAX_BLOCKS; ++b) {
        if (b >= nblocks) break;
        const int k0 = 128 * b + 2 * lane;
        xa[xa_index(m, k0 >> 6, nsteps_cap, k0 & 63)] = (uint16_t)(v[b] & 0xffffu);
        xa[xa_index(m, (k0 + 1) >> 6, nsteps_cap, (k0 + 1) & 63)] = (uint16_t)(v[b] >> 16);
    }
}

template <bool DEV = true>
__device__ __forceinline__ void copy_row(const uint16_t* src, uint16_t* xa, int m, int nblocks, int nsteps_cap) {
    uint32_t v[HAD_MAX_BLOCKS];
    copy_row_load<DEV>(src, nblocks, v);
    copy_row_store(v, xa, m, nblocks, nsteps_cap);
}

// Writes the 16 accumulators of one item (rows < R) as fp32 partials
// dst[row * ld + col], col = 16 * (n-tile) + n within the 256-column block,
// with device-scope stores (another wave reduces them).  The MFMA result
// layout (lane = n-tile + 16 * row group, register = column in the tile) is
// transposed through LDS (`tbuf`, >= R KB, free at this point) so every store
// instruction writes one contiguous 1 KB row.  rowmap (LDS, optional): row r
// goes to dst + rowmap[r] * ld instead of dst + r * ld.  DEV: device-scope stores (the
// reader runs in the same launch); otherwise plain stores (a later launch).
template <bool DEV = true>
__device__ __forceinline__ void store_partials(const float4_t (&acc)[16], float* dst, size_t ld, int R,
                                               int cols_valid, float* tbuf, const int16_t* rowmap = nullptr) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int c = lane & 15, rg = lane >> 4;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 4 * rg + i;
        if (row < R) {
            float4_t* t = reinterpret_cast<float4_t*>(tbuf + row * COLS + 16 * c);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                t[q] = float4_t{acc[4 * q][i], acc[4 * q + 1][i], acc[4 * q + 2][i], acc[4 * q + 3][i]};
        }
    }
    __syncthreads();
    if (4 * lane < cols_valid)
        for (int row = 0; row < R; ++row) {
            const float4_t v = reinterpret_cast<const float4_t*>(tbuf + row * COLS)[lane];
            float* d = dst + (size_t)(rowmap ? rowmap[row] : row) * ld + 4 * lane;
            if constexpr (DEV) st_dev4(d, v);
            else *reinterpret_cast<float4_t*>(d) = v;
        }
}

}  // namespace exl3
