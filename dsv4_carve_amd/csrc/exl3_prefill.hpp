// Routed-MoE layer for many tokens (prefill): the same mathematics as the
// decode kernel (gate/up, clamped SiLU*mul, down, slot-order fp32 sum), done as
// grouped GEMMs so every decoded weight is applied to up to 32 rows.
//
// Launch sequence (one stream, no host synchronisation, no persistent state):
//   1. plan:     route (token, slot) pairs by expert (counting sort in LDS),
//                cut each expert's rows into tiles: narrow tiles of up to
//                PF_RB rows for an expert with at most PF_RB rows (and for a
//                remainder of at most PF_RB), wide tiles of up to PF_RB_WIDE
//                rows otherwise.
//   2. rotate:   Xh[proj][pair] = half(H (half(x[token] * suh[e])) / sqrt(128))
//                for the gate and up projections.
//   3. gemm:     gate/up tiles: decode each weight step once per tile and
//                feed it to the MFMAs of every 16-row block (two in a narrow
//                tile, four in a wide one); epilogue output Hadamard + svh ->
//                fp32 [pair][I].
//   4. act:      half(silu(min(g, L)) * clamp(u, -L, L)), x down_suh, input
//                Hadamard -> fp16 down input [pair][I].
//   5. gemm:     down tiles, same kernel -> fp32 [pair][H].
//   6. gather:   out[t] = sum over slots j of w[t][j] * D[pair(t, j)] in slot
//                order, one cast.
// Rounding points follow the decode kernel (lna_moe_ticket.cu:5-12), so a
// token's result equals the decode kernel's up to fp32 summation order.
// Reference counterpart: exl3_moe's M16 inner path / reconstruct_hgemm for
// many rows (recipe-lna/exllamav3/exl3.py.lna:161-218), which dequantizes the
// whole weight to HBM first.
#pragma once

#include "exl3_gemv.hpp"
#include "exl3_route.hpp"
#include "exl3_capi_util.hpp"

namespace exl3 {
namespace prefill {

constexpr int PF_RB = 32;                 // rows per narrow tile (two MFMA row blocks)
constexpr int PF_RB_WIDE = 64;            // rows per wide tile (four MFMA row blocks)
constexpr int PF_A_PAD_ROWS = 16;         // rows after each A buffer that a wide tile may read
constexpr int PF_MAX_EXPERTS = 2048;
constexpr int PF_MAX_TOPK = 9;
constexpr int PF_MAX_PAIRS = 65536;

// Words of the meta block at the head of the scratch.  The error word sits at
// byte 4, as in the decode scratch; the plan launch rewrites it every call.
constexpr int PF_META_PAIRS = 0, PF_META_ERROR = 1, PF_META_TILES = 2;
constexpr int PF_ERR_WIDTH = 1;          // an expert width outside bits_mask was routed (it contributed nothing)

struct PfLayout {
    int64_t meta, eoff, toff, tile_e, tile_r0, tile_n, tile_w, pair_slot, pair_e, pos, Xh, GU, AD, D, total;
    int64_t max_tiles;
    int ks_up, ks_down;     // k-splits: GU is [ks_up][2][pairs][I], D is [ks_down][pairs][H]
};

__host__ __device__ inline int64_t pf_al(int64_t v) { return (v + 255) / 256 * 256; }

// Tile-table entries of an expert with c routed rows: one narrow tile up to
// PF_RB rows; above that two per wide tile of up to PF_RB_WIDE rows, and one
// for a last part of at most PF_RB rows.  Never more than ceil(c / PF_RB).
__host__ __device__ inline int pf_tile_entries(int c) {
    if (c <= PF_RB) return c > 0 ? 1 : 0;
    const int full = c / PF_RB_WIDE, rem = c - full * PF_RB_WIDE;
    return 2 * full + (rem > PF_RB ? 2 : rem > 0 ? 1 : 0);
}

// k-splits of the gate/up (K = hidden) and down (K = intermediate) GEMMs: as
// many as keep an even number of 64-row steps per part, up to the cap.  More
// parts give more, shorter items, so a launch's last round leaves less of the
// GPU idle; fewer parts halve the partials written and read again.  With many
// (token, slot) pairs the launches run several rounds anyway, so the caps drop
// to 1 there: the down GEMM from 4096 pairs, the gate/up GEMM (twice the items
// per tile) from 8192.  Each part writes its own fp32 output (the output
// Hadamard and svh are linear, so they apply per part); the activation and
// gather kernels add the parts in order, so results do not depend on
// scheduling (they do depend on the pair count through the split).
constexpr int64_t PF_KS_DOWN_ONE_PAIRS = 4096, PF_KS_UP_ONE_PAIRS = 8192;
inline int pf_ksplit(int64_t K, int cap) {
    int ks = cap;
    while (ks > 1 && K % (2 * STEP_K * ks)) ks /= 2;
    return ks;
}

inline PfLayout pf_layout(int64_t pairs, int64_t H, int64_t I, int64_t E) {
    PfLayout L;
    L.ks_up = pf_ksplit(H, pairs >= PF_KS_UP_ONE_PAIRS ? 1 : 2);
    L.ks_down = pf_ksplit(I, pairs >= PF_KS_DOWN_ONE_PAIRS ? 1 : 2);
    // An expert with c rows has at most ceil(c / PF_RB) tile entries (a wide
    // tile is two entries, one per half of the column blocks).
    L.max_tiles = E + (pairs + PF_RB - 1) / PF_RB;
    int64_t o = 0;
    L.meta = o;      o = pf_al(o + 64);
    L.eoff = o;      o = pf_al(o + (E + 1) * 4);
    L.toff = o;      o = pf_al(o + (E + 1) * 4);
    L.tile_e = o;    o = pf_al(o + L.max_tiles * 4);
    L.tile_r0 = o;   o = pf_al(o + L.max_tiles * 4);
    L.tile_n = o;    o = pf_al(o + L.max_tiles * 4);
    L.tile_w = o;    o = pf_al(o + L.max_tiles * 4);
    L.pair_slot = o; o = pf_al(o + pairs * 4);
    L.pair_e = o;    o = pf_al(o + pairs * 4);
    L.pos = o;       o = pf_al(o + pairs * 4);
    // A wide tile's last row block may read up to 15 rows past its last row
    // (pf_tile_wide): the A buffers end with that many rows of padding.
    L.Xh = o;        o = pf_al(o + (2 * pairs + PF_A_PAD_ROWS) * H * 2);
    L.GU = o;        o = pf_al(o + (int64_t)L.ks_up * 2 * pairs * I * 4);
    L.AD = o;        o = pf_al(o + (pairs + PF_A_PAD_ROWS) * I * 2);
    L.D = o;         o = pf_al(o + (int64_t)L.ks_down * pairs * H * 4);
    L.total = o;
    return L;
}

struct PfParams {
    const void* x; int x_kind;
    void* out; int out_kind;
    int T, H, I, E, topk, P;             // tokens, hidden, intermediate, experts, top-k, pair slots
    const int64_t* gt; const int64_t* gsu; const int64_t* gsv;
    const int64_t* ut; const int64_t* usu; const int64_t* usv;
    const int64_t* dt; const int64_t* dsu; const int64_t* dsv;
    Route rt;                            // top-k ids / weights / expert map
    const int8_t* ebits; int bits;
    uint32_t mask;                       // widths with a GEMM launch (bit b = b-bit experts)
    float limit;
    char* scratch;
    PfLayout L;
};

template <typename T>
__device__ __forceinline__ T* pat(char* base, int64_t off) { return reinterpret_cast<T*>(base + off); }

// ---------------------------------------------------------------- 3/5. grouped GEMM tile

// Duplicated A operand for k-group r from the 16 halves of this lane's row and
// k-slice (w[j] = halves 2j, 2j+1): the four k of group r are 2r, 2r+1, 2r+8,
// 2r+9 (the order mma_tile's windows use), each twice (lo/hi addends).
__device__ __forceinline__ half8_t a_from_words(const u32x4_t& lo, const u32x4_t& hi, int r) {
    const uint32_t a = lo[r & 3], b = hi[r & 3];
    // one byte permute per register: (lo, lo) and (hi, hi) of each word
    u32x4_t d;
    d[0] = __builtin_amdgcn_perm(a, a, 0x01000100u);
    d[1] = __builtin_amdgcn_perm(a, a, 0x03020302u);
    d[2] = __builtin_amdgcn_perm(b, b, 0x01000100u);
    d[3] = __builtin_amdgcn_perm(b, b, 0x03020302u);
    return __builtin_bit_cast(half8_t, d);
}

// MFMA i of a tile: column group n and k-group r, ordered (n & 7, r, n >> 3)
// rather than mma_tile's n-outer order, so the MFMAs of columns n and n + 8
// at one k-group, whose eight windows are consecutive in the stream, run back
// to back: a funnel shared by the windows that straddle one word boundary
// then lives only across them (in the n-outer order the 32-row accumulators
// leave no registers for those funnels and the kernel spills).  Each
// accumulator still takes its k-groups in order, so the sums are bitwise the
// same.
__host__ __device__ constexpr int pf_mma_n(int i) { return (i >> 3) + 8 * (i & 1); }
__host__ __device__ constexpr int pf_mma_r(int i) { return (i >> 1) & 3; }

// The 64 MFMAs of one decoded tile in pf_mma order, each B operand applied to
// both row blocks.
// Software-pipelined by one operand: row block 1's MFMA on the previous B is
// issued halfway through decoding the next B, so no two MFMAs are adjacent
// (back to back, the second waits for the matrix pipe).
// TWO false: row block 0 only (a tile of at most 16 rows), the same MFMA
// sequence on acc[0] without block 1's.
template <int BITS, int CB, bool TWO = true>
__device__ __forceinline__ void mma_tile2(const uint32_t* W, const u32x4_t (&a)[2][2], float4_t (&acc)[2][16]) {
    half8_t A0[4], A1[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        A0[r] = a_from_words(a[0][0], a[0][1], r);
        if constexpr (TWO) A1[r] = a_from_words(a[1][0], a[1][1], r);
    }
    half8_t Bprev;
    static_for<64>([&](auto II) {
        constexpr int i = decltype(II)::value;
        constexpr int n = pf_mma_n(i), r = pf_mma_r(i);
        constexpr int T0 = 32 * (n & 7) + 8 * r + 4 * (n >> 3);
        u32x4_t b;
        b[0] = decode_pair<BITS, CB, T0 + 0>(W);
        b[1] = decode_pair<BITS, CB, T0 + 1>(W);
        if constexpr (TWO && i > 0) {
            constexpr int np = pf_mma_n(i - 1), rp = pf_mma_r(i - 1);
            acc[1][np] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1[rp], Bprev, acc[1][np], 0, 0, 0);
        }
        b[2] = decode_pair<BITS, CB, T0 + 2>(W);
        b[3] = decode_pair<BITS, CB, T0 + 3>(W);
        const half8_t B = __builtin_bit_cast(half8_t, b);
        acc[0][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0[r], B, acc[0][n], 0, 0, 0);
        Bprev = B;
    });
    if constexpr (TWO) acc[1][15] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1[3], Bprev, acc[1][15], 0, 0, 0);
}

// One (tile, 256-column block) of C[rows, N] = A[rows, K] . Wq[K, N], rows of A
// at A + (row0 + i) * K (fp16, already rotated), i < nrows <= 32; epilogue
// y = (H c / sqrt(128)) * svh written as fp32 to out + (row0 + i) * N.
// `valid` false: no item (the wave returns).
template <int BITS, int CB>
__device__ __forceinline__ void pf_tile(bool valid, const uint16_t* A, int row0, int nrows,
                                        const int16_t* trellis, const uint16_t* svh, int K, int k0, int nsteps,
                                        int N, int cb, float* out) {
    if (!valid) return;
    const int lane = threadIdx.x & (WAVE - 1);
    const int g = lane >> 4, c = lane & 15;
    const int n16 = N / 16;
    const u32x4_t* tp = tile_ptr<BITS>(trellis, n16, k0 / 16, cb * 16);
    const size_t tstep = (size_t)4 * n16 * tile_vecs<BITS>();
    // A rows of this lane: c and c + 16, k-slice g of each step.  A row past
    // nrows reads row nrows - 1 instead (valid memory, no branch in the loop):
    // its accumulator rows are never written out.
    const int ra0 = min(c, nrows - 1), ra1 = min(c + 16, nrows - 1);
    const u32x4_t* a0 = reinterpret_cast<const u32x4_t*>(A + (size_t)(row0 + max(ra0, 0)) * K + k0 + 16 * g);
    const u32x4_t* a1 = reinterpret_cast<const u32x4_t*>(A + (size_t)(row0 + max(ra1, 0)) * K + k0 + 16 * g);
    const int astep = STEP_K / 8;        // 16-byte vectors per 64 k

    float4_t acc[2][16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[0][i] = acc[1][i] = float4_t{0.f, 0.f, 0.f, 0.f};

    // nsteps (64 k-rows each, from k0) is even
    TileRegs<BITS> t0, t1;
    // A tile of at most 16 rows (most tiles under skewed routing) runs a loop
    // without row block 1's A loads and MFMAs; its rows are the same.
    auto steps = [&](auto two) {
        constexpr bool TWO = decltype(two)::value;
        // A and the tile of step s + 1 are both requested before step s's
        // MFMAs: the wait for step s's operands (loads complete in issue
        // order) leaves both prefetches in flight.
        u32x4_t ac0[2][2], ac1[2][2];
        auto load_a = [&](u32x4_t (&ac)[2][2], int s) {
            ac[0][0] = a0[s * astep]; ac[0][1] = a0[s * astep + 1];
            if constexpr (TWO) { ac[1][0] = a1[s * astep]; ac[1][1] = a1[s * astep + 1]; }
        };
        load_tile<BITS>(t0, tp);
        load_a(ac0, 0);
        for (int s = 0; s < nsteps; s += 2) {
            load_tile<BITS>(t1, tp + (s + 1) * tstep);
            load_a(ac1, s + 1);
            mma_tile2<BITS, CB, TWO>(t0.words(), ac0, acc);
            // the last iteration reloads its own step (valid addresses, unused)
            const int sn = min(s + 2, nsteps - 1);
            load_tile<BITS>(t0, tp + sn * tstep);
            load_a(ac0, sn);
            mma_tile2<BITS, CB, TWO>(t1.words(), ac1, acc);
        }
    };
    if (nrows > 16) steps(std::true_type{});
    else steps(std::false_type{});

    // Epilogue in registers.  Accumulator acc[rb][n][i] is C[16 rb + 4 g + i]
    // [16 c + n]: a 128-column Hadamard block is 8 lanes' (c = 8 h .. 8 h + 7)
    // 16 values, so butterflies h = 1..8 run over n in registers and
    // h = 16, 32, 64 across lanes c ^ 1, 2, 4 -- the stage order and pairs of
    // the row transform, so the values are bitwise those of transforming the
    // row whole.  Each lane then stores 16 consecutive columns of its rows.
    float sv[16];
    {
        const u32x4_t* sp = reinterpret_cast<const u32x4_t*>(svh + cb * COLS + 16 * c);
        const u32x4_t s0 = sp[0], s1 = sp[1];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            sv[2 * q] = f16_bits_to_f32((uint16_t)(s0[q] & 0xffffu));
            sv[2 * q + 1] = f16_bits_to_f32((uint16_t)(s0[q] >> 16));
            sv[8 + 2 * q] = f16_bits_to_f32((uint16_t)(s1[q] & 0xffffu));
            sv[8 + 2 * q + 1] = f16_bits_to_f32((uint16_t)(s1[q] >> 16));
        }
    }
    const float s1 = (c & 1) ? -1.f : 1.f, s2 = (c & 2) ? -1.f : 1.f, s4 = (c & 4) ? -1.f : 1.f;
    const int nrb = nrows > 16 ? 2 : 1;
    for (int rb = 0; rb < nrb; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v[16];
#pragma unroll
            for (int n = 0; n < 16; ++n) v[n] = rb ? acc[1][n][i] : acc[0][n][i];
#pragma unroll
            for (int h = 1; h < 16; h <<= 1)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int a = (j / h) * 2 * h + (j % h);
                    const float x0 = v[a], x1 = v[a + h];
                    v[a] = x0 + x1;
                    v[a + h] = x0 - x1;
                }
#pragma unroll
            for (int n = 0; n < 16; ++n) v[n] = bfly(v[n], dpp_xor<1>(v[n]), s1);
#pragma unroll
            for (int n = 0; n < 16; ++n) v[n] = bfly(v[n], dpp_xor<2>(v[n]), s2);
#pragma unroll
            for (int n = 0; n < 16; ++n) v[n] = bfly(v[n], dpp_xor<4>(v[n]), s4);
            const int row = 16 * rb + 4 * g + i;
            if (row < nrows) {
                float4_t* o = reinterpret_cast<float4_t*>(out + (size_t)(row0 + row) * N + cb * COLS + 16 * c);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    o[q] = float4_t{v[4 * q] * HAD_NORM * sv[4 * q], v[4 * q + 1] * HAD_NORM * sv[4 * q + 1],
                                    v[4 * q + 2] * HAD_NORM * sv[4 * q + 2], v[4 * q + 3] * HAD_NORM * sv[4 * q + 3]};
            }
        }
}

// ---------------------------------------------------------------- 3/5b. wide tiles
//
// An expert with more than PF_RB routed rows is cut into tiles of PF_RB_WIDE
// rows (a remainder of at most PF_RB rows goes to a narrow tile), so its
// weights are decoded once per 64 rows instead of once per 32.  A wide tile is
// two entries of the tile table, one per half of the column blocks, so a
// group's blocks are the same count as a narrow tile's: the two waves of a
// block share one 256-column block, 128 columns (8 n-tiles) each, and each
// wave applies every decoded B operand to four 16-row blocks.
//
// Lane c of a wave holds n-tile c >> 1 and the eight columns n = 2m + p of it,
// p = c & 1 (MFMA column c is tile column 2m + p of n-tile c >> 1).  By the
// tile permutation (tile_t), column 2m + 1's windows sit 32 elements after
// column 2m's, so a lane of parity 1 loads its tile rotated by one 32-element
// block (BITS words) and decodes the windows of the even columns at their
// compile-time positions; the stream is circular, so each rotated window holds
// the bits of the window it stands for.
//
// Accumulator acc[rb][m][i] is C[16 rb + 4 g + i][16 (c >> 1) + 2 m + (c & 1)].
// Each accumulator takes the same k-groups in the same order as a narrow
// tile's, with the same MFMA operands, and the epilogue pairs the same
// elements in the same stage order, so every row's output is bitwise what a
// narrow tile gives.

// N consecutive words at byte offset voff + soff of a buffer, in loads of at
// most four words (4-byte alignment suffices).  Constant offsets go into the
// uniform soff, so every load of a tile shares the lane's one voff.
template <int N>
__device__ __forceinline__ void load_words(uint32_t* dst, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    if constexpr (N >= 4) {
        const u32x4_t v = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
        dst[0] = v[0]; dst[1] = v[1]; dst[2] = v[2]; dst[3] = v[3];
        if constexpr (N > 4) load_words<N - 4>(dst + 4, r, voff, soff + 16);
    } else if constexpr (N == 3) {
        typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));
        const u32x3_t v = __builtin_bit_cast(u32x3_t, __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, 0));
        dst[0] = v[0]; dst[1] = v[1]; dst[2] = v[2];
    } else if constexpr (N == 2) {
        const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
        dst[0] = v.x; dst[1] = v.y;
    } else {
        dst[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
    }
}

// The words of a lane's tile that its columns' windows read, rotated by p (0
// or 1) blocks of BITS words (buffer block b is stream block (b + p) & 7).
// The even columns' windows lie in the even blocks of the rotated stream and
// reach at most 16 - BITS bits back, into the last word of the block before:
// 4 (BITS + 1) of the 8 BITS words.  The other words are never written or
// read, so they take no registers.
template <int BITS>
struct WideTile {
    uint32_t w[8 * BITS];
};

// vrot: byte offset of the lane's rotated tile (its first word plus p blocks),
// vlast: of the word before rotated block 0; soff: the step's byte offset.
template <int BITS>
__device__ __forceinline__ void load_tile_rot(WideTile<BITS>& d, __amdgpu_buffer_rsrc_t r, uint32_t vrot,
                                              uint32_t vlast, uint32_t soff) {
    load_words<BITS>(d.w, r, vrot, soff);
    load_words<1>(d.w + 8 * BITS - 1, r, vlast, soff);
#pragma unroll
    for (int b = 2; b < 8; b += 2) load_words<BITS + 1>(d.w + b * BITS - 1, r, vrot, soff + 4 * (b * BITS - 1));
}

// The MFMAs of one decoded wide-tile step: k-group r outer (the four row
// blocks' A operands of one k-group live at a time), then the lane's columns
// in pairs n, n + 8 whose eight windows are consecutive in the stream.  Row
// block 0's MFMA follows its B; blocks 1-3 take the previous B between the
// next B's window decodes, and the k-group's last B after its own.
template <int BITS, int CB>
__device__ __forceinline__ void mma_tile_wide(const uint32_t* W, const u32x4_t (&a)[4][2], float4_t (&acc)[4][8]) {
    static_for<4>([&](auto RI) {
        constexpr int r = decltype(RI)::value;
        // keeps each k-group's operand builds and decodes within the k-group,
        // so no more than one k-group's A operands are live
        __builtin_amdgcn_sched_barrier(0);
        half8_t Ar[4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) Ar[rb] = a_from_words(a[rb][0], a[rb][1], r);
        half8_t Bprev;
        static_for<8>([&](auto II) {
            constexpr int i = decltype(II)::value;
            constexpr int n = 2 * (i >> 1) + 8 * (i & 1), m = n / 2;
            constexpr int ip = i > 0 ? i - 1 : 0;
            constexpr int mp = (2 * (ip >> 1) + 8 * (ip & 1)) / 2;
            constexpr int T0 = 32 * (n & 7) + 8 * r + 4 * (n >> 3);
            u32x4_t b;
            static_for<4>([&](auto QI) {
                constexpr int q = decltype(QI)::value;
                b[q] = decode_pair<BITS, CB, T0 + q>(W);
                if constexpr (i > 0 && q < 3)
                    acc[q + 1][mp] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ar[q + 1], Bprev, acc[q + 1][mp], 0, 0, 0);
            });
            const half8_t B = __builtin_bit_cast(half8_t, b);
            acc[0][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ar[0], B, acc[0][m], 0, 0, 0);
            Bprev = B;
        });
        static_for<3>([&](auto BI) {
            constexpr int rb = 1 + decltype(BI)::value;
            acc[rb][7] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ar[rb], Bprev, acc[rb][7], 0, 0, 0);
        });
    });
}

// One (wide tile, 128-column block c128) of C[rows, N] = A[rows, K] . Wq[K, N]:
// as pf_tile, for nrows <= 64 rows of A from row0.
// A wave-uniform pointer in scalar registers.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

template <int BITS, int CB>
__device__ __forceinline__ void pf_tile_wide(bool valid, const uint16_t* A, int row0, int nrows,
                                             const int16_t* trellis, const uint16_t* svh, int K, int k0, int nsteps,
                                             int N, int c128, float* out) {
    if (!valid) return;
    // every argument is the same across the wave; in scalar registers, the
    // buffer resources below need no per-lane handling
    A = uniform_ptr(A);
    trellis = uniform_ptr(trellis);
    svh = uniform_ptr(svh);
    out = uniform_ptr(out);
    row0 = __builtin_amdgcn_readfirstlane(row0);
    nrows = __builtin_amdgcn_readfirstlane(nrows);
    k0 = __builtin_amdgcn_readfirstlane(k0);
    const int lane = threadIdx.x & (WAVE - 1);
    const int g = lane >> 4, c = lane & 15, j = c >> 1, p = c & 1;
    const int n16 = N / 16;
    const int nt = 8 * c128 + j;                      // N is a multiple of 256, c128 < N / 128
    constexpr int TW = 8 * BITS;                      // words per tile
    // one matrix's trellis is below 2 GiB, so byte offsets fit 32 bits
    const __amdgpu_buffer_rsrc_t trsrc = dev_rsrc(trellis);
    const uint32_t vtile = ((uint32_t)(k0 / 16 + g) * (uint32_t)n16 + (uint32_t)nt) * (uint32_t)(TW * 4);
    const uint32_t vrot = vtile + 4 * p * BITS, vlast = vtile + 4 * (p ? BITS - 1 : TW - 1);
    const uint32_t tstep = 4u * 4u * (uint32_t)n16 * TW;   // bytes between steps
    // A rows of this lane: 16 rb + c, k-slice g of each step.  A row block
    // wholly past nrows re-reads block 0; in the last block that holds rows,
    // lanes past nrows read up to 15 rows beyond the tile's last row (other
    // pairs' rows, or the padding rows that end each A buffer).  Their
    // accumulator rows are never stored.  So one lane offset serves every row
    // block, the block's offset going in the uniform part.
    const __amdgpu_buffer_rsrc_t arsrc = dev_rsrc(A + (size_t)row0 * K + k0);
    const uint32_t avo = ((uint32_t)c * (uint32_t)K + 16u * g) * 2u;
    uint32_t arb[4];                                   // byte offset of each row block's rows
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) arb[rb] = 16 * rb < nrows ? 32u * (uint32_t)K * rb : 0u;

    float4_t acc[4][8];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int m = 0; m < 8; ++m) acc[rb][m] = float4_t{0.f, 0.f, 0.f, 0.f};

    WideTile<BITS> t0, t1;
    u32x4_t ac[4][2];
    auto load_a = [&](int s) {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            ac[rb][0] = __builtin_bit_cast(u32x4_t, ld_dev4_buf<CPOL_PLAIN>(arsrc, avo, (uint32_t)s * 128u + arb[rb]));
            ac[rb][1] =
                __builtin_bit_cast(u32x4_t, ld_dev4_buf<CPOL_PLAIN>(arsrc, avo, (uint32_t)s * 128u + arb[rb] + 16u));
        }
    };
    // nsteps is even; the step's A loads go out before the next step's tile
    load_tile_rot<BITS>(t0, trsrc, vrot, vlast, 0u);
    for (int s = 0; s < nsteps; s += 2) {
        load_a(s);
        load_tile_rot<BITS>(t1, trsrc, vrot, vlast, (uint32_t)(s + 1) * tstep);
        mma_tile_wide<BITS, CB>(t0.w, ac, acc);
        load_a(s + 1);
        // the last iteration reloads its own step (a valid address, unused)
        load_tile_rot<BITS>(t0, trsrc, vrot, vlast, (uint32_t)min(s + 2, nsteps - 1) * tstep);
        mma_tile_wide<BITS, CB>(t1.w, ac, acc);
    }

    // Epilogue in registers.  The 128 columns of the wave are one Hadamard
    // block, column 16 j + 2 m + p: stage h = 1 pairs lanes c, c ^ 1; h = 2, 4,
    // 8 run over m in registers; h = 16, 32, 64 pair lanes c ^ 2, 4, 8.  Then
    // each lane swaps half its values with lane c ^ 1 so that it stores eight
    // consecutive columns, 16 j + 8 p .. + 7, of each of its rows.
    float sv[8];
    {
        const u32x4_t* sp = reinterpret_cast<const u32x4_t*>(svh + (size_t)16 * nt);
        const u32x4_t s0 = sp[0], s1 = sp[1];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            sv[m] = f16_bits_to_f32((uint16_t)(p ? s0[m] >> 16 : s0[m] & 0xffffu));
            sv[4 + m] = f16_bits_to_f32((uint16_t)(p ? s1[m] >> 16 : s1[m] & 0xffffu));
        }
    }
    const float sg1 = (c & 1) ? -1.f : 1.f, sg2 = (c & 2) ? -1.f : 1.f;
    const float sg4 = (c & 4) ? -1.f : 1.f, sg8 = (c & 8) ? -1.f : 1.f;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        if (16 * rb >= nrows) break;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v[8];
#pragma unroll
            for (int m = 0; m < 8; ++m) v[m] = acc[rb][m][i];
#pragma unroll
            for (int m = 0; m < 8; ++m) v[m] = bfly(v[m], dpp_xor<1>(v[m]), sg1);
#pragma unroll
            for (int h = 1; h < 8; h <<= 1)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int a = (q / h) * 2 * h + (q % h);
                    const float x0 = v[a], x1 = v[a + h];
                    v[a] = x0 + x1;
                    v[a + h] = x0 - x1;
                }
#pragma unroll
            for (int m = 0; m < 8; ++m) v[m] = bfly(v[m], dpp_xor<2>(v[m]), sg2);
#pragma unroll
            for (int m = 0; m < 8; ++m) v[m] = bfly(v[m], dpp_xor<4>(v[m]), sg4);
#pragma unroll
            for (int m = 0; m < 8; ++m) v[m] = bfly(v[m], dpp_xor<8>(v[m]), sg8);
            float y[8], o[8];
#pragma unroll
            for (int m = 0; m < 8; ++m) y[m] = v[m] * HAD_NORM * sv[m];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                // parity 0 keeps columns 2q (own) and 2q + 1 (partner's y[q]);
                // parity 1 keeps 8 + 2q (partner's y[4 + q]) and 9 + 2q (own)
                const float r = dpp_xor<1>(p ? y[q] : y[4 + q]);
                o[2 * q] = p ? r : y[q];
                o[2 * q + 1] = p ? y[4 + q] : r;
            }
            const int row = 16 * rb + 4 * g + i;
            if (row < nrows) {
                float4_t* dst = reinterpret_cast<float4_t*>(out + (size_t)(row0 + row) * N + 128 * c128 + 16 * j + 8 * p);
                dst[0] = float4_t{o[0], o[1], o[2], o[3]};
                dst[1] = float4_t{o[4], o[5], o[6], o[7]};
            }
        }
    }
}

// Items: gate/up (DOWN = false) = (tile, projection, k-part, column block of
// I); down (DOWN = true) = (tile, k-part, column block of H).  The items of
// one (tile, projection, k-part) -- a group -- read the same rows of A.  Two
// waves per block take two neighbouring column blocks of a group (the
// epilogue needs no LDS, so the waves share nothing but their A rows in L2).
//
// Workgroups go to the eight XCDs in turn (block b to XCD b % 8), and each XCD
// has its own L2.  Group g is given to XCD g % 8 as consecutive blocks of that
// XCD's sequence, so its A rows are read into one L2 and shared there by
// every block of the group; with eight (projection, k-part) pairs per tile,
// each XCD also keeps the same pair across tiles, so consecutive tiles of a
// hot expert find that pair's weight slice in its L2.  Groups go round the
// XCDs in tile order, so the tiles of one width (a leading range of the
// planned tiles) spread over all of them.
//
// One launch per bit width present (one width per kernel keeps the registers
// at two waves per SIMD); items past the planned tile count, past the column
// blocks or of another width are skipped, and a block with none returns at
// once.
__host__ __device__ inline int pf_group_blocks(int ncb) { return (ncb + 1) / 2; }
__host__ __device__ inline int64_t pf_gemm_grid(int64_t tiles, int combos, int ncb) {
    const int64_t groups = tiles * combos;
    return 8 * (int64_t)pf_group_blocks(ncb) * ((groups + 7) / 8);
}

// BITS2 = 0: the experts of one width, BITS.  BITS2 > 0: the experts of either
// width BITS or BITS2 in one launch (a tile's width is the same for both waves
// of its block), so one launch's tail is paid where two would each pay one.
template <int BITS, int BITS2, int CB, bool DOWN>
// Up to 3 bits the kernel fits two waves per SIMD (at most 256 registers);
// the request keeps the compiler there with both step loops of pf_tile.
__global__ __launch_bounds__(2 * WAVE)
__attribute__((amdgpu_waves_per_eu((BITS <= 3 && BITS2 <= 3) ? 2 : 1, (BITS <= 3 && BITS2 <= 3) ? 2 : 8)))
void pf_gemm_kernel(PfParams P) {
    const PfLayout& L = P.L;
    const int ncb = (DOWN ? P.H : P.I) / COLS;
    const int KS = DOWN ? L.ks_down : L.ks_up;
    const int combos = DOWN ? KS : 2 * KS;             // groups per tile
    const int G = pf_group_blocks(ncb);
    const int wave = threadIdx.x / WAVE;
    const int jj = (int)(blockIdx.x >> 3);              // this block's place in its XCD's sequence
    const int g = 8 * (jj / G) + (int)(blockIdx.x & 7);
    const int cb = 2 * (jj % G) + wave;
    const int t = g / combos, c = g - t * combos;
    const bool tile_ok = t < pat<int>(P.scratch, L.meta)[PF_META_TILES];
    const int e = tile_ok ? pat<int>(P.scratch, L.tile_e)[t] : 0;
    // wide tile entry: its half of the column blocks, both waves on one block
    const int half = tile_ok ? pat<int>(P.scratch, L.tile_w)[t] : -1;
    const int cbx = half < 0 ? cb : half * G + (jj % G);      // 256-column block
    const int width = P.ebits ? (int)P.ebits[e] : P.bits;    // the same for the block's two waves
    const bool valid = tile_ok && cbx < ncb && (width == BITS || (BITS2 > 0 && width == BITS2));
    if (!__syncthreads_or(valid)) return;
    const int proj = DOWN ? 0 : c / KS, ks = c % KS;
    const int row0 = valid ? pat<int>(P.scratch, L.tile_r0)[t] : 0;
    const int nrows = valid ? pat<int>(P.scratch, L.tile_n)[t] : 0;
    const int K = DOWN ? P.I : P.H, N = DOWN ? P.H : P.I;
    const int kpart = K / KS;
    const uint16_t* A = DOWN ? pat<uint16_t>(P.scratch, L.AD)
                             : pat<uint16_t>(P.scratch, L.Xh) + (size_t)proj * P.P * P.H;
    const int16_t* tr = reinterpret_cast<const int16_t*>((DOWN ? P.dt : (proj ? P.ut : P.gt))[e]);
    const uint16_t* svh = reinterpret_cast<const uint16_t*>((DOWN ? P.dsv : (proj ? P.usv : P.gsv))[e]);
    float* out = DOWN ? pat<float>(P.scratch, L.D) + (size_t)ks * P.P * P.H
                      : pat<float>(P.scratch, L.GU) + ((size_t)ks * 2 + proj) * P.P * P.I;
    constexpr int B2 = BITS2 > 0 ? BITS2 : BITS;
    if (half >= 0) {
        if (BITS2 == 0 || width == BITS)
            pf_tile_wide<BITS, CB>(valid, A, row0, nrows, tr, svh, K, ks * kpart, kpart / STEP_K, N,
                                   2 * cbx + wave, out);
        else
            pf_tile_wide<B2, CB>(valid, A, row0, nrows, tr, svh, K, ks * kpart, kpart / STEP_K, N, 2 * cbx + wave,
                                 out);
    } else if (BITS2 == 0 || width == BITS) {
        pf_tile<BITS, CB>(valid, A, row0, nrows, tr, svh, K, ks * kpart, kpart / STEP_K, N, cb, out);
    } else {
        pf_tile<B2, CB>(valid, A, row0, nrows, tr, svh, K, ks * kpart, kpart / STEP_K, N, cb, out);
    }
}

// Launchers of the grouped GEMM for one bit width, and for widths 3 and 2
// together (exl3_prefill_inst.hip).
template <int BITS>
int launch_pf_gemm(const PfParams& P, int codebook, bool down, int blocks, hipStream_t stream);
int launch_pf_gemm_32(const PfParams& P, int codebook, bool down, int blocks, hipStream_t stream);

}  // namespace prefill
}  // namespace exl3
