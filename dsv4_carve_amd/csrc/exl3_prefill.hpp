// Routed-MoE layer for many tokens (prefill): the same mathematics as the
// decode kernel (gate/up, clamped SiLU*mul, down, slot-order fp32 sum), done as
// grouped GEMMs so every decoded weight is applied to up to 32 rows.
//
// Launch sequence (one stream, no host synchronisation, no persistent state):
//   1. plan:     route (token, slot) pairs by expert (counting sort in LDS),
//                cut each expert's rows into tiles of PF_RB rows.
//   2. rotate:   Xh[proj][pair] = half(H (half(x[token] * suh[e])) / sqrt(128))
//                for the gate and up projections.
//   3. gemm:     gate/up tiles: decode each 64x256 weight step once per tile
//                and feed it to the MFMAs of both 16-row blocks; epilogue
//                output Hadamard + svh -> fp32 [pair][I].
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

constexpr int PF_RB = 32;                 // rows per tile (two MFMA row blocks)
constexpr int PF_MAX_EXPERTS = 2048;
constexpr int PF_MAX_TOPK = 9;
constexpr int PF_MAX_PAIRS = 65536;

// Words of the meta block at the head of the scratch.  The error word sits at
// byte 4, as in the decode scratch; the plan launch rewrites it every call.
constexpr int PF_META_PAIRS = 0, PF_META_ERROR = 1, PF_META_TILES = 2;
constexpr int PF_ERR_WIDTH = 1;          // an expert width outside bits_mask was routed (it contributed nothing)

struct PfLayout {
    int64_t meta, eoff, toff, tile_e, tile_r0, tile_n, pair_slot, pair_e, pos, Xh, GU, AD, D, total;
    int64_t max_tiles;
    int ks_up, ks_down;     // k-splits: GU is [ks_up][2][pairs][I], D is [ks_down][pairs][H]
};

__host__ __device__ inline int64_t pf_al(int64_t v) { return (v + 255) / 256 * 256; }

// k-splits of the gate/up (K = hidden) and down (K = intermediate) GEMMs: as
// many as keep an even number of 64-row steps per part, up to 2 each (on the
// 512-token layer 2/2 measured faster than 4/2, 1/2 and 2/1: fewer parts halve
// the partials the activation reads, more parts shorten the launches' last
// round).  Each part writes its own fp32 output (the output Hadamard and svh
// are linear, so they apply per part); the activation and gather kernels add
// the parts in order, so results do not depend on scheduling.
inline int pf_ksplit(int64_t K, int cap) {
    int ks = cap;
    while (ks > 1 && K % (2 * STEP_K * ks)) ks /= 2;
    return ks;
}

inline PfLayout pf_layout(int64_t pairs, int64_t H, int64_t I, int64_t E) {
    PfLayout L;
    L.ks_up = pf_ksplit(H, 2);
    L.ks_down = pf_ksplit(I, 2);
    L.max_tiles = E + (pairs + PF_RB - 1) / PF_RB;
    int64_t o = 0;
    L.meta = o;      o = pf_al(o + 64);
    L.eoff = o;      o = pf_al(o + (E + 1) * 4);
    L.toff = o;      o = pf_al(o + (E + 1) * 4);
    L.tile_e = o;    o = pf_al(o + L.max_tiles * 4);
    L.tile_r0 = o;   o = pf_al(o + L.max_tiles * 4);
    L.tile_n = o;    o = pf_al(o + L.max_tiles * 4);
    L.pair_slot = o; o = pf_al(o + pairs * 4);
    L.pair_e = o;    o = pf_al(o + pairs * 4);
    L.pos = o;       o = pf_al(o + pairs * 4);
    L.Xh = o;        o = pf_al(o + 2 * pairs * H * 2);
    L.GU = o;        o = pf_al(o + (int64_t)L.ks_up * 2 * pairs * I * 4);
    L.AD = o;        o = pf_al(o + pairs * I * 2);
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
    u32x4_t ac[2][2];
    // Each step's A loads are issued before the next step's tile loads: the
    // wait for A (needed at once) then leaves the tile prefetch in flight
    // (loads complete in issue order, so A issued after it would wait for it).
    // A tile of at most 16 rows (most tiles under skewed routing) runs a loop
    // without row block 1's A loads and MFMAs; its rows are the same.
    auto steps = [&](auto two) {
        constexpr bool TWO = decltype(two)::value;
        auto load_a = [&](int s) {
            ac[0][0] = a0[s * astep]; ac[0][1] = a0[s * astep + 1];
            if constexpr (TWO) { ac[1][0] = a1[s * astep]; ac[1][1] = a1[s * astep + 1]; }
        };
        load_tile<BITS>(t0, tp);
        for (int s = 0; s < nsteps; s += 2) {
            load_a(s);
            load_tile<BITS>(t1, tp + (s + 1) * tstep);
            mma_tile2<BITS, CB, TWO>(t0.words(), ac, acc);
            load_a(s + 1);
            // the last iteration reloads its own step (a valid address, unused)
            load_tile<BITS>(t0, tp + min(s + 2, nsteps - 1) * tstep);
            mma_tile2<BITS, CB, TWO>(t1.words(), ac, acc);
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
    const int width = P.ebits ? (int)P.ebits[e] : P.bits;    // the same for the block's two waves
    const bool valid = tile_ok && cb < ncb && (width == BITS || (BITS2 > 0 && width == BITS2));
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
    if (BITS2 == 0 || width == BITS)
        pf_tile<BITS, CB>(valid, A, row0, nrows, tr, svh, K, ks * kpart, kpart / STEP_K, N, cb, out);
    else
        pf_tile<(BITS2 > 0 ? BITS2 : BITS), CB>(valid, A, row0, nrows, tr, svh, K, ks * kpart, kpart / STEP_K, N,
                                                cb, out);
}

// Launchers of the grouped GEMM for one bit width, and for widths 3 and 2
// together (exl3_prefill_inst.hip).
template <int BITS>
int launch_pf_gemm(const PfParams& P, int codebook, bool down, int blocks, hipStream_t stream);
int launch_pf_gemm_32(const PfParams& P, int codebook, bool down, int blocks, hipStream_t stream);

}  // namespace prefill
}  // namespace exl3
