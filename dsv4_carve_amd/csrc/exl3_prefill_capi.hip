// C ABI of the routed-MoE prefill path (grouped GEMMs over tokens routed to
// the same expert):
//   exl3_moe_prefill_scratch_bytes, exl3_moe_prefill  <- exllamav3_ext.exl3_moe
//   for many rows (recipe-lna/vllm_exl3_exl3.py.lna:1597-1704, its fat-chunk
//   path) and LinearEXL3.reconstruct_hgemm (recipe-lna/exllamav3/exl3.py.lna:161-218)
#include <cmath>
#include <mutex>

#include "exl3_prefill.hpp"

namespace exl3 {
namespace prefill {

// ---------------------------------------------------------------- 1. plan (one workgroup of 1024 threads)

// Exclusive scan of n ints in LDS by wave 0 (64 at a time, carrying the sum).
__device__ __forceinline__ void wave0_scan(int* v, int n, int* total) {
    if (threadIdx.x >= WAVE) return;
    const int lane = threadIdx.x;
    int carry = 0;
    for (int i0 = 0; i0 < n; i0 += WAVE) {
        const int x = i0 + lane < n ? v[i0 + lane] : 0;
        int s = x;
#pragma unroll
        for (int d = 1; d < WAVE; d <<= 1) {
            const int y = __shfl_up(s, d, WAVE);
            if (lane >= d) s += y;
        }
        if (i0 + lane < n) v[i0 + lane] = carry + s - x;
        carry += __shfl(s, WAVE - 1, WAVE);
    }
    if (lane == 0) *total = carry;
}

// Local experts of PF_PLAN_N slots per thread (s0, s0 + nt, ...), -1 for
// none.  An expert whose width is outside the call's bits_mask (no GEMM
// launch covers it) is routed nowhere, so it contributes nothing, and sets
// `bad`.  Every slot's id loads, then its map and width loads, are in flight
// together, so a round pays one chain of dependent loads instead of one per
// slot.
constexpr int PF_PLAN_N = 8;

__device__ __forceinline__ void pf_local_n(const PfParams& P, int s0, int nt, int (&e)[PF_PLAN_N], int* bad) {
    int s[PF_PLAN_N];
#pragma unroll
    for (int i = 0; i < PF_PLAN_N; ++i) s[i] = s0 + i * nt;
    P.rt.local_n(s, P.P, P.E, e);
    if (P.ebits) {
        int b[PF_PLAN_N];
#pragma unroll
        for (int i = 0; i < PF_PLAN_N; ++i) b[i] = P.ebits[e[i] >= 0 ? e[i] : 0];
#pragma unroll
        for (int i = 0; i < PF_PLAN_N; ++i)
            if (e[i] >= 0 && !((P.mask >> (b[i] & 31)) & 1u)) {
                *bad = 1;
                e[i] = -1;
            }
    }
}

__global__ __launch_bounds__(1024) void pf_plan_kernel(PfParams P) {
    __shared__ int cnt[PF_MAX_EXPERTS + 1];
    __shared__ int off[PF_MAX_EXPERTS + 1];
    __shared__ int tof[PF_MAX_EXPERTS + 1];
    __shared__ int totals[2];
    __shared__ int bad;
    const PfLayout& L = P.L;
    const int tid = threadIdx.x, nt = blockDim.x;
    const int round = nt * PF_PLAN_N;
    // up to `round` pairs, each thread's experts stay in registers for the
    // placement pass; beyond that the placement pass looks them up again
    const bool one_round = P.P <= round;
    int ev[PF_PLAN_N];
    for (int e = tid; e < P.E; e += nt) cnt[e] = 0;
    if (tid == 0) bad = 0;
    __syncthreads();
    for (int s0 = tid; s0 < P.P; s0 += round) {
        pf_local_n(P, s0, nt, ev, &bad);
#pragma unroll
        for (int i = 0; i < PF_PLAN_N; ++i)
            if (ev[i] >= 0) atomicAdd(&cnt[ev[i]], 1);
    }
    __syncthreads();
    for (int e = tid; e < P.E; e += nt) {
        off[e] = cnt[e];
        tof[e] = pf_tile_entries(cnt[e]);
    }
    __syncthreads();
    wave0_scan(off, P.E, &totals[0]);
    wave0_scan(tof, P.E, &totals[1]);
    __syncthreads();
    int* eoff = pat<int>(P.scratch, L.eoff);
    int* toff = pat<int>(P.scratch, L.toff);
    int* tile_e = pat<int>(P.scratch, L.tile_e);
    int* tile_r0 = pat<int>(P.scratch, L.tile_r0);
    int* tile_n = pat<int>(P.scratch, L.tile_n);
    int* tile_w = pat<int>(P.scratch, L.tile_w);
    for (int e = tid; e < P.E; e += nt) {
        eoff[e] = off[e];
        toff[e] = tof[e];
        const int c = cnt[e];
        int k = tof[e];
        auto entry = [&](int r0, int n, int w) {
            tile_e[k] = e;
            tile_r0[k] = r0;
            tile_n[k] = n;
            tile_w[k] = w;
            ++k;
        };
        if (c <= PF_RB) {
            if (c > 0) entry(off[e], c, -1);
        } else {
            // wide tiles of PF_RB_WIDE rows, two entries each (column-block
            // halves); a remainder of at most PF_RB rows in a narrow tile
            for (int r = 0; r < c; r += PF_RB_WIDE) {
                const int n = min(PF_RB_WIDE, c - r);
                if (n > PF_RB) {
                    entry(off[e] + r, n, 0);
                    entry(off[e] + r, n, 1);
                } else {
                    entry(off[e] + r, n, -1);
                }
            }
        }
    }
    if (tid == 0) {
        eoff[P.E] = totals[0];
        toff[P.E] = totals[1];
        pat<int>(P.scratch, L.meta)[PF_META_PAIRS] = totals[0];
        pat<int>(P.scratch, L.meta)[PF_META_ERROR] = bad ? PF_ERR_WIDTH : 0;
        pat<int>(P.scratch, L.meta)[PF_META_TILES] = totals[1];
    }
    __syncthreads();
    // place the pairs: any order within an expert (a row's result does not
    // depend on its position in the tile; the gather sums in slot order)
    for (int e = tid; e < P.E; e += nt) cnt[e] = off[e];
    __syncthreads();
    int* pair_slot = pat<int>(P.scratch, L.pair_slot);
    int* pair_e = pat<int>(P.scratch, L.pair_e);
    int* pos = pat<int>(P.scratch, L.pos);
    for (int s0 = tid; s0 < P.P; s0 += round) {
        if (!one_round) pf_local_n(P, s0, nt, ev, &bad);
#pragma unroll
        for (int i = 0; i < PF_PLAN_N; ++i) {
            const int s = s0 + i * nt;
            if (s >= P.P) break;
            int p = -1;
            if (ev[i] >= 0) {
                p = atomicAdd(&cnt[ev[i]], 1);
                pair_slot[p] = s;
                pair_e[p] = ev[i];
            }
            pos[s] = p;
        }
    }
}

// ---------------------------------------------------------------- 2. input rotation (one wave per pair and 512 columns, both projections)
//
// Each lane holds 8 consecutive columns (16-byte loads and stores): lanes
// 16 b .. 16 b + 15 cover 128-block b, so the block's Hadamard runs in
// registers and DPP moves (fwht128_x8).  The pair's expert comes from the plan
// (no route lookup), and one wave rotates the gate and the up input of its
// columns, so the chain of dependent loads (pair -> scale pointers -> x and
// scales) is paid once for both.

// half(x * s) of 8 packed inputs (fp16 or bf16 x, fp16 s), as fp32.
__device__ __forceinline__ void pf_scaled8(const u32x4_t& xv, const u32x4_t& sv, int x_kind, float (&v)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint16_t xb = (uint16_t)(h ? xv[i] >> 16 : xv[i] & 0xffffu);
            const uint16_t x16 = x_kind != 0 ? f32_to_f16_bits(bf16_to_f32(xb)) : xb;
            const uint16_t s16 = (uint16_t)(h ? sv[i] >> 16 : sv[i] & 0xffffu);
            // the fp32 product of two halves is exact, so one RNE cast = half mul
            v[2 * i + h] = f16_bits_to_f32(f32_to_f16_bits(f16_bits_to_f32(x16) * f16_bits_to_f32(s16)));
        }
    }
}

__device__ __forceinline__ u32x4_t pf_rotated8(float (&v)[8]) {
    fwht128_x8(v);
    u32x4_t o;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        o[i] = (uint32_t)f32_to_f16_bits(v[2 * i] * HAD_NORM) | ((uint32_t)f32_to_f16_bits(v[2 * i + 1] * HAD_NORM) << 16);
    return o;
}

__global__ __launch_bounds__(64) void pf_rotate_kernel(PfParams P) {
    const PfLayout& L = P.L;
    const int nch = (P.H + 511) / 512;
    const int p = blockIdx.x / nch, ch = blockIdx.x - p * nch;
    if (p >= pat<int>(P.scratch, L.meta)[PF_META_PAIRS]) return;
    const int s = pat<int>(P.scratch, L.pair_slot)[p];
    const int e = pat<int>(P.scratch, L.pair_e)[p];
    const int tok = s / P.topk;
    const int lane = threadIdx.x;
    // H is a multiple of 256: a lane whose 128-block is past H has no columns
    const int col = ch * 512 + 8 * lane;
    const bool live = col < P.H;
    const int cl = live ? col : ch * 512;
    const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(P.x) + (size_t)tok * P.H + cl);
    const u32x4_t gs = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(P.gsu[e]) + cl);
    const u32x4_t us = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(P.usu[e]) + cl);
    float vg[8], vu[8];
    pf_scaled8(xv, gs, P.x_kind, vg);
    pf_scaled8(xv, us, P.x_kind, vu);
    const u32x4_t og = pf_rotated8(vg), ou = pf_rotated8(vu);
    uint16_t* xh = pat<uint16_t>(P.scratch, L.Xh);
    if (live) {
        *reinterpret_cast<u32x4_t*>(xh + (size_t)p * P.H + col) = og;
        *reinterpret_cast<u32x4_t*>(xh + ((size_t)P.P + p) * P.H + col) = ou;
    }
}

// ---------------------------------------------------------------- 4. activation + down input rotation (one wave per pair and 512 columns)
//
// Lane l holds 8 consecutive columns, lanes 16 b .. 16 b + 15 one 128-block of
// the down input (fwht128_x8), as in the input rotation.

__global__ __launch_bounds__(64) void pf_act_kernel(PfParams P) {
    const PfLayout& L = P.L;
    const int nch = (P.I + 511) / 512;
    const int p = blockIdx.x / nch, ch = blockIdx.x - p * nch;
    if (p >= pat<int>(P.scratch, L.meta)[PF_META_PAIRS]) return;
    const int lane = threadIdx.x;
    const int e = pat<int>(P.scratch, L.pair_e)[p];
    // I is a multiple of 256: a lane whose 128-block is past I has no columns
    const int col = ch * 512 + 8 * lane;
    const bool live = col < P.I;
    const int cl = live ? col : ch * 512;
    const float* G = pat<float>(P.scratch, L.GU) + (size_t)p * P.I + cl;
    const float* U = pat<float>(P.scratch, L.GU) + ((size_t)P.P + p) * P.I + cl;
    const size_t kstride = (size_t)2 * P.P * P.I;     // between k-parts
    const u32x4_t ds = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(P.dsu[e]) + cl);
    // every k-part's loads first, then the sums in k-part order
    float4_t gp[2][2], up[2][2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
        if (ks < L.ks_up) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                gp[ks][h] = *reinterpret_cast<const float4_t*>(G + ks * kstride + 4 * h);
                up[ks][h] = *reinterpret_cast<const float4_t*>(U + ks * kstride + 4 * h);
            }
        }
    float dv[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float4_t g4 = gp[0][h], u4 = up[0][h];
        if (L.ks_up > 1) {
            g4 += gp[1][h];
            u4 += up[1][h];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float gg = g4[i], uu = u4[i];
            if (gg > P.limit) gg = P.limit;
            if (uu < -P.limit) uu = -P.limit;
            if (uu > P.limit) uu = P.limit;
            const uint16_t act = f32_to_f16_bits((gg / (1.0f + expf(-gg))) * uu);
            const int j = 4 * h + i;
            const uint16_t s16 = (uint16_t)((j & 1) ? ds[j >> 1] >> 16 : ds[j >> 1] & 0xffffu);
            dv[j] = f16_bits_to_f32(f32_to_f16_bits(f16_bits_to_f32(act) * f16_bits_to_f32(s16)));
        }
    }
    fwht128_x8(dv);
    u32x4_t packed;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        packed[i] = (uint32_t)f32_to_f16_bits(dv[2 * i] * HAD_NORM) | ((uint32_t)f32_to_f16_bits(dv[2 * i + 1] * HAD_NORM) << 16);
    if (live) *reinterpret_cast<u32x4_t*>(pat<uint16_t>(P.scratch, L.AD) + (size_t)p * P.I + col) = packed;
}

// ---------------------------------------------------------------- 6. gather (one wave per token and 256-column block)

__global__ __launch_bounds__(64) void pf_gather_kernel(PfParams P) {
    const PfLayout& L = P.L;
    const int ncb = P.H / COLS;
    const int tok = blockIdx.x / ncb, cb = blockIdx.x - (blockIdx.x / ncb) * ncb;
    const int lane = threadIdx.x;
    const int col = cb * COLS + 4 * lane;
    const int* pos = pat<int>(P.scratch, L.pos);
    const float* D = pat<float>(P.scratch, L.D);
    // every slot's loads first (pair index, weight, both k-parts), then the
    // fp32 sum in top-k slot order
    int pp[PF_MAX_TOPK];
    float wt[PF_MAX_TOPK];
#pragma unroll
    for (int j = 0; j < PF_MAX_TOPK; ++j) {
        pp[j] = j < P.topk ? pos[tok * P.topk + j] : -1;
        wt[j] = j < P.topk ? P.rt.weight(tok * P.topk + j) : 0.f;
    }
    float4_t d0[PF_MAX_TOPK], d1[PF_MAX_TOPK];
#pragma unroll
    for (int j = 0; j < PF_MAX_TOPK; ++j)
        if (pp[j] >= 0) {
            d0[j] = *reinterpret_cast<const float4_t*>(D + (size_t)pp[j] * P.H + col);
            if (L.ks_down > 1) d1[j] = *reinterpret_cast<const float4_t*>(D + ((size_t)P.P + pp[j]) * P.H + col);
        }
    float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < PF_MAX_TOPK; ++j) {
        if (pp[j] < 0) continue;
        float4_t d = d0[j];
        if (L.ks_down > 1) d += d1[j];                // k-parts added in order
#pragma unroll
        for (int i = 0; i < 4; ++i) s4[i] = s4[i] + wt[j] * d[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) store_out(P.out, (size_t)tok * P.H + col + i, P.out_kind, s4[i]);
}


template <> int launch_pf_gemm<1>(const PfParams&, int, bool, int, hipStream_t);
template <> int launch_pf_gemm<2>(const PfParams&, int, bool, int, hipStream_t);
template <> int launch_pf_gemm<3>(const PfParams&, int, bool, int, hipStream_t);
template <> int launch_pf_gemm<4>(const PfParams&, int, bool, int, hipStream_t);
template <> int launch_pf_gemm<5>(const PfParams&, int, bool, int, hipStream_t);
template <> int launch_pf_gemm<6>(const PfParams&, int, bool, int, hipStream_t);
template <> int launch_pf_gemm<7>(const PfParams&, int, bool, int, hipStream_t);
template <> int launch_pf_gemm<8>(const PfParams&, int, bool, int, hipStream_t);

// Grouped GEMM over every width in `mask`: one launch for the 3- and 2-bit
// experts together when both are present, one launch for each other width.
static int launch_widths(const PfParams& P, uint32_t mask, int codebook, bool down, int blocks, hipStream_t s) {
    int (*const fn[9])(const PfParams&, int, bool, int, hipStream_t) = {
        nullptr, &launch_pf_gemm<1>, &launch_pf_gemm<2>, &launch_pf_gemm<3>, &launch_pf_gemm<4>,
        &launch_pf_gemm<5>, &launch_pf_gemm<6>, &launch_pf_gemm<7>, &launch_pf_gemm<8>};
    constexpr uint32_t W32 = (1u << 3) | (1u << 2);
    if ((mask & W32) == W32) {
        const int rc = launch_pf_gemm_32(P, codebook, down, blocks, s);
        if (rc) return rc;
        mask &= ~W32;
    }
    for (int b = 1; b <= 8; ++b)
        if (mask & (1u << b)) {
            const int rc = fn[b](P, codebook, down, blocks, s);
            if (rc) return rc;
        }
    return 0;
}

}  // namespace prefill
}  // namespace exl3

using namespace exl3;
using namespace exl3::prefill;

static_assert(PF_META_ERROR * 4 == 4, "prefill error word at byte 4, as in the decode scratch");

extern "C" {

int64_t exl3_moe_prefill_scratch_bytes(int64_t tokens, int64_t hidden, int64_t intermediate, int64_t topk,
                                       int64_t n_experts) {
    clear_error();
    if (tokens < 1 || topk < 1 || topk > PF_MAX_TOPK || tokens * topk > PF_MAX_PAIRS)
        return fail("tokens * topk must be in 1..65536 with topk in 1..9");
    if (hidden <= 0 || hidden % COLS || intermediate <= 0 || intermediate % COLS)
        return fail("hidden and intermediate must be positive multiples of 256");
    if (n_experts < 1 || n_experts > PF_MAX_EXPERTS) return fail("expert count out of range (1..2048)");
    return pf_layout(tokens * topk, hidden, intermediate, n_experts).total;
}

}  // extern "C"

// The prefill layer for one routing descriptor; both entry points below.
static int moe_prefill_impl(const void* x, int x_kind, void* out, int out_kind, int64_t tokens, int64_t hidden,
                            int64_t intermediate, int64_t n_experts, int64_t topk,
                            const int64_t* gate_trellis, const int64_t* gate_suh, const int64_t* gate_svh,
                            const int64_t* up_trellis, const int64_t* up_suh, const int64_t* up_svh,
                            const int64_t* down_trellis, const int64_t* down_suh, const int64_t* down_svh,
                            const Route& rt, const int8_t* expert_bits, int bits, int bits_mask, int codebook,
                            float swiglu_limit, void* scratch, int64_t scratch_bytes, void* stream) {
    if (!x || !out || !rt.ids || !rt.w || !scratch) return fail("null pointer");
    if (!gate_trellis || !gate_suh || !gate_svh || !up_trellis || !up_suh || !up_svh || !down_trellis ||
        !down_suh || !down_svh)
        return fail("null pointer table");
    if (x_kind != 0 && x_kind != 1) return fail("x must be fp16 or bf16");
    if (reinterpret_cast<uintptr_t>(x) % 16) return fail("x must be 16-byte aligned (the input rotation reads 16-byte rows)");
    if (out_kind < OUT_F16 || out_kind > OUT_F32) return fail("out must be fp16, bf16 or fp32");
    const int64_t need = exl3_moe_prefill_scratch_bytes(tokens, hidden, intermediate, topk, n_experts);
    if (need < 0) return (int)need;
    if (!(swiglu_limit > 0.0f) || !std::isfinite(swiglu_limit)) return fail("requires a finite positive SwiGLU limit");
    if (codebook < CB_3INST || codebook > CB_MUL1) return fail("codebook must be 0, 1 or 2");
    uint32_t mask;
    if (expert_bits) {
        mask = (uint32_t)bits_mask;
        if (mask == 0 || (mask & ~0x1FEu)) return fail("bits_mask must name widths in 1..8");
    } else {
        if (bits < 1 || bits > 8) return fail("bits must be in 1..8");
        mask = 1u << bits;
    }
    if (scratch_bytes < need) return fail("scratch too small (see exl3_moe_prefill_scratch_bytes)");

    PfParams P;
    P.x = x; P.x_kind = x_kind; P.out = out; P.out_kind = out_kind;
    P.T = (int)tokens; P.H = (int)hidden; P.I = (int)intermediate; P.E = (int)n_experts; P.topk = (int)topk;
    P.P = (int)(tokens * topk);
    P.gt = gate_trellis; P.gsu = gate_suh; P.gsv = gate_svh;
    P.ut = up_trellis; P.usu = up_suh; P.usv = up_svh;
    P.dt = down_trellis; P.dsu = down_suh; P.dsv = down_svh;
    P.rt = rt;
    P.ebits = expert_bits; P.bits = bits; P.mask = mask;
    P.limit = swiglu_limit;
    P.scratch = reinterpret_cast<char*>(scratch);
    P.L = pf_layout(P.P, hidden, intermediate, n_experts);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    int rc;
    hipLaunchKernelGGL(pf_plan_kernel, dim3(1), dim3(1024), 0, s, P);
    if ((rc = check_launch())) return rc;
    hipLaunchKernelGGL(pf_rotate_kernel, dim3(P.P * ((hidden + 511) / 512)), dim3(WAVE), 0, s, P);
    if ((rc = check_launch())) return rc;
    const int64_t tiles = P.L.max_tiles;
    if ((rc = launch_widths(P, mask, codebook, false,
                            (int)pf_gemm_grid(tiles, 2 * P.L.ks_up, (int)(intermediate / COLS)), s)))
        return rc;
    hipLaunchKernelGGL(pf_act_kernel, dim3(P.P * ((intermediate + 511) / 512)), dim3(WAVE), 0, s, P);
    if ((rc = check_launch())) return rc;
    if ((rc = launch_widths(P, mask, codebook, true, (int)pf_gemm_grid(tiles, P.L.ks_down, (int)(hidden / COLS)), s)))
        return rc;
    hipLaunchKernelGGL(pf_gather_kernel, dim3((unsigned)(tokens * (hidden / COLS))), dim3(WAVE), 0, s, P);
    return check_launch();
}

extern "C" {

int exl3_moe_prefill(const void* x, int x_kind, void* out, int out_kind, int64_t tokens, int64_t hidden,
                     int64_t intermediate, int64_t n_experts, int64_t topk,
                     const int64_t* gate_trellis, const int64_t* gate_suh, const int64_t* gate_svh,
                     const int64_t* up_trellis, const int64_t* up_suh, const int64_t* up_svh,
                     const int64_t* down_trellis, const int64_t* down_suh, const int64_t* down_svh,
                     const int32_t* expert_ids, const float* routing_weights,
                     const int8_t* expert_bits, int bits, int bits_mask, int codebook,
                     float swiglu_limit, void* scratch, int64_t scratch_bytes, void* stream) {
    clear_error();
    const Route rt{expert_ids, routing_weights, nullptr, IDS_I32, OUT_F32, 0};
    return moe_prefill_impl(x, x_kind, out, out_kind, tokens, hidden, intermediate, n_experts, topk, gate_trellis,
                            gate_suh, gate_svh, up_trellis, up_suh, up_svh, down_trellis, down_suh, down_svh, rt,
                            expert_bits, bits, bits_mask, codebook, swiglu_limit, scratch, scratch_bytes, stream);
}

int exl3_moe_prefill_routed(const void* x, int x_kind, void* out, int out_kind, int64_t tokens, int64_t hidden,
                            int64_t intermediate, int64_t n_experts, int64_t topk,
                            const int64_t* gate_trellis, const int64_t* gate_suh, const int64_t* gate_svh,
                            const int64_t* up_trellis, const int64_t* up_suh, const int64_t* up_svh,
                            const int64_t* down_trellis, const int64_t* down_suh, const int64_t* down_svh,
                            const void* topk_ids, int ids_kind, const void* topk_weights, int weights_kind,
                            const int64_t* expert_map, int64_t n_global,
                            const int8_t* expert_bits, int bits, int bits_mask, int codebook,
                            float swiglu_limit, void* scratch, int64_t scratch_bytes, void* stream) {
    clear_error();
    Route rt;
    if (int rc = make_route(topk_ids, ids_kind, topk_weights, weights_kind, expert_map, n_global, rt)) return rc;
    return moe_prefill_impl(x, x_kind, out, out_kind, tokens, hidden, intermediate, n_experts, topk, gate_trellis,
                            gate_suh, gate_svh, up_trellis, up_suh, up_svh, down_trellis, down_suh, down_svh, rt,
                            expert_bits, bits, bits_mask, codebook, swiglu_limit, scratch, scratch_bytes, stream);
}

}  // extern "C"
