// EXL3 trellis decode primitives for gfx950 (CDNA4, wave64).
//
// Layout decision: one lane owns one whole 16x16 tile (16*BITS int16 =
// 8*BITS dwords, loaded with 16-byte vector loads).  Every window of the
// tile then sits at a bit position known at compile time, so a window costs
// at most one v_alignbit_b32 and never a per-lane variable shift.  Compare the
// reference's per-lane runtime shifts (orders/F1-ref/exl3_dq.cuh:15-31, 96-161).
//
// Bitstream contract (orders/F1-ref/exl3_dq.cuh:18-29, exl3_dequant.cuh:109-127):
//   word i = u16[2i] | u16[2i+1] << 16; stream bit p = bit 31-(p&31) of word p>>5;
//   the window of element t is the 16 stream bits ending at ((t+1)*BITS) mod
//   256*BITS, read circularly, first bit most significant.
// Codebooks (exl3_dequant.cuh:73-92; GPU canon recipe-lna/lna2/primitive_gate.cu:25-31):
//   MCG:   x = w*0xCBAC1FED; x = (x & 0x8fff8fff) ^ 0x3b603b60; h = half(lo)+half(hi)
//   3INST: x = w*89226354 + 64248484, then as MCG
//   MUL1:  x = w*0x83DCD12D; s = 0x6400 + bytesum(x); h = fma(s, 0x1eee, 0xc931)
// Tile permutation (recipe-lna/lna2/bindings.cpp:33-77):
//   W[k][n] = decode(t), t = 8*(4*(n&7) + ((k&7)>>1)) + 4*(n>>3) + 2*(k>>3) + (k&1)
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <utility>

namespace exl3 {

enum Codebook : int { CB_3INST = 0, CB_MCG = 1, CB_MUL1 = 2 };

constexpr float HAD_NORM = 0.08838834764831845f;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Global-address-space views.  Pointers that reach a kernel through a device
// table (the MoE weight tables) are generic to the compiler, which would emit
// flat loads (these also count against the LDS counter and force broader
// waits); casting them to address space 1 keeps the loads on the vector memory path.
template <typename T>
using gptr_t = const __attribute__((address_space(1))) T*;
template <typename T>
__device__ __forceinline__ gptr_t<T> as_global(const T* p) {
    return (gptr_t<T>)p;
}

// ---------------------------------------------------------------- compile-time loops

template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(std::forward<F>(f), std::make_integer_sequence<int, N>{});
}

// ---------------------------------------------------------------- windows

// Element t of a (k, n) position in the tile.
__host__ __device__ constexpr int tile_t(int k, int n) {
    return 8 * (4 * (n & 7) + ((k & 7) >> 1)) + 4 * (n >> 3) + 2 * (k >> 3) + (k & 1);
}

// A 32-bit funnel of the tile stream whose LOW 16 bits are the window of
// element T (bits above are the stream bits that precede the window).  When
// 16 % BITS == 0 the high 16 bits are exactly the window of element T - 16/BITS.
template <int BITS, int T>
__device__ __forceinline__ uint32_t win_lo(const uint32_t* W) {
    constexpr int NB = 256 * BITS, NW = 8 * BITS;
    constexpr int E0 = ((T + 1) * BITS) % NB;
    constexpr int E = E0 == 0 ? NB : E0;          // exclusive end bit in (0, NB]
    constexpr int I1 = (E - 1) >> 5;              // word holding the window's last bit
    constexpr int O = E - 32 * I1;                // 1..32
    if constexpr (O == 32) {
        return W[I1];
    } else {
        constexpr int I0 = (I1 + NW - 1) % NW;
        return __builtin_amdgcn_alignbit(W[I0], W[I1], 32 - O);
    }
}

// ---------------------------------------------------------------- codebooks

// x = (w * MULT + ADD) mod 2^32 for the 16-bit window w held in the low (HI=false)
// or high (HI=true) half of `src`, then (x & 0x8fff8fff) ^ 0x3b603b60.
// Two ops for the multiply (a 16x16-bit multiply and v_pk_mad_u16, both reading
// the window from its register half, so `src` needs no masking) plus the
// masked xor (v_bitop3_b32).  The dequant kernels decode this way; the GEMV
// kernels isolate each window and use codebook_word.
template <bool HI, uint32_t MULT, uint32_t ADD>
__device__ __forceinline__ uint32_t mcg_bits(uint32_t src) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    constexpr uint32_t MLO = MULT & 0xffffu;
    constexpr unsigned short MHI = (unsigned short)(MULT >> 16);
    const uint32_t w = HI ? (src >> 16) : (src & 0xffffu);
    // p = w * MLO + ADD (16x16 -> 32 bit): p.lo16 is x.lo16, p.hi16 the carry into x.hi16
    const uint32_t p = w * MLO + ADD;
    // x.lo16 = p.lo16 ; x.hi16 = w * (MULT >> 16) + p.hi16  (mod 2^16)
    const u16x2 sv = __builtin_bit_cast(u16x2, src);
    const u16x2 wv = HI ? sv.yy : sv.xx;
    const u16x2 x = wv * (u16x2){0, MHI} + __builtin_bit_cast(u16x2, p);
    return (__builtin_bit_cast(uint32_t, x) & 0x8fff8fffu) ^ 0x3b603b60u;
}

template <int CB>
struct CbConst;
template <> struct CbConst<CB_MCG>   { static constexpr uint32_t MULT = 0xCBAC1FEDu, ADD = 0u; };
template <> struct CbConst<CB_3INST> { static constexpr uint32_t MULT = 89226354u, ADD = 64248484u; };

// The same x for an isolated window w (w < 2^16), as one full 32-bit multiply:
// x = w * MULT + ADD (mod 2^32), then the masked xor.  On gfx950 v_mul_lo_u32
// issues at the rate of each 16-bit multiply it replaces, and the masks and
// shifts that isolate a window issue at twice that rate.
template <int CB>
__device__ __forceinline__ uint32_t codebook_word(uint32_t w) {
    const uint32_t x = w * CbConst<CB>::MULT + CbConst<CB>::ADD;
    return (x & 0x8fff8fffu) ^ 0x3b603b60u;
}

// Codebook output as a packed pair of fp16 ADDENDS (lo, hi) whose sum is the
// weight, for MCG/3INST; for MUL1 the pair is (weight, 0).  GEMV kernels feed
// both addends to the MFMA against a duplicated activation, so the codebook's
// final half add is performed exactly instead of rounded (bounded by 2^-11 of
// each weight, far inside the fp tolerance); dequant kernels round it (RNE).
template <int CB, bool HI>
__device__ __forceinline__ uint32_t codebook_pair(uint32_t src) {
    if constexpr (CB == CB_MUL1) {
        const uint32_t w = HI ? (src >> 16) : (src & 0xffffu);
        const uint32_t x = w * 0x83DCD12Du;
        const uint32_t s = __builtin_amdgcn_udot4(x, 0x01010101u, 0x6400u, false);
        const _Float16 hs = __builtin_bit_cast(_Float16, (uint16_t)s);
        const _Float16 r = __builtin_fmaf16(hs, __builtin_bit_cast(_Float16, (uint16_t)0x1eee),
                                            __builtin_bit_cast(_Float16, (uint16_t)0xc931));
        return (uint32_t)__builtin_bit_cast(uint16_t, r);
    } else {
        return mcg_bits<HI, CbConst<CB>::MULT, CbConst<CB>::ADD>(src);
    }
}

// Fully rounded codebook value (binary16 bits), bit-exact with the canon.
template <int CB, bool HI>
__device__ __forceinline__ uint16_t codebook_half(uint32_t src) {
    const uint32_t pr = codebook_pair<CB, HI>(src);
    if constexpr (CB == CB_MUL1) {
        return (uint16_t)pr;
    } else {
        const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(pr & 0xffffu));
        const _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(pr >> 16));
        return __builtin_bit_cast(uint16_t, (_Float16)(lo + hi));
    }
}

// Decode the window of compile-time element T of a tile held in registers.
template <int BITS, int CB, int T>
__device__ __forceinline__ uint32_t decode_pair_t(const uint32_t* W) {
    return codebook_pair<CB, false>(win_lo<BITS, T>(W));
}
template <int BITS, int CB, int T>
__device__ __forceinline__ uint16_t decode_half_t(const uint32_t* W) {
    return codebook_half<CB, false>(win_lo<BITS, T>(W));
}

// ---------------------------------------------------------------- fp16 / bf16

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);   // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
// fp32 -> fp16 (RNE) of a value that has been rounded to fp32 first.  The
// register barrier keeps the compiler from fusing a preceding multiply into the
// conversion (v_fma_mixlo_f16 rounds once, straight to half), which would skip
// the fp32 rounding point the reference's float-then-half code has.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);     // v_cvt_f16_f32, RNE
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// Output element kinds shared by every entry point: 0 = fp16, 1 = bf16, 2 = fp32.
enum OutKind : int { OUT_F16 = 0, OUT_BF16 = 1, OUT_F32 = 2 };

__device__ __forceinline__ void store_out(void* out, size_t idx, int kind, float v) {
    if (kind == OUT_F32) reinterpret_cast<float*>(out)[idx] = v;
    else if (kind == OUT_F16) reinterpret_cast<uint16_t*>(out)[idx] = f32_to_f16_bits(v);
    else reinterpret_cast<uint16_t*>(out)[idx] = f32_to_bf16_rne(v);
}

// ---------------------------------------------------------------- wave shuffles

__device__ __forceinline__ float shfl_xor(float v, int mask) {
    return __shfl_xor(v, mask, 64);
}

}  // namespace exl3
