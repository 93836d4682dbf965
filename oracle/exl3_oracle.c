/*
 * EXL3 trellis-decode ORACLE -- test infrastructure only.
 *
 * A plain-C restatement of the reference's CPU decode path, used by the tests,
 * by __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker.
 * Nothing in the product path may link or call this file.
 *
 * Followed reference sources (paths relative to the reference tree):
 *   window extraction   orders/F1-ref/exl3_dq.cuh:15-31 (dq<bits,cb>),
 *                       orders/F1-ref/exl3_dequant.cuh:109-134 (read_window,
 *                       decode_weight), recipe-lna/lna2/primitive_gate.cu:33-45
 *   codebooks           orders/F1-ref/exl3_dequant.cuh:73-92 (decode_codebook_bits),
 *                       recipe-lna/lna2/primitive_gate.cu:25-31 (lna_mcg, __hadd)
 *                       -- with IEEE binary16 round-to-nearest-even where the
 *                       reference CPU helper truncates (exl3_dequant.cuh:40-53);
 *                       the GPU canon rounds (__hadd), see primitive_gate.cu:30.
 *   tile permutation    recipe-lna/lna2/bindings.cpp:33-77 (fragment swizzle)
 *   128-point Hadamard  orders/F1-ref/exl3_dequant.cuh:136-147
 *   full dequant        recipe-lna/lna2/bindings.cpp:16-101 (dequant_cpu order)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ---------------- binary16 helpers ---------------- */

float ora_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) & 1u;
    const int exp = (h >> 10) & 0x1f;
    const uint32_t mant = h & 0x3ffu;
    double v;
    if (exp == 0) {
        v = ldexp((double)mant, -24);
    } else if (exp == 31) {
        if (mant) return NAN;
        v = INFINITY;
    } else {
        v = ldexp(1024.0 + (double)mant, exp - 25);
    }
    return (float)(sign ? -v : v);
}

/* Correctly rounded (round to nearest, ties to even) double -> binary16. */
uint16_t ora_double_to_half(double v) {
    if (isnan(v)) return 0x7e00;
    uint16_t sign = signbit(v) ? 0x8000 : 0;
    v = fabs(v);
    if (v == 0.0) return sign;
    if (isinf(v)) return (uint16_t)(sign | 0x7c00);
    int e;
    (void)frexp(v, &e);
    int E = e - 1;                    /* v = 1.f * 2^E */
    if (E < -14) {                    /* subnormal range: units of 2^-24 */
        double r = rint(ldexp(v, 24));    /* default rounding mode: ties-to-even */
        return (uint16_t)(sign | (uint16_t)r);   /* r == 1024 becomes min normal */
    }
    double r = rint(ldexp(v, 10 - E));   /* in [1024, 2048] */
    if (r >= 2048.0) { r = 1024.0; E += 1; }
    if (E > 15) return (uint16_t)(sign | 0x7c00);
    return (uint16_t)(sign | ((E + 15) << 10) | ((int)r - 1024));
}

uint16_t ora_float_to_half(float f) { return ora_double_to_half((double)f); }

/* ---------------- A.2 trellis window ---------------- */

/* Tile = 16*bits uint16 = 8*bits uint32 words, word i = u16[2i] | u16[2i+1]<<16.
 * Stream bit p sits in word p>>5 at bit 31-(p&31) (MSB first).  The window of
 * element t is the 16 stream bits ending (exclusive) at ((t+1)*bits) mod 256*bits,
 * read circularly, first bit = MSB.  This is the bit-serial form of the
 * funnel-shift windows in exl3_dq.cuh:18-30 / exl3_dequant.cuh:109-127. */
uint16_t ora_window(const uint16_t* tile, int bits, int t) {
    const int nbits = 256 * bits;
    const int end = ((t + 1) * bits) % nbits;
    uint32_t w = 0;
    for (int i = 0; i < 16; ++i) {
        const int p = (end - 16 + i + nbits) % nbits;
        const uint32_t word = (uint32_t)tile[2 * (p >> 5)] |
                              ((uint32_t)tile[2 * (p >> 5) + 1] << 16);
        w = (w << 1) | ((word >> (31 - (p & 31))) & 1u);
    }
    return (uint16_t)w;
}

/* ---------------- A.3 codebooks ---------------- */

#define ORA_MCG_MULT 0xCBAC1FEDu
#define ORA_MUL1_MULT 0x83DCD12Du

/* MUL1's value: a single-rounded half FMA s*h(0x1eee) + h(0xc931); the double
 * product of two halves is exact and so is the sum here, so this is the FMA's
 * exact result before its one rounding. */
static double mul1_fma_exact(uint16_t window) {
    const uint32_t x = (uint32_t)window * ORA_MUL1_MULT;
    const uint32_t s = 0x6400u + (x & 0xffu) + ((x >> 8) & 0xffu) + ((x >> 16) & 0xffu) + ((x >> 24) & 0xffu);
    return (double)ora_half_to_float((uint16_t)s) * (double)ora_half_to_float(0x1eee) +
           (double)ora_half_to_float(0xc931);
}

/* The exact sum, in a double, of the binary16 addends whose rounded sum is
 * the codebook value: for 3INST and MCG the two masked halves; MUL1 is one
 * single-rounded half FMA, so its one addend is the binary16 value itself.
 * (The GPU GEMV and MoE kernels hand these addends to the matrix core, which
 * adds them exactly, so this is the weight they use.)
 * cb: 0 = 3INST, 1 = MCG, 2 = MUL1 (exl3_gemm.cu.lna:186-189 numbering) */
double ora_codebook_addend_sum(uint16_t window, int cb) {
    if (cb == 2) return (double)ora_half_to_float(ora_double_to_half(mul1_fma_exact(window)));
    uint32_t x = window;
    if (cb == 0) x = x * 89226354u + 64248484u;
    else x = x * ORA_MCG_MULT;
    x = (x & 0x8fff8fffu) ^ 0x3b603b60u;   /* lop3 0x6a */
    /* the double sum of two binary16 values is exact */
    return (double)ora_half_to_float((uint16_t)(x & 0xffffu)) + (double)ora_half_to_float((uint16_t)(x >> 16));
}

/* The codebook value: that sum rounded to nearest even (a binary16 addend of
 * MUL1 is unchanged by it). */
uint16_t ora_codebook(uint16_t window, int cb) {
    return ora_double_to_half(ora_codebook_addend_sum(window, cb));
}

void ora_codebook_lut(int cb, uint16_t* lut /* [65536] */) {
    for (uint32_t w = 0; w < 65536u; ++w) lut[w] = ora_codebook((uint16_t)w, cb);
}

void ora_codebook_addend_sum_lut(int cb, double* lut /* [65536] */) {
    for (uint32_t w = 0; w < 65536u; ++w) lut[w] = ora_codebook_addend_sum((uint16_t)w, cb);
}

/* ---------------- A.4 tile permutation ---------------- */

/* W_tile[k][n] = decode(t(k, n)); k = input row in the 16x16 tile, n = output col. */
int ora_tile_t(int k, int n) {
    return 8 * (4 * (n & 7) + ((k & 7) >> 1)) + 4 * (n >> 3) + 2 * (k >> 3) + (k & 1);
}

/* trellis: int16 [K/16][N/16][16*bits]; out: binary16 bits [K][N] row-major. */
void ora_reconstruct(const uint16_t* trellis, int K, int N, int bits, int cb, uint16_t* out) {
    const int kt_n = K / 16, nt_n = N / 16, tw = 16 * bits;
    uint16_t dec[256];
    for (int kt = 0; kt < kt_n; ++kt) {
        for (int nt = 0; nt < nt_n; ++nt) {
            const uint16_t* tile = trellis + ((size_t)kt * nt_n + nt) * tw;
            for (int t = 0; t < 256; ++t) dec[t] = ora_codebook(ora_window(tile, bits, t), cb);
            for (int k = 0; k < 16; ++k)
                for (int n = 0; n < 16; ++n)
                    out[(size_t)(kt * 16 + k) * N + nt * 16 + n] = dec[ora_tile_t(k, n)];
        }
    }
}

/* ---------------- A.5 Hadamard ---------------- */

/* Natural (Sylvester) order fast Walsh-Hadamard transform, unnormalised, fp32. */
void ora_fwht(float* v, int n) {
    for (int stride = 1; stride < n; stride <<= 1)
        for (int base = 0; base < n; base += stride << 1)
            for (int i = 0; i < stride; ++i) {
                const float a = v[base + i];
                const float b = v[base + stride + i];
                v[base + i] = a + b;
                v[base + stride + i] = a - b;
            }
}

#define ORA_HAD_NORM 0.08838834764831845f

/* Input rotation, lna2 rounding points (lna_moe_ticket.cu:119-144):
 * x (binary16) * suh in half precision (RNE), fp32 butterflies, * 1/sqrt(128)
 * in fp32, then RNE to binary16.  x: [rows][K], K % 128 == 0. */
void ora_had_in(const uint16_t* x, const uint16_t* suh, int rows, int K, uint16_t* out) {
    float line[128];
    for (int r = 0; r < rows; ++r)
        for (int b = 0; b < K; b += 128) {
            for (int i = 0; i < 128; ++i) {
                const double p = (double)ora_half_to_float(x[(size_t)r * K + b + i]) *
                                 (double)ora_half_to_float(suh[b + i]);
                line[i] = ora_half_to_float(ora_double_to_half(p));
            }
            ora_fwht(line, 128);
            for (int i = 0; i < 128; ++i)
                out[(size_t)r * K + b + i] = ora_float_to_half(line[i] * ORA_HAD_NORM);
        }
}

/* Output rotation: y = (H c) / sqrt(128) * svh, all fp32.  c: [rows][N]. */
void ora_had_out(const float* c, const uint16_t* svh, int rows, int N, float* out) {
    float line[128];
    for (int r = 0; r < rows; ++r)
        for (int b = 0; b < N; b += 128) {
            memcpy(line, c + (size_t)r * N + b, sizeof(line));
            ora_fwht(line, 128);
            for (int i = 0; i < 128; ++i)
                out[(size_t)r * N + b + i] = line[i] * ORA_HAD_NORM * ora_half_to_float(svh[b + i]);
        }
}

/* Full dequant W = diag(suh) H Wq H diag(svh) / 128 -> binary16, in the operation
 * order of dequant_cpu (bindings.cpp:80-99): per 128x128 block, row transforms
 * then column transforms, value = line*norm*su*sv left to right in fp32. */
void ora_dequant_full(const uint16_t* trellis, int K, int N, int bits, int cb,
                      const uint16_t* suh, const uint16_t* svh,
                      float* scratch /* [K*N] */, uint16_t* wq /* [K*N] */, uint16_t* out) {
    ora_reconstruct(trellis, K, N, bits, cb, wq);
    for (size_t i = 0; i < (size_t)K * N; ++i) scratch[i] = ora_half_to_float(wq[i]);
    float line[128];
    for (int r0 = 0; r0 < K; r0 += 128)
        for (int c0 = 0; c0 < N; c0 += 128) {
            for (int r = 0; r < 128; ++r) {
                float* row = scratch + (size_t)(r0 + r) * N + c0;
                memcpy(line, row, sizeof(line));
                ora_fwht(line, 128);
                for (int c = 0; c < 128; ++c) row[c] = line[c] * ORA_HAD_NORM;
            }
            for (int c = 0; c < 128; ++c) {
                for (int r = 0; r < 128; ++r) line[r] = scratch[(size_t)(r0 + r) * N + c0 + c];
                ora_fwht(line, 128);
                for (int r = 0; r < 128; ++r) {
                    float v = line[r] * ORA_HAD_NORM;
                    v = v * ora_half_to_float(suh[r0 + r]);
                    v = v * ora_half_to_float(svh[c0 + c]);
                    out[(size_t)(r0 + r) * N + c0 + c] = ora_float_to_half(v);
                }
            }
        }
}

/* Second restatement of reconstruct, in the funnel-shift form of exl3_dq.cuh:18-30
 * (two 32-bit words and one right shift per window) with a precomputed codebook
 * LUT; ~100x faster than the bit-serial spec above and pinned against it. */
void ora_reconstruct_fast(const uint16_t* trellis, int K, int N, int bits, const uint16_t* lut,
                          uint16_t* out) {
    const int kt_n = K / 16, nt_n = N / 16, nw = 8 * bits;
    int i0[256], i1[256], sh[256], pos[256];
    for (int t = 0; t < 256; ++t) {
        const int b0 = (t + 257) * bits - 16, b1 = b0 + 16;
        const int j1 = (b1 - 1) / 32;
        i0[t] = (b0 / 32) % nw;
        i1[t] = j1 % nw;
        sh[t] = (j1 + 1) * 32 - b1;
    }
    for (int k = 0; k < 16; ++k)
        for (int n = 0; n < 16; ++n) pos[ora_tile_t(k, n)] = k * N + n;
    uint32_t words[64];
    for (int kt = 0; kt < kt_n; ++kt)
        for (int nt = 0; nt < nt_n; ++nt) {
            const uint16_t* tile = trellis + ((size_t)kt * nt_n + nt) * 16 * bits;
            for (int i = 0; i < nw; ++i) words[i] = (uint32_t)tile[2 * i] | ((uint32_t)tile[2 * i + 1] << 16);
            uint16_t* dst = out + (size_t)kt * 16 * N + nt * 16;
            for (int t = 0; t < 256; ++t) {
                const uint64_t merged = ((uint64_t)words[i0[t]] << 32) | words[i1[t]];
                dst[pos[t]] = lut[(merged >> sh[t]) & 0xffffu];
            }
        }
}
