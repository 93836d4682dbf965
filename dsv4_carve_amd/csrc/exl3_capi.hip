// C-ABI entry points for the dense path (declared in include/exl3_amd.h):
//   exl3_dequant            <- dequant_trellis  recipe-lna/lna2/bindings.cpp:118-133
//                              (raw variant  <- exllamav3 `reconstruct`, recipe-lna/exllamav3/exl3.py.lna:197)
//   exl3_gemm               <- exl3_gemm        recipe-lna/exllamav3/exl3_gemm.cu.lna:336-364
//                              (and the exl3_gemv entry, recipe-lna/lna2/bindings.cpp:135-148)
//   exl3_dequant_nk            the same weight stored [n][k], for reconstruct_hgemm's GEMM
//   exl3_had_rows           <- exllamav3_ext.had_r_128  recipe-lna/exllamav3/exl3.py.lna:190, 214
//   exl3_gemm_scratch_bytes    scratch sizing for exl3_gemm
//   exl3_gemm_group         <- exl3_mgemm with a broadcast A (same-input fan)
//                              recipe-lna/vllm_exl3_exl3.py.lna:546-613
//   exl3_gemm_group_scratch_bytes
//   exl3_last_error            message of the last failed call on this thread
#include <cmath>

#include "exl3_dense.hpp"

namespace exl3 {
// ---------------------------------------------------------------- dispatch tables

#define EXL3_BITS_SWITCH(BITS_VAR, ...)                       \
    switch (BITS_VAR) {                                        \
        case 1: { constexpr int B_ = 1; __VA_ARGS__; } break;  \
        case 2: { constexpr int B_ = 2; __VA_ARGS__; } break;  \
        case 3: { constexpr int B_ = 3; __VA_ARGS__; } break;  \
        case 4: { constexpr int B_ = 4; __VA_ARGS__; } break;  \
        case 5: { constexpr int B_ = 5; __VA_ARGS__; } break;  \
        case 6: { constexpr int B_ = 6; __VA_ARGS__; } break;  \
        case 7: { constexpr int B_ = 7; __VA_ARGS__; } break;  \
        case 8: { constexpr int B_ = 8; __VA_ARGS__; } break;  \
        default: return fail("bits must be in 1..8");          \
    }

}  // namespace exl3

using namespace exl3;

static int dequant_impl(const int16_t* trellis, int64_t k, int64_t n, int bits, int codebook, const uint16_t* suh,
                        const uint16_t* svh, uint16_t* out, void* stream, bool nk) {
    if (!trellis || !out) return fail("null pointer");
    if (k <= 0 || n <= 0 || k % 16 || n % 16) return fail("k and n must be positive multiples of 16");
    const bool had = suh != nullptr || svh != nullptr;
    if (had && (!suh || !svh)) return fail("suh and svh must both be given or both be null");
    if (had && (k % 128 || n % 128)) return fail("Hadamard-folded dequant needs k, n multiples of 128");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int k16 = (int)(k / 16), n16 = (int)(n / 16);
    if (codebook < CB_3INST || codebook > CB_MUL1) return fail("codebook must be 0 (3inst), 1 (mcg) or 2 (mul1)");
    const DequantArgs args{trellis, k16, n16, codebook, had ? suh : nullptr, had ? svh : nullptr, out, s, nk};
    EXL3_BITS_SWITCH(bits, return launch_dequant<B_>(args));
    return 0;
}

extern "C" {

int exl3_dequant(const int16_t* trellis, int64_t k, int64_t n, int bits, int codebook,
                 const uint16_t* suh, const uint16_t* svh, uint16_t* out, void* stream) {
    clear_error();
    return dequant_impl(trellis, k, n, bits, codebook, suh, svh, out, stream, false);
}

int exl3_dequant_nk(const int16_t* trellis, int64_t k, int64_t n, int bits, int codebook,
                    const uint16_t* suh, const uint16_t* svh, uint16_t* out, void* stream) {
    clear_error();
    return dequant_impl(trellis, k, n, bits, codebook, suh, svh, out, stream, true);
}

int exl3_had_rows(const void* x, int x_kind, void* y, int y_kind, int64_t rows, int64_t cols,
                  const uint16_t* pre_scale, const uint16_t* post_scale, float scale, void* stream) {
    clear_error();
    if (!x || !y) return fail("null pointer");
    if (x_kind < OUT_F16 || x_kind > OUT_F32 || y_kind < OUT_F16 || y_kind > OUT_F32)
        return fail("kinds must be 0 (fp16), 1 (bf16) or 2 (fp32)");
    if (rows < 1 || cols < 128 || cols % 128) return fail("rows must be positive and cols a positive multiple of 128");
    if (x == y && x_kind != y_kind) return fail("in place needs the same element kind");
    const int64_t waves = rows * ((cols / 128 + 1) / 2);
    if (waves > 0x7fffffffLL) return fail("too many rows");
    if (!std::isfinite(scale)) return fail("scale must be finite");
    hipLaunchKernelGGL(had_rows_kernel<0>, dim3((unsigned)waves), dim3(64), 0, reinterpret_cast<hipStream_t>(stream), x,
                       x_kind, y, y_kind, (int)cols, pre_scale, post_scale, scale);
    return check_launch();
}

int64_t exl3_gemm_scratch_bytes(int64_t m, int64_t k, int64_t n) {
    clear_error();
    if (m <= 0 || k <= 0 || n <= 0) return fail("dimensions must be positive");
    return gemv_scratch_bytes(m, k, n, device_cus());
}

int exl3_gemm(const uint16_t* a, int64_t m, int64_t k, const int16_t* b, int64_t n, int bits,
              int codebook, const uint16_t* suh, const uint16_t* svh, void* c, int c_kind,
              void* scratch, int64_t scratch_bytes, void* stream) {
    clear_error();
    if (!a || !b || !c || !suh || !svh || !scratch) return fail("null pointer");
    if (m <= 0) return fail("m must be positive");
    if (codebook < CB_3INST || codebook > CB_MUL1) return fail("codebook must be 0 (3inst), 1 (mcg) or 2 (mul1)");
    if (k <= 0 || k % 128) return fail("k must be a positive multiple of 128");
    if (n <= 0 || n % 128) return fail("n must be a positive multiple of 128");
    if (c_kind < OUT_F16 || c_kind > OUT_F32) return fail("c_kind must be 0 (fp16), 1 (bf16) or 2 (fp32)");
    const int cus = device_cus();
    if (scratch_bytes < gemv_scratch_bytes(m, k, n, cus)) return fail("scratch too small");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const GemvPlan p = gemv_plan(m, k, n, cus);
    int* counters = reinterpret_cast<int*>(scratch);
    float* partials = reinterpret_cast<float*>(reinterpret_cast<char*>(scratch) +
                                               align_up((int64_t)p.n_cb * 4, 256));
    const size_t c_elem = c_kind == OUT_F32 ? 4 : 2;
    const int64_t block = gemv_block_rows(m);
    for (int64_t r0 = 0; r0 < m; r0 += block) {
        const int R = (int)(m - r0 < block ? m - r0 : block);
        const uint16_t* ar = a + r0 * k;
        void* cr = reinterpret_cast<char*>(c) + (size_t)r0 * n * c_elem;
        const GemvArgs args{ar, b, suh, svh, cr, c_kind, R, (int)k, (int)n, p, codebook, counters, partials, s};
        int rc = 0;
        EXL3_BITS_SWITCH(bits, rc = launch_gemv<B_>(args));
        if (rc) return rc;
        if (p.split_reduce) {
            hipLaunchKernelGGL(gemv_reduce_kernel<RED_BATCH>, dim3((int)(n / 128) * R), dim3(64), 0, s, partials, svh, cr,
                               c_kind, R, (int)n, p.n_kc, p.xcd ? 1 : 0);
            if ((rc = check_launch())) return rc;
        }
    }
    return 0;
}

// Fan scratch: per member, its split-K partials (gemv_partial_bytes), each
// member's region 256-byte aligned.
static int64_t fan_scratch(int64_t m, int64_t k, int64_t count, const int64_t* n_list, int cus, GemvPlan* plan,
                           int64_t* offsets) {
    int64_t total_cb = 0;
    for (int64_t j = 0; j < count; ++j) total_cb += (n_list[j] + COLS - 1) / COLS;
    const GemvPlan p = gemv_fan_plan(m, k, total_cb, cus);
    const int64_t rows = m < GEMV_MAX_ROWS ? m : GEMV_MAX_ROWS;
    int64_t o = 0;
    for (int64_t j = 0; j < count; ++j) {
        if (offsets) offsets[j] = o;
        o = align_up(o + gemv_partial_bytes(rows, (n_list[j] + COLS - 1) / COLS, p.n_kc), 256);
    }
    if (plan) *plan = p;
    return o;
}

static int check_fan(int64_t m, int64_t k, int64_t count, const int64_t* n_list) {
    if (m <= 0) return fail("m must be positive");
    if (k <= 0 || k % 128) return fail("k must be a positive multiple of 128");
    if (count < 1 || count > MAX_FAN) return fail("a fan has 1..8 matrices");
    if (!n_list) return fail("null pointer");
    for (int64_t j = 0; j < count; ++j)
        if (n_list[j] <= 0 || n_list[j] % 128) return fail("every n must be a positive multiple of 128");
    return 0;
}

int64_t exl3_gemm_group_scratch_bytes(int64_t m, int64_t k, int64_t count, const int64_t* n_list) {
    clear_error();
    if (int rc = check_fan(m, k, count, n_list)) return rc;
    return fan_scratch(m, k, count, n_list, device_cus(), nullptr, nullptr);
}

int exl3_gemm_group(const uint16_t* a, int64_t m, int64_t k, int64_t count, const int16_t* const* trellis,
                    const uint16_t* const* suh, const uint16_t* const* svh, const int64_t* n_list,
                    const int32_t* bits_list, int codebook, void* const* c, int c_kind, void* scratch,
                    int64_t scratch_bytes, void* stream) {
    clear_error();
    if (int rc = check_fan(m, k, count, n_list)) return rc;
    if (!a || !trellis || !suh || !svh || !bits_list || !c || !scratch) return fail("null pointer");
    if (codebook < CB_3INST || codebook > CB_MUL1) return fail("codebook must be 0 (3inst), 1 (mcg) or 2 (mul1)");
    if (c_kind < OUT_F16 || c_kind > OUT_F32) return fail("c_kind must be 0 (fp16), 1 (bf16) or 2 (fp32)");
    uint32_t widths = 0;
    for (int64_t j = 0; j < count; ++j) {
        if (!trellis[j] || !suh[j] || !svh[j] || !c[j]) return fail("null pointer");
        if (bits_list[j] < 1 || bits_list[j] > 8) return fail("bits must be in 1..8");
        widths |= 1u << bits_list[j];
    }
    const int cus = device_cus();
    GemvPlan p;
    int64_t offsets[MAX_FAN];
    if (scratch_bytes < fan_scratch(m, k, count, n_list, cus, &p, offsets)) return fail("scratch too small");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const size_t c_elem = c_kind == OUT_F32 ? 4 : 2;
    const int64_t block = gemv_block_rows(m);
    for (int64_t r0 = 0; r0 < m; r0 += block) {
        const int R = (int)(m - r0 < block ? m - r0 : block);
        FanParams P{};
        P.x = a + r0 * k;
        P.R = R; P.K = (int)k; P.nsteps = p.nsteps; P.n_kc = p.n_kc; P.count = (int)count; P.out_kind = c_kind;
        int blocks = 0, rblocks = 0;
        bool whole = true;
        for (int64_t j = 0; j < count; ++j) {
            const int n_cb = (int)((n_list[j] + COLS - 1) / COLS);
            P.trellis[j] = trellis[j]; P.suh[j] = suh[j]; P.svh[j] = svh[j];
            P.out[j] = reinterpret_cast<char*>(c[j]) + (size_t)r0 * n_list[j] * c_elem;
            P.partials[j] = reinterpret_cast<float*>(reinterpret_cast<char*>(scratch) + offsets[j]);
            P.N[j] = (int)n_list[j];
            P.bits[j] = bits_list[j];
            P.block0[j] = blocks;
            P.rblock0[j] = rblocks;
            blocks += n_cb * p.n_kc;
            rblocks += (int)(n_list[j] / 128) * R;
            whole = whole && n_list[j] % COLS == 0;
        }
        P.block0[count] = blocks;
        P.rblock0[count] = rblocks;
        P.xcd = xcd_order_allowed() && whole && (blocks / p.n_kc) % N_XCD == 0 ? 1 : 0;
        for (int b = 1; b <= 8; ++b) {
            if (!(widths & (1u << b))) continue;
            int rc = 0;
            EXL3_BITS_SWITCH(b, rc = launch_gemv_fan<B_>(P, codebook, p.waves, blocks, s));
            if (rc) return rc;
        }
        hipLaunchKernelGGL(gemv_fan_reduce_kernel<RED_BATCH>, dim3(rblocks), dim3(64), 0, s, P);
        if (int rc = check_launch()) return rc;
    }
    return 0;
}

}  // extern "C"

extern "C" const char* exl3_last_error(void) { return exl3::g_last_error; }
