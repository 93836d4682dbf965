// C-ABI entry points of the routed-MoE decode (declared in include/exl3_amd.h):
//   exl3_moe_decode         <- lna2_moe_decode   recipe-lna/lna2/lna_moe_ticket.cu:507-581
//   exl3_moe_scratch_bytes  <- lna2_moe_scratch_bytes  :481 (16 rows)
//   exl3_moe_scratch_bytes_rows   (the same for up to `rows` rows; the reference
//                                  sizes its scratch for LNA2_MAX_M at build time, :40-53)
//   exl3_moe_max_rows       <- lna2_moe_max_rows       :484
//   exl3_moe_info           <- lna2_moe_info           :494-505
//   exl3_moe_decode_noalloc    (no counterpart: the routed decode on a fixed scratch)
//   exl3_moe_noalloc_error     (no counterpart: that fixed scratch's error word)
#include <math.h>
#include <stddef.h>
#include <stdlib.h>

#include "exl3_moe.hpp"

namespace exl3 {
namespace moe {

// Instantiated (mask, codebook) pairs; the first whose mask covers the
// requested widths is used.  Keep in sync with MOE_UNITS in build.py.
#define EXL3_MOE_INSTANCES(X)                 \
    X(0x004u, 1) X(0x008u, 1) X(0x010u, 1)    \
    X(0x040u, 1) X(0x00Cu, 1) X(0x01Cu, 1)    \
    X(0x04Cu, 1)                              \
    X(0x1FEu, 1) X(0x1FEu, 0) X(0x1FEu, 2)

#define EXL3_DECL(M, C)                                                          \
    template <> int launch_moe<M, C>(const Params&, int, int, hipStream_t);     \
    template <> int launch_phased<M, C>(const Params&, int, hipStream_t);       \
    template <> int moe_waves_per_cu<M, C>(int);
EXL3_MOE_INSTANCES(EXL3_DECL)
#undef EXL3_DECL

struct Instance {
    uint32_t mask;
    int cb;
    int (*launch)(const Params&, int, int, hipStream_t);
    int (*phased)(const Params&, int, hipStream_t);
    int (*waves)(int);
};

#define EXL3_ENTRY(M, C) {M, C, &launch_moe<M, C>, &launch_phased<M, C>, &moe_waves_per_cu<M, C>},
static const Instance kInstances[] = {EXL3_MOE_INSTANCES(EXL3_ENTRY)};
#undef EXL3_ENTRY

// Resident single-wave workgroups per CU for an instance at a dynamic LDS size
// (1..MAX_LDS_KB KB), asked of the occupancy API once per device.
constexpr int MAX_LDS_KB = 16;
static int cached_waves(int idx, int lds_kb) {
    static int cache[MAX_DEVICES][sizeof(kInstances) / sizeof(kInstances[0])][MAX_LDS_KB + 1] = {};
    static std::mutex mu;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) dev = 0;
    std::lock_guard<std::mutex> lock(mu);
    if (!cache[dev][idx][lds_kb]) cache[dev][idx][lds_kb] = kInstances[idx].waves(lds_kb);
    return cache[dev][idx][lds_kb];
}

// Phased launches: down items assemble their own input (no activation launch)
// while the layer's activation is small, m * topk * intermediate <=
// FUSE_ACT_MAX_ELEMS; beyond, the redundant assembly (every H block repeats
// it) costs more than the extra launch.  Measured, us, assembled / separate:
// 256-expert layer (intermediate 2048, top-8), 1 row 52 / 52, 2 rows 81 / 80,
// 4 rows 139 / 133, 16 rows 387 / 375; one GPU's TP8 share (intermediate 256,
// top-6), 1 row 27 / 30, 16 rows 76 / 80.  EXL3_MOE_FUSE_ACT_MAX_ROWS, when
// set, replaces the rule by a row count.
constexpr int64_t FUSE_ACT_MAX_ELEMS = 32768;
static bool fuse_act(int64_t m, int64_t topk, int64_t intermediate) {
    const char* v = getenv("EXL3_MOE_FUSE_ACT_MAX_ROWS");
    if (v && *v) return m <= atoi(v);
    return m * topk * intermediate <= FUSE_ACT_MAX_ELEMS;
}

// Schedule choice.  The phased launches are the default: on the 256-expert
// layer they beat the ticket kernel at every row count (1 / 2 / 4 / 8 / 16
// rows: 50 / 78 / 134 / 225 / 360 us against 82 / 100 / 159 / 248 / 379), and
// one GPU's TP8 share likewise.  The ticket kernel (one persistent launch,
// device-scope hand-offs) stays available: EXL3_MOE_PHASED_MAX_ROWS, when
// set, selects by row count (0: always the ticket kernel).
static bool use_phased(int64_t m) {
    if (m > TICKET_MAX_M) return true;        // the ticket kernel's plan holds 16 rows
    const char* v = getenv("EXL3_MOE_PHASED_MAX_ROWS");
    if (v && *v) return m <= atoi(v);
    return true;
}

// Row capacity of a call's data regions: 16 rows (the default scratch) up to
// 16 rows, else the call's row count.
static int scratch_rows(int64_t m) { return m > SCRATCH_ROWS ? (int)m : SCRATCH_ROWS; }

}  // namespace moe
}  // namespace exl3

using namespace exl3;
using namespace exl3::moe;

extern "C" {

int64_t exl3_moe_scratch_bytes_rows(int64_t hidden, int64_t intermediate, int64_t topk, int64_t rows) {
    clear_error();
    if (hidden <= 0 || hidden % COLS || intermediate <= 0 || intermediate % COLS)
        return fail("hidden and intermediate must be positive multiples of 256");
    if (hidden > COLS * MAX_BLOCKS || intermediate > COLS * MAX_BLOCKS)
        return fail("hidden and intermediate must be at most 16384");
    if (topk < 1 || topk > MAX_TOPK) return fail("topk must be in 1..9");
    if (rows < 1 || rows > MAX_M) return fail("row count out of range (1 <= rows <= exl3_moe_max_rows())");
    return layout((int)hidden, (int)intermediate, (int)topk, 2, 2, scratch_rows(rows)).total + trace_bytes();
}

int64_t exl3_moe_scratch_bytes(int64_t hidden, int64_t intermediate, int64_t topk) {
    return exl3_moe_scratch_bytes_rows(hidden, intermediate, topk, SCRATCH_ROWS);
}

int exl3_moe_max_rows(void) { return MAX_M; }

int64_t exl3_moe_error_offset(void) {
    static_assert(offsetof(Ctrl, error) == 4, "error word at byte 4 of the control block");
    return layout(COLS, COLS, 1).ctrl + (int64_t)offsetof(Ctrl, error);
}

int exl3_moe_info(int64_t* out, int n) {
    clear_error();
    if (!out || n < 0) return fail("bad output buffer");
    const int cus = device_cus();
    const int kb = moe_lds_kb(MAX_M, 256);
    const int64_t lds = (int64_t)kb * 1024 + (int64_t)sizeof(Plan);
    const int64_t v[] = {cus, (int64_t)cus * cached_waves(4, kb), WAVE, MAX_M, PHASED_MAX_SLOTS, STEP_K, COLS,
                         layout(COLS, COLS, 1).PA, lds};
    const int k = n < 9 ? n : 9;
    for (int i = 0; i < k; ++i) out[i] = v[i];
    return k;
}

}  // extern "C"

// The decode layer for one routing descriptor; both entry points below.
static int moe_decode_impl(const void* x, int x_kind, void* out, int out_kind, int64_t m, int64_t hidden,
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
    if (out_kind < OUT_F16 || out_kind > OUT_F32) return fail("out must be fp16, bf16 or fp32");
    if (m < 1 || m > MAX_M) return fail("row count out of range (1 <= m <= exl3_moe_max_rows())");
    if (hidden <= 0 || hidden % COLS || intermediate <= 0 || intermediate % COLS)
        return fail("hidden and intermediate must be positive multiples of 256");
    if (hidden > COLS * MAX_BLOCKS || intermediate > COLS * MAX_BLOCKS)
        return fail("hidden and intermediate must be at most 16384");
    if (n_experts < 1 || n_experts > MAX_EXPERTS) return fail("expert count out of range (1..2048)");
    if (topk < 1 || topk > MAX_TOPK) return fail("topk must be in 1..9");
    if (!(swiglu_limit > 0.0f) || !isfinite(swiglu_limit)) return fail("requires a finite positive SwiGLU limit");
    if (codebook < CB_3INST || codebook > CB_MUL1) return fail("codebook must be 0, 1 or 2");
    uint32_t mask;
    if (expert_bits) {
        mask = (uint32_t)bits_mask;
        if (mask == 0 || (mask & ~0x1FEu)) return fail("bits_mask must name widths in 1..8");
    } else {
        if (bits < 1 || bits > 8) return fail("bits must be in 1..8");
        mask = 1u << bits;
    }
    const int rows = scratch_rows(m);
    const int64_t trace_off = layout((int)hidden, (int)intermediate, (int)topk, 2, 2, rows).total;
    if (scratch_bytes < trace_off + trace_bytes())
        return fail(m > SCRATCH_ROWS ? "scratch too small for this row count (see exl3_moe_scratch_bytes_rows)"
                                     : "scratch too small (see exl3_moe_scratch_bytes)");

    int idx = -1;
    const int ninst = (int)(sizeof(kInstances) / sizeof(kInstances[0]));
    for (int i = 0; i < ninst; ++i)
        if (kInstances[i].cb == codebook && (kInstances[i].mask & mask) == mask) { idx = i; break; }
    if (idx < 0) return fail("no kernel instance for this bit-width set / codebook");

    // Distinct experts are at most min(E, m * topk); size the items for that.
    const int64_t groups = n_experts < m * topk ? n_experts : m * topk;
    const int lds_kb = moe_lds_kb(m, n_experts);
    static_assert(MAX_ROWS * NSTEP_CAP * STEP_K * 2 <= MAX_LDS_KB * 1024 && 6 * MAX_EXPERTS <= MAX_LDS_KB * 1024,
                  "dynamic LDS bound");
    const int64_t resident = (int64_t)device_cus() * cached_waves(idx, lds_kb);
    const int stepsA = item_steps((int)hidden, groups * 2 * (intermediate / COLS), resident);
    const int stepsB = item_steps((int)intermediate, groups * (hidden / COLS), resident);
    const Layout L = layout((int)hidden, (int)intermediate, (int)topk, stepsA, stepsB, rows);

    Params P;
    P.x = x; P.x_kind = x_kind; P.out = out; P.out_kind = out_kind;
    P.m = (int)m; P.H = (int)hidden; P.I = (int)intermediate; P.E = (int)n_experts; P.topk = (int)topk;
    P.gt = gate_trellis; P.gsu = gate_suh; P.gsv = gate_svh;
    P.ut = up_trellis; P.usu = up_suh; P.usv = up_svh;
    P.dt = down_trellis; P.dsu = down_suh; P.dsv = down_svh;
    P.rt = rt;
    P.ebits = expert_bits; P.bits = bits;
    P.limit = swiglu_limit;
    P.scratch = reinterpret_cast<char*>(scratch);
    P.L = L;
    P.trace_off = trace_off;
    P.fuse_act = fuse_act(m, topk, intermediate) ? 1 : 0;

    if (use_phased(m))
        return kInstances[idx].phased(P, lds_kb, reinterpret_cast<hipStream_t>(stream));

    const int64_t items = groups * (2LL * L.nI * L.SA + (int64_t)L.nH * L.SB) + (int64_t)L.nH * m;
    const int waves = (int)(items < resident ? items : resident);
    // one gate/up ticket class per XCD (32 CUs each on this part); any class
    // count is correct, this one only spreads the first draws
    const int cus = device_cus();
    const int nxcd = (cus >= 64 && cus % 32 == 0) ? cus / 32 : 1;
    P.nclass = nxcd <= MAX_CLASSES ? nxcd : MAX_CLASSES;
    return kInstances[idx].launch(P, waves, lds_kb, reinterpret_cast<hipStream_t>(stream));
}

extern "C" {

int exl3_moe_decode(const void* x, int x_kind, void* out, int out_kind, int64_t m, int64_t hidden,
                    int64_t intermediate, int64_t n_experts, int64_t topk,
                    const int64_t* gate_trellis, const int64_t* gate_suh, const int64_t* gate_svh,
                    const int64_t* up_trellis, const int64_t* up_suh, const int64_t* up_svh,
                    const int64_t* down_trellis, const int64_t* down_suh, const int64_t* down_svh,
                    const int32_t* expert_ids, const float* routing_weights,
                    const int8_t* expert_bits, int bits, int bits_mask, int codebook,
                    float swiglu_limit, void* scratch, int64_t scratch_bytes, void* stream) {
    clear_error();
    const Route rt{expert_ids, routing_weights, nullptr, IDS_I32, OUT_F32, 0};
    return moe_decode_impl(x, x_kind, out, out_kind, m, hidden, intermediate, n_experts, topk, gate_trellis,
                           gate_suh, gate_svh, up_trellis, up_suh, up_svh, down_trellis, down_suh, down_svh, rt,
                           expert_bits, bits, bits_mask, codebook, swiglu_limit, scratch, scratch_bytes, stream);
}

int exl3_moe_decode_routed(const void* x, int x_kind, void* out, int out_kind, int64_t m, int64_t hidden,
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
    return moe_decode_impl(x, x_kind, out, out_kind, m, hidden, intermediate, n_experts, topk, gate_trellis,
                           gate_suh, gate_svh, up_trellis, up_suh, up_svh, down_trellis, down_suh, down_svh, rt,
                           expert_bits, bits, bits_mask, codebook, swiglu_limit, scratch, scratch_bytes, stream);
}

}  // extern "C"

// ---------------------------------------------------------------- fixed scratch (no allocation)
//
// The scratch of exl3_moe_decode_noalloc: one array per GPU inside the
// library's code object, held until the process ends.  Host code never passes
// the array's name to a kernel: hipGetSymbolAddress gives each device's own
// address, kept per device, and only that address is used.

constexpr int64_t NOALLOC_SCRATCH_BYTES = (int64_t)128 << 20;
static __device__ __align__(256) char fixed_scratch[NOALLOC_SCRATCH_BYTES];

__global__ __launch_bounds__(256) void zero_fill_kernel(uint4* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// Clears one 32-bit word (the error word; the words around it keep their values).
__global__ __launch_bounds__(64) void clear_word_kernel(int* p) {
    if (threadIdx.x == 0) *p = 0;
}

// This device's fixed scratch.  On the first call on a device its control
// words (the fixed region at the head of every layout) are zeroed by a fill
// kernel on `stream`, ahead of the layer's launches.  A fill recorded into a
// graph being captured is not remembered: the next call outside a capture
// fills again.
static int fixed_scratch_for(hipStream_t stream, char** out) {
    static char* addr[MAX_DEVICES] = {};
    static bool zeroed[MAX_DEVICES] = {};
    static std::mutex mu;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return fail("no HIP device");
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(fixed_scratch)) != hipSuccess || !p)
            return fail("cannot locate the fixed MoE scratch on this device");
        addr[dev] = reinterpret_cast<char*>(p);
    }
    if (!zeroed[dev]) {
        const int64_t ctrl_bytes = layout(COLS, COLS, 1).PA;     // the same for every shape
        hipLaunchKernelGGL(zero_fill_kernel, dim3(256), dim3(256), 0, stream, reinterpret_cast<uint4*>(addr[dev]),
                           ctrl_bytes / 16);
        if (int rc = check_launch()) return rc;
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &st) == hipSuccess && st == hipStreamCaptureStatusNone) zeroed[dev] = true;
    }
    *out = addr[dev];
    return 0;
}

extern "C" {

int64_t exl3_moe_noalloc_scratch_bytes(void) { return NOALLOC_SCRATCH_BYTES; }

int exl3_moe_decode_noalloc(const void* x, int x_kind, void* out, int out_kind, int64_t m, int64_t hidden,
                            int64_t intermediate, int64_t n_experts, int64_t topk,
                            const int64_t* gate_trellis, const int64_t* gate_suh, const int64_t* gate_svh,
                            const int64_t* up_trellis, const int64_t* up_suh, const int64_t* up_svh,
                            const int64_t* down_trellis, const int64_t* down_suh, const int64_t* down_svh,
                            const void* topk_ids, int ids_kind, const void* topk_weights, int weights_kind,
                            const int64_t* expert_map, int64_t n_global,
                            const int8_t* expert_bits, int bits, int bits_mask, int codebook,
                            float swiglu_limit, void* stream) {
    clear_error();
    const int64_t need = exl3_moe_scratch_bytes_rows(hidden, intermediate, topk, m);
    if (need < 0) return (int)need;
    if (need > NOALLOC_SCRATCH_BYTES)
        return fail("layer needs more scratch than the fixed 128 MiB (see exl3_moe_scratch_bytes_rows)");
    Route rt;
    if (int rc = make_route(topk_ids, ids_kind, topk_weights, weights_kind, expert_map, n_global, rt)) return rc;
    char* scratch = nullptr;
    if (int rc = fixed_scratch_for(reinterpret_cast<hipStream_t>(stream), &scratch)) return rc;
    return moe_decode_impl(x, x_kind, out, out_kind, m, hidden, intermediate, n_experts, topk, gate_trellis,
                           gate_suh, gate_svh, up_trellis, up_suh, up_svh, down_trellis, down_suh, down_svh, rt,
                           expert_bits, bits, bits_mask, codebook, swiglu_limit, scratch, NOALLOC_SCRATCH_BYTES,
                           stream);
}

int exl3_moe_noalloc_error(int clear, void* stream) {
    clear_error();
    if (clear < 0 || clear > 2) return fail("clear must be 0 (read), 1 (clear the bits) or 2 (reset every control word)");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
        return fail("the error word is read with a stream synchronisation: not inside a graph capture");
    char* scratch = nullptr;
    if (int rc = fixed_scratch_for(st, &scratch)) return rc;
    int* word = reinterpret_cast<int*>(scratch + exl3_moe_error_offset());
    int value = 0;
    if (hipMemcpyAsync(&value, word, sizeof(int), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return fail("cannot read the fixed scratch's error word");
    if (clear == 2) {
        // every counter, flag and the epoch back to zero, as at the first call
        const int64_t ctrl_bytes = layout(COLS, COLS, 1).PA;
        hipLaunchKernelGGL(zero_fill_kernel, dim3(256), dim3(256), 0, st, reinterpret_cast<uint4*>(scratch),
                           ctrl_bytes / 16);
        if (int rc = check_launch()) return rc;
    } else if (clear == 1 && value) {
        hipLaunchKernelGGL(clear_word_kernel, dim3(1), dim3(64), 0, st, word);
        if (int rc = check_launch()) return rc;
    }
    return value;
}

}  // extern "C"
