// Routed-MoE decode layer for gfx950: one launch computes, for up to 16 rows,
//   out[r] = sum_j w[r][j] * down_e(half(silu(min(gate_e(x_r), L)) * clamp(up_e(x_r), -L, L)))
// over the top-k experts e of each row (precision boundaries of the lna2 canon,
// recipe-lna/lna2/lna_moe_ticket.cu:5-12).
//
// Scheduler (re-derived for 256 CUs, no grid barrier, no co-residency assumption):
//   * Persistent single-wave workgroups run items in ticket order.
//   * Ticket order: every gate/up item of every active expert, then every
//     down item.  Item = (expert group, projection, 256-column block, k-chunk).
//   * gate/up items write fp32 partials; the last arriver of a (group, column
//     block) sums them in fixed order, applies the output Hadamard + svh, the
//     clamped SwiGLU, the down projection's suh + input Hadamard, stores the
//     fp16 down input and publishes an epoch flag.
//   * Gate/up tickets come from one counter per XCD class (class c hands out
//     c, c+C, c+2C, ...; a wave draws from its own XCD's class, hardware
//     XCC_ID, then from the others), which spreads the launch-time burst of
//     first draws over eight counters.  Down and gather tickets come from one
//     counter, drawn only after the drawing wave saw every class spent.
//   * A down item spins on the flags of the column blocks it reads; a gather
//     item on the flag of its H-block.  Gate/up items never wait, and every
//     one of them was drawn by a running wave before any down or gather item
//     was drawn; down and gather items wait only on items with smaller tickets
//     of the one ordered counter (or on gate/up items).  So everything waited
//     for is held by a running wave or done, and every wait ends whatever the
//     number of resident waves (other kernels may hold CUs; no co-residency
//     or dispatch order is assumed).
//   * A wave draws its next ticket while it finishes the current item, but
//     only once that item is past its last wait: the item it holds ahead
//     starts after a finite amount of work, so the argument above still holds
//     (the smallest unfinished ticket is always some wave's current item, and
//     everything it waits for is smaller).  The first ticket is drawn while
//     the route plan is built.
//   * down items write partials; the last arriver of a (group, H-block) applies
//     the output Hadamard + svh; the last group to finish an H-block gathers the
//     block of `out` in top-k slot order (fp32) and casts once.
//   * Counters are reset by whoever consumes them; flags compare against an
//     epoch the last retiring wave advances, so the control block is zeroed once.
// Short layers run the same items as three or four plain launches instead
// (the phased launches below, keyed by top-k slot), with bitwise the same
// result.
// Reference counterpart: lna2_kernel<K> (lna_moe_ticket.cu:240-429), whose expert
// teams need co-resident CTAs and a team barrier (lna_moe_ticket.cu:459-466).
#pragma once

#include "exl3_gemv.hpp"
#include "exl3_route.hpp"
#include "exl3_capi_util.hpp"

namespace exl3 {
namespace moe {

// Rows per call: up to 32 on the phased launches (the reference's lna2 takes
// 24, lna_moe_ticket.cu:40-51), up to 16 on the ticket kernel, whose route
// plan and control words are sized for 16.  The scratch size function without
// a row count covers 16 rows; larger batches ask exl3_moe_scratch_bytes_rows.
constexpr int MAX_M = 32;
constexpr int TICKET_MAX_M = 16;
constexpr int SCRATCH_ROWS = 16;
constexpr int MAX_TOPK = 9;                   // e.g. 8 routed slots + a shared expert
constexpr int MAX_SLOTS = TICKET_MAX_M * MAX_TOPK;   // ticket kernel: bound on groups and pairs
constexpr int PHASED_MAX_SLOTS = MAX_M * MAX_TOPK;   // phased launches: slots of one call
constexpr int MAX_EXPERTS = 2048;             // route-plan bitmask capacity
constexpr int MAX_BLOCKS = 64;                // hidden/256 and intermediate/256 (both <= 16384)
constexpr int NSTEP_CAP = 8;
constexpr int MAX_CLASSES = 8;                // gate/up ticket classes, one per XCD
// Gate/up ticket counters, one per class, each in its own 4 KB so concurrent
// atomics on different classes do not serialise on one line or channel.
constexpr int64_t CLASS_STRIDE = 4096;
// Each completion counter and flag in its own 256 bytes.
constexpr int64_t WORD_STRIDE = 256;

// Steps (64 k-rows each) per item: a power of two in 2..8 dividing k/64.  The
// host starts from 8 and halves while the items would not give every resident
// wave at least one (small batches read few experts and need short items to
// spread them over the whole GPU).
__host__ __device__ inline int item_steps(int k, int64_t units, int64_t waves) {
    const int ks = k / STEP_K;
    int s = NSTEP_CAP;
    while (s > 2 && (ks % s != 0 || units * (ks / s) < waves)) s /= 2;
    return s;
}

struct Layout {
    int nI, nH, SA, SB, stepsA, stepsB;
    int64_t ctrl, cls, cntA, doneA, cntB, cntG, doneB, PA, DI, PB, DC, total;
};
constexpr int64_t PLAN_BYTES = 4096;          // bound on the route plan (LDS)

__host__ __device__ inline int64_t al(int64_t v) { return (v + 255) / 256 * 256; }

// stepsA/stepsB: steps per gate/up and per down item (2, 4 or 8; the scratch
// size is taken at 2, the most partials).  rows: the row capacity the data
// regions are laid out for (the call's row count, at least 16).  Split-K partials are fp32
// PA [pair][projection][I-block][k-chunk][256] and PB [pair][H-block][k-chunk][256]:
// the finish of one (pair, column block) reads its k-chunks from one
// contiguous range (the same offset read in every k-chunk of a
// [k-chunk][columns] layout fell on a few memory channels).
__host__ __device__ inline Layout layout(int H, int I, int topk, int stepsA = 2, int stepsB = 2,
                                        int rows = SCRATCH_ROWS) {
    Layout L;
    L.nI = I / COLS;
    L.nH = H / COLS;
    L.stepsA = stepsA;
    L.stepsB = stepsB;
    L.SA = H / STEP_K / L.stepsA;
    L.SB = I / STEP_K / L.stepsB;
    const int64_t P = (int64_t)rows * topk;       // max pairs = max groups
    // The control words sit at fixed offsets with fixed strides whatever the
    // geometry, so one scratch buffer can serve layers of different shapes:
    // every counter is back at zero after a launch and every flag holds an
    // older epoch, whichever shape used the slot last.
    int64_t o = 0;
    L.ctrl = o;  o += 3 * CLASS_STRIDE;
    L.cls = o;   o += MAX_CLASSES * CLASS_STRIDE;
    L.cntA = o;  o += (int64_t)MAX_SLOTS * MAX_BLOCKS * WORD_STRIDE;
    L.doneA = o; o += (int64_t)MAX_SLOTS * MAX_BLOCKS * WORD_STRIDE;
    L.cntB = o;  o += (int64_t)MAX_SLOTS * MAX_BLOCKS * WORD_STRIDE;
    L.cntG = o;  o += (int64_t)MAX_BLOCKS * WORD_STRIDE;
    L.doneB = o; o += (int64_t)MAX_BLOCKS * WORD_STRIDE;
    o = al(o);
    L.PA = o;    o = al(o + P * 2 * L.SA * I * 4);
    L.DI = o;    o = al(o + P * I * 2);
    L.PB = o;    o = al(o + P * L.SB * H * 4);
    L.DC = o;    o = al(o + P * H * 4);
    L.total = o;
    return L;
}

// Bits of the error word (Ctrl::error).  The kernels only set bits; the word is
// zero in a freshly zeroed scratch and the host reads and clears it.
constexpr int ERR_WIDTH = 1;     // an expert width outside the kernel's instance
constexpr int ERR_WAIT = 2;      // a bounded wait gave up (ticket kernel)

// Control words at the head of the scratch buffer.  The two counters every
// wave updates sit 4 KB apart and away from the words that are only read.
struct Ctrl {
    int epoch;
    int error;                     // ERR_* bits (see dispatch_bits and wait_flag)
    int pad0[1022];
    int later;                     // down and gather items, in order (see draw_ticket)
    int pad1[1023];
    int retire;
};
static_assert(sizeof(Ctrl) <= 3 * CLASS_STRIDE, "control words fit their slot");


struct Params {
    const void* x; int x_kind;
    void* out; int out_kind;
    int m, H, I, E, topk;
    const int64_t* gt; const int64_t* gsu; const int64_t* gsv;
    const int64_t* ut; const int64_t* usu; const int64_t* usv;
    const int64_t* dt; const int64_t* dsu; const int64_t* dsv;
    Route rt;            // top-k ids / weights / expert map
    const int8_t* ebits; int bits;
    float limit;
    char* scratch;
    Layout L;
    int64_t trace_off;   // start of the phase-trace region (EXL3_TRACE builds)
    int nclass;          // ticket classes: the XCD count, or 1 for small grids
    int fuse_act;        // phased launches: down items compute their own input
};

template <typename T>
__device__ __forceinline__ T* at(char* base, int64_t off) { return reinterpret_cast<T*>(base + off); }
// Counter or flag i of the array at `off` (one per WORD_STRIDE bytes).
__device__ __forceinline__ int* word(char* base, int64_t off, int i) {
    return reinterpret_cast<int*>(base + off + (int64_t)i * WORD_STRIDE);
}

// ---------------------------------------------------------------- phase tracing
//
// Built with -DEXL3_TRACE=1, every wave appends (event, argument, time) records
// to a region after the scratch layout (TRACE_EVENTS per wave, TRACE_WAVES
// waves); time is s_memrealtime (100 MHz).  Off by default: no code, no bytes.
#ifndef EXL3_TRACE
#define EXL3_TRACE 0
#endif
constexpr int TRACE_EVENTS = 128;
constexpr int TRACE_WAVES = 4096;
enum TraceEvent : uint32_t {
    EV_START = 1, EV_PLAN, EV_A_BEGIN, EV_A_MMA, EV_A_END, EV_EPI_A_END, EV_B_BEGIN, EV_B_WAITED,
    EV_B_MMA, EV_B_END, EV_EPI_B_END, EV_GATHER_END, EV_RETIRE, EV_STORED, EV_FENCED
};
inline int64_t trace_bytes() { return EXL3_TRACE ? (int64_t)TRACE_WAVES * TRACE_EVENTS * 8 + 256 : 0; }

struct Tracer {
#if EXL3_TRACE
    uint2* buf = nullptr;
    int n = 0;
    // records of workgroup b go to wave slot slot0 + b (phased launches use
    // disjoint slot ranges so one call's launches do not overwrite each other)
    __device__ void init(char* base, int slot0 = 0) {
        const int slot = slot0 + (int)blockIdx.x;
        if (slot < TRACE_WAVES) buf = reinterpret_cast<uint2*>(base) + (size_t)slot * TRACE_EVENTS;
    }
    __device__ void operator()(uint32_t ev, uint32_t arg = 0) {
        if (buf && n < TRACE_EVENTS - 1 && threadIdx.x == 0) {
            const uint64_t t = __builtin_amdgcn_s_memrealtime();
            buf[n] = make_uint2((ev << 24) | (arg & 0xffffffu), (uint32_t)t);
            buf[n + 1] = make_uint2(0u, 0u);
        }
        ++n;
    }
#else
    __device__ void init(char*, int = 0) {}
    __device__ void operator()(uint32_t, uint32_t = 0) {}
#endif
};

// ---------------------------------------------------------------- route plan

struct Plan {
    int U;                       // active expert groups (ascending expert id)
    int gexp[MAX_SLOTS];
    int gpair[MAX_SLOTS];        // first pair index of the group
    uint32_t gmask[MAX_SLOTS];   // row bitmask
    int8_t gbits[MAX_SLOTS];
    int16_t slotpair[MAX_SLOTS]; // pair of slot (row*topk + j), -1 if invalid
};
static_assert(sizeof(Plan) <= PLAN_BYTES && sizeof(Plan) % 4 == 0, "plan size bound");

// Expert-major row bitmask, then a wave-wide exclusive scan over experts
// (lna_moe_ticket.cu:167-214 computes the same plan with block scans).
// `tmp` (>= 6 * E bytes of LDS) is only used during planning.
__device__ inline void build_plan(const Params& P, Plan& pl, char* tmp) {
    const int lane = threadIdx.x;
    uint32_t* rowmask = reinterpret_cast<uint32_t*>(tmp);
    int16_t* epair = reinterpret_cast<int16_t*>(tmp + 4 * P.E);
    for (int e = lane; e < P.E; e += WAVE) rowmask[e] = 0u;
    __syncthreads();
    const int slots = P.m * P.topk;
    for (int s = lane; s < slots; s += WAVE) {
        const int id = P.rt.local(s, P.E);
        if (id >= 0) atomicOr(&rowmask[id], 1u << (s / P.topk));
    }
    __syncthreads();
    const int chunk = (P.E + WAVE - 1) / WAVE;
    const int e0 = lane * chunk, e1 = min(P.E, e0 + chunk);
    int ng = 0, np = 0;
    for (int e = e0; e < e1; ++e) {
        const uint32_t mk = rowmask[e];
        ng += mk != 0u;
        np += __popc(mk);
    }
    int sg = ng, sp = np;   // inclusive scans
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        const int a = __shfl_up(sg, d, WAVE), b = __shfl_up(sp, d, WAVE);
        if (lane >= d) { sg += a; sp += b; }
    }
    int gx = sg - ng, px = sp - np;
    for (int e = e0; e < e1; ++e) {
        const uint32_t mk = rowmask[e];
        epair[e] = (int16_t)px;
        if (mk) {
            pl.gexp[gx] = e;
            pl.gpair[gx] = px;
            pl.gmask[gx] = mk;
            pl.gbits[gx] = (int8_t)(P.ebits ? P.ebits[e] : P.bits);
            ++gx;
            px += __popc(mk);
        }
    }
    if (lane == WAVE - 1) pl.U = sg;
    __syncthreads();
    for (int s = lane; s < slots; s += WAVE) {
        const int id = P.rt.local(s, P.E);
        int16_t pr = -1;
        if (id >= 0) {
            const int row = s / P.topk;
            pr = (int16_t)(epair[id] + __popc(rowmask[id] & ((1u << row) - 1u)));
        }
        pl.slotpair[s] = pr;
    }
    __syncthreads();
}

// ---------------------------------------------------------------- device sync helpers

// One atomic per wave (its lane 0), the old value broadcast to the wave.
__device__ __forceinline__ int wave_atomic_add(int* p, int v) {
    int old = 0;
    if ((threadIdx.x & (WAVE - 1)) == 0) old = atomicAdd(p, v);
    return __shfl(old, 0, WAVE);
}

// Spins until a device-scope flag reaches `target`.  The producer set it after
// completing the device-scope stores it publishes, so reads that follow (also
// device-scope) see that data.  Every wait ends by construction (see the
// scheduler notes at the top); the poll bound (~2^24 polls, several seconds)
// only turns a broken invariant into an error word instead of a hung GPU.
#ifndef EXL3_POLL_SLEEP
#define EXL3_POLL_SLEEP 2
#endif
__device__ __forceinline__ void wait_flag(int* flag, int target, int* err) {
    if (threadIdx.x == 0) {
        for (uint32_t n = 0; __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != target; ++n) {
            if (n == (1u << 24)) {
                __hip_atomic_fetch_or(err, ERR_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(EXL3_POLL_SLEEP);
        }
    }
    __syncthreads();
}

// Hardware id of the XCD this wave runs on (HW_REG_XCC_ID, bits 3:0).
__device__ __forceinline__ int xcc_id() {
    return (int)__builtin_amdgcn_s_getreg((4 - 1) << 11 | 0 << 6 | 20) & 15;
}

// Next ticket.  Gate/up tickets [0, nA): class c hands out c, c + C, c + 2C,
// ... (C = nclass); a wave draws from the class of its own XCD and, once that
// is spent, from the others in turn (`home` remembers where it found work;
// -1 once every class is spent).  Only then does it draw down and gather
// tickets [nA, total) from the one counter `later`, in order.  So every
// gate/up ticket is drawn, by a running wave, before the first later ticket.
__device__ __forceinline__ int draw_ticket(Ctrl* ctrl, char* cls, int nclass, int& home, int nA, int total) {
    while (home >= 0) {
        // One look at every class, the loads in flight together: a spent
        // class costs no atomic.  A failed atomic leaves its class spent for
        // good, so this loop ends after at most nclass draws.
        int v[MAX_CLASSES];
#pragma unroll
        for (int k = 0; k < MAX_CLASSES; ++k)
            if (k < nclass)
                v[k] = __hip_atomic_load(reinterpret_cast<int*>(cls + k * CLASS_STRIDE), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
        uint32_t avail = 0;
#pragma unroll
        for (int k = 0; k < MAX_CLASSES; ++k)
            if (k < nclass && k + nclass * v[k] < nA) avail |= 1u << k;
        if (!avail) {
            home = -1;
            break;
        }
        const uint32_t from_home = avail >> home;       // first open class at or after home, cyclically
        const int c = from_home ? home + __ffs((int)from_home) - 1 : __ffs((int)avail) - 1;
        const int t = c + nclass * wave_atomic_add(reinterpret_cast<int*>(cls + c * CLASS_STRIDE), 1);
        if (t < nA) {
            home = c;
            return t;
        }
    }
    return nA + wave_atomic_add(&ctrl->later, 1);
}

// The next ticket, drawn while the current item runs.  A gate/up item (which
// never waits) draws at its start; a down item once its waits are over.  So
// the draw's latency overlaps the item, and a ticket held ahead never waits
// behind a wait of its holder.  A wave on a gate/up item draws from its
// class; a wave past every class draws from `later`, in order, as draw_ticket
// would.  `want` is set by the scheduler only while enough tickets remain
// that the draw is likely to succeed (an empty draw is one more atomic on a
// contended counter).  The value is read after the item.
struct NextTicket {
    int* ctr = nullptr;      // counter drawn from, null if none was issued
    bool later = false;
    bool want = false;
    int old = 0;
    __device__ __forceinline__ void issue(Ctrl* ctrl, char* cls, int home) {
        if (!want) return;
        later = home < 0;
        ctr = later ? &ctrl->later : reinterpret_cast<int*>(cls + home * CLASS_STRIDE);
        if (threadIdx.x == 0) old = atomicAdd(ctr, 1);
    }
    // The drawn ticket, or -1 when none was drawn or the class was spent.
    __device__ __forceinline__ int take(int home, int nclass, int nA) {
        if (!ctr) return -1;
        const int v = __shfl(old, 0, WAVE);
        const int t = later ? nA + v : home + nclass * v;
        ctr = nullptr;
        return later || t < nA ? t : -1;
    }
};

__device__ __forceinline__ void reset_counter(int* p) {
    if (threadIdx.x == 0) __hip_atomic_store(p, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float silu_clamped(float g, float u, float limit) {
    // comparisons leave NaN untouched, as in lna_moe_ticket.cu:350-352
    if (g > limit) g = limit;
    if (u < -limit) u = -limit;
    if (u > limit) u = limit;
    return (g / (1.0f + expf(-g))) * u;
}

// Four consecutive fp16 scale values starting at element `col` of the vector
// whose address is `addr` (col is a multiple of 4, so one 8-byte load).
__device__ __forceinline__ void load_half4(uint16_t (&v)[4], int64_t addr, int col) {
    gptr_t<uint32_t> p = as_global(reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(addr) + col));
    const uint32_t a = p[0], b = p[1];
    v[0] = (uint16_t)a;
    v[1] = (uint16_t)(a >> 16);
    v[2] = (uint16_t)b;
    v[3] = (uint16_t)(b >> 16);
}

// ---------------------------------------------------------------- item parts
//
// Shared by the two schedules: the ticket kernel (one launch; DEV = true:
// device-scope stores and loads, the data handed over inside the launch) and
// the phased launches for small batches (DEV = false: plain stores and loads,
// each phase a launch of its own).  Item bodies are instantiated once per bit
// width; the kernels dispatch on the expert's width at item granularity (a
// uniform branch per wave).

// gate/up partial sums of (expert e, pairs pb.., rows `mask`, projection p,
// 256-column block cb, k-chunk kc).  rowmap (LDS, optional): the pair of the
// r-th row is rowmap[r] instead of pb + r.
template <int B, int CB, bool DEV>
__device__ __forceinline__ void gateup_partials(const Params& P, int e, int pb, uint32_t mask, uint16_t* xa, int p,
                                                int cb, int kc, Tracer& tr, const int16_t* rowmap = nullptr) {
    const Layout& L = P.L;
    const int R = __popc(mask);
    const int kchunk = L.stepsA * STEP_K;
    const int k0 = kc * kchunk;

    float4_t acc[16];
    if constexpr (B == 0) {
        zero_acc(acc);              // a width outside the instance (see dispatch_bits)
    } else {
        // step-0 weights are in flight while the input rotation runs
        const u32x4_t* tp = tile_ptr<B>(reinterpret_cast<const int16_t*>((p ? P.ut : P.gt)[e]), P.I / 16, k0 / 16,
                                        cb * 16);
        const uint16_t* suh = reinterpret_cast<const uint16_t*>((p ? P.usu : P.gsu)[e]);
        TileRegs<B> first;
        rotate_rows_and_load<B>(P.x, P.H, k0, P.x_kind, suh + k0, mask, xa, kchunk / 128, NSTEP_CAP, first, tp);
        __syncthreads();
        tr(EV_STORED);                  // input rotated (trace builds)
        mma_steps<B, CB, true>(first, tp, P.I / 16, L.stepsA, xa, NSTEP_CAP, R, acc);
        tr(EV_A_MMA);
    }

    float* PA = at<float>(P.scratch, L.PA);
    store_partials<DEV>(acc, PA + ((((size_t)(rowmap ? 0 : pb) * 2 + p) * L.nI + cb) * L.SA + kc) * COLS,
                        (size_t)2 * L.SA * P.I, R, COLS, reinterpret_cast<float*>(xa), rowmap);
}

// Four fp16 down-input values of one pair at columns col..col+3 of the
// intermediate (col % 4 == 0; each half-wave holds one 128-block): the gate/up
// split-K sums in chunk order, output Hadamard + svh, clamped SwiGLU, fp16, the
// down projection's suh and input Hadamard.  gsv/usv/dsu: the expert's scales
// at those columns.
template <int CPOL>
__device__ __forceinline__ uint2 down_input4(const Params& P, int pair, int col, const uint16_t (&gsv)[4],
                                             const uint16_t (&usv)[4], const uint16_t (&dsu)[4]) {
    const Layout& L = P.L;
    const float* PA = at<float>(P.scratch, L.PA);
    float4_t ga, ua;
    // uniform buffer bases, the pair in the per-lane offset: `pair` may differ
    // between the half-waves (< 1 GB of partials, inside the 32-bit offset)
    const uint32_t cb = (uint32_t)col / COLS, c = (uint32_t)col % COLS;
    sum_partials2<CPOL>(PA, PA + (size_t)L.SA * P.I,
                        ((uint32_t)pair * 2u * (uint32_t)(L.SA * P.I) + cb * (uint32_t)(L.SA * COLS) + c) * 4u,
                        COLS, L.SA, ga, ua);
    float gv[4] = {ga[0], ga[1], ga[2], ga[3]}, uv[4] = {ua[0], ua[1], ua[2], ua[3]};
    fwht128_x4(gv);
    fwht128_x4(uv);
    float dv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float gg = gv[i] * HAD_NORM * f16_bits_to_f32(gsv[i]);
        const float uu = uv[i] * HAD_NORM * f16_bits_to_f32(usv[i]);
        const uint16_t act = f32_to_f16_bits(silu_clamped(gg, uu, P.limit));
        // down input rotation: half(act * down_suh), fp32 butterflies
        dv[i] = f16_bits_to_f32(f32_to_f16_bits(f16_bits_to_f32(act) * f16_bits_to_f32(dsu[i])));
    }
    fwht128_x4(dv);
    uint2 packed;
    packed.x = (uint32_t)f32_to_f16_bits(dv[0] * HAD_NORM) | ((uint32_t)f32_to_f16_bits(dv[1] * HAD_NORM) << 16);
    packed.y = (uint32_t)f32_to_f16_bits(dv[2] * HAD_NORM) | ((uint32_t)f32_to_f16_bits(dv[3] * HAD_NORM) << 16);
    return packed;
}

// gate/up finish of (expert e, pairs pb..pb+R-1, column block cb): stores the
// fp16 down input DI of every pair.
template <bool DEV>
__device__ __forceinline__ void gateup_finish(const Params& P, int e, int pb, int R, int cb) {
    const Layout& L = P.L;
    const int lane = threadIdx.x & (WAVE - 1);
    const int col = cb * COLS + 128 * (lane >> 5) + 4 * (lane & 31);
    // scales first: their loads are in flight during the partial sums
    uint16_t gsv[4], usv[4], dsu[4];
    load_half4(gsv, P.gsv[e], col);
    load_half4(usv, P.usv[e], col);
    load_half4(dsu, P.dsu[e], col);
    uint16_t* DI = at<uint16_t>(P.scratch, L.DI);
    for (int r = 0; r < R; ++r) {
        const int pair = pb + r;
        const uint2 packed = down_input4<DEV ? CPOL_SC1 : CPOL_PLAIN>(P, pair, col, gsv, usv, dsu);
        uint32_t* dst = reinterpret_cast<uint32_t*>(DI + (size_t)pair * P.I + col);
        if constexpr (DEV) st_dev2(dst, packed);
        else *reinterpret_cast<uint2*>(dst) = packed;
    }
}

// down partial sums of (pairs pb..pb+R-1, 256-column block cb of hidden,
// k-chunk kc of intermediate); `first` holds the step-0 tile of `tp`.
template <int B, int CB, bool DEV>
__device__ __forceinline__ void down_partials(const Params& P, int pb, int R, uint16_t* xa, int cb, int kc,
                                              TileRegs<B>& first, const u32x4_t* tp, Tracer& tr) {
    const Layout& L = P.L;
    const int kchunk = L.stepsB * STEP_K;
    const int k0 = kc * kchunk;
    float4_t acc[16];
    if constexpr (B == 0) {
        zero_acc(acc);
    } else {
        const uint16_t* DI = at<uint16_t>(P.scratch, L.DI);
        for (int r = 0; r < R; ++r) copy_row<DEV>(DI + (size_t)(pb + r) * P.I + k0, xa, r, kchunk / 128, NSTEP_CAP);
        __syncthreads();
        mma_steps<B, CB, true>(first, tp, P.H / 16, L.stepsB, xa, NSTEP_CAP, R, acc);
        tr(EV_B_MMA);
    }

    float* PB = at<float>(P.scratch, L.PB);
    store_partials<DEV>(acc, PB + (((size_t)pb * L.nH + cb) * L.SB + kc) * COLS, (size_t)L.SB * P.H, R, COLS,
                        reinterpret_cast<float*>(xa));
}

// Down output of one pair for the lane's four columns `col` (expert scales
// dsv): the split-K sum in chunk order, output Hadamard, svh (fp32).
template <int CPOL>
__device__ __forceinline__ float4_t down_value(const Params& P, int pair, const uint16_t (&dsv)[4], int col) {
    const Layout& L = P.L;
    const uint32_t cb = (uint32_t)col / COLS, c = (uint32_t)col % COLS;
    const float4_t t = sum_partials<CPOL>(at<float>(P.scratch, L.PB) + (size_t)pair * L.SB * P.H,
                                          (cb * (uint32_t)(L.SB * COLS) + c) * 4u, COLS, L.SB);
    float v[4] = {t[0], t[1], t[2], t[3]};
    fwht128_x4(v);
    float4_t o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = v[i] * HAD_NORM * f16_bits_to_f32(dsv[i]);
    return o;
}

// ---------------------------------------------------------------- ticket items

// gate/up item: (group g, projection p, 256-column block cb, k-chunk kc)
template <int B, int CB>
__device__ void item_a_body(const Params& P, const Plan& pl, uint16_t* xa, int g, int p, int cb, int kc,
                            int epoch, Tracer& tr, NextTicket& nt, int home) {
    const Layout& L = P.L;
    nt.issue(at<Ctrl>(P.scratch, L.ctrl), P.scratch + L.cls, home);
    gateup_partials<B, CB, true>(P, pl.gexp[g], pl.gpair[g], pl.gmask[g], xa, p, cb, kc, tr);
    tr(EV_STORED);
    publish_fence();
    tr(EV_FENCED);
    int* cnt = word(P.scratch, L.cntA, g * MAX_BLOCKS + cb);
    const bool last = wave_atomic_add(cnt, 1) == 2 * L.SA - 1;
    tr(EV_A_END, last);
    if (!last) return;

    // Last arriver: gate/up finish for (group g, column block cb), then the flag.
    gateup_finish<true>(P, pl.gexp[g], pl.gpair[g], __popc(pl.gmask[g]), cb);
    reset_counter(cnt);
    publish_fence();
    if (threadIdx.x == 0)
        __hip_atomic_store(word(P.scratch, L.doneA, g * MAX_BLOCKS + cb), epoch + 1, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    tr(EV_EPI_A_END);
}

// down item: (group g, 256-column block cb of hidden, k-chunk kc of intermediate)
template <int B, int CB>
__device__ void item_b_body(const Params& P, const Plan& pl, uint16_t* xa, int g, int cb, int kc, int epoch,
                            Tracer& tr, NextTicket& nt) {
    const Layout& L = P.L;
    const int e = pl.gexp[g], pb = pl.gpair[g];
    const int R = __popc(pl.gmask[g]);
    const int kchunk = L.stepsB * STEP_K;
    const int k0 = kc * kchunk;

    const u32x4_t* tp = tile_ptr<B>(reinterpret_cast<const int16_t*>(P.dt[e]), P.H / 16, k0 / 16, cb * 16);
    TileRegs<B> first;
    if constexpr (B != 0) load_tile<B>(first, tp);

    // wait for the gate/up column blocks this chunk reads
    for (int c = k0 / COLS; c <= (k0 + kchunk - 1) / COLS; ++c)
        wait_flag(word(P.scratch, L.doneA, g * MAX_BLOCKS + c), epoch + 1, &at<Ctrl>(P.scratch, L.ctrl)->error);
    tr(EV_B_WAITED);
    nt.issue(at<Ctrl>(P.scratch, L.ctrl), P.scratch + L.cls, -1);

    down_partials<B, CB, true>(P, pb, R, xa, cb, kc, first, tp, tr);
    tr(EV_STORED);
    publish_fence();
    tr(EV_FENCED);
    int* cnt = word(P.scratch, L.cntB, g * MAX_BLOCKS + cb);
    const bool last = wave_atomic_add(cnt, 1) == L.SB - 1;
    tr(EV_B_END, last);
    if (!last) return;

    // Last arriver for (group, H block): output rotation + svh.
    const int lane = threadIdx.x;
    const int col = cb * COLS + 128 * (lane >> 5) + 4 * (lane & 31);
    uint16_t dsv[4];
    load_half4(dsv, P.dsv[e], col);
    float* DC = at<float>(P.scratch, L.DC);
    for (int r = 0; r < R; ++r) st_dev4(DC + (size_t)(pb + r) * P.H + col, down_value<CPOL_SC1>(P, pb + r, dsv, col));
    reset_counter(cnt);
    publish_fence();
    int* cg = word(P.scratch, L.cntG, cb);
    const bool done = wave_atomic_add(cg, 1) == pl.U - 1;
    tr(EV_EPI_B_END, done);
    if (!done) return;
    // Every group has finished this H block: publish it to the gather items.
    reset_counter(cg);
    publish_fence();
    if (lane == 0)
        __hip_atomic_store(word(P.scratch, L.doneB, cb), epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// gather item: (H block cb, row) -- out[row][block] = sum over the row's top-k
// slots, in slot order, of weight * down output (fp32), one cast.
__device__ void item_g(const Params& P, const Plan& pl, int t, int epoch, Tracer& tr) {
    const Layout& L = P.L;
    const int cb = t / P.m, row = t - (t / P.m) * P.m;
    wait_flag(word(P.scratch, L.doneB, cb), epoch + 1, &at<Ctrl>(P.scratch, L.ctrl)->error);
    const int lane = threadIdx.x;
    const int col = cb * COLS + 128 * (lane >> 5) + 4 * (lane & 31);
    compiler_barrier();
    const __amdgpu_buffer_rsrc_t dc = dev_rsrc(at<float>(P.scratch, L.DC));
    float4_t d[MAX_TOPK];
    float wt[MAX_TOPK];
    int pr[MAX_TOPK];
#pragma unroll
    for (int j = 0; j < MAX_TOPK; ++j) {       // every slot's load issued first
        pr[j] = j < P.topk ? pl.slotpair[row * P.topk + j] : -1;
        wt[j] = pr[j] >= 0 ? P.rt.weight(row * P.topk + j) : 0.f;
        if (pr[j] >= 0) d[j] = ld_dev4_buf(dc, (uint32_t)col * 4u, (uint32_t)pr[j] * (uint32_t)P.H * 4u);
    }
    float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < MAX_TOPK; ++j) {       // fp32 sum in top-k slot order
        if (pr[j] < 0) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) s4[i] = s4[i] + wt[j] * d[j][i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) store_out(P.out, (size_t)row * P.H + col + i, P.out_kind, s4[i]);
    tr(EV_GATHER_END);
}

// Width dispatch: runs body<B> for the instantiated width B == bits.  A width
// outside MASK (the host rejects such tables before launch) sets bit 0 of the
// error word and runs body<0>: the item writes zero partials and still takes
// part in every counter and flag, so the layer completes with that expert's
// contribution zero and the scratch's control words stay consistent.
template <uint32_t MASK, typename F>
__device__ __forceinline__ void dispatch_bits(int bits, int* err, F&& body) {
    bool done = false;
    static_for<8>([&](auto BI) {
        constexpr int B = decltype(BI)::value + 1;
        if constexpr ((MASK >> B) & 1u) {
            if (!done && bits == B) {
                body(std::integral_constant<int, B>{});
                done = true;
            }
        }
    });
    if (!done) {
        if ((threadIdx.x & (WAVE - 1)) == 0) atomicOr(err, ERR_WIDTH);
        body(std::integral_constant<int, 0>{});
    }
}

template <uint32_t MASK, int CB>
__device__ void item_a(const Params& P, const Plan& pl, uint16_t* xa, int t, int epoch, Tracer& tr, NextTicket& nt,
                       int home) {
    const Layout& L = P.L;
    const int per_g = 2 * L.nI * L.SA;
    const int g = t / per_g;
    int rem = t - g * per_g;
    const int p = rem / (L.nI * L.SA);
    rem -= p * L.nI * L.SA;
    const int cb = rem / L.SA, kc = rem - (rem / L.SA) * L.SA;
    dispatch_bits<MASK>(pl.gbits[g], &at<Ctrl>(P.scratch, L.ctrl)->error, [&](auto BI) {
        item_a_body<decltype(BI)::value, CB>(P, pl, xa, g, p, cb, kc, epoch, tr, nt, home);
    });
}

template <uint32_t MASK, int CB>
__device__ void item_b(const Params& P, const Plan& pl, uint16_t* xa, int t, int epoch, Tracer& tr, NextTicket& nt) {
    const Layout& L = P.L;
    const int per_g = L.nH * L.SB;
    const int g = t / per_g;
    const int rem = t - g * per_g;
    const int cb = rem / L.SB, kc = rem - (rem / L.SB) * L.SB;
    dispatch_bits<MASK>(pl.gbits[g], &at<Ctrl>(P.scratch, L.ctrl)->error, [&](auto BI) {
        item_b_body<decltype(BI)::value, CB>(P, pl, xa, g, cb, kc, epoch, tr, nt);
    });
}

// Dynamic LDS of one workgroup: the activation tile of an item (rows x
// NSTEP_CAP steps x 64 halves, which is also the fp32 transpose buffer of its
// partials, 1 KB per row) or the route-plan workspace, whichever is larger.
// Sized by the batch, so small batches leave room for more resident waves.
inline int moe_lds_kb(int64_t m, int64_t n_experts) {
    const int64_t rows = m < MAX_ROWS ? m : MAX_ROWS;     // an item takes at most 16 rows per pass
    const int64_t a = rows * NSTEP_CAP * STEP_K * 2, b = 6 * n_experts;
    return (int)(((a > b ? a : b) + 1023) / 1024);
}

template <uint32_t MASK, int CB>
__global__ __launch_bounds__(64, 2) void moe_kernel(Params P) {   // 2 waves per SIMD: <= 256 registers
    extern __shared__ __align__(16) uint16_t xa[];   // moe_lds_kb(m, E) KB
    __shared__ Plan pl;
    const Layout& L = P.L;
    Tracer tr;
    tr.init(P.scratch + P.trace_off);
    tr(EV_START);
    Ctrl* ctrl = at<Ctrl>(P.scratch, L.ctrl);
    const int epoch = __hip_atomic_load(&ctrl->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int nclass = P.nclass;
    int home = nclass > 1 ? xcc_id() % nclass : 0;
    char* cls = P.scratch + L.cls;
    // The first ticket is drawn from this wave's class while the plan is built
    // (a ticket past the gate/up items only means the class is spent).
    NextTicket nt;
    nt.want = true;
    nt.issue(ctrl, cls, home);

    build_plan(P, pl, reinterpret_cast<char*>(xa));
    tr(EV_PLAN);
    const int U = pl.U;
    const int nA = U * 2 * L.nI * L.SA;
    const int nAB = nA + U * L.nH * L.SB;
    const int total = U ? nAB + L.nH * P.m : 0;

    if (U == 0 && blockIdx.x == 0) {   // nothing routed: the layer output is zero
        for (int i = threadIdx.x; i < P.m * P.H; i += WAVE) store_out(P.out, i, P.out_kind, 0.f);
    }

    // Ticket order: gate/up items, down items, gather items; every ticket is
    // drawn from the counter by the wave that will run it.
    int t = nt.take(home, nclass, nA);
    if (t < 0) t = draw_ticket(ctrl, cls, nclass, home, nA, total);
    const int ahead = (int)gridDim.x;      // draw ahead while this many tickets remain beyond t
    while (t < total) {
        nt.want = t + ahead < (t < nA ? nA : total);
        if (t < nA) {
            tr(EV_A_BEGIN, t);
            item_a<MASK, CB>(P, pl, xa, t, epoch, tr, nt, home);
        } else if (t < nAB) {
            tr(EV_B_BEGIN, t - nA);
            item_b<MASK, CB>(P, pl, xa, t - nA, epoch, tr, nt);
        } else {
            item_g(P, pl, t - nAB, epoch, tr);
        }
        __syncthreads();   // xa is rewritten by the next item
        t = nt.take(home, nclass, nA);
        if (t < 0) t = draw_ticket(ctrl, cls, nclass, home, nA, total);
    }

    // Retire; the last wave out resets the queue and advances the epoch.
    tr(EV_RETIRE);
    publish_fence();
    if (threadIdx.x == 0) {
        const int r = atomicAdd(&ctrl->retire, 1);
        if (r == (int)gridDim.x - 1) {
            for (int c = 0; c < nclass; ++c)
                __hip_atomic_store(reinterpret_cast<int*>(cls + c * CLASS_STRIDE), 0, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&ctrl->later, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&ctrl->retire, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&ctrl->epoch, epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---------------------------------------------------------------- phased launches (short layers)
//
// Plain launches on one stream (gate/up, the activation for larger batches,
// down, finish), keyed by top-k slot instead of the
// expert-sorted route plan: an item's slot o names its expert e, the item runs
// only when o is e's first slot, and it finds the rows routed to e itself (one
// ballot over the call's slot ids: no plan, no barrier before the first weight
// load).  The pair (row r, expert e) is indexed by the first slot of row r
// that holds e, so partial sums and down outputs are found by slot and the
// last launch sums a row's slots directly.  Item sizes, the sums and their
// order are the ticket kernel's, so both schedules give bitwise the same out.

struct SlotGroup {
    int e, R, bits;
    uint32_t mask;     // rows routed to e
};

// Expert of slot o, its rows and each row's pair slot (pslot[r], LDS, for the
// r-th row in ascending order).  False when slot o holds no valid expert or is
// not the first slot holding it.
constexpr int SLOTS_PER_LANE = (PHASED_MAX_SLOTS + WAVE - 1) / WAVE;
__device__ __forceinline__ bool slot_group(const Params& P, int o, SlotGroup& g, int16_t* pslot) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int S = P.m * P.topk;                 // <= PHASED_MAX_SLOTS: SLOTS_PER_LANE slots per lane
    int sl[SLOTS_PER_LANE];
#pragma unroll
    for (int i = 0; i < SLOTS_PER_LANE; ++i) sl[i] = lane + i * WAVE;
    int v[SLOTS_PER_LANE];
    P.rt.local_n(sl, S, P.E, v);
    const int oi = o / WAVE;
    int vo = v[0];
#pragma unroll
    for (int i = 1; i < SLOTS_PER_LANE; ++i)
        if (oi == i) vo = v[i];
    const int e = __builtin_amdgcn_readlane(vo, o & (WAVE - 1));
    if (e < 0) return false;
    uint64_t mk[SLOTS_PER_LANE];
#pragma unroll
    for (int i = 0; i < SLOTS_PER_LANE; ++i) mk[i] = __ballot(v[i] == e);
    int first = -1;
#pragma unroll
    for (int i = SLOTS_PER_LANE - 1; i >= 0; --i)
        if (mk[i]) first = WAVE * i + __builtin_ctzll(mk[i]);
    if (first != o) return false;
    uint32_t mask = 0u;
    int R = 0;
#pragma unroll
    for (int i = 0; i < SLOTS_PER_LANE; ++i) {
        uint64_t bits = mk[i];
        while (bits) {
            const int s = WAVE * i + __builtin_ctzll(bits);
            bits &= bits - 1u;
            const int row = s / P.topk;
            if (!((mask >> row) & 1u)) {
                mask |= 1u << row;
                if (lane == 0) pslot[R] = (int16_t)s;
                ++R;
            }
        }
    }
    g.e = e;
    g.R = R;
    g.mask = mask;
    g.bits = P.ebits ? P.ebits[e] : P.bits;
    __syncthreads();
    return true;
}

// Down input of the rows pslot[0..R) at intermediate columns [k0, k0 + kchunk)
// (kchunk a multiple of 128), written into the LDS A tile: each half-wave
// computes one (row, 128-block) unit per pass (its butterflies never leave the
// half-wave, so a half-wave without a unit skips the pass).
__device__ __forceinline__ void down_input_chunk(const Params& P, int e, int R, const int16_t* pslot, uint16_t* xa,
                                                 int k0, int kchunk) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int nblk = kchunk / 128;
    const int units = R * nblk;
    for (int u0 = 0; u0 < units; u0 += 2) {
        const int u = u0 + (lane >> 5);
        if (u < units) {
            const int r = u / nblk, b = u - r * nblk;
            const int kk = 128 * b + 4 * (lane & 31);      // column within the chunk
            const int col = k0 + kk;
            uint16_t gsv[4], usv[4], dsu[4];
            load_half4(gsv, P.gsv[e], col);
            load_half4(usv, P.usv[e], col);
            load_half4(dsu, P.dsu[e], col);
            const uint2 pk = down_input4<CPOL_PLAIN>(P, pslot[r], col, gsv, usv, dsu);
            const uint16_t h[4] = {(uint16_t)(pk.x & 0xffffu), (uint16_t)(pk.x >> 16), (uint16_t)(pk.y & 0xffffu),
                                   (uint16_t)(pk.y >> 16)};
#pragma unroll
            for (int i = 0; i < 4; ++i) xa[xa_index(r, (kk + i) >> 6, NSTEP_CAP, (kk + i) & 63)] = h[i];
        }
    }
}

// The rows of `mask` from the `skip`-th set bit on, at most MAX_ROWS of them:
// an expert routed by more than 16 rows of a batch runs its item in passes of
// 16 rows (each pass streams and decodes the item's weights again; the LDS
// A tile stays at 16 rows, so residency does not depend on the batch).
__device__ __forceinline__ uint32_t row_pass(uint32_t mask, int skip) {
    for (int i = 0; i < skip; ++i) mask &= mask - 1u;
    uint32_t pass = 0u;
    for (int i = 0; i < MAX_ROWS && mask; ++i) {
        pass |= mask & (0u - mask);
        mask &= mask - 1u;
    }
    return pass;
}

// Launch 1: item = (slot, projection, column block of I, k-chunk).
template <uint32_t MASK, int CB>
__global__ __launch_bounds__(64, 2) void moe_slot_gateup(Params P) {
    extern __shared__ __align__(16) uint16_t xa[];   // moe_lds_kb(m, E) KB
    __shared__ int16_t pslot[MAX_M];
    const Layout& L = P.L;
    Tracer tr;
    tr.init(P.scratch + P.trace_off);
    tr(EV_START);
    const int per_o = 2 * L.nI * L.SA;
    const int o = blockIdx.x / per_o;
    SlotGroup g;
    if (!slot_group(P, o, g, pslot)) return;
    tr(EV_PLAN);
    int rem = blockIdx.x - o * per_o;
    const int p = rem / (L.nI * L.SA);
    rem -= p * L.nI * L.SA;
    const int cb = rem / L.SA, kc = rem - (rem / L.SA) * L.SA;
    dispatch_bits<MASK>(g.bits, &at<Ctrl>(P.scratch, L.ctrl)->error, [&](auto BI) {
        for (int r0 = 0; r0 < g.R; r0 += MAX_ROWS) {
            if (r0) __syncthreads();                  // the previous pass is done with xa
            gateup_partials<decltype(BI)::value, CB, false>(P, g.e, 0, row_pass(g.mask, r0), xa, p, cb, kc, tr,
                                                            pslot + r0);
        }
    });
    tr(EV_A_END);
}

// Launch 2 (large batches only): item = (slot, column block of I).  A slot
// that is the pair slot of its (row, expert), i.e. the first slot of its row
// holding that expert, stores that pair's fp16 down input DI; one row per item,
// so all rows run at once.
template <int DUMMY = 0>
__global__ __launch_bounds__(64) void moe_slot_act(Params P) {
    const Layout& L = P.L;
    const int s = blockIdx.x / L.nI, cb = blockIdx.x - (blockIdx.x / L.nI) * L.nI;
    const int lane = threadIdx.x & (WAVE - 1);
    const int s0 = (s / P.topk) * P.topk;
    const int sl[1] = {s0 + (lane < P.topk ? lane : P.topk)};          // lanes past top-k read nothing
    int vv[1];
    P.rt.local_n(sl, s0 + P.topk, P.E, vv);
    const int v = vv[0];                                               // the row's experts, one per lane
    const int e = __builtin_amdgcn_readlane(v, s - s0);
    if (e < 0 || s0 + __builtin_ctzll(__ballot(v == e)) != s) return;
    const int col = cb * COLS + 128 * (lane >> 5) + 4 * (lane & 31);
    uint16_t gsv[4], usv[4], dsu[4];
    load_half4(gsv, P.gsv[e], col);
    load_half4(usv, P.usv[e], col);
    load_half4(dsu, P.dsu[e], col);
    uint16_t* DI = at<uint16_t>(P.scratch, L.DI);
    *reinterpret_cast<uint2*>(DI + (size_t)s * P.I + col) = down_input4<CPOL_PLAIN>(P, s, col, gsv, usv, dsu);
}

// Launch 3: item = (slot, column block of H, k-chunk of I).  For small
// batches (fuse_act) the item first computes its chunk of the down input (the
// activation of the gate/up sums) into LDS while its first weight tile is in
// flight; otherwise it copies that chunk from the activation launch's DI.
template <uint32_t MASK, int CB>
__global__ __launch_bounds__(64, 2) void moe_slot_down(Params P) {
    extern __shared__ __align__(16) uint16_t xa[];   // moe_lds_kb(m, E) KB
    __shared__ int16_t pslot[MAX_M];
    const Layout& L = P.L;
    Tracer tr;
    tr.init(P.scratch + P.trace_off, TRACE_WAVES / 2);
    tr(EV_B_BEGIN);
    const int per_o = L.nH * L.SB;
    const int o = blockIdx.x / per_o;
    SlotGroup g;
    if (!slot_group(P, o, g, pslot)) return;
    tr(EV_PLAN);
    const int rem = blockIdx.x - o * per_o;
    const int cb = rem / L.SB, kc = rem - (rem / L.SB) * L.SB;
    dispatch_bits<MASK>(g.bits, &at<Ctrl>(P.scratch, L.ctrl)->error, [&](auto BI) {
        constexpr int B = decltype(BI)::value;
        const int kchunk = L.stepsB * STEP_K;
        for (int r0 = 0; r0 < g.R; r0 += MAX_ROWS) {
            const int R = min(g.R - r0, MAX_ROWS);
            const int16_t* ps = pslot + r0;
            if (r0) __syncthreads();                  // the previous pass is done with xa
            float4_t acc[16];
            if constexpr (B == 0) {
                zero_acc(acc);
            } else {
                const u32x4_t* tp = tile_ptr<B>(reinterpret_cast<const int16_t*>(P.dt[g.e]), P.H / 16,
                                                kc * kchunk / 16, cb * 16);
                TileRegs<B> first;
                if (P.fuse_act) {
                    load_tile<B>(first, tp);
                    down_input_chunk(P, g.e, R, ps, xa, kc * kchunk, kchunk);
                } else {
                    // the first rows' input is requested before the step-0 tile, so
                    // waiting for it (loads complete in issue order) skips the tile
                    const uint16_t* DI = at<uint16_t>(P.scratch, L.DI) + (size_t)kc * kchunk;
                    uint32_t v[IN_AHEAD][HAD_MAX_BLOCKS];
#pragma unroll
                    for (int i = 0; i < IN_AHEAD; ++i)
                        if (i < R) copy_row_load<false>(DI + (size_t)ps[i] * P.I, kchunk / 128, v[i]);
                    load_tile<B>(first, tp);
#pragma unroll
                    for (int i = 0; i < IN_AHEAD; ++i)
                        if (i < R) copy_row_store(v[i], xa, i, kchunk / 128, NSTEP_CAP);
                    for (int r = IN_AHEAD; r < R; ++r)
                        copy_row<false>(DI + (size_t)ps[r] * P.I, xa, r, kchunk / 128, NSTEP_CAP);
                }
                __syncthreads();
                tr(EV_B_WAITED);
                mma_steps<B, CB, true>(first, tp, P.H / 16, L.stepsB, xa, NSTEP_CAP, R, acc);
                tr(EV_B_MMA);
            }
            store_partials<false>(acc, at<float>(P.scratch, L.PB) + ((size_t)cb * L.SB + kc) * COLS,
                                  (size_t)L.SB * P.H, R, COLS, reinterpret_cast<float*>(xa), ps);
        }
    });
    tr(EV_B_END);
}

// Launch 4: item = (column block of H, row), one wave per top-k slot: each
// wave finishes its slot's down output (the split-K sum, output Hadamard,
// svh), so every slot's loads are in flight at once; wave 0 then adds them in
// top-k slot order (fp32) and casts once.
template <int DUMMY = 0>
__global__ __launch_bounds__(MAX_TOPK * WAVE) void moe_slot_finish(Params P) {
    __shared__ float4_t slot_val[MAX_TOPK][WAVE];
    const int cb = blockIdx.x / P.m, row = blockIdx.x - (blockIdx.x / P.m) * P.m;
    const int j = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
    const int col = cb * COLS + 128 * (lane >> 5) + 4 * (lane & 31);
    const int s0 = row * P.topk;
    const int sl[1] = {s0 + (lane < P.topk ? lane : P.topk)};         // lanes past top-k read nothing
    int vv[1];
    P.rt.local_n(sl, s0 + P.topk, P.E, vv);
    const int v = vv[0];                                              // the row's experts, one per lane
    const int e = __builtin_amdgcn_readlane(v, j);
    if (e >= 0) {
        const int pair = s0 + __builtin_ctzll(__ballot(v == e));       // the row's first slot with e
        uint16_t dsv[4];
        load_half4(dsv, P.dsv[e], col);
        slot_val[j][lane] = down_value<CPOL_PLAIN>(P, pair, dsv, col);
    }
    __syncthreads();
    if (j != 0) return;
    float s4[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < P.topk; ++k) {      // fp32 sum in top-k slot order
        if (__builtin_amdgcn_readlane(v, k) < 0) continue;
        const float w = P.rt.weight(s0 + k);
        const float4_t o = slot_val[k][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) s4[i] = s4[i] + w * o[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) store_out(P.out, (size_t)row * P.H + col + i, P.out_kind, s4[i]);
}

// Launcher for one (bit-width mask, codebook) instantiation; defined in exl3_moe_inst.hip.
template <uint32_t MASK, int CB>
int launch_moe(const Params& P, int waves, int lds_kb, hipStream_t stream);

// The phased launches (three, or four with a separate activation launch).
template <uint32_t MASK, int CB>
int launch_phased(const Params& P, int lds_kb, hipStream_t stream);

template <uint32_t MASK, int CB>
int moe_waves_per_cu(int lds_kb);

}  // namespace moe
}  // namespace exl3
