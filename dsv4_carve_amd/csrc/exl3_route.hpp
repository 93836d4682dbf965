// Top-k routing input as the serving layer hands it over, read inside the
// routed-expert kernels' planning and gathering steps: expert ids (int32 or
// int64), routing weights (fp32, fp16 or bf16, already scaled) and an optional
// global -> local expert map (int64, negative for experts another rank owns).
//
// A slot's local expert is valid when the id is inside the map (or, without a
// map, inside [0, E)) and the mapped id is inside [0, E); any other slot
// contributes nothing.  This is map_topk_to_local's rule
// (recipe-lna/vllm_exl3_exl3.py.lna:963-985) with its sentinel read as "skip",
// so the plugin's id mapping, dtype casts and contiguity copies before the
// kernel are no longer separate launches.
#pragma once

#include "exl3_decode.hpp"
#include "exl3_capi_util.hpp"

namespace exl3 {

enum IdsKind : int { IDS_I32 = 0, IDS_I64 = 1 };
constexpr int64_t MAX_MAP = 1 << 20;   // longest global expert map

struct Route {
    const void* ids;        // [rows][topk], IdsKind
    const void* w;          // [rows][topk], OutKind codes (fp16, bf16, fp32)
    const int64_t* emap;    // [n_global] or null
    int ids_kind, w_kind, n_global;

    // Global id of slot s as stored.
    __device__ __forceinline__ int64_t raw(int s) const {
        return ids_kind == IDS_I64 ? static_cast<const int64_t*>(ids)[s] : (int64_t) static_cast<const int32_t*>(ids)[s];
    }

    // Local expert of global id g, or -1.
    __device__ __forceinline__ int map(int64_t g, int E) const {
        if (emap) {
            if (g < 0 || g >= n_global) return -1;
            g = emap[g];
        }
        return (g >= 0 && g < E) ? (int)g : -1;
    }

    // Local expert of slot s, or -1.
    __device__ __forceinline__ int local(int s, int E) const { return map(raw(s), E); }

    // local() for N slots per lane (slots >= S give -1), branch-free so all N
    // id loads, then all N map loads, are in flight together.
    template <int N>
    __device__ __forceinline__ void local_n(const int (&s)[N], int S, int E, int (&out)[N]) const {
        int64_t g[N];
        if (ids_kind == IDS_I64) {
            const int64_t* p = static_cast<const int64_t*>(ids);
#pragma unroll
            for (int i = 0; i < N; ++i) g[i] = p[s[i] < S ? s[i] : S - 1];
        } else {
            const int32_t* p = static_cast<const int32_t*>(ids);
#pragma unroll
            for (int i = 0; i < N; ++i) g[i] = p[s[i] < S ? s[i] : S - 1];
        }
        if (emap) {
            int64_t mg[N];
#pragma unroll
            for (int i = 0; i < N; ++i) mg[i] = emap[g[i] < 0 ? 0 : g[i] >= n_global ? n_global - 1 : g[i]];
#pragma unroll
            for (int i = 0; i < N; ++i) g[i] = (g[i] < 0 || g[i] >= n_global) ? -1 : mg[i];
        }
#pragma unroll
        for (int i = 0; i < N; ++i) out[i] = (s[i] < S && g[i] >= 0 && g[i] < E) ? (int)g[i] : -1;
    }

    __device__ __forceinline__ float weight(int s) const {
        if (w_kind == OUT_F32) return static_cast<const float*>(w)[s];
        const uint16_t h = static_cast<const uint16_t*>(w)[s];
        return w_kind == OUT_BF16 ? bf16_to_f32(h) : f16_bits_to_f32(h);
    }
};

// Host side: fills `rt` after checking the kinds and the map length; 0 when
// usable, else the library error code.
inline int make_route(const void* ids, int ids_kind, const void* w, int w_kind, const int64_t* emap,
                      int64_t n_global, Route& rt) {
    if (ids_kind != IDS_I32 && ids_kind != IDS_I64) return fail("expert ids must be int32 or int64");
    if (w_kind < OUT_F16 || w_kind > OUT_F32) return fail("routing weights must be fp16, bf16 or fp32");
    if (emap && (n_global < 1 || n_global > MAX_MAP)) return fail("expert map length out of range (1..1048576)");
    rt = Route{ids, w, emap, ids_kind, w_kind, emap ? (int)n_global : 0};
    return 0;
}

}  // namespace exl3
