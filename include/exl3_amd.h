/*
 * exl3_amd.h -- C ABI of libexl3_amd.so, the MI355X (gfx950) EXL3 decode path.
 *
 * Plain pointers, sizes and an opaque stream (a hipStream_t passed as void*;
 * NULL = the default stream).  Every device pointer is HBM memory on the
 * current HIP device.  Functions return 0 (or a non-negative size) on success
 * and a negative value on an argument or launch error; exl3_last_error()
 * returns the message of the last failure on the calling thread.  No call
 * allocates device memory, synchronises the stream or queries the clock, so
 * every launch can be captured into a HIP graph.
 *
 * Element kinds: x_kind 0 = fp16, 1 = bf16; out_kind 0 = fp16, 1 = bf16, 2 = fp32.
 * Codebooks: 0 = 3INST, 1 = MCG (production), 2 = MUL1.
 * Weight ABI per projection (recipe-lna/vllm_exl3_exl3.py.lna:50-54, 2083-2122):
 *   trellis int16 [in/16][out/16][16*bits], suh fp16 [in], svh fp16 [out].
 */
#ifndef EXL3_AMD_H
#define EXL3_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failed call on this thread ("" if none). */
const char* exl3_last_error(void);

/*
 * Trellis -> fp16 weight matrix [k][n] (row-major).
 * suh == svh == NULL: the raw codebook matrix Wq (exllamav3 `reconstruct`,
 *   called at recipe-lna/exllamav3/exl3.py.lna:197); k, n multiples of 16.
 * suh, svh given: W = diag(suh) H Wq H diag(svh) / 128 with 128-blocks
 *   (replaces vllm_exl3_c.dequant_trellis, recipe-lna/lna2/bindings.cpp:118-133,
 *   computed on the GPU instead of bindings.cpp:16-101); k, n multiples of 128.
 * Bit-exact with the round-to-nearest-even decode canon.
 */
int exl3_dequant(const int16_t* trellis, int64_t k, int64_t n, int bits, int codebook,
                 const uint16_t* suh, const uint16_t* svh, uint16_t* out, void* stream);

/*
 * The same matrix written transposed, out[n][k] (row-major), bit for bit the
 * values exl3_dequant writes.  No counterpart in the reference: its
 * reconstruct writes [k][n]; LinearEXL3.reconstruct_hgemm
 * (recipe-lna/exllamav3/exl3.py.lna:161-218) uses this layout because
 * hipBLASLt's fp16 GEMM reads a [n][k] operand faster on MI355X.
 */
int exl3_dequant_nk(const int16_t* trellis, int64_t k, int64_t n, int bits, int codebook,
                    const uint16_t* suh, const uint16_t* svh, uint16_t* out, void* stream);

/*
 * Row Hadamard: for every row r and 128-block b of x [rows][cols]
 *   y[r][128b + i] = (H128 v / sqrt(128))[i] * scale * post_scale[128b + i],
 *   v = x[r][128b ..] * pre_scale rounded to fp16 (as the GEMV input rotation
 *   does; x converted to fp16 first), or x itself when pre_scale is NULL.
 * Butterflies in fp32; either scale pointer may be NULL.  Replaces
 * exllamav3_ext.had_r_128(input, output, pre_scale, post_scale, scale) as
 * LinearEXL3.reconstruct_hgemm calls it around the fp16 GEMM
 * (recipe-lna/exllamav3/exl3.py.lna:186-190, 213-214).  x_kind / y_kind:
 * 0 = fp16, 1 = bf16, 2 = fp32; cols % 128 == 0; y may be x (same kind).
 */
int exl3_had_rows(const void* x, int x_kind, void* y, int y_kind, int64_t rows, int64_t cols,
                  const uint16_t* pre_scale, const uint16_t* post_scale, float scale, void* stream);

/*
 * c[m][n] = had_out(had_in(a . suh) . Wq) . svh, fp32 accumulation.
 * Replaces exllamav3 `exl3_gemm` (recipe-lna/exllamav3/exl3_gemm.cu.lna:336-364,
 * limits k % 16, n % 128 at :35-37) as used by LinearEXL3.forward for rows <= 144
 * (recipe-lna/exllamav3/exl3.py.lna:114-139), and vllm_exl3_c.exl3_gemv
 * (recipe-lna/lna2/bindings.cpp:135-148).  a: fp16 [m][k]; k % 128 == 0,
 * n % 128 == 0; any m (processed in blocks of 16 rows).  scratch: device
 * buffer of at least exl3_gemm_scratch_bytes(m, k, n) bytes, zeroed once
 * before its first use; the kernels leave its counters zero again, so one
 * buffer serves every later call on the same stream (one call at a time).
 */
int64_t exl3_gemm_scratch_bytes(int64_t m, int64_t k, int64_t n);
int exl3_gemm(const uint16_t* a, int64_t m, int64_t k, const int16_t* b, int64_t n, int bits,
              int codebook, const uint16_t* suh, const uint16_t* svh, void* c, int c_kind,
              void* scratch, int64_t scratch_bytes, void* stream);

/*
 * Same-input fan: c_j[m][n_j] = had_out(had_in(a . suh_j) . Wq_j) . svh_j for
 * count (1..8) matrices that read one input a (fp16 [m][k], k % 128 == 0): one
 * launch of split-K partial sums over every member per bit width present, one
 * finishing launch over all of them.  Replaces exllamav3 `exl3_mgemm` with a
 * broadcast A (bszm_in == 1), as the plugin's dense groups call it
 * (recipe-lna/vllm_exl3_exl3.py.lna:546-613); unlike it, members may differ in
 * bit width and need not be ordered widest first.  trellis/suh/svh/c: host
 * arrays of count device pointers; n_list: host int64 [count], each a multiple
 * of 128; bits_list: host int32 [count] in 1..8; every c_j has c_kind.
 * scratch: >= exl3_gemm_group_scratch_bytes(m, k, count, n_list) bytes (no
 * zeroing needed); one call at a time per scratch buffer.
 */
int64_t exl3_gemm_group_scratch_bytes(int64_t m, int64_t k, int64_t count, const int64_t* n_list);
int exl3_gemm_group(const uint16_t* a, int64_t m, int64_t k, int64_t count, const int16_t* const* trellis,
                    const uint16_t* const* suh, const uint16_t* const* svh, const int64_t* n_list,
                    const int32_t* bits_list, int codebook, void* const* c, int c_kind, void* scratch,
                    int64_t scratch_bytes, void* stream);

/*
 * Routed-MoE decode layer: for every row r and top-k slot j with a
 * valid expert e = expert_ids[r][j] (0 <= e < n_experts; others are skipped):
 *   g = had_out(had_in(x[r] . gate_suh[e]) . Wgate[e]) . gate_svh[e]   (fp32)
 *   u = same with up;  act = half(silu(min(g, L)) * clamp(u, -L, L))
 *   d = had_out(had_in(act . down_suh[e]) . Wdown[e]) . down_svh[e]    (fp32)
 *   out[r] = sum_j routing_weights[r][j] * d   (fp32, slot order), one cast.
 * Replaces vllm_exl3_c.lna2_moe_decode (recipe-lna/lna2/lna_moe_ticket.cu:507-581)
 * and generalises its fixed geometry (H=4096, I=256, top-6, one K per launch,
 * :34-36, 532) to any hidden and intermediate that are multiples of 256 up to
 * 16384, topk <= 9 (room for a shared expert as one more slot of weight 1)
 * and a per-expert bit width.
 *   x: [m][hidden] (x_kind), out: [m][hidden] (out_kind), 1 <= m <= exl3_moe_max_rows().
 *   Pointer tables: device int64 [n_experts] of data pointers (as built by
 *     build_exl3_fused_state, recipe-lna/vllm_exl3_exl3.py.lna:1543-1569).
 *   expert_ids int32 [m][topk], routing_weights fp32 [m][topk] (already scaled).
 *   expert_bits: device int8 [n_experts] bit widths, or NULL when every expert
 *     uses `bits`.  bits_mask: bit b set for every width b present (ignored
 *     when expert_bits is NULL).
 *   swiglu_limit: finite and > 0 (lna_moe_ticket.cu:552-553).
 *   scratch: >= exl3_moe_scratch_bytes(hidden, intermediate, topk) bytes for
 *     m <= 16, >= exl3_moe_scratch_bytes_rows(hidden, intermediate, topk, m)
 *     beyond; zeroed once before first use; self-resetting afterwards, and one
 *     buffer may serve layers of different shapes (its control words have
 *     fixed offsets).  One call at a time per scratch buffer.
 * Rows: 1 <= m <= exl3_moe_max_rows() = 32 (the reference's lna2 takes up to
 * LNA2_MAX_M = 24 rows, lna_moe_ticket.cu:40-51).  An expert routed by more
 * than 16 rows of the batch runs its items in passes of 16 rows.
 * Schedule: plain launches keyed by top-k slot (gate/up, an activation launch
 * when m * topk * intermediate > 32768, down, finish), or, up to 16 rows, one
 * persistent ticket-kernel launch; both give bitwise the same result.  The
 * launches are the default at every batch size.  The environment variable
 * EXL3_MOE_PHASED_MAX_ROWS, when set, picks by row count instead up to 16 rows
 * (0: always the ticket kernel there).  Every launch is on `stream`; nothing
 * is allocated or synchronised, so a call can be captured in a graph.
 * exl3_moe_scratch_bytes replaces lna2_moe_scratch_bytes (:481) and covers 16
 * rows; exl3_moe_scratch_bytes_rows covers up to `rows` rows (the reference
 * fixes its row capacity at build time instead).
 */
int64_t exl3_moe_scratch_bytes(int64_t hidden, int64_t intermediate, int64_t topk);
int64_t exl3_moe_scratch_bytes_rows(int64_t hidden, int64_t intermediate, int64_t topk, int64_t rows);
int exl3_moe_max_rows(void);

/*
 * Byte offset of the int32 error word inside a decode or prefill scratch
 * buffer (the host-side counterpart of the reference's TORCH_CHECK failures
 * and LNA_EXL3_DEBUG_FINITE signal, recipe-lna/lna2/lna_moe_ticket.cu:516-553,
 * lna_moe_decode.cu:707; there no error crosses the kernel boundary).  Bits:
 *   1  an expert of a width outside bits_mask was routed and not decoded
 *      (decode: a width the kernel instance chosen for bits_mask lacks;
 *      prefill: any width outside bits_mask); its contribution is zero and
 *      the items still complete, so the scratch stays consistent;
 *   2  (decode, ticket schedule) a bounded wait gave up.
 * Decode scratch: the word is zero in the zeroed buffer, the kernels only set
 * bits, and the caller reads and clears it (a 4-byte copy, outside any
 * captured region).  Prefill scratch: the first launch of every call rewrites
 * it, so it reports that call.  Widths are also checked where the entry points
 * can see them: a host-side caller that builds expert_bits should check it
 * against bits_mask before launching (the kernels cannot refuse a launch).
 */
int64_t exl3_moe_error_offset(void);
int exl3_moe_decode(const void* x, int x_kind, void* out, int out_kind, int64_t m, int64_t hidden,
                    int64_t intermediate, int64_t n_experts, int64_t topk,
                    const int64_t* gate_trellis, const int64_t* gate_suh, const int64_t* gate_svh,
                    const int64_t* up_trellis, const int64_t* up_suh, const int64_t* up_svh,
                    const int64_t* down_trellis, const int64_t* down_suh, const int64_t* down_svh,
                    const int32_t* expert_ids, const float* routing_weights,
                    const int8_t* expert_bits, int bits, int bits_mask, int codebook,
                    float swiglu_limit, void* scratch, int64_t scratch_bytes, void* stream);

/*
 * exl3_moe_decode over the top-k tensors as the serving layer holds them: the
 * global-to-local expert mapping, id widening and weight cast that the plugin
 * runs as separate launches before the kernel (map_topk_to_local,
 * recipe-lna/vllm_exl3_exl3.py.lna:963-985, and the .to(int32)/.to(float32)
 * copies of _apply_lna2_moe, :1234-1236) are done inside the kernels' route
 * planning instead.  Results are bitwise those of exl3_moe_decode on the
 * mapped int32 ids and fp32 weights.
 *   topk_ids: [m][topk], ids_kind 0 = int32, 1 = int64.
 *   topk_weights: [m][topk], weights_kind 0 = fp16, 1 = bf16, 2 = fp32.
 *   expert_map: device int64 [n_global] (global id -> local id, negative for
 *     experts of other ranks), or NULL when the ids are already local.  A slot
 *     whose id is outside the map, or whose mapped id is outside
 *     [0, n_experts), contributes nothing.
 * Other arguments as exl3_moe_decode.
 */
int exl3_moe_decode_routed(const void* x, int x_kind, void* out, int out_kind, int64_t m, int64_t hidden,
                           int64_t intermediate, int64_t n_experts, int64_t topk,
                           const int64_t* gate_trellis, const int64_t* gate_suh, const int64_t* gate_svh,
                           const int64_t* up_trellis, const int64_t* up_suh, const int64_t* up_svh,
                           const int64_t* down_trellis, const int64_t* down_suh, const int64_t* down_svh,
                           const void* topk_ids, int ids_kind, const void* topk_weights, int weights_kind,
                           const int64_t* expert_map, int64_t n_global,
                           const int8_t* expert_bits, int bits, int bits_mask, int codebook,
                           float swiglu_limit, void* scratch, int64_t scratch_bytes, void* stream);

/*
 * exl3_moe_decode_routed without a scratch argument.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * scratch is a fixed device array inside the library, one per GPU, of
 * exl3_moe_noalloc_scratch_bytes() = 128 MiB, held until the process ends; a
 * call whose exl3_moe_scratch_bytes_rows(hidden, intermediate, topk, m)
 * exceeds it is rejected (hidden 4096, intermediate 2048, top-9 needs about
 * 126 MB up to 16 rows, so larger batches of that layer are rejected).  The
 * call allocates nothing.  Its control words are zeroed by a fill kernel on
 * `stream` at the first call on each device and reset themselves afterwards.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other threads) race, so issue them on one stream.  Results
 * are bitwise those of exl3_moe_decode_routed.
 */
int64_t exl3_moe_noalloc_scratch_bytes(void);
int exl3_moe_decode_noalloc(const void* x, int x_kind, void* out, int out_kind, int64_t m, int64_t hidden,
                            int64_t intermediate, int64_t n_experts, int64_t topk,
                            const int64_t* gate_trellis, const int64_t* gate_suh, const int64_t* gate_svh,
                            const int64_t* up_trellis, const int64_t* up_suh, const int64_t* up_svh,
                            const int64_t* down_trellis, const int64_t* down_suh, const int64_t* down_svh,
                            const void* topk_ids, int ids_kind, const void* topk_weights, int weights_kind,
                            const int64_t* expert_map, int64_t n_global,
                            const int8_t* expert_bits, int bits, int bits_mask, int codebook,
                            float swiglu_limit, void* stream);

/*
 * The error word of this device's fixed scratch (the ERR bits of
 * exl3_moe_decode_noalloc's calls: 1 = an expert of a width outside bits_mask
 * was routed and contributed zero, 2 = a bounded wait gave up), read after
 * the work queued on `stream`.  No counterpart in the reference; it serves
 * the same callers as exl3_moe_decode_noalloc, which cannot see the fixed
 * array's address.  clear: 0 reads only; 1 also clears the bits; 2 also
 * resets every control word to zero, as at the first call (recovery after a
 * call that did not complete).  Synchronises `stream`, so it is refused inside
 * a graph capture; allocates nothing.  Returns the word (>= 0) or < 0.
 */
int exl3_moe_noalloc_error(int clear, void* stream);

/*
 * Routed-MoE layer for many tokens (prefill), same mathematics as
 * exl3_moe_decode: tokens are routed by expert on the device and each expert's
 * weights are decoded once per 32 routed rows, feeding fp16 MFMA with fp32
 * accumulation (grouped GEMMs; six launches on `stream`, no host sync).
 * Replaces exllamav3_ext.exl3_moe on the many-row path
 * (recipe-lna/vllm_exl3_exl3.py.lna:1597-1704) and LinearEXL3.reconstruct_hgemm
 * per expert (recipe-lna/exllamav3/exl3.py.lna:161-218), which dequantize whole
 * weights to HBM first.  Arguments as exl3_moe_decode, with tokens in place of
 * m (1 <= tokens * topk <= 65536, topk <= 9, n_experts <= 2048).  scratch:
 * >= exl3_moe_prefill_scratch_bytes(...) bytes; no zeroing needed, nothing is
 * kept between calls; one call at a time per scratch buffer.
 */
int64_t exl3_moe_prefill_scratch_bytes(int64_t tokens, int64_t hidden, int64_t intermediate, int64_t topk,
                                       int64_t n_experts);
int exl3_moe_prefill(const void* x, int x_kind, void* out, int out_kind, int64_t tokens, int64_t hidden,
                     int64_t intermediate, int64_t n_experts, int64_t topk,
                     const int64_t* gate_trellis, const int64_t* gate_suh, const int64_t* gate_svh,
                     const int64_t* up_trellis, const int64_t* up_suh, const int64_t* up_svh,
                     const int64_t* down_trellis, const int64_t* down_suh, const int64_t* down_svh,
                     const int32_t* expert_ids, const float* routing_weights,
                     const int8_t* expert_bits, int bits, int bits_mask, int codebook,
                     float swiglu_limit, void* scratch, int64_t scratch_bytes, void* stream);

/*
 * exl3_moe_prefill over the serving layer's top-k tensors and expert map, as
 * exl3_moe_decode_routed is to exl3_moe_decode (replaces the plugin's
 * map_topk_to_local and casts before the fused MoE,
 * recipe-lna/vllm_exl3_exl3.py.lna:1616-1620).
 */
int exl3_moe_prefill_routed(const void* x, int x_kind, void* out, int out_kind, int64_t tokens, int64_t hidden,
                            int64_t intermediate, int64_t n_experts, int64_t topk,
                            const int64_t* gate_trellis, const int64_t* gate_suh, const int64_t* gate_svh,
                            const int64_t* up_trellis, const int64_t* up_suh, const int64_t* up_svh,
                            const int64_t* down_trellis, const int64_t* down_suh, const int64_t* down_svh,
                            const void* topk_ids, int ids_kind, const void* topk_weights, int weights_kind,
                            const int64_t* expert_map, int64_t n_global,
                            const int8_t* expert_bits, int bits, int bits_mask, int codebook,
                            float swiglu_limit, void* scratch, int64_t scratch_bytes, void* stream);

/*
 * Launch geometry for diagnostics (replaces lna2_moe_info,
 * recipe-lna/lna2/lna_moe_ticket.cu:494-505): writes up to n values
 * {cus, waves_per_launch, threads_per_wave, max_rows, max_pairs, step_k, cols,
 *  ctrl_bytes (the fixed control region at the head of the scratch),
 *  lds_bytes (per single-wave workgroup)} and returns how many were written.
 */
int exl3_moe_info(int64_t* out, int n);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_AMD_H */
