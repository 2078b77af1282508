/*
 * llmgen_attn.h -- C-ABI of the MI355X (gfx950) attention path for llmgen: libllmgen_attn.so.
 *
 * Each entry point replaces one extern of the reference engine's CUDA backend with the same argument list,
 * meaning, ownership and error behaviour (citations relative to the reference repository root):
 *   - the three attention launchers: src/backend/cuda/attention/attention_v1.zig:10-48
 *   - the device context:            src/backend/cuda/cuda_context.zig:1-11, cuda_context.cu:13-126
 *   - device memory helpers:         src/backend/cuda/memory/memory.zig:1-11
 * A host that binds `cuda_X` today binds `hip_X` here, with the same argument list.
 *
 * Conventions (same as the reference):
 *   - bf16 tensors are passed as uint16_t bit patterns; index tensors are int32; all pointers are device
 *     pointers except the host sides of the copy helpers.
 *   - Every launcher enqueues on the library's one stream (created by hip_init, or the caller's stream after
 *     hip_set_stream) and returns without synchronising.  Launchers allocate nothing, never synchronise and
 *     derive grid sizes only from their integer arguments, so they may be called inside graph capture.
 *   - Launchers return void.  Unsupported shapes print one line to stderr and launch nothing.  Device faults
 *     surface through hip_last_error() after hip_sync().
 *   - T <= 0, S <= 0 and n_tiles <= 0 are no-ops.
 */
#ifndef LLMGEN_ATTN_H
#define LLMGEN_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------------------------------------
 * Attention launchers
 * ------------------------------------------------------------------------------------------------------- */

/* Replaces cuda_store_kv (attention_v1.zig:10; kernel semantics cpu/attention.zig:31-44).
 * k, v [T, nkv, hd] -> k_cache / v_cache [num_blocks, nkv, block_size, hd] at slot_mapping[t]
 * (block = slot / block_size, offset = slot % block_size); slot < 0 rows are skipped.  Bit-exact copy.
 * Accepts any hd that is a multiple of 8 (the reference requires hd == 128 and nkv <= 32). */
void hip_store_kv(const uint16_t *k, const uint16_t *v, const int32_t *slot_mapping, uint16_t *k_cache,
                  uint16_t *v_cache, int T, int nkv, int hd, int block_size);

/* Replaces cuda_attn_decode (attention_v1.zig:11-29).  One query token per sequence: q, out [S, nq, hd];
 * block_tables [S, max_blocks]; ctx_lens [S] = number of cached keys including this step's token.
 * Split-K scratch is owned by the caller: part_o [S, nq, max_parts, hd] f32 and part_ml [S, nq, max_parts, 2]
 * f32 (attention_v1.zig:51-57 partSize / maxParts; executor.zig:92-102 sizing).  Part p covers tokens
 * [p * part_size, (p + 1) * part_size); tokens past max_parts * part_size are not attended (as in the
 * reference).  ctx <= 0 rows output 0.  Requires hd == 128 and nq / nkv in {1, 2, 4, 8, 16}.
 * Split launches merge their partials in the kernel, elected by per-(sequence, kv head) counters in a library-owned
 * device array that return to 0 after every launch: launches of the decode entry points that overlap on one
 * device (two streams) race on them and must be serialised by the caller. */
void hip_attn_decode(uint16_t *out, const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                     const int32_t *block_tables, const int32_t *ctx_lens, int S, int nq, int nkv, int hd,
                     int max_blocks, int block_size, float scale, float *part_o, float *part_ml, int part_size,
                     int max_parts);

/* No single reference extern: the pair cuda_store_kv + cuda_attn_decode that PagedAttentionImpl issues for a decode
 * step (attention_v1.zig:65-95), fused into one launch.  k, v [S, nkv, hd] hold the step's one token per sequence,
 * slot_mapping[s] its cache slot, which must be the slot of position ctx_lens[s] - 1 under block_tables[s] (as
 * the engine's metadata guarantees).  The cache receives exactly what hip_store_kv would write (slot < 0: nothing)
 * and out equals hip_store_kv followed by hip_attn_decode.  Other arguments as hip_attn_decode. */
void hip_attn_decode_store_kv(uint16_t *out, const uint16_t *q, const uint16_t *k, const uint16_t *v,
                              const int32_t *slot_mapping, uint16_t *k_cache, uint16_t *v_cache,
                              const int32_t *block_tables, const int32_t *ctx_lens, int S, int nq, int nkv, int hd,
                              int max_blocks, int block_size, float scale, float *part_o, float *part_ml,
                              int part_size, int max_parts);

/* No reference counterpart.  hip_attn_decode for callers that cannot allocate or pass device memory (code under
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): the split-K partials live in the
 * library's own file-scope device array of 8 MiB per device instead of caller-owned part_o / part_ml, so the
 * call allocates nothing.  Arguments and output as hip_attn_decode (part_size / max_parts as the engine computes
 * them).  A launch with one part per (sequence, head) stores no partials and needs none of the array, whatever
 * its size.  A launch whose partials need more than 8 MiB (S * nq * parts-per-sequence * 520 bytes; the launcher
 * keeps parts-per-sequence near 512 / (S * nkv) or below, so in practice only single-sequence launches with over
 * 1000 parts at GQA 16 reach it) prints one line, launches nothing and records hipErrorInvalidValue, which the next
 * hip_last_error() returns.  All calls on one device share the array and also the per-(sequence, kv head) merge
 * counters that hip_attn_decode and hip_attn_decode_store_kv use: calls of any of the three that overlap on one
 * device (two streams) race on the counters and, for this entry point, on the array, and must be serialised by
 * the caller. */
void hip_attn_decode_noalloc(uint16_t *out, const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                             const int32_t *block_tables, const int32_t *ctx_lens, int S, int nq, int nkv, int hd,
                             int max_blocks, int block_size, float scale, int part_size, int max_parts);

/* Replaces cuda_attn_prefill (attention_v1.zig:30-47).  Causal varlen attention over the paged cache: sequence
 * s owns rows [cu_q[s], cu_q[s+1]) of q / out [T, nq, hd]; ctx_lens[s] = keys after this step; row j sits at
 * position ctx - q_len + j and attends to keys 0..pos.  Sequences with ctx < q_len are padding: rows of 0.
 * tile_seq / tile_q0 [n_tiles] list the query tiles of hip_attn_prefill_tile() rows (executor.zig:843-850).
 * Also used for mixed chunked-prefill + decode steps.  Requires hd == 128 and nq / nkv in {1, 2, 4, 8, 16}
 * (the reference kernel accepts only 1 and 2). */
void hip_attn_prefill(uint16_t *out, const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                      const int32_t *block_tables, const int32_t *ctx_lens, const int32_t *cu_q,
                      const int32_t *tile_seq, const int32_t *tile_q0, int n_tiles, int nq, int nkv, int hd,
                      int max_blocks, int block_size, float scale);

/* hip_attn_prefill for a caller that knows how many segments of the step have one query row (the decode rows of
 * a mixed step, and padding rows): single_rows == 0 skips the work that serves such rows, > 0 runs it, < 0 means
 * unknown and behaves as hip_attn_prefill.  No reference counterpart (the reference kernel runs decode rows as
 * one-row prefill tiles); the executor slice (llmgen_paged_attention) passes the count llmgen_fill_meta returned.
 * The count must be exact when it is 0: a step that has single-row segments but is passed 0 leaves those rows
 * unwritten (pass -1 when unsure).  With a count > 0 at G = 2 or 4 the whole step is one launch in which workgroups
 * take either a prefill unit or a decode row; it is fastest when the list holds the single-row tiles first (as
 * llmgen_fill_meta orders it) and gives the same result for any order.  For GQA >= 2 a count of 0 also selects,
 * on steps of at most 2.5 (query tile, KV head, head pair) units per CU, the key-split prefill kernel, and at
 * GQA 2 on steps of up to 5 units per CU the heavy-tile split kernel, whose split units keep their partials in a
 * library-owned device array (two such launches running at once on different streams of one GPU race on it;
 * launches on one stream and graph replays are safe).  Which
 * kernel runs (hip_attn_prefill_plan) changes the summation order, so the same rows computed in steps of different
 * composition or with a different count can differ in their last bits (same tolerance); one call is always
 * bit-reproducible. */
void hip_attn_prefill_rows(uint16_t *out, const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                           const int32_t *block_tables, const int32_t *ctx_lens, const int32_t *cu_q,
                           const int32_t *tile_seq, const int32_t *tile_q0, int n_tiles, int nq, int nkv, int hd,
                           int max_blocks, int block_size, float scale, int single_rows);

/* No reference counterpart; for tests and tuning.  The launch hip_attn_prefill_rows makes for a step of this shape
 * (n_tiles tiles, single_rows as passed to it): one LLMGEN_PREFILL_* kernel value, plus LLMGEN_PREFILL_ROWS_LAUNCH
 * when a separate decode-row launch also runs on the library's side stream.  0 = nothing is launched (n_tiles <= 0),
 * -1 = unsupported shape.  The choice depends only on these integers and the device's compute-unit count. */
enum {
    LLMGEN_PREFILL_MIXED = 1,     /* mixed step in one launch: prefill units and decode rows as workgroup roles */
    LLMGEN_PREFILL_KEYSPLIT = 2,  /* 8-wave workgroups, two heads, key tiles split over two groups of 4 waves */
    LLMGEN_PREFILL_W2 = 3,        /* 2-wave workgroups, one head (G = 1) */
    LLMGEN_PREFILL_W4 = 4,        /* 4-wave workgroups, two heads */
    LLMGEN_PREFILL_W8 = 5,        /* 8-wave workgroups, four heads */
    LLMGEN_PREFILL_SPLIT = 6,     /* 4-wave workgroups, the heaviest tiles' units split over two workgroups */
    LLMGEN_PREFILL_PIECES = 7,    /* 4-wave workgroups, each unit's key tiles split over up to 8 workgroups */
    LLMGEN_PREFILL_ROWS_LAUNCH = 16
};
int hip_attn_prefill_plan(int n_tiles, int nq, int nkv, int hd, int block_size, int single_rows);

/* Replaces cuda_attn_prefill_tile (attention_v1.zig:48): query rows per prefill tile (64). */
int hip_attn_prefill_tile(void);

/* Launcher options.  No reference counterpart except LLMGEN_OPT_ATTN_PART_MIN, which restates the reference's
 * SV_ATTN_PART switch (attention.cu:219-229): split-K parts of at least that many tokens (0 = off; it can only
 * lengthen parts, so max_parts and the scratch stay valid).  The others select paths that the default launch
 * heuristics reach only on rare shapes, so that they can be tested and tuned:
 *   LLMGEN_OPT_DECODE_ROW_WAVES    4 (default) or 8 waves per workgroup for the decode rows of a prefill step;
 *   LLMGEN_OPT_DECODE_MERGE_KERNEL 1: merge split-K partials in a separate merge kernel (the path of launches with
 *                                  more than 2^18 (sequence, kv head) pairs), 0 (default): in the decode kernel.
 *   LLMGEN_OPT_PREFILL_SPLIT_TILES -1 (default): the launcher's own count of heavy tiles whose units a pure
 *                                  prefill step at G = 2 splits over two workgroups (LLMGEN_PREFILL_SPLIT);
 *                                  0: no split; n > 0: the n heaviest tiles (at most what the scratch holds).
 * Defaults are read from the environment (SV_ATTN_PART, LLMGEN_DECODE_ROW_WAVES, LLMGEN_DECODE_MERGE,
 * LLMGEN_PREFILL_SPLIT_TILES) on first use.  Returns the previous value, or -1 (and prints one line) for an unknown
 * option or a bad value (for LLMGEN_OPT_PREFILL_SPLIT_TILES, -1 is also its automatic setting).  Not
 * thread-safe; set options between launches. */
enum {
    LLMGEN_OPT_ATTN_PART_MIN = 0,
    LLMGEN_OPT_DECODE_ROW_WAVES = 1,
    LLMGEN_OPT_DECODE_MERGE_KERNEL = 2,
    LLMGEN_OPT_PREFILL_SPLIT_TILES = 3,
    LLMGEN_OPT_COUNT = 4
};
int hip_attn_set_option(int option, int value);

/* ---------------------------------------------------------------------------------------------------------
 * Device context (cuda_context.zig:1-11, cuda_context.cu:13-126)
 * ------------------------------------------------------------------------------------------------------- */

/* Replaces cuda_init: selects device 0 and creates the non-blocking stream.  0 = ok, 1 = no device,
 * 2 = stream creation failed.  ws_bytes is accepted for signature parity and unused (no library workspace). */
int hip_init(size_t ws_bytes);
/* Replaces cuda_sync: waits for the stream. */
void hip_sync(void);
/* Replaces cuda_last_error: 0 = no error.  Returns an error the library recorded when it rejected a launch on the
 * host (hip_attn_decode_noalloc), else hipGetLastError(); either is cleared by the read. */
int hip_last_error(void);
/* Replace cuda_graph_begin / _end / _launch / _destroy: capture on the stream (thread-local mode),
 * end + instantiate (returns a hipGraphExec_t or NULL), replay, destroy. */
int hip_graph_begin(void);
void *hip_graph_end(void);
void hip_graph_launch(void *exec);
void hip_graph_destroy(void *exec);
/* Replace cuda_device_count / cuda_mem_info / cuda_device_info (arch receives e.g. 950 for gfx950). */
int hip_device_count(void);
void hip_mem_info(size_t *free_mem, size_t *total_mem);
void hip_device_info(int dev, char *name, int name_cap, size_t *total_mem, int *arch);

/* No reference counterpart: route launches onto a caller-owned stream (e.g. PyTorch's current stream);
 * NULL selects the legacy default stream.  A stream created by hip_init is destroyed. */
void hip_set_stream(void *stream);
void *hip_get_stream(void);

/* ---------------------------------------------------------------------------------------------------------
 * Memory helpers (memory.zig:1-11)
 * ------------------------------------------------------------------------------------------------------- */
void *hip_malloc(size_t bytes);
void hip_free(void *p);
void *hip_host_alloc(size_t bytes);
void hip_host_free(void *p);
void hip_h2d(void *dst_dev, const void *src_host, size_t bytes);
void hip_d2h(void *dst_host, const void *src_dev, size_t bytes);
void hip_d2d(void *dst_dev, const void *src_dev, size_t bytes);
void hip_h2d_async(void *dst_dev, const void *src_host, size_t bytes);
void hip_d2h_async(void *dst_host, const void *src_dev, size_t bytes);

/* ---------------------------------------------------------------------------------------------------------
 * Timing on the launch stream (no reference counterpart; used by the benchmark to time kernels on the
 * stream they run on)
 * ------------------------------------------------------------------------------------------------------- */
void *hip_timer_create(void);
void hip_timer_record(void *ev);
float hip_timer_elapsed_ms(void *start, void *stop);
void hip_timer_destroy(void *ev);

#ifdef __cplusplus
}
#endif

#endif /* LLMGEN_ATTN_H */
