/*
 * llmgen_host.h -- C-ABI of the host-side executor slice around the attention path, in libllmgen_attn.so.
 *
 * The reference engine's executor (Zig) prepares every step for the attention kernels: it packs the step
 * metadata into one buffer and uploads it with one copy, publishes the device addresses of that buffer's
 * segments in g_step, dispatches PagedAttentionImpl per layer, splits oversized batches into passes of at most
 * max_tokens tokens and replays decode steps from captured graph buckets.  This header is the C++ restatement of
 * that slice (citations relative to the reference repository root):
 *   llmgen_layout_init        src/executor.zig:139-202      (Layout: byte offsets of the packed metadata)
 *   llmgen_fill_meta          src/executor.zig:772-861      (fillMeta, incl. graph-bucket padding rows)
 *   llmgen_bind_step          src/executor.zig:864-895      (bindStep -> StepState, common.zig:10-41)
 *   llmgen_paged_attention    src/backend/cuda/attention/attention_v1.zig:60-120 (PagedAttentionImpl.execute)
 *   llmgen_part_size / llmgen_max_parts   attention_v1.zig:51-57
 *   llmgen_workspace          src/executor.zig:92-102       (Workspace.of: meta / part_o / part_ml / sample bytes)
 *   llmgen_decode_buckets     src/executor.zig:609-632      (captureGraphs bucket sizes)
 *   llmgen_plan_passes        src/executor.zig:986-1043     (execute: passes of <= max_tokens, flushPass)
 *   llmgen_graphs_*           src/executor.zig:530-575, 609-660 (forward's bucket replay, captureGraphs)
 * Conventions: host pointers unless named *_dev; bf16 as uint16_t bits; launches on the library stream
 * (include/llmgen_attn.h).  Functions returning int return 0 on success and a negative value on bad arguments.
 */
#ifndef LLMGEN_HOST_H
#define LLMGEN_HOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* executor.zig:139-202: byte offsets of the segments of one step's packed metadata. */
typedef struct llmgen_layout {
    size_t seed, ids, pos, slots, cu_q, ctx, last, temps, tile_seq, tile_q0, bt, total;
} llmgen_layout;

/* A sequence as the executor sees it (runner/sequence: all token ids so far, block table, sampling temperature). */
typedef struct llmgen_seq {
    const int32_t *token_ids;
    int32_t n_tokens;
    const int32_t *block_table;
    int32_t n_blocks;
    float temperature;
} llmgen_seq;

/* runner/batching.zig:93-103: this step computes positions [q_start, q_start + q_len) of sequence `seq`. */
typedef struct llmgen_entry {
    int32_t seq;
    int32_t q_start;
    int32_t q_len;
} llmgen_entry;

/* common.zig:10-41 StepState; pointers are device addresses inside the uploaded metadata buffer. */
typedef struct llmgen_step_state {
    int32_t n_tok, n_seq, n_tiles, decode;
    int32_t hidden, n_head, n_kv_head, head_dim;
    float attn_scale;
    int32_t block_size, max_blocks;
    size_t max_model_len;
    void *seed, *pos, *slots, *cu_q, *ctx, *last, *temps, *tile_seq, *tile_q0, *block_tables;
    void *cos_sin, *part_o, *part_ml, *sample_scratch;
    int32_t single_rows; /* segments with one query row (decode / padding rows); -1 = unknown.  Not in the
                            reference's StepState: llmgen_fill_meta returns the count and llmgen_bind_step stores
                            it; llmgen_paged_attention passes it to hip_attn_prefill_rows. */
} llmgen_step_state;

llmgen_layout llmgen_layout_init(size_t n_tok, size_t n_seq, size_t n_tiles, size_t max_blocks);

/* Entry.emits (batching.zig:98-100): the entry reaches the sequence's last known token. */
int llmgen_entry_emits(const llmgen_seq *seqs, const llmgen_entry *e);

/* executor.zig:530-552: decode step iff every entry has q_len == 1 and emits; prefill tiles per entry. */
int llmgen_step_is_decode(const llmgen_seq *seqs, const llmgen_entry *entries, int n_entries);
int llmgen_step_tiles(const llmgen_entry *entries, int n_entries, int pf_tile);
/* Segments of the step with one query row: entries with q_len == 1 plus the seq_num - n_entries padding rows. */
int llmgen_single_rows(const llmgen_entry *entries, int n_entries, int seq_num);

/* executor.zig:772-861.  Writes the step into meta_host (lay.total bytes).  seq_num >= n_entries adds padding
 * rows (id 0, pos 0, slot -1, ctx 0, temperature 0, zero block-table row); in a step with prefill tiles
 * (n_tiles > 0) each padding row also gets a tile of its own, so n_tiles must count them.  *step_seed advances by
 * the golden-ratio increment and is stored in the seed segment.  slot = block_table[p / bs] * bs + p % bs
 * (batching.zig:74-77).  Prefill tiles are listed lightest first (by the keys a tile needs, stable), the reverse
 * of the prefill kernel's dispatch order, so that the heaviest tiles start first; the reference lists them in
 * entry order.  Returns the step's count of single-row segments (>= 0, llmgen_single_rows), which
 * llmgen_bind_step takes, or a negative value if the step does not fit the layout or is malformed. */
int llmgen_fill_meta(uint8_t *meta_host, llmgen_layout lay, const llmgen_seq *seqs, const llmgen_entry *entries,
                     int n_entries, int seq_num, int n_tiles, int pf_tile, int block_size, int max_blocks,
                     uint64_t *step_seed);

/* executor.zig:864-895: fill st with the step's sizes, the model's head shape and the device addresses of the
 * metadata segments in meta_dev (attn_scale = 1 / sqrtf(head_dim)).  single_rows is llmgen_fill_meta's return
 * value for this step (-1 if unknown: the prefill launcher then always runs its single-row launch and never the
 * key-split kernel). */
void llmgen_bind_step(llmgen_step_state *st, void *meta_dev, llmgen_layout lay, int n_tok, int n_seq, int n_tiles,
                      int decode, int hidden, int n_head, int n_kv_head, int head_dim, int block_size, int max_blocks,
                      size_t max_model_len, void *part_o, void *part_ml, void *sample_scratch, int single_rows);

/* attention_v1.zig:60-120 PagedAttentionImpl.execute for one layer: store_kv of the step's k / v (unless
 * store_kv == 0: already written, e.g. by hip_qk_norm_rope_store_kv), then split-K decode or causal prefill.
 * Decode steps issue store_kv and decode as one launch (hip_attn_decode_store_kv). */
int llmgen_paged_attention(const llmgen_step_state *st, uint16_t *out, const uint16_t *q, const uint16_t *k,
                           const uint16_t *v, uint16_t *k_cache, uint16_t *v_cache, int store_kv);

int llmgen_part_size(int n_seq);
int llmgen_max_parts(int n_seq, size_t max_model_len);

/* executor.zig:92-102: bytes of the metadata buffer (Layout at the largest step), part_o, part_ml and the
 * sampling scratch.  out[4] = {meta, part_o, part_ml, sample}. */
void llmgen_workspace(int n_head, int head_dim, int max_seqs, size_t max_tokens, size_t max_model_len,
                      int block_size, int pf_tile, size_t out[4]);

/* executor.zig:614-632: 1, 2, 4, 8, multiples of 16 up to max_seqs, then max_seqs.  Returns the count. */
int llmgen_decode_buckets(int max_seqs, int *out, int cap);

/* executor.zig:986-1043: split entries into passes of at most max_tokens tokens (an entry's query range may be
 * cut).  pieces[i] is the i-th piece, owner[i] the index of the entry it came from, pass[i] its pass number.
 * Returns the number of pieces (or -1 if cap is too small).  Only the piece that ends an entry carries that
 * entry's sampled token. */
int llmgen_plan_passes(const llmgen_entry *entries, int n_entries, size_t max_tokens, llmgen_entry *pieces,
                       int *owner, int *pass, int cap);

/* Decode graph buckets over n_layers attention layers (executor.zig:609-660): one captured graph per bucket
 * size, each recording llmgen_paged_attention for every layer over the bucket's own q / k / v / out and
 * metadata buffers.  k_caches / v_caches: n_layers device pointers.  Returns NULL on failure. */
void *llmgen_graphs_create(int n_layers, uint16_t *const *k_caches, uint16_t *const *v_caches, int n_head,
                           int n_kv_head, int head_dim, int block_size, size_t max_model_len, int max_seqs,
                           const int *buckets, int n_buckets);
/* forward's replay path (executor.zig:541-575): pick the smallest bucket >= n_entries, fill and upload the
 * metadata (one copy), copy the step's q / k / v (device, n_entries rows) into the bucket, replay, copy the
 * first n_entries rows of the output to out_dev.  Asynchronous on the library stream.  Returns the bucket size
 * used, or a negative value (no bucket fits, not a decode step). */
int llmgen_graphs_step(void *graphs, const llmgen_seq *seqs, const llmgen_entry *entries, int n_entries,
                       const uint16_t *q_dev, const uint16_t *k_dev, const uint16_t *v_dev, uint16_t *out_dev);
/* Replay the graph of the bucket used last (no metadata upload): for timing repeated identical steps. */
int llmgen_graphs_replay(void *graphs);
void llmgen_graphs_destroy(void *graphs);

#ifdef __cplusplus
}
#endif

#endif /* LLMGEN_HOST_H */
