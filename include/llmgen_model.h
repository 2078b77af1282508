/*
 * llmgen_model.h -- C-ABI of the non-attention ops the Qwen3 forward needs around the attention path, in
 * libllmgen_attn.so.  They exist for the end-to-end greedy-token check, not as tuned kernels: each one computes
 * every output value in the same order and with the same roundings as the reference CPU backend
 * (the src/backend/cpu/ ops), so that a forward built from them differs from the CPU backend's only through the
 * attention kernels.  Each entry point replaces one extern of the reference CUDA backend with the same argument
 * list (citations relative to the reference repository root):
 *   hip_embedding    src/backend/cuda/embedding/embedding.zig:7      (CPU: src/backend/cpu/embedding.zig)
 *   hip_rmsnorm      src/backend/cuda/norm/norm.zig:5                 (CPU: src/backend/cpu/norm.zig:57-89)
 *   hip_linear       src/backend/cuda/linear/linear.zig:7-15          (CPU: src/backend/cpu/linear.zig:7-28)
 *   hip_rope         src/backend/cuda/rope/rope.zig:9-18              (CPU: src/backend/cpu/rope.zig:6-36)
 *   hip_silu         src/backend/cuda/activation/activation.zig:5     (CPU: src/backend/cpu/activation.zig)
 *   hip_add/hip_mul  src/backend/cuda/arithmetic/arithmetic.zig:7,27  (CPU: src/backend/cpu/arithmetic.zig)
 *   hip_gather_rows  src/backend/cuda/memory/memcpy.zig:34-40         (CPU: GatherLast, src/backend/cpu/memcpy.zig)
 *   hip_sample       src/backend/cuda/sample/sample.zig:4-14          (CPU: src/backend/cpu/sample.zig:12-40)
 * Conventions are those of llmgen_attn.h: device pointers, bf16 as uint16_t bits, launches on the library
 * stream, no allocation and no synchronisation (capturable); unsupported shapes print one line to stderr and
 * launch nothing.  Every f32 operation is a separately rounded IEEE multiply, add, divide or square root (no
 * fused multiply-add), as in the reference's Zig code.
 */
#ifndef LLMGEN_MODEL_H
#define LLMGEN_MODEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* out [T, H] bf16 = weight[ids[t]] (weight [vocab, H] bf16).  H % 8 == 0.  Ids are not range-checked (as in
 * the reference CUDA kernel): the caller validates them. */
void hip_embedding(uint16_t *out, const int32_t *ids, const uint16_t *weight, int T, int H);

/* out [rows, D] bf16 = bf16(bf16(x * scale) * w), scale = 1 / sqrt(sum(x^2) / D + eps), the sum taken in index
 * order in f32.  x bf16, w f32 [D] (GGUF norm gains are f32).  D % 8 == 0 and D <= 8192. */
void hip_rmsnorm(uint16_t *out, const uint16_t *x, const float *w, long rows, int D, float eps);

/* y [M, N] = x [M, K] * w [N, K]^T with f32 accumulation over k = 0..K-1 in order; y is bf16 (RNE) or, with
 * y_f32 != 0, f32.  K % 8 == 0. */
void hip_linear(void *y, int y_f32, const uint16_t *x, const uint16_t *w, int M, int N, int K);

/* NEOX rotary embedding, in place allowed: for i < hd/2, out[i] = x[i]*cos[p][i] - x[i+hd/2]*sin[p][i] and
 * out[i+hd/2] = x[i+hd/2]*cos[p][i] + x[i]*sin[p][i], p = positions[t]; tables [max_seq, hd] f32.  hd even. */
void hip_rope(uint16_t *out, const uint16_t *x, const float *cos_tab, const float *sin_tab, const int32_t *positions,
              int T, int n_head, int hd);

/* Elementwise over n bf16 values: silu(x) = x / (1 + exp(-x)); a + b; a * b. */
void hip_silu(uint16_t *out, const uint16_t *x, size_t n);
void hip_add(uint16_t *out, const uint16_t *a, const uint16_t *b, size_t n);
void hip_mul(uint16_t *out, const uint16_t *a, const uint16_t *b, size_t n);

/* out [S, H] bf16 = x[idx[s]] (gather_last).  H % 8 == 0. */
void hip_gather_rows(uint16_t *out, const uint16_t *x, const int32_t *idx, int S, int H);

/* out_ids [S] = argmax over logits [S, V] bf16 per row: greedy when temps[s] <= 0 (the first index of the maximum),
 * else Gumbel-max of logits / temp with splitmix64 noise keyed by (*seed, s, index).  No scratch is used:
 * hip_sample_scratch_bytes returns 0 and scratch may be NULL (both kept for the reference's argument list). */
void hip_sample(int32_t *out_ids, const uint16_t *logits, const float *temps, const uint64_t *seed, int S, int V,
                void *scratch);
size_t hip_sample_scratch_bytes(int max_S);

/* Fused per-head q/k RMSNorm + NEOX RoPE + paged KV write.  No single reference extern: it replaces the sequence
 * the reference graph runs before attention -- cuda_rmsnorm over q and k rows (norm/norm.zig:5, D = hd), cuda_rope
 * over q and k (rope/rope.zig:9-18) and cuda_store_kv (attention/attention_v1.zig:10) -- the fusion the reference
 * docs list as the next step (docs/llmgen-serving-unfused/23-switches-debug.html).  q, k, v [T, n, hd] bf16;
 * q_out [T, nq, hd] (may alias q) receives the normed, rotated q; the normed, rotated k and the unchanged v go to
 * k_cache / v_cache [num_blocks, nkv, block_size, hd] at slot_mapping[t] (slot < 0: not written).  Gains f32 [hd];
 * tables [max_seq, hd] f32.  Outputs are bit-identical to hip_rmsnorm + hip_rope + hip_store_kv.  hd == 128. */
void hip_qk_norm_rope_store_kv(uint16_t *q_out, uint16_t *k_cache, uint16_t *v_cache, const uint16_t *q,
                               const uint16_t *k, const uint16_t *v, const float *q_norm_w, const float *k_norm_w,
                               float eps, const float *cos_tab, const float *sin_tab, const int32_t *positions,
                               const int32_t *slot_mapping, int T, int nq, int nkv, int hd, int block_size);

#ifdef __cplusplus
}
#endif

#endif /* LLMGEN_MODEL_H */
