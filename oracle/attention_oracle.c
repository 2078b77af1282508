/*
 * attention_oracle.c -- CPU restatement of the llmgen reference CPU backend's paged attention.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP attention path.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the product library
 * (llmgen_amd/libllmgen_attn.so) never links or calls it.
 *
 * What each function restates (paths relative to the reference repository root):
 *   ora_f32_to_bf16 / ora_bf16_to_f32 : src/backend/cpu/common.zig:55-65 (RNE, NaN -> 0x7FC0, bf16 = high half)
 *   ora_store_kv                      : src/backend/cpu/attention.zig:31-44 (storeKv)
 *   ora_attend                        : src/backend/cpu/attention.zig:64-118 (attend: online softmax in f32)
 *   ora_attend_rows / _omp            : the same per-(token, head) computation, restricted to a list of token
 *                                       rows (sampling for large configs) or spread over OpenMP threads
 *                                       (multi-core CPU baseline).  Per-row arithmetic is identical.
 *   ora_ref_two_pass                  : src/backend/cuda/kernel_test.zig:117-149 and
 *                                       src/backend/cpu/attention.zig:162-186 (two-pass f32 reference).
 *
 * Arithmetic follows the Zig source statement by statement: f32 accumulation in key order and dimension order,
 * no fused multiply-add (build with -ffp-contract=off; Zig's default float mode does not contract), expf for
 * Zig's @exp, the division acc/l, then RNE to bf16.  Besides the bf16 output the oracle can return the f32
 * value acc/l before rounding, which is what the parity tolerance is measured against.
 *
 * Pinning: tests/test_oracle.py checks every function here against the reference's own literal cases
 * (attention.zig:188-274, kernel_test.zig:151-232 re-expressed), an independent float64 numpy softmax
 * attention, and closed-form invariants (single key -> v, equal scores -> mean of V, block-table
 * permutation invariance, padding rows -> 0, chunked prefill == tail of full prefill).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORA_MAX_HD 256 /* cpu/attention.zig:12 */

uint16_t ora_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0; /* NaN stays NaN */
    uint32_t bias = 0x7FFFu + ((u >> 16) & 1u);         /* ties to even */
    return (uint16_t)((u + bias) >> 16);
}

float ora_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void ora_f32_to_bf16_array(const float *src, uint16_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = ora_f32_to_bf16(src[i]);
}

void ora_bf16_to_f32_array(const uint16_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = ora_bf16_to_f32(src[i]);
}

/* cpu/attention.zig:31-44.  Cache layout per block: [kv_head][slot][hd]. */
void ora_store_kv(const uint16_t *k, const uint16_t *v, const int32_t *slots, uint16_t *kc, uint16_t *vc,
                  int64_t n_tok, int64_t nkv, int64_t hd, int64_t bs) {
    for (int64_t t = 0; t < n_tok; ++t) {
        if (slots[t] < 0) continue;
        int64_t slot = slots[t];
        int64_t blk = slot / bs, off = slot % bs;
        for (int64_t h = 0; h < nkv; ++h) {
            int64_t dst = ((blk * nkv + h) * bs + off) * hd;
            int64_t src = (t * nkv + h) * hd;
            memcpy(kc + dst, k + src, (size_t)hd * 2);
            memcpy(vc + dst, v + src, (size_t)hd * 2);
        }
    }
}

typedef struct {
    uint16_t *out;      /* [T, nq, hd] bf16, may be NULL */
    float *out_f32;     /* [T, nq, hd] f32 acc/l before rounding, may be NULL */
    const uint16_t *q;  /* [T, nq, hd] */
    const uint16_t *kc; /* [blocks, nkv, bs, hd] */
    const uint16_t *vc;
    const int32_t *block_tables; /* [n_seq, max_blocks] */
    const int32_t *ctx_lens;     /* [n_seq] */
    const int32_t *cu_q;         /* [n_seq + 1] */
    int64_t n_seq, nq, nkv, hd, max_blocks, bs;
    float scale;
} OraArgs;

/* One (token t of sequence s, head h) output row: the body of attention.zig:78-115. */
static void attend_one(const OraArgs *a, int64_t s, int64_t t, int64_t h) {
    const int64_t q_beg = a->cu_q[s], q_end = a->cu_q[s + 1];
    const int64_t q_len = q_end - q_beg;
    const int64_t ctx = a->ctx_lens[s];
    const int32_t *bt = a->block_tables + s * a->max_blocks;
    const int64_t j = t - q_beg;
    const int64_t group = a->nq / a->nkv;
    const int64_t hd = a->hd;
    const int64_t orow = (t * a->nq + h) * hd;
    if (ctx < q_len) { /* padding row: nothing to attend to */
        for (int64_t d = 0; d < hd; ++d) {
            if (a->out) a->out[orow + d] = 0;
            if (a->out_f32) a->out_f32[orow + d] = 0.0f;
        }
        return;
    }
    const int64_t n_keys = ctx - q_len + j + 1;
    const int64_t kvh = h / group;
    const uint16_t *qr = a->q + orow;
    float acc[ORA_MAX_HD];
    for (int64_t d = 0; d < hd; ++d) acc[d] = 0.0f;
    float m = -INFINITY, l = 0.0f;
    for (int64_t p = 0; p < n_keys; ++p) {
        const int64_t blk = bt[p / a->bs];
        const int64_t row = ((blk * a->nkv + kvh) * a->bs + p % a->bs) * hd;
        float dot = 0.0f;
        for (int64_t d = 0; d < hd; ++d) dot += ora_bf16_to_f32(qr[d]) * ora_bf16_to_f32(a->kc[row + d]);
        const float score = dot * a->scale;
        const float m_new = m > score ? m : score;
        const float corr = expf(m - m_new);
        const float w = expf(score - m_new);
        l = l * corr + w;
        for (int64_t d = 0; d < hd; ++d) acc[d] = acc[d] * corr + w * ora_bf16_to_f32(a->vc[row + d]);
        m = m_new;
    }
    for (int64_t d = 0; d < hd; ++d) {
        const float r = acc[d] / l;
        if (a->out) a->out[orow + d] = ora_f32_to_bf16(r);
        if (a->out_f32) a->out_f32[orow + d] = r;
    }
}

static int args_ok(const OraArgs *a) { return a->hd > 0 && a->hd <= ORA_MAX_HD && a->nkv > 0 && a->nq % a->nkv == 0; }

/* cpu/attention.zig:64-118, loop order seq -> token -> head. Returns 0 on success, -1 on bad shape. */
int ora_attend(uint16_t *out, float *out_f32, const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
               const int32_t *block_tables, const int32_t *ctx_lens, const int32_t *cu_q, int64_t n_seq, int64_t nq,
               int64_t nkv, int64_t hd, int64_t max_blocks, int64_t bs, float scale) {
    OraArgs a = {out, out_f32, q, kc, vc, block_tables, ctx_lens, cu_q, n_seq, nq, nkv, hd, max_blocks, bs, scale};
    if (!args_ok(&a)) return -1;
    for (int64_t s = 0; s < n_seq; ++s)
        for (int64_t t = cu_q[s]; t < cu_q[s + 1]; ++t)
            for (int64_t h = 0; h < nq; ++h) attend_one(&a, s, t, h);
    return 0;
}

static int64_t seq_of_row(const int32_t *cu_q, int64_t n_seq, int64_t t) {
    int64_t lo = 0, hi = n_seq - 1; /* last s with cu_q[s] <= t */
    while (lo < hi) {
        int64_t mid = (lo + hi + 1) / 2;
        if (cu_q[mid] <= t) lo = mid; else hi = mid - 1;
    }
    return lo;
}

/* Same computation as ora_attend for the listed token rows only (every head of each row).  Rows not listed are
 * left untouched in out / out_f32. */
int ora_attend_rows(uint16_t *out, float *out_f32, const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                    const int32_t *block_tables, const int32_t *ctx_lens, const int32_t *cu_q, int64_t n_seq,
                    int64_t nq, int64_t nkv, int64_t hd, int64_t max_blocks, int64_t bs, float scale,
                    const int32_t *rows, int64_t n_rows) {
    OraArgs a = {out, out_f32, q, kc, vc, block_tables, ctx_lens, cu_q, n_seq, nq, nkv, hd, max_blocks, bs, scale};
    if (!args_ok(&a)) return -1;
    for (int64_t i = 0; i < n_rows; ++i) {
        const int64_t t = rows[i];
        const int64_t s = seq_of_row(cu_q, n_seq, t);
        for (int64_t h = 0; h < nq; ++h) attend_one(&a, s, t, h);
    }
    return 0;
}

/* Multi-core variant for the CPU baseline: (row, head) pairs spread over OpenMP threads; identical per-row
 * arithmetic, so its outputs equal ora_attend_rows bit for bit. */
int ora_attend_rows_omp(uint16_t *out, float *out_f32, const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                        const int32_t *block_tables, const int32_t *ctx_lens, const int32_t *cu_q, int64_t n_seq,
                        int64_t nq, int64_t nkv, int64_t hd, int64_t max_blocks, int64_t bs, float scale,
                        const int32_t *rows, int64_t n_rows, int n_threads) {
    OraArgs a = {out, out_f32, q, kc, vc, block_tables, ctx_lens, cu_q, n_seq, nq, nkv, hd, max_blocks, bs, scale};
    if (!args_ok(&a)) return -1;
    const int64_t total = n_rows * nq;
#pragma omp parallel for schedule(dynamic, 4) num_threads(n_threads)
    for (int64_t w = 0; w < total; ++w) {
        const int64_t t = rows[w / nq];
        const int64_t s = seq_of_row(cu_q, n_seq, t);
        attend_one(&a, s, t, w % nq);
    }
    return 0;
}

/* kernel_test.zig:117-149 generalised to a varlen batch: scores, max, exp, sum, then sum_p (e_p/sum)*v_p in f32.
 * Writes f32 [T, nq, hd]; padding rows (ctx < q_len) are 0. */
int ora_ref_two_pass(float *out, const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                     const int32_t *block_tables, const int32_t *ctx_lens, const int32_t *cu_q, int64_t n_seq,
                     int64_t nq, int64_t nkv, int64_t hd, int64_t max_blocks, int64_t bs, float scale) {
    if (hd <= 0 || nkv <= 0 || nq % nkv) return -1;
    const int64_t group = nq / nkv;
    int64_t max_ctx = 1;
    for (int64_t s = 0; s < n_seq; ++s) max_ctx = ctx_lens[s] > max_ctx ? ctx_lens[s] : max_ctx;
    float *scores = (float *)malloc((size_t)max_ctx * sizeof(float));
    if (!scores) return -2;
    for (int64_t s = 0; s < n_seq; ++s) {
        const int64_t q_beg = cu_q[s], q_len = cu_q[s + 1] - cu_q[s], ctx = ctx_lens[s];
        const int32_t *bt = block_tables + s * max_blocks;
        for (int64_t j = 0; j < q_len; ++j) {
            const int64_t t = q_beg + j;
            for (int64_t h = 0; h < nq; ++h) {
                float *o = out + (t * nq + h) * hd;
                if (ctx < q_len) {
                    for (int64_t d = 0; d < hd; ++d) o[d] = 0.0f;
                    continue;
                }
                const int64_t n_keys = ctx - q_len + j + 1, kvh = h / group;
                float mx = -INFINITY;
                for (int64_t p = 0; p < n_keys; ++p) {
                    const int64_t base = (((int64_t)bt[p / bs] * nkv + kvh) * bs + p % bs) * hd;
                    float dd = 0.0f;
                    for (int64_t e = 0; e < hd; ++e)
                        dd += ora_bf16_to_f32(q[(t * nq + h) * hd + e]) * ora_bf16_to_f32(kc[base + e]);
                    scores[p] = dd * scale;
                    mx = scores[p] > mx ? scores[p] : mx;
                }
                float sum = 0.0f;
                for (int64_t p = 0; p < n_keys; ++p) {
                    scores[p] = expf(scores[p] - mx);
                    sum += scores[p];
                }
                for (int64_t e = 0; e < hd; ++e) {
                    float acc = 0.0f;
                    for (int64_t p = 0; p < n_keys; ++p) {
                        const int64_t base = (((int64_t)bt[p / bs] * nkv + kvh) * bs + p % bs) * hd;
                        acc += scores[p] * ora_bf16_to_f32(vc[base + e]);
                    }
                    o[e] = acc / sum;
                }
            }
        }
    }
    free(scores);
    return 0;
}
