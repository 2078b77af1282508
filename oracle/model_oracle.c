/*
 * model_oracle.c -- CPU restatement of the reference CPU backend's non-attention ops, for the Qwen3 forward of the
 * greedy-token parity test.  TEST INFRASTRUCTURE ONLY (see attention_oracle.c): only tests/, the smoke entry and
 * the benchmark's CPU baseline may load it.
 *
 * Like the reference, every op reads its tensors as f32 whatever their storage (elemF32,
 * src/backend/cpu/common.zig) and stores through storeF32, which rounds to bf16 (RNE) when the output tensor is
 * bf16.  Each tensor argument therefore comes with a dtype flag: 0 = f32, 1 = bf16 (uint16 bit pattern).
 *   ora_embedding : src/backend/cpu/embedding.zig          row gather (id out of range -> -1)
 *   ora_rmsnorm   : src/backend/cpu/norm.zig:57-89          ss in f32, index order; scale = 1/sqrt(ss/n + eps);
 *                                                           bf16 output rounds x*scale to bf16 before the gain
 *   ora_linear    : src/backend/cpu/linear.zig:7-28         y[s][o] = sum_i x[s][i]*w[o][i], f32, i ascending
 *   ora_rope_table: src/backend/cpu/rope.zig:38-68          inv_freq, angle in f64; cos/sin -> f32 in both halves
 *   ora_rope      : src/backend/cpu/rope.zig:6-36           NEOX pairs (i, i + rope_dim/2); tail dims copied
 *   ora_silu      : src/backend/cpu/activation.zig          v / (1 + exp(-v))
 *   ora_add/mul   : src/backend/cpu/arithmetic.zig          elementwise in f32, b broadcast by index % bn
 *   ora_gather    : src/backend/cpu/memcpy.zig GatherLast    out[s] = x[last[s]]
 *   ora_sample    : src/backend/cpu/sample.zig:12-40        greedy when temp == 0 (strictly greater: ties keep
 *                                                           the smaller index), Gumbel-max with splitmix64 else
 * Built with -ffp-contract=off like the rest of the oracle, so a*b - c*d is two rounded products and a rounded
 * difference, as in the reference.  OpenMP splits only independent outputs (rows or output features), so each
 * value is computed in the reference's order.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

uint16_t ora_f32_to_bf16(float f);
float ora_bf16_to_f32(uint16_t b);

static inline float ld(const void *p, int64_t i, int bf) {
    return bf ? ora_bf16_to_f32(((const uint16_t *)p)[i]) : ((const float *)p)[i];
}
static inline void st(void *p, int64_t i, int bf, float v) {
    if (bf)
        ((uint16_t *)p)[i] = ora_f32_to_bf16(v);
    else
        ((float *)p)[i] = v;
}

int ora_embedding(const int32_t *ids, const void *table, int tdt, void *out, int odt, int64_t n, int64_t vocab,
                  int64_t hidden) {
    for (int64_t s = 0; s < n; ++s) {
        if (ids[s] < 0 || ids[s] >= vocab) return -1;
        for (int64_t h = 0; h < hidden; ++h) st(out, s * hidden + h, odt, ld(table, (int64_t)ids[s] * hidden + h, tdt));
    }
    return 0;
}

void ora_rmsnorm(const void *x, int xdt, const void *gain, int gdt, void *out, int odt, int64_t rows, int64_t n,
                 float eps, float w_offset) {
#pragma omp parallel for schedule(static)
    for (int64_t s = 0; s < rows; ++s) {
        float ss = 0.0f;
        for (int64_t h = 0; h < n; ++h) {
            const float v = ld(x, s * n + h, xdt);
            ss += v * v;
        }
        const float scale = 1.0f / sqrtf(ss / (float)n + eps);
        for (int64_t h = 0; h < n; ++h) {
            float normed = ld(x, s * n + h, xdt) * scale;
            if (odt) normed = ora_bf16_to_f32(ora_f32_to_bf16(normed));
            st(out, s * n + h, odt, normed * (ld(gain, h, gdt) + w_offset));
        }
    }
}

/* x [rows, in_dim], w [out_dim, in_dim], out [rows, out_dim].  Four rows are accumulated side by side (four
 * independent chains, each in the reference's order) so the scalar loop is not bound by one add latency. */
void ora_linear(const void *x, int xdt, const void *w, int wdt, void *out, int odt, int64_t rows, int64_t in_dim,
                int64_t out_dim) {
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < out_dim; ++o) {
        int64_t s = 0;
        for (; s + 4 <= rows; s += 4) {
            float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
            for (int64_t i = 0; i < in_dim; ++i) {
                const float wv = ld(w, o * in_dim + i, wdt);
                a0 += ld(x, (s + 0) * in_dim + i, xdt) * wv;
                a1 += ld(x, (s + 1) * in_dim + i, xdt) * wv;
                a2 += ld(x, (s + 2) * in_dim + i, xdt) * wv;
                a3 += ld(x, (s + 3) * in_dim + i, xdt) * wv;
            }
            st(out, (s + 0) * out_dim + o, odt, a0);
            st(out, (s + 1) * out_dim + o, odt, a1);
            st(out, (s + 2) * out_dim + o, odt, a2);
            st(out, (s + 3) * out_dim + o, odt, a3);
        }
        for (; s < rows; ++s) {
            float acc = 0.0f;
            for (int64_t i = 0; i < in_dim; ++i) acc += ld(x, s * in_dim + i, xdt) * ld(w, o * in_dim + i, wdt);
            st(out, s * out_dim + o, odt, acc);
        }
    }
}

void ora_rope_table(float *cos_t, float *sin_t, int64_t max_seq, int64_t head_dim, double theta) {
    const int64_t half = head_dim / 2;
    for (int64_t s = 0; s < max_seq; ++s) {
        for (int64_t i = 0; i < half; ++i) {
            const double inv = 1.0 / pow(theta, (2.0 * (double)i) / (double)head_dim);
            const double angle = (double)s * inv;
            cos_t[s * head_dim + i] = cos_t[s * head_dim + i + half] = (float)cos(angle);
            sin_t[s * head_dim + i] = sin_t[s * head_dim + i + half] = (float)sin(angle);
        }
    }
}

/* x / out [T, n_head, head_dim] (out may alias x); tables [max_seq, rope_dim]; pos[T] */
void ora_rope(const void *x, int xdt, void *out, int odt, const int32_t *pos, const float *cos_t, const float *sin_t,
              int64_t T, int64_t n_head, int64_t head_dim, int64_t rope_dim) {
    const int64_t half = rope_dim / 2;
    for (int64_t t = 0; t < T; ++t) {
        const float *cr = cos_t + (int64_t)pos[t] * rope_dim;
        const float *sr = sin_t + (int64_t)pos[t] * rope_dim;
        for (int64_t h = 0; h < n_head; ++h) {
            const int64_t b = (t * n_head + h) * head_dim;
            for (int64_t i = 0; i < half; ++i) {
                const float x0 = ld(x, b + i, xdt), x1 = ld(x, b + i + half, xdt);
                st(out, b + i, odt, x0 * cr[i] - x1 * sr[i]);
                st(out, b + i + half, odt, x1 * cr[i] + x0 * sr[i]);
            }
            for (int64_t i = rope_dim; i < head_dim; ++i) st(out, b + i, odt, ld(x, b + i, xdt));
        }
    }
}

void ora_silu(const void *x, int xdt, void *out, int odt, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float v = ld(x, i, xdt);
        st(out, i, odt, v / (1.0f + expf(-v)));
    }
}

void ora_add(const void *a, int adt, const void *b, int bdt, void *out, int odt, int64_t n, int64_t bn) {
    for (int64_t i = 0; i < n; ++i) st(out, i, odt, ld(a, i, adt) + ld(b, i % bn, bdt));
}

void ora_mul(const void *a, int adt, const void *b, int bdt, void *out, int odt, int64_t n, int64_t bn) {
    for (int64_t i = 0; i < n; ++i) st(out, i, odt, ld(a, i, adt) * ld(b, i % bn, bdt));
}

void ora_gather(const void *x, void *out, const int32_t *last, int64_t n_seq, int64_t row_bytes) {
    for (int64_t s = 0; s < n_seq; ++s)
        memcpy((char *)out + s * row_bytes, (const char *)x + (int64_t)last[s] * row_bytes, (size_t)row_bytes);
}

uint64_t ora_splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

/* logits [n_seq, vocab]; temps [n_seq]; one u64 seed for the step */
void ora_sample(const void *logits, int ldt, int32_t *out, const float *temps, uint64_t step_seed, int64_t n_seq,
                int64_t vocab) {
    for (int64_t r = 0; r < n_seq; ++r) {
        const float temp = temps[r];
        const uint64_t seed = ora_splitmix64(step_seed ^ ((uint64_t)r << 40));
        float best = -INFINITY;
        int64_t bi = 0;
        for (int64_t i = 0; i < vocab; ++i) {
            float v = ld(logits, r * vocab + i, ldt);
            if (temp > 0.0f) {
                const uint64_t rr = ora_splitmix64(seed + (uint64_t)i);
                const float u = ((float)(rr >> 40) + 0.5f) * (1.0f / 16777216.0f);
                v = v / temp - logf(-logf(u));
            }
            if (v > best) {
                best = v;
                bi = i;
            }
        }
        out[r] = (int32_t)bi;
    }
}
