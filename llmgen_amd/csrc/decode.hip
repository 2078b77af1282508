// decode.hip -- split-K flash-decoding over the paged KV cache with GQA head sharing (gfx950, wave64).
//
// Contract: src/backend/cuda/attention/attention_v1.zig:11-29 (cuda_attn_decode argument list) with the semantics
// of src/backend/cuda/attention/attention.cu:51-253: q [S, nq, 128] (one query token per sequence, whose K/V is
// already in the cache), ctx_lens[s] = keys to attend, split-K scratch part_o [S, nq, max_parts, 128] f32 and
// part_ml [S, nq, max_parts, 2] f32 owned by the caller, part p covering tokens [p*part_size, (p+1)*part_size).
// Output: bf16(softmax(scale * q K^T) V) per (s, head), 0 for ctx <= 0 (cpu/attention.zig:80-83).
//
// Design (one workgroup = one (kv head, sequence, part), 4 waves):
//   * every wave owns 16-token tiles of the part; per round a wave issues all of its K and V loads at once as
//     16-byte vectors (K: the MFMA B-operand layout, 16 tokens x 64 B per instruction; V: 4 full 256-byte rows
//     per instruction), so a workgroup keeps up to 128 KB in flight;
//   * QK^T runs on the matrix cores: v_mfma_f32_16x16x32_bf16 with the G query heads of the group as the 16 A
//     rows, so the K bytes are read once for all G heads (GQA sharing).  Scores land one token per lane column,
//     one head per row, and the softmax max / sum reduce over a 16-lane DPP row;
//   * softmax is in base 2 (scale * log2 e folded in), fp32 throughout; the probabilities go through a small
//     per-wave LDS buffer to the PV lanes, which hold 8 head dims of 4 tokens per 16-byte V vector and
//     accumulate all G heads in fp32 registers;
//   * the four waves merge (max, sum, unnormalised o) through LDS; a part that is the only part of its
//     sequence writes the final bf16 row directly, otherwise (o, m, l) go to the caller's scratch and
//     attn_decode_reduce merges the parts with the log-sum-exp rule (attention.cu:186-207).
// Grid = (nkv, S, max_parts) from host integers only, so the launch is graph-capturable; parts past ctx exit.
#include "hip_common.h"

#include <math.h>

namespace {

constexpr int HD = 128;
constexpr int DEC_WAVES = 4;
constexpr int DEC_THREADS = 64 * DEC_WAVES;

// Physical row offset (in elements) of logical token t of one sequence, for KV head kvh.
__device__ __forceinline__ long kv_row(const int *__restrict__ bt, int t, int block_size, int bs_shift, long head_off,
                                       long blk_stride) {
    const int bi = bs_shift >= 0 ? (t >> bs_shift) : (t / block_size);
    const int off = t - bi * block_size;
    return (long)bt[bi] * blk_stride + head_off + (long)off * HD;
}

// G = query heads per KV head (1..16); NT = 16-token tiles per wave per round.
template <int G, int NT>
__global__ void __launch_bounds__(DEC_THREADS)
    attn_decode_split_kernel(bf16_t *__restrict__ out, float *__restrict__ part_o, float *__restrict__ part_ml,
                             const bf16_t *__restrict__ q, const bf16_t *__restrict__ kc,
                             const bf16_t *__restrict__ vc, const int *__restrict__ block_tables,
                             const int *__restrict__ ctx_lens, int nq, int nkv, int max_blocks, int block_size,
                             int bs_shift, float scale_log2, int part_size, int max_parts, int rounds) {
    constexpr int WTOK = NT * 16;      // tokens per wave per round
    const int kvh = blockIdx.x, s = blockIdx.y, part = blockIdx.z;
    const int ctx = ctx_lens[s];
    const int t0 = part * part_size;
    if (t0 >= ctx) return;
    const int n = min(ctx - t0, part_size);
    const int np = (ctx + part_size - 1) / part_size;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, rgrp = lane >> 4;

    __shared__ float p_lds[DEC_WAVES][WTOK][G];
    __shared__ float corr_lds[DEC_WAVES][G];
    __shared__ float o_lds[DEC_WAVES][G][HD];
    __shared__ float m_lds[DEC_WAVES][G];
    __shared__ float l_lds[DEC_WAVES][G];

    const int *bt = block_tables + (long)s * max_blocks;
    const long blk_stride = (long)nkv * block_size * HD;
    const long head_off = (long)kvh * block_size * HD;

    // A operand: row g = col holds head kvh*G+g; lane group rgrp holds dims c*32 + rgrp*8 .. +8 of chunk c.
    bf16x8_t qa[4];
    {
        const bf16_t *qrow = q + ((long)s * nq + (long)kvh * G + (col < G ? col : 0)) * HD + rgrp * 8;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            u32x4_t v = ld16(qrow + c * 32);
            if (col >= G) v = u32x4_t{0, 0, 0, 0};
            qa[c] = __builtin_bit_cast(bf16x8_t, v);
        }
    }

    float m_run[4], l_run[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m_run[i] = -INFINITY;
        l_run[i] = 0.f;
    }
    float o[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < 8; ++k) o[g][k] = 0.f;

    for (int r = 0; r < rounds; ++r) {
        const int wbase = r * DEC_WAVES * WTOK + wave * WTOK;  // first token (within the part) of this wave

        // ---- issue every K and V load of the round ----
        u32x4_t kf[NT][4];
#pragma unroll
        for (int tau = 0; tau < NT; ++tau) {
            const int i = min(wbase + tau * 16 + col, n - 1);  // clamp: masked later, address stays valid
            const bf16_t *kr = kc + kv_row(bt, t0 + i, block_size, bs_shift, head_off, blk_stride) + rgrp * 8;
#pragma unroll
            for (int c = 0; c < 4; ++c) kf[tau][c] = ld16(kr + c * 32);
        }
        u32x4_t vf[4 * NT];
#pragma unroll
        for (int j = 0; j < 4 * NT; ++j) {
            const int i = min(wbase + rgrp + 4 * j, n - 1);
            vf[j] = ld16(vc + kv_row(bt, t0 + i, block_size, bs_shift, head_off, blk_stride) + col * 8);
        }

        // ---- scores on the matrix cores: D[g][token] = sum_d q[g][d] k[token][d] ----
        f32x4_t sc[NT];
#pragma unroll
        for (int tau = 0; tau < NT; ++tau) {
            f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 4; ++c)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[c], __builtin_bit_cast(bf16x8_t, kf[tau][c]), acc,
                                                              0, 0, 0);
            const bool valid = wbase + tau * 16 + col < n;
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[tau][i] = valid ? acc[i] * scale_log2 : -INFINITY;
        }

        // ---- online softmax for this round (row rgrp*4+i of the MFMA output = head g; rows past G hold the
        //      zero query rows and are computed but never stored) ----
        float corr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float mx = sc[0][i];
#pragma unroll
            for (int tau = 1; tau < NT; ++tau) mx = fmaxf(mx, sc[tau][i]);
            mx = row16_max(mx);
            const float m_new = fmaxf(m_run[i], mx);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            corr[i] = fast_exp2(m_run[i] - m_use);
            float sum = 0.f;
#pragma unroll
            for (int tau = 0; tau < NT; ++tau) {
                const float p = fast_exp2(sc[tau][i] - m_use);
                sc[tau][i] = p;
                sum += p;
            }
            l_run[i] = l_run[i] * corr[i] + sum;
            m_run[i] = m_new;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int g = rgrp * 4 + i;
            if (g < G) {
#pragma unroll
                for (int tau = 0; tau < NT; ++tau) p_lds[wave][tau * 16 + col][g] = sc[tau][i];
                if (col == 0) corr_lds[wave][g] = corr[i];
            }
        }
        __syncthreads();

        // ---- P V on the vector ALUs: lane holds dims col*8.. of tokens rgrp + 4j ----
        float cr[G];
#pragma unroll
        for (int g = 0; g < G; ++g) cr[g] = corr_lds[wave][g];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int k = 0; k < 8; ++k) o[g][k] *= cr[g];
#pragma unroll
        for (int j = 0; j < 4 * NT; ++j) {
            float f[8];
            unpack_bf16x8(vf[j], f);
            const float *pp = p_lds[wave][rgrp + 4 * j];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float p = pp[g];
#pragma unroll
                for (int k = 0; k < 8; ++k) o[g][k] += p * f[k];
            }
        }
        __syncthreads();  // p_lds / corr_lds are rewritten next round
    }

    // ---- per-wave totals ----
#pragma unroll
    for (int i = 0; i < 4; ++i) l_run[i] = row16_sum(l_run[i]);
    if (col == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int g = rgrp * 4 + i;
            if (g < G) {
                m_lds[wave][g] = m_run[i];
                l_lds[wave][g] = l_run[i];
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            float x = o[g][k];
            x += lane_xor(x, 16);
            x += lane_xor(x, 32);
            o[g][k] = x;
        }
    if (lane < 16) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int k = 0; k < 8; ++k) o_lds[wave][g][lane * 8 + k] = o[g][k];
    }
    __syncthreads();

    // ---- merge the waves (LDS split-K merge) ----
    for (int idx = tid; idx < G * HD; idx += DEC_THREADS) {
        const int g = idx / HD, d = idx % HD;
        float M = m_lds[0][g];
#pragma unroll
        for (int w = 1; w < DEC_WAVES; ++w) M = fmaxf(M, m_lds[w][g]);
        float acc = 0.f, L = 0.f;
#pragma unroll
        for (int w = 0; w < DEC_WAVES; ++w) {
            const float e = fast_exp2(m_lds[w][g] - M);
            acc += e * o_lds[w][g][d];
            L += e * l_lds[w][g];
        }
        const long h = (long)kvh * G + g;
        if (np == 1) {
            out[((long)s * nq + h) * HD + d] = __builtin_bit_cast(bf16_t, (__bf16)(acc / L));
        } else {
            const long slot = ((long)s * nq + h) * max_parts + part;
            part_o[slot * HD + d] = acc;
            if (d == 0) {
                part_ml[slot * 2] = M;
                part_ml[slot * 2 + 1] = L;
            }
        }
    }
}

// attention.cu:186-207 semantics: out = sum_p 2^(m_p - M) o_p / sum_p 2^(m_p - M) l_p (m in base 2 here).
__global__ void __launch_bounds__(HD) attn_decode_reduce_kernel(bf16_t *__restrict__ out,
                                                                const float *__restrict__ part_o,
                                                                const float *__restrict__ part_ml,
                                                                const int *__restrict__ ctx_lens, int nq,
                                                                int part_size, int max_parts) {
    const int h = blockIdx.x, s = blockIdx.y, d = threadIdx.x;
    const int ctx = ctx_lens[s];
    bf16_t *o = out + ((long)s * nq + h) * HD;
    if (ctx <= 0) {
        o[d] = 0;
        return;
    }
    int np = (ctx + part_size - 1) / part_size;
    if (np == 1) return;  // the split kernel wrote the final row
    np = min(np, max_parts);
    const float *ml = part_ml + ((long)s * nq + h) * max_parts * 2;
    const float *po = part_o + ((long)s * nq + h) * max_parts * HD;
    float M = -INFINITY;
    for (int p = 0; p < np; ++p) M = fmaxf(M, ml[2 * p]);
    float num = 0.f, den = 0.f;
    for (int p = 0; p < np; ++p) {
        const float w = fast_exp2(ml[2 * p] - M);
        num += w * po[(long)p * HD + d];
        den += w * ml[2 * p + 1];
    }
    o[d] = __builtin_bit_cast(bf16_t, (__bf16)(num / den));
}

template <int G, int NT>
void launch_split(dim3 grid, bf16_t *out, const bf16_t *q, const bf16_t *kc, const bf16_t *vc, const int *bt,
                  const int *ctx, int nq, int nkv, int max_blocks, int block_size, int bs_shift, float sl2,
                  float *part_o, float *part_ml, int part_size, int max_parts, int rounds) {
    hipLaunchKernelGGL((attn_decode_split_kernel<G, NT>), grid, dim3(DEC_THREADS), 0, g_llmgen_stream, out, part_o,
                       part_ml, q, kc, vc, bt, ctx, nq, nkv, max_blocks, block_size, bs_shift, sl2, part_size,
                       max_parts, rounds);
}

template <int G>
bool dispatch_nt(int nt, dim3 grid, bf16_t *out, const bf16_t *q, const bf16_t *kc, const bf16_t *vc, const int *bt,
                 const int *ctx, int nq, int nkv, int max_blocks, int block_size, int bs_shift, float sl2,
                 float *part_o, float *part_ml, int part_size, int max_parts, int rounds) {
#define LLMGEN_NT(N)                                                                                              \
    case N:                                                                                                       \
        launch_split<G, N>(grid, out, q, kc, vc, bt, ctx, nq, nkv, max_blocks, block_size, bs_shift, sl2, part_o, \
                           part_ml, part_size, max_parts, rounds);                                                \
        return true;
    switch (nt) {
        LLMGEN_NT(1)
        LLMGEN_NT(2)
        LLMGEN_NT(3)
        LLMGEN_NT(4)
        default:
            return false;
    }
#undef LLMGEN_NT
}

}  // namespace

extern "C" void hip_attn_decode(bf16_t *out, const bf16_t *q, const bf16_t *k_cache, const bf16_t *v_cache,
                                const int *block_tables, const int *ctx_lens, int S, int nq, int nkv, int hd,
                                int max_blocks, int block_size, float scale, float *part_o, float *part_ml,
                                int part_size, int max_parts) {
    if (S <= 0) return;
    if (hd != HD) {
        fprintf(stderr, "[llmgen-hip] attn_decode: only head_dim=128 is supported (got %d)\n", hd);
        return;
    }
    if (nkv <= 0 || nq <= 0 || nq % nkv != 0 || block_size <= 0 || part_size <= 0 || max_parts <= 0) {
        fprintf(stderr, "[llmgen-hip] attn_decode: bad shape nq=%d nkv=%d block_size=%d part_size=%d max_parts=%d\n",
                nq, nkv, block_size, part_size, max_parts);
        return;
    }
    const int G = nq / nkv;
    const int nt_cap = G <= 4 ? 4 : (G == 8 ? 2 : 1);  // register budget: o holds G*8 floats per lane
    int nt = (part_size + 63) / 64;
    if (nt > nt_cap) nt = nt_cap;
    const int per_round = DEC_WAVES * 16 * nt;
    const int rounds = (part_size + per_round - 1) / per_round;
    const int bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
    const float sl2 = scale * LLMGEN_LOG2E;
    const dim3 grid(nkv, S, max_parts);
    bool ok = false;
    switch (G) {
        case 1: ok = dispatch_nt<1>(nt, grid, out, q, k_cache, v_cache, block_tables, ctx_lens, nq, nkv, max_blocks,
                                    block_size, bs_shift, sl2, part_o, part_ml, part_size, max_parts, rounds); break;
        case 2: ok = dispatch_nt<2>(nt, grid, out, q, k_cache, v_cache, block_tables, ctx_lens, nq, nkv, max_blocks,
                                    block_size, bs_shift, sl2, part_o, part_ml, part_size, max_parts, rounds); break;
        case 4: ok = dispatch_nt<4>(nt, grid, out, q, k_cache, v_cache, block_tables, ctx_lens, nq, nkv, max_blocks,
                                    block_size, bs_shift, sl2, part_o, part_ml, part_size, max_parts, rounds); break;
        case 8: ok = dispatch_nt<8>(nt, grid, out, q, k_cache, v_cache, block_tables, ctx_lens, nq, nkv, max_blocks,
                                    block_size, bs_shift, sl2, part_o, part_ml, part_size, max_parts, rounds); break;
        case 16: ok = dispatch_nt<16>(nt, grid, out, q, k_cache, v_cache, block_tables, ctx_lens, nq, nkv, max_blocks,
                                      block_size, bs_shift, sl2, part_o, part_ml, part_size, max_parts, rounds); break;
        default: break;
    }
    if (!ok) {
        fprintf(stderr, "[llmgen-hip] attn_decode: unsupported GQA group size %d\n", G);
        return;
    }
    hipLaunchKernelGGL(attn_decode_reduce_kernel, dim3(nq, S), dim3(HD), 0, g_llmgen_stream, out, part_o, part_ml,
                       ctx_lens, nq, part_size, max_parts);
}
