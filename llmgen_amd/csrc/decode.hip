// decode.hip -- split-K flash-decoding over the paged KV cache with GQA head sharing (gfx950, wave64).
//
// Contract: src/backend/cuda/attention/attention_v1.zig:11-29 (cuda_attn_decode argument list) with the semantics
// of src/backend/cuda/attention/attention.cu:51-253: q [S, nq, 128] (one query token per sequence, whose K/V is
// already in the cache), ctx_lens[s] = keys to attend, split-K scratch part_o [S, nq, max_parts, 128] f32 and
// part_ml [S, nq, max_parts, 2] f32 owned by the caller, part p covering tokens [p*part_size, (p+1)*part_size).
// Output: bf16(softmax(scale * q K^T) V) per (s, head), 0 for ctx <= 0 (cpu/attention.zig:80-83).
//
// Design (one workgroup = one (kv head, sequence, span of parts), 4 or 8 waves):
//   * every wave owns 16-token tiles of the part; per round a wave issues all of its K and V loads at once as
//     16-byte nontemporal vectors, four whole 256-byte rows per instruction, so a workgroup keeps up to 128 KB in
//     flight.  K rows then pass through a wave-private LDS slice into the MFMA B-operand layout (16 tokens x 64 B
//     per fragment); loading that layout directly reads each 128-byte line in two halves, which streams worse;
//   * QK^T runs on the matrix cores: v_mfma_f32_16x16x32_bf16 with the G query heads of the group as the 16 A
//     rows, so the K bytes are read once for all G heads (GQA sharing).  Scores land one token per lane column,
//     one head per row, and the softmax max / sum reduce over a 16-lane DPP row;
//   * softmax is in base 2 (scale * log2 e folded in), fp32 throughout.  P V runs on the matrix cores for
//     G >= 8 and in 8-wave workgroups (v_mfma_f32_16x16x16_bf16: P from a per-wave LDS slice as A, V^T read
//     transposed out of the wave's LDS slice as B); otherwise the probabilities go through the per-wave LDS
//     slice to PV lanes that hold 8 head dims of 4 tokens per 16-byte V vector and accumulate all G heads in fp32;
//   * the W waves merge (max, sum, unnormalised o) through LDS; a part that is the only part of its
//     sequence writes the final bf16 row directly, otherwise (o, m, l) go to the caller's scratch and the last
//     workgroup of the (sequence, kv head) to finish merges the parts with the log-sum-exp rule
//     (attention.cu:186-207), elected by a self-resetting counter (attn_decode_reduce_kernel when the launch
//     has more pairs than counters);
//   * hip_attn_decode_store_kv also writes the step's token into the cache (the store_kv of a decode step),
//     reading that token's K/V from the step's k / v rather than from the slot being written.
// Grid = (nkv, S, parts) from host integers only, so the launch is graph-capturable; parts past ctx exit.
#include "hip_common.h"

#include <math.h>
#include <stdlib.h>

#include <algorithm>

namespace {

// K and V rows are read once, whole (four full 256-byte rows per instruction): nontemporal loads keep them from
// displacing cache lines (c5d 362 -> 330 us).
__device__ __forceinline__ u32x4_t ld16_stream(const void *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
}
constexpr int HD = 128;
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
// LDS read with transpose: a 16-lane group whose lane 4j+m addresses four 16-bit values (dims 4m..4m+3) of row j
// receives, in lane i, rows 0..3's value of dim i
__device__ __forceinline__ s16x4_t ds_read_tr(const bf16_t *p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)p);
}
constexpr int DEC_THREADS = 256;  // the separate merge kernel's workgroup

// Block-table lookup of logical token t (POW2: block_size == 1 << bs_shift).
template <bool POW2>
__device__ __forceinline__ int blk_index(int t, int block_size, int bs_shift) {
    return POW2 ? (t >> bs_shift) : (t / block_size);
}

// G = query heads per KV head (1..16); NT = 16-token tiles per wave per round (a round is W waves x 16*NT
// tokens); W = waves per workgroup (4 or 8); FUSE = also write the step's token into the cache.  Each workgroup
// streams `span` tokens of one (kv head, sequence) pair, one round at a time with a single register buffer
// (three waves per SIMD hide each other's load latency).
template <int G, int NT, bool POW2, bool FUSE, int W>
__global__ void __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(3)))
    attn_decode_split_kernel(bf16_t *__restrict__ out, float *__restrict__ part_o, float *__restrict__ part_ml,
                             const bf16_t *__restrict__ q, const bf16_t *__restrict__ kc,
                             const bf16_t *__restrict__ vc, const int *__restrict__ block_tables,
                             const int *__restrict__ ctx_lens, int nq, int nkv, int max_blocks, int block_size,
                             int bs_shift, float scale_log2, int span, int max_parts, int nparts,
                             int *__restrict__ counters, const int *__restrict__ cu_q,
                             const int *__restrict__ tile_seq, const bf16_t *__restrict__ k_new,
                             const bf16_t *__restrict__ v_new, const int *__restrict__ slots,
                             bf16_t *__restrict__ kc_w, bf16_t *__restrict__ vc_w) {
    constexpr int WTOK = NT * 16;              // tokens per wave per round
    constexpr int RTOK = W * WTOK;             // tokens per round
    constexpr int NTH = 64 * W;
    const int kvh = blockIdx.x, part = blockIdx.z;
    // decode launch: blockIdx.y is the sequence and its query row.  Prefill-metadata launch (cu_q != null):
    // blockIdx.y counts query tiles from the end of the list; only single-row segments (decode rows of a mixed
    // step) are handled here.  The tile list runs lightest first (by key end), so the longest contexts are
    // dispatched first and the shortest fill the tail.
    int s = blockIdx.y, row = blockIdx.y;
    if (cu_q) {
        s = tile_seq[gridDim.y - 1 - blockIdx.y];
        row = cu_q[s];
        if (cu_q[s + 1] - row != 1) return;
    }
    const int ctx = ctx_lens[s];
    const int t0 = part * span;
    // Fused KV write (decode launch only): this step's token sits at position ctx - 1.  Part 0 copies its K/V
    // rows into the cache slot; the workgroup whose span holds position ctx - 1 reads them from k_new / v_new,
    // so no workgroup of this launch reads the slot being written.
    constexpr bool fuse = FUSE;
    const long new_row = ((long)row * nkv + kvh) * HD;
    if (fuse && part == 0 && ctx > 0 && threadIdx.x < 32) {
        const int slot = slots[row];
        if (slot >= 0) {
            const long dst = (((long)(slot / block_size) * nkv + kvh) * block_size + slot % block_size) * HD;
            const int c = threadIdx.x & 15;
            if (threadIdx.x < 16)
                *reinterpret_cast<u32x4_t *>(kc_w + dst + c * 8) = ld16(k_new + new_row + c * 8);
            else
                *reinterpret_cast<u32x4_t *>(vc_w + dst + c * 8) = ld16(v_new + new_row + c * 8);
        }
    }
    if (t0 >= ctx) {
        if (ctx <= 0 && part == 0) {  // padding row: zeros (cpu/attention.zig:80-83)
            for (int idx = threadIdx.x; idx < G * HD; idx += NTH)
                out[((long)row * nq + (long)kvh * G + idx / HD) * HD + idx % HD] = 0;
        }
        return;
    }
    const int n = min(ctx - t0, span);
    const int np = min((ctx + span - 1) / span, nparts);
    const int rounds = (n + RTOK - 1) / RTOK;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, rgrp = lane >> 4;

    __shared__ u32x4_t k_lds[W][WTOK][16];  // K rows of this round, 16-byte chunks XOR-swizzled by the token
    __shared__ __attribute__((aligned(16))) float p_lds[W][WTOK][G];
    __shared__ float corr_lds[W][G];
    __shared__ float o_lds[W][G][HD];
    __shared__ float m_lds[W][G];
    __shared__ float l_lds[W][G];

    const int *bt = block_tables + (long)s * max_blocks;
    const long blk_stride = (long)nkv * block_size * HD;
    const bf16_t *kbase = kc + (long)kvh * block_size * HD;
    const bf16_t *vbase = vc + (long)kvh * block_size * HD;

    // A operand: row g = col holds head kvh*G+g; lane group rgrp holds dims c*32 + rgrp*8 .. +8 of chunk c.
    bf16x8_t qa[4];
    {
        const bf16_t *qrow = q + ((long)row * nq + (long)kvh * G + (col < G ? col : 0)) * HD + rgrp * 8;
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
    // MPV (G >= 8, and every 8-wave workgroup): P V on the matrix cores; o4[db] is the 16 x 16 block (rows: heads rgrp*4 + i, columns: dims
    // db*16 + col) of O.  Otherwise o[g][k]: dims col*8 + k of head g over this lane's tokens.
    constexpr bool MPV = G >= 8 || W == 8;
    float o[G][8];
    f32x4_t o4[8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < 8; ++k) o[g][k] = 0.f;
#pragma unroll
    for (int db = 0; db < 8; ++db) o4[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // K and V: token rgrp + 4j, dims col*8 (four whole 256-byte rows per load instruction).
    struct Buf {
        u32x4_t kr[4 * NT];
        u32x4_t vf[4 * NT];
    };
    auto load = [&](int r, Buf &b) {
        const int wbase = r * RTOK + wave * WTOK;
        int vt[4 * NT], vblk[4 * NT];
#pragma unroll
        for (int j = 0; j < 4 * NT; ++j) vt[j] = t0 + min(wbase + rgrp + 4 * j, n - 1);
        if (POW2 && block_size >= WTOK) {
            // the wave's WTOK tokens touch at most two blocks: two scalar block-table reads (scalar cache,
            // their own wait counter), then a per-lane select
            const int b0 = __builtin_amdgcn_readfirstlane((t0 + min(wbase, n - 1)) >> bs_shift);
            const int b1 = __builtin_amdgcn_readfirstlane((t0 + min(wbase + WTOK - 1, n - 1)) >> bs_shift);
            const int p0 = bt[b0], p1 = bt[b1];
#pragma unroll
            for (int j = 0; j < 4 * NT; ++j) vblk[j] = (vt[j] >> bs_shift) == b0 ? p0 : p1;
        } else {
            // all block-table reads first (independent), then all K/V reads
#pragma unroll
            for (int j = 0; j < 4 * NT; ++j) vblk[j] = bt[blk_index<POW2>(vt[j], block_size, bs_shift)];
        }
#pragma unroll
        for (int j = 0; j < 4 * NT; ++j) {
            const int off = vt[j] - blk_index<POW2>(vt[j], block_size, bs_shift) * block_size;
            const long row = (long)vblk[j] * blk_stride + (long)off * HD + col * 8;
            const bool mine = fuse && vt[j] == ctx - 1;
            b.kr[j] = ld16_stream(mine ? k_new + new_row + col * 8 : kbase + row);
        }
#pragma unroll
        for (int j = 0; j < 4 * NT; ++j) {
            const int off = vt[j] - blk_index<POW2>(vt[j], block_size, bs_shift) * block_size;
            const bf16_t *vr = vbase + (long)vblk[j] * blk_stride + (long)off * HD + col * 8;
            if (fuse && vt[j] == ctx - 1) vr = v_new + new_row + col * 8;
            b.vf[j] = ld16_stream(vr);
        }
    };

    auto compute = [&](int r, const Buf &b) {
        const int wbase = r * RTOK + wave * WTOK;
        // ---- K rows into this wave's LDS slice, then the MFMA B fragments back out of it (tile tau, chunk c =
        //      dims c*32 + rgrp*8 of token tau*16 + col); the XOR swizzle keeps both directions conflict-free ----
#pragma unroll
        for (int j = 0; j < 4 * NT; ++j) {
            const int tok = rgrp + 4 * j;
            k_lds[wave][tok][col ^ (tok & 15)] = b.kr[j];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        u32x4_t kf[NT][4];
#pragma unroll
        for (int tau = 0; tau < NT; ++tau)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int tok = tau * 16 + col;
                kf[tau][c] = k_lds[wave][tok][(c * 4 + rgrp) ^ (tok & 15)];
            }
        // ---- scores on the matrix cores: D[g][token] = sum_d q[g][d] k[token][d] ----
        f32x4_t sc[NT];
#pragma unroll
        for (int tau = 0; tau < NT; ++tau) {
            f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 4; ++c)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[c], __builtin_bit_cast(bf16x8_t, kf[tau][c]),
                                                              acc, 0, 0, 0);
            const bool valid = wbase + tau * 16 + col < n;
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[tau][i] = valid ? acc[i] * scale_log2 : -INFINITY;
        }
        // ---- online softmax (row rgrp*4+i of the MFMA output = head g; rows past G hold the zero query
        //      rows and are computed but never stored) ----
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
        if constexpr (MPV) {
            // ---- P V on the matrix cores (v_mfma_f32_16x16x16_bf16): A = P (rows: heads, k: tokens) from this
            //      wave's LDS slice laid out [head][token]; B = V (k: tokens, columns: dims) read transposed from the
            //      wave's K slice, which now holds this round's V rows (the K fragments are in registers) ----
            float *pw = &p_lds[wave][0][0];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int g = rgrp * 4 + i;
                if (g < G) {
#pragma unroll
                    for (int tau = 0; tau < NT; ++tau) pw[g * WTOK + tau * 16 + col] = sc[tau][i];
                }
            }
#pragma unroll
            for (int j = 0; j < 4 * NT; ++j) {
                const int t = rgrp + 4 * j;
                k_lds[wave][t][col ^ ((t << 2) & 15)] = b.vf[j];
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int db = 0; db < 8; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) o4[db][i] *= corr[i];
            const bf16_t *vb = reinterpret_cast<const bf16_t *>(&k_lds[wave][0][0]);
            const int jj = col >> 2, mm = col & 3;
#pragma unroll
            for (int kb = 0; kb < NT; ++kb) {
                f32x4_t pv = {0.f, 0.f, 0.f, 0.f};
                if (col < G) pv = *reinterpret_cast<const f32x4_t *>(&pw[col * WTOK + kb * 16 + rgrp * 4]);
                u32x2_t pa;
                pa[0] = pack_bf16x2(pv[0], pv[1]);
                pa[1] = pack_bf16x2(pv[2], pv[3]);
                const s16x4_t a = __builtin_bit_cast(s16x4_t, pa);
                const int key = kb * 16 + rgrp * 4 + jj;
#pragma unroll
                for (int db = 0; db < 8; ++db) {
                    const int dim = db * 16 + 4 * mm;
                    const int off = key * HD + (((dim >> 3) ^ ((key << 2) & 15)) << 3) + (dim & 7);
                    o4[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, ds_read_tr(vb + off), o4[db], 0, 0, 0);
                }
            }
            // the next round rewrites both slices: keep every lane's reads ahead of those writes
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            return;
        }
        // probabilities to this wave's LDS slice (wave-private: a wavefront fence orders write -> read)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int g = rgrp * 4 + i;
            if (g < G) {
#pragma unroll
                for (int tau = 0; tau < NT; ++tau) p_lds[wave][tau * 16 + col][g] = sc[tau][i];
                if (col == 0) corr_lds[wave][g] = corr[i];
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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
            unpack_bf16x8(b.vf[j], f);
            const float *pp = p_lds[wave][rgrp + 4 * j];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float p = pp[g];
#pragma unroll
                for (int k = 0; k < 8; ++k) o[g][k] += p * f[k];
            }
        }
        // the next round rewrites p_lds: keep every lane's reads ahead of those writes
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    Buf buf;
    for (int r = 0; r < rounds; ++r) {
        load(r, buf);
        compute(r, buf);
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
    if constexpr (MPV) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int g = rgrp * 4 + i;
            if (g < G) {
#pragma unroll
                for (int db = 0; db < 8; ++db) o_lds[wave][g][db * 16 + col] = o4[db][i];
            }
        }
    } else {
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
    }
    __syncthreads();

    // ---- merge the waves (LDS split-K merge) ----
    for (int idx = tid; idx < G * HD; idx += NTH) {
        const int g = idx / HD, d = idx % HD;
        float M = m_lds[0][g];
#pragma unroll
        for (int w = 1; w < W; ++w) M = fmaxf(M, m_lds[w][g]);
        float acc = 0.f, L = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float e = fast_exp2(m_lds[w][g] - M);
            acc += e * o_lds[w][g][d];
            L += e * l_lds[w][g];
        }
        const long h = (long)kvh * G + g;
        if (np == 1) {
            out[((long)row * nq + h) * HD + d] = __builtin_bit_cast(bf16_t, (__bf16)(acc / L));
        } else {
            const long slot = ((long)s * nq + h) * max_parts + part;
            if (counters) {  // device-coherent (write-through) stores: read by another workgroup below
                __hip_atomic_store(part_o + slot * HD + d, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (d == 0) {
                    __hip_atomic_store(part_ml + slot * 2, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(part_ml + slot * 2 + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            } else {
                part_o[slot * HD + d] = acc;
                if (d == 0) {
                    part_ml[slot * 2] = M;
                    part_ml[slot * 2 + 1] = L;
                }
            }
        }
    }
    if (np == 1 || !counters) return;

    // ---- cross-workgroup merge: the last workgroup of this (kv head, sequence) to finish combines the np
    //      partial results (attention.cu:186-207 semantics, m in base 2).  The partials were written with
    //      device-coherent stores; each thread waits for its stores to complete before the barrier, then one
    //      counter increment per workgroup elects the merger, which reads the partials with device-coherent
    //      loads.  No cache-wide fence (an L2 write-back + invalidate per workgroup costs more than the whole
    //      merge).  The merger resets the counter, so it is zero again when the kernel ends. ----
    __shared__ int s_last;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int *cnt = counters + (long)s * nkv + kvh;
    if (tid == 0) s_last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == np - 1;
    __syncthreads();
    if (!s_last) return;
    // acquire at agent scope: the other workgroups' partials, published before their ticket increments, are read
    // after this point (the loads below are agent-scope atomics as well)
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    for (int idx = tid; idx < G * HD; idx += NTH) {
        const int g = idx / HD, d = idx % HD;
        const long h = (long)kvh * G + g;
        float *ml = part_ml + ((long)s * nq + h) * max_parts * 2;
        float *po = part_o + ((long)s * nq + h) * max_parts * HD + d;
        float M = -INFINITY;
        for (int p = 0; p < np; ++p)
            M = fmaxf(M, __hip_atomic_load(ml + 2 * p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        float num = 0.f, den = 0.f;
        for (int p = 0; p < np; ++p) {
            const float w =
                fast_exp2(__hip_atomic_load(ml + 2 * p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - M);
            num += w * __hip_atomic_load(po + (long)p * HD, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            den += w * __hip_atomic_load(ml + 2 * p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        out[((long)s * nq + h) * HD + d] = __builtin_bit_cast(bf16_t, (__bf16)(num / den));
    }
    if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// attention.cu:186-207 semantics: out = sum_p 2^(m_p - M) o_p / sum_p 2^(m_p - M) l_p (m in base 2 here).
// One workgroup per (kv head, sequence) covers the G heads of the group; a sequence whose context fits one span
// was finished by the split kernel.
__global__ void __launch_bounds__(DEC_THREADS) attn_decode_reduce_kernel(bf16_t *__restrict__ out,
                                                                        const float *__restrict__ part_o,
                                                                        const float *__restrict__ part_ml,
                                                                        const int *__restrict__ ctx_lens, int nq,
                                                                        int G, int span, int nparts, int max_parts) {
    const int kvh = blockIdx.x, s = blockIdx.y;
    const int ctx = ctx_lens[s];
    if (ctx > 0 && (ctx + span - 1) / span == 1) return;
    const int np = ctx > 0 ? min((ctx + span - 1) / span, nparts) : 0;
    for (int idx = threadIdx.x; idx < G * HD; idx += DEC_THREADS) {
        const int g = idx / HD, d = idx % HD;
        const long h = (long)kvh * G + g;
        bf16_t *o = out + ((long)s * nq + h) * HD + d;
        if (np == 0) {
            *o = 0;
            continue;
        }
        const float *ml = part_ml + ((long)s * nq + h) * max_parts * 2;
        const float *po = part_o + ((long)s * nq + h) * max_parts * HD + d;
        float M = -INFINITY;
        for (int p = 0; p < np; ++p) M = fmaxf(M, ml[2 * p]);
        float num = 0.f, den = 0.f;
#pragma unroll 4
        for (int p = 0; p < np; ++p) {
            const float w = fast_exp2(ml[2 * p] - M);
            num += w * po[(long)p * HD];
            den += w * ml[2 * p + 1];
        }
        *o = __builtin_bit_cast(bf16_t, (__bf16)(num / den));
    }
}

struct DecodeArgs {
    bf16_t *out;
    const bf16_t *q, *kc, *vc;
    const int *bt, *ctx;
    int nq, nkv, max_blocks, block_size, bs_shift;
    float sl2;
    float *part_o, *part_ml;
    int span, max_parts, nparts;
    int *counters;  // merge counters (nullptr: the separate merge kernel runs)
    const int *cu_q = nullptr, *tile_seq = nullptr;  // prefill-metadata launch (single-row segments)
    hipStream_t stream = nullptr;                    // nullptr: the library's launch stream
    const bf16_t *k_new = nullptr, *v_new = nullptr;  // fused KV write of this step's token (decode launch)
    const int *slots = nullptr;
    bf16_t *kc_w = nullptr, *vc_w = nullptr;
    int waves = 4;  // waves per workgroup (4 or 8)
};

template <int G, int NT, bool POW2, int W>
void launch_split_w(dim3 grid, const DecodeArgs &a) {
    auto kern = a.k_new ? attn_decode_split_kernel<G, NT, POW2, true, W>
                        : attn_decode_split_kernel<G, NT, POW2, false, W>;
    hipLaunchKernelGGL(kern, grid, dim3(64 * W), 0,
                       a.stream ? a.stream : g_llmgen_stream, a.out,
                       a.part_o, a.part_ml, a.q, a.kc, a.vc, a.bt, a.ctx, a.nq, a.nkv, a.max_blocks, a.block_size,
                       a.bs_shift, a.sl2, a.span, a.max_parts, a.nparts, a.counters, a.cu_q, a.tile_seq, a.k_new,
                       a.v_new, a.slots, a.kc_w, a.vc_w);
}

template <int G, int NT, bool POW2>
void launch_split(dim3 grid, const DecodeArgs &a) {
    if constexpr (G <= 4) {
        if (a.waves == 8) {
            launch_split_w<G, NT, POW2, 8>(grid, a);
            return;
        }
    }
    launch_split_w<G, NT, POW2, 4>(grid, a);
}

template <int G, int NT>
void launch_pow2(dim3 grid, const DecodeArgs &a) {
    if (a.bs_shift >= 0)
        launch_split<G, NT, true>(grid, a);
    else
        launch_split<G, NT, false>(grid, a);
}


// Merge counters for the in-kernel split-K merge, one per (sequence, kv head).  They start at zero when the
// library loads and every merging workgroup resets its own, so they are zero between launches.  Launches that
// overlap on two streams must not share the library (as they must not share part_o / part_ml).
constexpr int MAX_MERGE_SEGMENTS = 1 << 18;
__device__ int g_merge_counters[MAX_MERGE_SEGMENTS];

int *merge_counters() {
    static int *ptr[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    if (!ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_merge_counters)) != hipSuccess) return nullptr;
        ptr[dev] = (int *)p;
    }
    return ptr[dev];
}

// Waves per workgroup: 8 when the launch has enough (sequence, kv head) pairs to fill the chip with 8-wave
// workgroups (fewer, longer workgroups: less split-K merging, fewer partial results), else 4.
int decode_waves(int G, long pairs) {
    if (G > 4) return 4;
    return pairs * 2 >= llmgen_num_cus() ? 8 : 4;
}

// The decode rows of a mixed step (4-wave workgroups, no fused KV write): 64 tokens per wave and round (NT = 4)
// for G <= 4, twice the bytes in flight per wave and half the rounds, with 72 KB of LDS per workgroup.
template <int G>
void launch_rows_nt4(dim3 grid, const DecodeArgs &a) {
    auto kern = a.bs_shift >= 0 ? attn_decode_split_kernel<G, 4, true, false, 4>
                                : attn_decode_split_kernel<G, 4, false, false, 4>;
    hipLaunchKernelGGL(kern, grid, dim3(64 * 4), 0, a.stream ? a.stream : g_llmgen_stream, a.out, a.part_o,
                       a.part_ml, a.q, a.kc, a.vc, a.bt, a.ctx, a.nq, a.nkv, a.max_blocks, a.block_size, a.bs_shift,
                       a.sl2, a.span, a.max_parts, a.nparts, a.counters, a.cu_q, a.tile_seq, a.k_new, a.v_new,
                       a.slots, a.kc_w, a.vc_w);
}

void launch_decode_rows(dim3 grid, const DecodeArgs &a, int G) {
    switch (G) {
        case 1: launch_pow2<1, 2>(grid, a); break;
        case 2: launch_pow2<2, 2>(grid, a); break;
        case 4: launch_pow2<4, 2>(grid, a); break;
        case 8: launch_pow2<8, 2>(grid, a); break;
        default: launch_pow2<16, 1>(grid, a); break;
    }
}


// Split-K scratch of hip_attn_decode_noalloc: a file-scope device array (each device holds its own copy for the
// life of the process).  Host code never passes the array's name to a kernel: its device address is taken once
// per device with hipGetSymbolAddress and kept here.  Every call on a device shares that device's array, so calls
// that overlap on one device (two streams) race; the partials need no clearing (each slot is written before it
// is read) and the merge counters reset themselves.
constexpr size_t NOALLOC_SCRATCH_FLOATS = (size_t)2 << 20;  // 8 MiB
__device__ __align__(256) float scratch[NOALLOC_SCRATCH_FLOATS];

float *noalloc_scratch() {
    static float *ptr[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    if (!ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            fprintf(stderr, "[llmgen-hip] attn_decode_noalloc: hipGetSymbolAddress failed: %s\n",
                    hipGetErrorString(e));
            return nullptr;
        }
        ptr[dev] = (float *)p;
    }
    return ptr[dev];
}

// own_scratch: part_o / part_ml are ignored and the partials go to the library's array above, packed with a
// stride of the launch's own part count instead of max_parts.
void decode_launch(bf16_t *out, const bf16_t *q, const bf16_t *k_new, const bf16_t *v_new, const int *slots,
                   bf16_t *k_cache, bf16_t *v_cache, const int *block_tables, const int *ctx_lens, int S, int nq,
                   int nkv, int hd, int max_blocks, int block_size, float scale, float *part_o, float *part_ml,
                   int part_size, int max_parts, bool own_scratch = false) {
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
    if (G != 1 && G != 2 && G != 4 && G != 8 && G != 16) {
        fprintf(stderr, "[llmgen-hip] attn_decode: unsupported GQA group size %d\n", G);
        return;
    }
    // SV_ATTN_PART (attention.cu:219-229): parts only ever get longer, so max_parts slots still suffice
    const int part_min = llmgen_opt(LLMGEN_OPT_ATTN_PART_MIN);
    if (part_min > part_size) part_size = part_min;
    if ((long)part_size * max_parts > 0x7fffffffL) {  // token positions are int32 throughout
        fprintf(stderr, "[llmgen-hip] attn_decode: part_size * max_parts (%d * %d) exceeds the int32 token range\n",
                part_size, max_parts);
        return;
    }
    // Each workgroup takes k consecutive parts (span = k * part_size tokens, one partial result).  k grows
    // with the launch so that a long-context launch has about 8 waves per compute unit (two 4-wave or one
    // 8-wave workgroup), each streaming a long span, instead of many short workgroups; partial slots stay
    // < max_parts.
    const long total = (long)nkv * S * max_parts;
    constexpr int wg_per_cu = 2;
    const int W = decode_waves(G, (long)S * nkv);
    const long target = (long)wg_per_cu * llmgen_num_cus() * 4 / W;
    // ... and a span is at least one round (W waves x 32 tokens, 16 at G = 16), so that no wave of a workgroup
    // idles: small batches have 64-token parts (c1: 9.4 -> 8.0 us)
    const int round_tokens = W * (G >= 16 ? 16 : 32);
    const int k = std::max((int)(total > target ? total / target : 1),
                           (int)(((long)round_tokens + part_size - 1) / part_size));
    const int nparts = (max_parts + k - 1) / k;
    const int span = (int)std::min((long)part_size * k, 1L << 30);  // tokens per workgroup (no int overflow)
    int stride = max_parts;  // partial slots per (sequence, head) in part_o / part_ml
    // With one part per (sequence, head) every workgroup writes its rows directly and no partial is stored or
    // read (the merge kernel returns early), so the library's array is not needed.
    if (own_scratch && nparts == 1) {
        part_o = part_ml = nullptr;
        stride = 1;
    } else if (own_scratch) {
        const size_t rows = (size_t)S * nq * nparts;
        if (rows * (HD + 2) > NOALLOC_SCRATCH_FLOATS) {
            fprintf(stderr,
                    "[llmgen-hip] attn_decode_noalloc: this launch needs %zu bytes of split-K scratch, more than the "
                    "library's %zu; use hip_attn_decode with caller-owned scratch\n",
                    rows * (HD + 2) * sizeof(float), NOALLOC_SCRATCH_FLOATS * sizeof(float));
            llmgen_record_error(hipErrorInvalidValue);
            return;
        }
        float *base = noalloc_scratch();
        if (!base) {
            llmgen_record_error(hipErrorInvalidSymbol);
            return;
        }
        part_o = base;
        part_ml = base + rows * HD;
        stride = nparts;
    }
    int *counters = (long)S * nkv <= MAX_MERGE_SEGMENTS && !llmgen_opt(LLMGEN_OPT_DECODE_MERGE_KERNEL)
                        ? merge_counters()
                        : nullptr;
    DecodeArgs a{out, q, k_cache, v_cache, block_tables, ctx_lens, nq, nkv, max_blocks, block_size,
                 (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1, scale * LLMGEN_LOG2E,
                 part_o, part_ml, span, stride, nparts, counters};
    a.k_new = k_new;
    a.v_new = v_new;
    a.slots = slots;
    a.kc_w = k_cache;
    a.vc_w = v_cache;
    a.waves = W;
    launch_decode_rows(dim3(nkv, S, nparts), a, G);
    if (!counters)  // batches beyond the counter array merge in a second kernel
        hipLaunchKernelGGL(attn_decode_reduce_kernel, dim3(nkv, S), dim3(DEC_THREADS), 0, g_llmgen_stream, out,
                           part_o, part_ml, ctx_lens, nq, G, a.span, nparts, stride);
}

}  // namespace

extern "C" void hip_attn_decode(bf16_t *out, const bf16_t *q, const bf16_t *k_cache, const bf16_t *v_cache,
                                const int *block_tables, const int *ctx_lens, int S, int nq, int nkv, int hd,
                                int max_blocks, int block_size, float scale, float *part_o, float *part_ml,
                                int part_size, int max_parts) {
    decode_launch(out, q, nullptr, nullptr, nullptr, const_cast<bf16_t *>(k_cache), const_cast<bf16_t *>(v_cache),
                  block_tables, ctx_lens, S, nq, nkv, hd, max_blocks, block_size, scale, part_o, part_ml, part_size,
                  max_parts);
}

// hip_attn_decode with the split-K partials in the library's own device array: allocates nothing, takes no
// scratch from the caller.
extern "C" void hip_attn_decode_noalloc(bf16_t *out, const bf16_t *q, const bf16_t *k_cache, const bf16_t *v_cache,
                                        const int *block_tables, const int *ctx_lens, int S, int nq, int nkv, int hd,
                                        int max_blocks, int block_size, float scale, int part_size, int max_parts) {
    decode_launch(out, q, nullptr, nullptr, nullptr, const_cast<bf16_t *>(k_cache), const_cast<bf16_t *>(v_cache),
                  block_tables, ctx_lens, S, nq, nkv, hd, max_blocks, block_size, scale, nullptr, nullptr, part_size,
                  max_parts, true);
}

// store_kv of the step's one token per sequence fused into the decode launch (one kernel instead of two).
extern "C" void hip_attn_decode_store_kv(bf16_t *out, const bf16_t *q, const bf16_t *k, const bf16_t *v,
                                         const int *slot_mapping, bf16_t *k_cache, bf16_t *v_cache,
                                         const int *block_tables, const int *ctx_lens, int S, int nq, int nkv, int hd,
                                         int max_blocks, int block_size, float scale, float *part_o, float *part_ml,
                                         int part_size, int max_parts) {
    if (S > 0 && (k == nullptr || v == nullptr || slot_mapping == nullptr)) {
        fprintf(stderr, "[llmgen-hip] attn_decode_store_kv: k, v and slot_mapping are required\n");
        return;
    }
    decode_launch(out, q, k, v, slot_mapping, k_cache, v_cache, block_tables, ctx_lens, S, nq, nkv, hd, max_blocks,
                  block_size, scale, part_o, part_ml, part_size, max_parts);
}

// Decode rows of a prefill / mixed step (segments with q_len == 1): one workgroup per (kv head, tile) streams the
// whole context and writes the row directly; no split-K scratch is needed.  The MFMA prefill kernel skips these
// tiles.  Called by hip_attn_prefill.
void llmgen_decode_rows_of_prefill(bf16_t *out, const bf16_t *q, const bf16_t *k_cache, const bf16_t *v_cache,
                                   const int *block_tables, const int *ctx_lens, const int *cu_q,
                                   const int *tile_seq, int n_tiles, int nq, int nkv, int max_blocks,
                                   int block_size, float scale, hipStream_t stream) {
    const int G = nq / nkv;
    DecodeArgs a{out, q, k_cache, v_cache, block_tables, ctx_lens, nq, nkv, max_blocks, block_size,
                 (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1, scale * LLMGEN_LOG2E,
                 nullptr, nullptr, 1 << 30, 1, 1, nullptr, cu_q, tile_seq, stream};
    // one workgroup per (row, kv head) and no split: many generations of workgroups per CU, which overlap their
    // start and end better as 4-wave workgroups (c4 262 -> 249 us; the split decode launch sizes its grid to about
    // one generation and prefers 8)
    a.waves = llmgen_opt(LLMGEN_OPT_DECODE_ROW_WAVES) == 8 ? 8 : 4;
    const dim3 grid(nkv, n_tiles, 1);
    if (a.waves == 4 && G <= 4) {  // 64 tokens per wave and round: c4 236 -> 226 us
        if (G == 1) launch_rows_nt4<1>(grid, a);
        else if (G == 2) launch_rows_nt4<2>(grid, a);
        else launch_rows_nt4<4>(grid, a);
        return;
    }
    launch_decode_rows(grid, a, G);
}

