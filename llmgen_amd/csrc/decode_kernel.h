// decode_kernel.h -- the split-K paged decode workgroup (gfx950), shared by the decode launchers (decode.hip) and
// the mixed-step kernel (mixed.hip).  What it computes and how is described in decode.hip.
#pragma once
#include "hip_common.h"

#include <math.h>

#include <type_traits>

namespace llmgen_decode {

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
template <int G, int NT, int W>
struct DecodeLds {
    u32x4_t k[W][NT * 16][16];  // K rows of this round, 16-byte chunks XOR-swizzled by the token
    __attribute__((aligned(16))) float p[W][NT * 16][G];
    float corr[W][G];
    float o[W][G][HD];
    float m[W][G];
    float l[W][G];
    int last;
};

// The split-K decode workgroup's work, as a device function so that other kernels can run it as one of their
// workgroup roles.  (bx, by, bz) play the part of the grid position (kv head, sequence or list entry, span);
// n_list is the length of the tile list in a prefill-metadata launch; lds holds a DecodeLds<G, NT, W>.
template <int G, int NT, bool POW2, bool FUSE, int W>
__device__ __forceinline__ void decode_split_body(bf16_t *__restrict__ out, float *__restrict__ part_o, float *__restrict__ part_ml,
                             const bf16_t *__restrict__ q, const bf16_t *__restrict__ kc,
                             const bf16_t *__restrict__ vc, const int *__restrict__ block_tables,
                             const int *__restrict__ ctx_lens, int nq, int nkv, int max_blocks, int block_size,
                             int bs_shift, float scale_log2, int span, int max_parts, int nparts,
                             int *__restrict__ counters, const int *__restrict__ cu_q,
                             const int *__restrict__ tile_seq, const bf16_t *__restrict__ k_new,
                             const bf16_t *__restrict__ v_new, const int *__restrict__ slots,
                             bf16_t *__restrict__ kc_w, bf16_t *__restrict__ vc_w, int bx, int by, int bz, int n_list, unsigned char *lds) {
    constexpr int WTOK = NT * 16;              // tokens per wave per round
    constexpr int RTOK = W * WTOK;             // tokens per round
    constexpr int NTH = 64 * W;
    const int kvh = bx, part = bz;
    // decode launch: by is the sequence and its query row.  Prefill-metadata launch (cu_q != null): by counts
    // query tiles from the end of the list; only single-row segments (decode rows of a mixed
    // step) are handled here.  The tile list runs lightest first (by key end), so the longest contexts are
    // dispatched first and the shortest fill the tail.
    int s = by, row = by;
    if (cu_q) {
        s = tile_seq[n_list - 1 - by];
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

    DecodeLds<G, NT, W> &sm = *reinterpret_cast<DecodeLds<G, NT, W> *>(lds);
    auto &k_lds = sm.k;
    auto &p_lds = sm.p;
    auto &corr_lds = sm.corr;
    auto &o_lds = sm.o;
    auto &m_lds = sm.m;
    auto &l_lds = sm.l;

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

    // K rows go straight from HBM into this wave's LDS slice (LDS DMA, no registers); V rows into registers,
    // token rgrp + 4j, dims col*8 (four whole 256-byte rows per load instruction).
    struct Buf {
        u32x4_t knew;  // the fused token's K row chunk (FUSE only)
        u32x4_t vf[4 * NT];
    };
    bf16_t *k_lds_flat = reinterpret_cast<bf16_t *>(&k_lds[0][0][0]);
    int kb0_blk = 0;
    __amdgpu_buffer_rsrc_t krs0, krs1;
    int vt_keep[4 * NT];  // this round's (clamped) token of load j, for the fused-token fix-up
    // SCAL: the wave's rows lie in at most two blocks of a power-of-two size: scalar block-table reads and K rows
    // through one buffer descriptor per block.  The round loop is instantiated once per case.
    auto load = [&](int r, Buf &b, auto scal) {
        constexpr bool SCAL = decltype(scal)::value;
        const int wbase = r * RTOK + wave * WTOK;
        int vt[4 * NT], vblk[4 * NT];
#pragma unroll
        for (int j = 0; j < 4 * NT; ++j) vt[j] = t0 + min(wbase + rgrp + 4 * j, n - 1);
#pragma unroll
        for (int j = 0; j < 4 * NT; ++j) vt_keep[j] = vt[j];
        if (fuse) b.knew = ld16(k_new + new_row + col * 8);  // issued before the K rows: covered by their wait
        if (SCAL) {
            // the wave's WTOK tokens touch at most two blocks: two scalar block-table reads (scalar cache,
            // their own wait counter), then a per-lane select
            const int b0 = __builtin_amdgcn_readfirstlane((t0 + min(wbase, n - 1)) >> bs_shift);
            const int b1 = __builtin_amdgcn_readfirstlane((t0 + min(wbase + WTOK - 1, n - 1)) >> bs_shift);
            const int p0 = bt[b0], p1 = bt[b1];
#pragma unroll
            for (int j = 0; j < 4 * NT; ++j) vblk[j] = (vt[j] >> bs_shift) == b0 ? p0 : p1;
            kb0_blk = b0;
            krs0 = __builtin_amdgcn_make_buffer_rsrc((void *)(kbase + (long)p0 * blk_stride), (short)0,
                                                     block_size * HD * 2, 0x00020000);
            krs1 = __builtin_amdgcn_make_buffer_rsrc((void *)(kbase + (long)p1 * blk_stride), (short)0,
                                                     block_size * HD * 2, 0x00020000);
        } else {
            // all block-table reads first (independent), then all K/V reads
#pragma unroll
            for (int j = 0; j < 4 * NT; ++j) vblk[j] = bt[blk_index<POW2>(vt[j], block_size, bs_shift)];
        }
        // K: instruction j fills rows 4j..4j+3 of the slice (1 KB); lane l writes physical chunk l % 16 of row
        // 4j + l / 16, so it reads the logical chunk that the XOR swizzle puts there.  The four rows of an
        // instruction share a block (block sizes are multiples of 4 on this path), whose descriptor is picked per
        // instruction; other block sizes take per-lane addresses.  Nontemporal, as the V rows.
        if (SCAL) {
            const int wb = __builtin_amdgcn_readfirstlane(wbase);
#pragma unroll
            for (int j = 0; j < 4 * NT; ++j) {
                const int kch = col ^ ((rgrp + 4 * j) & 15);
                const int u = t0 + min(wb + 4 * j, n - 1);  // the instruction's first row (wave-uniform)
                const int voff = ((vt[j] & (block_size - 1)) * HD + kch * 8) * 2;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    (u >> bs_shift) == kb0_blk ? krs0 : krs1,
                    (__attribute__((address_space(3))) void *)&k_lds_flat[(wave * WTOK + 4 * j) * HD], 16, voff, 0,
                    0, LLMGEN_CPOL_NT);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4 * NT; ++j) {
                const int kch = col ^ ((rgrp + 4 * j) & 15);
                const int off = vt[j] - blk_index<POW2>(vt[j], block_size, bs_shift) * block_size;
                const long row = (long)vblk[j] * blk_stride + (long)off * HD + kch * 8;
                __builtin_amdgcn_global_load_lds(
                    (const __attribute__((address_space(1))) void *)(kbase + row),
                    (__attribute__((address_space(3))) void *)&k_lds_flat[(wave * WTOK + 4 * j) * HD], 16, 0,
                    LLMGEN_CPOL_NT);
            }
        }
        // the V loads below must be issued after these: compute() waits for the K rows by counting the V loads
        // still outstanding (vmcnt(4 NT)); the compiler does not order LDS-DMA writes against LDS reads itself
        __builtin_amdgcn_sched_barrier(0);
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
        // ---- this wave's K rows in its LDS slice, then the MFMA B fragments out of it (tile tau, chunk c =
        //      dims c*32 + rgrp*8 of token tau*16 + col); the XOR swizzle keeps both directions conflict-free ----
        // vmcnt(4 NT): the K rows (issued before the 4 NT V loads) have landed
        __builtin_amdgcn_s_waitcnt(LLMGEN_WAIT_VMCNT(4 * NT));
        if (fuse) {  // the step's own token: its row comes from k_new, not from the slot being written
#pragma unroll
            for (int j = 0; j < 4 * NT; ++j) {
                const int tok = rgrp + 4 * j;
                if (vt_keep[j] == ctx - 1) k_lds[wave][tok][col ^ (tok & 15)] = b.knew;
            }
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
    if (POW2 && block_size >= WTOK) {
        for (int r = 0; r < rounds; ++r) {
            load(r, buf, std::true_type{});
            compute(r, buf);
        }
    } else {
        for (int r = 0; r < rounds; ++r) {
            load(r, buf, std::false_type{});
            compute(r, buf);
        }
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
    int &s_last = sm.last;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int *cnt = counters + (long)s * nkv + kvh;
    if (tid == 0) s_last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == np - 1;
    __syncthreads();
    if (!s_last) return;
    // acquire at agent scope: the other workgroups' partials, published before their ticket increments, are read
    // after this point (the loads below are agent-scope atomics as well)
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // These device-coherent loads are served from memory, so the merge is written to pay few load latencies (read
    // one part at a time, a 32-part merge took ~30 us).  Up to MB parts: each output loads the (m, l, o) of all
    // parts at once.  More parts: the whole workgroup first loads every (m, l) of the np parts and G heads into the
    // LDS that the wave merge above has finished with, then each output reads its o values in batches of MB2
    // parts, all loads of a batch issued before any is used.  Either way the arithmetic and its order are those of
    // a part-by-part loop: M = the max over the parts, then w = 2^(m_p - M), num += w o_p, den += w l_p for
    // p = 0, 1, ...
    constexpr int MB = 16, MB2 = 32;
    auto ld = [](const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    float *mlb = &o_lds[0][0][0];  // [g][p][m, l]
    const bool staged = np > MB && np * 2 <= W * HD;
    if (staged) {
        for (int i = tid; i < G * np; i += NTH) {
            const int g = i / np, p = i - g * np;
            const float *ml = part_ml + ((long)s * nq + (long)kvh * G + g) * max_parts * 2 + 2 * p;
            mlb[2 * i] = ld(ml);
            mlb[2 * i + 1] = ld(ml + 1);
        }
        __syncthreads();
    }
    for (int idx = tid; idx < G * HD; idx += NTH) {
        const int g = idx / HD, d = idx % HD;
        const long h = (long)kvh * G + g;
        const float *ml = part_ml + ((long)s * nq + h) * max_parts * 2;
        const float *po = part_o + ((long)s * nq + h) * max_parts * HD + d;
        float M = -INFINITY, num = 0.f, den = 0.f;
        if (np <= MB) {
            float mv[MB], lv[MB], ov[MB];
#pragma unroll
            for (int j = 0; j < MB; ++j) {
                const bool ok = j < np;
                mv[j] = ok ? ld(ml + 2 * j) : -INFINITY;
                lv[j] = ok ? ld(ml + 2 * j + 1) : 0.f;
                ov[j] = ok ? ld(po + (long)j * HD) : 0.f;
            }
#pragma unroll
            for (int j = 0; j < MB; ++j) M = fmaxf(M, mv[j]);
#pragma unroll
            for (int j = 0; j < MB; ++j) {
                if (j < np) {
                    const float w = fast_exp2(mv[j] - M);
                    num += w * ov[j];
                    den += w * lv[j];
                }
            }
        } else if (staged) {
            const float *mlg = mlb + 2 * g * np;
            for (int p = 0; p < np; ++p) M = fmaxf(M, mlg[2 * p]);
            for (int p0 = 0; p0 < np; p0 += MB2) {
                float ov[MB2];
#pragma unroll
                for (int j = 0; j < MB2; ++j) ov[j] = p0 + j < np ? ld(po + (long)(p0 + j) * HD) : 0.f;
#pragma unroll
                for (int j = 0; j < MB2; ++j) {
                    if (p0 + j < np) {
                        const float w = fast_exp2(mlg[2 * (p0 + j)] - M);
                        num += w * ov[j];
                        den += w * mlg[2 * (p0 + j) + 1];
                    }
                }
            }
        } else {  // more parts than the LDS holds: part by part
            for (int p = 0; p < np; ++p) M = fmaxf(M, ld(ml + 2 * p));
            for (int p = 0; p < np; ++p) {
                const float w = fast_exp2(ld(ml + 2 * p) - M);
                num += w * ld(po + (long)p * HD);
                den += w * ld(ml + 2 * p + 1);
            }
        }
        out[((long)s * nq + h) * HD + d] = __builtin_bit_cast(bf16_t, (__bf16)(num / den));
    }
    if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace llmgen_decode
