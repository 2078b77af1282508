// prefill_kernel.h -- the FA2 prefill workgroup (gfx950), shared by the prefill launcher (prefill.hip) and the
// mixed-step kernel (mixed.hip).  What it computes and how is described in prefill.hip.
#pragma once
#include "hip_common.h"

#include <math.h>

#include <type_traits>

namespace llmgen_prefill {

constexpr int HD = 128;
constexpr int BQ = 64;               // query rows per tile (the value hip_attn_prefill_tile returns)
constexpr int BK = 64;               // keys per LDS tile
constexpr int TILE = BK * HD;        // bf16 elements of one K (or V) tile: 16 KB, rows of 256 B, no padding
constexpr float RESCALE_LOG2 = 8.f;  // lazy-rescale threshold (log2 units) of the tiles that take a row max
constexpr int KPF = 3;               // K fragment pairs read ahead of the S MFMAs
constexpr int VPF = 4;               // V^T fragments read ahead of the PV MFMAs

// DMA addressing: BLOCK = block_size is a power of two and a multiple of BK (a K/V tile lies inside one block:
// one descriptor per tile); ROW4 = block_size % 4 == 0 (the four rows of one DMA instruction lie inside one
// block: one descriptor per instruction); FLAT = any block size (global_load_lds with per-lane addresses).
enum DmaMode { DMA_FLAT = 0, DMA_BLOCK = 1, DMA_ROW4 = 2 };
constexpr unsigned BUF_WORD3 = 0x00020000u;  // raw buffer descriptor, 32-bit data format

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

// element offset of (row, 16-byte chunk) in a swizzled tile
__device__ __forceinline__ int k_off(int row, int chunk) { return row * HD + ((chunk ^ (row & 15)) << 3); }
__device__ __forceinline__ int v_off(int row, int chunk) { return row * HD + ((chunk ^ ((row << 2) & 15)) << 3); }

__device__ __forceinline__ s16x4_t ds_read_tr(const bf16_t *p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)p);
}

__device__ __forceinline__ void dma16(const bf16_t *gsrc, bf16_t *ldst) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)gsrc,
                                     (__attribute__((address_space(3))) void *)ldst, 16, 0, 0);
}

// 16 bytes per lane from (descriptor base + byte offset voff) into LDS at ldst (wave-uniform) + 16 * lane
__device__ __forceinline__ void bufdma16(__amdgpu_buffer_rsrc_t rs, int voff, bf16_t *ldst) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)ldst, 16, voff, 0, 0, 0);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const bf16_t *base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, bytes, BUF_WORD3);
}

// NW = waves per workgroup; MODE = DmaMode; KS = key groups.  The waves form KS key groups of NW / KS waves, two
// per head (rows 0-31 and 32-63 of the tile).  With KS = 2 group k takes the key tiles k, k + 2, k + 4, ... into
// its own LDS stages, so a unit of n key tiles takes ceil(n / 2) iterations; the two groups' (m, l, O) are merged
// through LDS at the end in a fixed order (bit-reproducible, and a tile's keys always go to the same group).
template <int NW, int KS>
struct PrefillLds {
    static constexpr bool ONE_STAGE = NW == 2;  // 2-wave workgroups (G = 1) keep one stage
    // stage buffers: one 64-key K and V tile per key group
    __attribute__((aligned(16))) bf16_t K0[KS * TILE];
    __attribute__((aligned(16))) bf16_t V0[KS * TILE];
    __attribute__((aligned(16))) bf16_t K1[ONE_STAGE ? 8 : KS * TILE];
    __attribute__((aligned(16))) bf16_t V1[ONE_STAGE ? 8 : KS * TILE];
};

// Split-K partial result of one unit (4 waves x 64 lanes): per wave, the unnormalised O^T accumulator values
// [64][lane], then m [lane] and l [lane] (before the half-wave sum).
constexpr int PART_WAVE_FLOATS = 66 * 64;
constexpr int PART_FLOATS = 4 * PART_WAVE_FLOATS;

// The prefill workgroup's work, as a device function so that other kernels can run it as one of their workgroup
// roles: bid plays the part of the 1-D grid position, lds holds a PrefillLds<NW, KS>.  With SK (one key group,
// four waves) the workgroup runs only key tiles [j0, j1) of the unit (j1 < 0: to the unit's last tile); if part
// is not null it leaves the unit's partial result there (device-coherent stores, PART_FLOATS floats) instead of
// storing rows.
template <int NW, int MODE, int KS, bool SK = false>
__device__ __forceinline__ void prefill_body(bf16_t *__restrict__ out, const bf16_t *__restrict__ q, const bf16_t *__restrict__ kc,
                        const bf16_t *__restrict__ vc, const int *__restrict__ block_tables,
                        const int *__restrict__ ctx_lens, const int *__restrict__ cu_q,
                        const int *__restrict__ tile_seq, const int *__restrict__ tile_q0, int n_tiles, int nq,
                        int nkv, int G, int head_groups, int max_blocks, int block_size, int bs_shift,
                        float scale_log2, int bid, unsigned char *lds, int j0 = 0, int j1 = 0,
                        float *__restrict__ part = nullptr) {
    static_assert(!SK || (KS == 1 && (NW == 4 || NW == 2)), "key ranges are for 4- or 2-wave, one-group workgroups");
    constexpr int NWG = NW / KS;     // waves per key group
    constexpr int LOADS = 16 / NWG;  // 4-row DMA instructions per wave per tile, for K and for V each

    // 2-wave workgroups (G = 1) keep one stage: 32 KB of LDS lets four of them share a CU (two waves per SIMD)
    constexpr bool ONE_STAGE = NW == 2;
    PrefillLds<NW, KS> &sm = *reinterpret_cast<PrefillLds<NW, KS> *>(lds);
    auto &K0 = sm.K0;
    auto &V0 = sm.V0;
    auto &K1 = sm.K1;
    auto &V1 = sm.V1;

    const int kvh = bid % nkv;
    const int rest = bid / nkv;
    const int hg = rest % head_groups;
    const int tile = n_tiles - 1 - rest / head_groups;
    const int s = tile_seq[tile], q0 = tile_q0[tile];
    const int q_beg = cu_q[s], q_len = cu_q[s + 1] - q_beg, ctx = ctx_lens[s];
    // The key group is taken through readfirstlane (it is uniform across the wave), so that the key-tile index
    // derived from it, and with it the DMA descriptors, stay in scalar registers; otherwise each DMA is wrapped in a
    // loop over distinct descriptor values.  The wave index itself stays a plain vector value: taking it through
    // readfirstlane as well measures slower (c5p 2104 against 1931 us, c3 85.6 against 82.2 us; only the
    // compiler's schedule differs).
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = tid >> 6;
    const int kg = KS == 1 ? 0 : __builtin_amdgcn_readfirstlane(wave) / NWG, wl = wave % NWG;
    const int g = hg * (NWG / 2) + (wl >> 1);    // head within the KV group
    const int head = kvh * G + g;
    const int r0 = q0 + (wl & 1) * 32;  // first query row (within the segment) of this wave
    const int l32 = lane & 31, hh = lane >> 5;

    if (q_len == 1) return;  // single-row segments (decode rows of a mixed step): streamed by the decode kernel
    if (ctx < q_len) {       // padding sequence: zero rows, no keys (cpu/attention.zig:80-83)
        const int row = r0 + l32;
        if (row < q_len) {
            bf16_t *o = out + ((long)(q_beg + row) * nq + head) * HD + hh * 64;
            for (int d = 0; d < 64; d += 8) *reinterpret_cast<u32x4_t *>(o + d) = u32x4_t{0, 0, 0, 0};
        }
        return;
    }

    const int *bt = block_tables + (long)s * max_blocks;
    const long blk_stride = (long)nkv * block_size * HD;
    const long head_off = (long)kvh * block_size * HD;
    const int base_pos = ctx - q_len;                // position of segment row 0
    const int kend = base_pos + min(q0 + BQ, q_len);  // keys needed by the whole tile
    const int n_all = (kend + BK - 1) / BK;  // key tiles of the unit
    const int n_iter = SK && j1 >= 0 ? min(j1, n_all) : n_all;  // SK: the end of this workgroup's key range
    const int it_base = SK ? j0 : 0;                             // first key tile
    const int n_super = SK ? n_iter - j0 : (n_iter + KS - 1) / KS;  // iterations: one tile per key group each

    // ---- Q fragments (B operand): lane holds row r0+l32, dims c*16 + hh*8 .. +8 ----
    const int my_row = r0 + l32;
    const bool row_valid = my_row < q_len;
    const int my_pos = base_pos + my_row;
    bf16x8_t qf[8];
    {
        const int rq = min(my_row, q_len - 1);
        const bf16_t *qp = q + ((long)(q_beg + rq) * nq + head) * HD + hh * 8;
#pragma unroll
        for (int c = 0; c < 8; ++c) qf[c] = __builtin_bit_cast(bf16x8_t, ld16(qp + c * 16));
    }
    const bool wave_active = r0 < q_len;
    const int wave_pos_min = base_pos + r0;
    const int wave_pos_max = base_pos + min(r0 + 31, q_len - 1);
    const bool wave_has_pad = r0 + 31 >= q_len;

    // ---- DMA of this group's K/V tile of iteration `it` into (Kd, Vd): wave instruction i covers rows
    //      4*(wl + NWG*i) .. +3; lane writes row + lane/16, physical chunk lane%16, so it reads the logical chunk
    //      that swizzles onto it ----
    const int drow = lane >> 4, dchunk = lane & 15;
    auto issue = [&](int it, bf16_t *Kd, bf16_t *Vd) {
        const int ti = it_base + it * KS + kg;
        if (KS > 1 && ti >= n_iter) return;  // the unit's last iteration has no tile for this group
        Kd += kg * TILE;
        Vd += kg * TILE;
        const int kb0 = ti * BK;
        const int last = kend - 1 - kb0;  // keys past kend reread the last valid key (finite data)
        __amdgpu_buffer_rsrc_t krs, vrs;
        if (MODE == DMA_BLOCK) {  // the whole tile lies in one block: one descriptor pair per tile
            const int phys = bt[__builtin_amdgcn_readfirstlane(kb0 >> bs_shift)];
            const long kbase = (long)phys * blk_stride + head_off + (long)(kb0 & (block_size - 1)) * HD;
            krs = make_rsrc(kc + kbase, TILE * 2);
            vrs = make_rsrc(vc + kbase, TILE * 2);
        }
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int rbase = 4 * (wl + NWG * i);
            const int r = rbase + drow;
            const int kswz = (dchunk ^ (r & 15)) << 4, vswz = (dchunk ^ ((r << 2) & 15)) << 4;  // bytes
            if (MODE == DMA_BLOCK) {
                const int voff = min(r, last) * (HD * 2);
                bufdma16(krs, voff + kswz, Kd + rbase * HD);
                bufdma16(vrs, voff + vswz, Vd + rbase * HD);
            } else if (MODE == DMA_ROW4) {
                // rows rbase..rbase+3 (clamped to last) lie in one block: key t0 + d, d in 0..3
                const int t0 = __builtin_amdgcn_readfirstlane(kb0 + min(rbase, last));
                const int bi = bs_shift >= 0 ? (t0 >> bs_shift) : t0 / block_size;
                const long base = (long)bt[bi] * blk_stride + head_off + (long)(t0 - bi * block_size) * HD;
                const int voff = (min(r, last) - min(rbase, last)) * (HD * 2);
                bufdma16(make_rsrc(kc + base, 4 * HD * 2), voff + kswz, Kd + rbase * HD);
                bufdma16(make_rsrc(vc + base, 4 * HD * 2), voff + vswz, Vd + rbase * HD);
            } else {
                const int t = kb0 + min(r, last);
                const int bi = t / block_size;
                const long src = (long)bt[bi] * blk_stride + head_off + (long)(t - bi * block_size) * HD;
                dma16(kc + src + (kswz >> 1), Kd + rbase * HD);
                dma16(vc + src + (vswz >> 1), Vd + rbase * HD);
            }
        }
    };

    f32x16_t o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    // per-lane LDS offsets of the V^T fragment reads (ds_read_b64_tr_b16): 16-lane group g4, lane i = 4j + m;
    // the fragment's k-slots (hh*8 + e) are keys kc16*16 + (e/4)*8 + hh*4 + e%4, so the two reads of a fragment
    // take keys hh*4 + j (+8) and dims db*32 + (g4&1)*16 + 4m .. +3
    int voff[4];
    {
        const int g4 = lane >> 4, i = lane & 15, j = i >> 2, m = i & 3;
        const int key = (g4 >> 1) * 4 + j;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const int dim = db * 32 + (g4 & 1) * 16 + 4 * m;
            voff[db] = v_off(key, dim >> 3) + (dim & 7);
        }
    }

    // per-lane LDS offsets of the K fragment reads (row l32, logical chunk 2c + hh); row 32 + l32 has the same
    // swizzle, so its offset is a constant 32 rows further
    int koff[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) koff[c] = k_off(l32, 2 * c + hh);

    // One 64-key tile for this wave: S^T = K Q^T, online softmax (base 2, scale folded into one FMA), O^T += V^T P^T.
    auto tile_step = [&](int kb0, const bf16_t *Ks, const bf16_t *Vs, auto masked) {
        constexpr bool MASK = decltype(masked)::value;
        f32x16_t sacc[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
        bf16x8_t ka[8], kb[8];  // K fragments of keys 0-31 and 32-63, read KPF steps ahead
#pragma unroll
        for (int c = 0; c < KPF; ++c) {
            ka[c] = *reinterpret_cast<const bf16x8_t *>(Ks + koff[c]);
            kb[c] = *reinterpret_cast<const bf16x8_t *>(Ks + koff[c] + 32 * HD);
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {  // two independent accumulation chains interleaved
            if (c + KPF < 8) {
                ka[c + KPF] = *reinterpret_cast<const bf16x8_t *>(Ks + koff[c + KPF]);
                kb[c + KPF] = *reinterpret_cast<const bf16x8_t *>(Ks + koff[c + KPF] + 32 * HD);
            }
            sacc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[c], qf[c], sacc[0], 0, 0, 0);
            sacc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kb[c], qf[c], sacc[1], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);  // keep the read-ahead order
        }
        // V^T fragment i = kc16 * 4 + db: keys kc16*16 + hh*4 + j (+8), dims db*32 + ...; the first VPF do not
        // depend on P and are read before the softmax
        bf16x8_t va[16];
        auto vread = [&](int i) {
            const bf16_t *vp = Vs + (i >> 2) * 16 * HD + voff[i & 3];
            const s16x4_t lo = ds_read_tr(vp);           // keys hh*4 + j
            const s16x4_t hi = ds_read_tr(vp + 8 * HD);  // keys 8 + hh*4 + j
            va[i] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        };
#pragma unroll
        for (int i = 0; i < VPF; ++i) vread(i);
        __builtin_amdgcn_sched_barrier(0);
        // lane holds row my_row, keys kb0 + kb*32 + (r/4)*8 + hh*4 + r%4 (raw dot products)
        if (MASK) {
            // key kb0 + off + hh*4 is masked when it lies past the row's position (or the row is padding): one
            // compare of the compile-time offset against a per-lane limit, then one select, per score
            const int lim = row_valid ? my_pos - kb0 - hh * 4 : -1;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int off = kb * 32 + (r >> 2) * 8 + (r & 3);
                    if (off > lim) sacc[kb][r] = -INFINITY;
                }
        }
        auto row_max = [&]() {
            float mx = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb][r]);
            return fmaxf(mx, lane_xor(mx, 32)) * scale_log2;  // scale > 0 commutes with max
        };
        float lsum;
        bf16x8_t pf[4];  // B fragments for the four 16-key steps of P V
        auto probs = [&](float m_use) {
            lsum = 0.f;
#pragma unroll
            for (int kc16 = 0; kc16 < 4; ++kc16) {
                const int kb = kc16 >> 1, half = kc16 & 1;
                float p[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    p[e] = fast_exp2(__builtin_fmaf(sacc[kb][half * 8 + e], scale_log2, -m_use));
                    lsum += p[e];
                }
                u32x4_t w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = pack_bf16x2(p[2 * e], p[2 * e + 1]);
                pf[kc16] = __builtin_bit_cast(bf16x8_t, w);
            }
        };
        // Once every row of the wave has a finite reference m_run, the tile's probabilities are taken against
        // it without a row max: they may exceed 1 (f32 and bf16 share the exponent range, and o / l is
        // unchanged by the common factor).  Only a row sum beyond 2^64 (scores far above the reference) moves
        // the reference, recomputing the tile against the new row max.
        bool grow = false;
        float m_new = m_run, corr = 1.f;
        if (!__all(m_run > -INFINITY)) {
            const float mx = row_max();
            grow = mx > m_run + RESCALE_LOG2;
            m_new = grow ? mx : m_run;
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            corr = grow ? fast_exp2(m_run - m_use) : 1.f;
            probs(m_use);
        } else {
            probs(m_run);
            if (__any(!(lsum <= 0x1p64f))) {
                const float mx = row_max();
                grow = mx > m_run;
                m_new = grow ? mx : m_run;
                corr = grow ? fast_exp2(m_run - m_new) : 1.f;
                probs(m_new);
            }
        }
        l_run = l_run * corr + lsum;
        m_run = m_new;
        if (__any(grow)) {  // corr == 1 in rows that did not move
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[db][r] *= corr;
        }
        // ---- O^T[dim][row] += V^T P^T: four independent accumulators per 16-key step ----
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if (i + VPF < 16) vread(i + VPF);
            o[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[i], pf[i >> 2], o[i & 3], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto compute = [&](int it, const bf16_t *Ks, const bf16_t *Vs) {
        const int ti = it_base + it * KS + kg;
        const int kb0 = ti * BK;
        Ks += kg * TILE;
        Vs += kg * TILE;
        if (wave_active && ti < n_iter && kb0 <= wave_pos_max) {
            // tiles wholly below the wave's diagonal (and with no padding rows) take the unmasked path
            if (wave_has_pad || kb0 + BK - 1 > wave_pos_min)
                tile_step(kb0, Ks, Vs, std::true_type{});
            else
                tile_step(kb0, Ks, Vs, std::false_type{});
        }
    };

    // two LDS stages; the loop is unrolled twice so every DMA targets a fixed buffer (the compiler can then see
    // that the reads of one stage never wait for the DMA into the other)
    if (ONE_STAGE) {
        for (int it = 0; it < n_super; ++it) {
            issue(it, K0, V0);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();  // the tile has landed for every wave
            compute(it, K0, V0);
            __syncthreads();  // every wave is done reading it
        }
    } else {
        if (n_super > 0) issue(0, K0, V0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        for (int it = 0; it < n_super; it += 2) {
            if (it + 1 < n_super) issue(it + 1, K1, V1);
            compute(it, K0, V0);
            __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA into stage 1 has landed
            __syncthreads();                // ... and everyone's; everyone is done reading stage 0
            if (it + 1 >= n_super) break;
            if (it + 2 < n_super) issue(it + 2, K0, V0);
            compute(it + 1, K1, V1);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
    }

    if constexpr (KS == 2) {
        // ---- merge the key groups: group 1 leaves (o, m, l) in LDS (the stage buffers are free: the loop ended
        //      on a barrier), group 0 combines them with its own, lane by lane (both groups hold the same rows in
        //      the same accumulator layout, and m is equal across a row's two half-waves) ----
        float *xo = reinterpret_cast<float *>(wl < 2 ? K0 : V0) + (wl & 1) * 64 * 64;  // [64 values][64 lanes]
        float *xm = reinterpret_cast<float *>(K1) + wl * 2 * 64;                       // [m, l][64 lanes]
        if (kg == 1) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) xo[(db * 16 + r) * 64 + lane] = o[db][r];
            xm[lane] = m_run;
            xm[64 + lane] = l_run;
        }
        __syncthreads();
        if (kg == 1) return;
        const float m1 = xm[lane], l1 = xm[64 + lane];
        const float M = fmaxf(m_run, m1);
        const float Mu = M == -INFINITY ? 0.f : M;
        const float c0 = fast_exp2(m_run - Mu), c1 = fast_exp2(m1 - Mu);
        l_run = l_run * c0 + l1 * c1;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[db][r] = o[db][r] * c0 + xo[(db * 16 + r) * 64 + lane] * c1;
    }

    if constexpr (SK) {
        if (part) {  // leave the partial result (the merging workgroup reads it with device-coherent loads)
            if (!wave_active) return;
            float *pw = part + wave * PART_WAVE_FLOATS + lane;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    __hip_atomic_store(pw + (db * 16 + r) * 64, o[db][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pw + 64 * 64, m_run, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pw + 65 * 64, l_run, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
    }
    // ---- normalise and store: lane holds dims db*32 + (r/4)*8 + hh*4 + r%4 of row my_row ----
    if (!wave_active) return;
    const float l_tot = l_run + lane_xor(l_run, 32);
    if (!row_valid) return;
    const float inv = 1.f / l_tot;
    bf16_t *orow = out + ((long)(q_beg + my_row) * nq + head) * HD + hh * 4;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            u32x2_t w;
            w[0] = pack_bf16x2(o[db][rr * 4 + 0] * inv, o[db][rr * 4 + 1] * inv);
            w[1] = pack_bf16x2(o[db][rr * 4 + 2] * inv, o[db][rr * 4 + 3] * inv);
            *reinterpret_cast<u32x2_t *>(orow + db * 32 + rr * 8) = w;
        }
}

// Merge the partial results of one unit (4-wave, one-group layout of prefill_body<4, *, 1, true>): the
// log-sum-exp combination of its key-range pieces in the order given, lane by lane (each lane holds the same row
// and dims in every piece), then the normalisation and bf16 store of prefill_body.  Device-coherent loads: the
// pieces were written by other workgroups.
template <int NP>
__device__ __forceinline__ void prefill_merge_store(bf16_t *__restrict__ out, const int *__restrict__ cu_q,
                                                    const int *__restrict__ tile_seq, const int *__restrict__ tile_q0,
                                                    int n_tiles, int nq, int nkv, int G, int head_groups, int bid,
                                                    const float *const (&pieces)[NP]) {
    const int kvh = bid % nkv, rest = bid / nkv, hg = rest % head_groups;
    const int tile = n_tiles - 1 - rest / head_groups;
    const int s = tile_seq[tile], q0 = tile_q0[tile];
    const int q_beg = cu_q[s], q_len = cu_q[s + 1] - q_beg;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int head = kvh * G + hg * 2 + (wave >> 1);
    const int r0 = q0 + (wave & 1) * 32, l32 = lane & 31, hh = lane >> 5;
    if (r0 >= q_len) return;  // an inactive wave left no partial
    auto ld = [&](const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    float M = -INFINITY;
#pragma unroll
    for (int p = 0; p < NP; ++p) M = fmaxf(M, ld(pieces[p] + wave * PART_WAVE_FLOATS + 64 * 64 + lane));
    const float Mu = M == -INFINITY ? 0.f : M;
    float o[64], l = 0.f;
#pragma unroll
    for (int v = 0; v < 64; ++v) o[v] = 0.f;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const float *pw = pieces[p] + wave * PART_WAVE_FLOATS + lane;
        const float c = fast_exp2(ld(pw + 64 * 64) - Mu);
        l += ld(pw + 65 * 64) * c;
#pragma unroll
        for (int v = 0; v < 64; ++v) o[v] += ld(pw + v * 64) * c;
    }
    const float l_tot = l + lane_xor(l, 32);
    const int my_row = r0 + l32;
    if (my_row >= q_len) return;
    const float inv = 1.f / l_tot;
    bf16_t *orow = out + ((long)(q_beg + my_row) * nq + head) * HD + hh * 4;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            u32x2_t w;
            w[0] = pack_bf16x2(o[db * 16 + rr * 4 + 0] * inv, o[db * 16 + rr * 4 + 1] * inv);
            w[1] = pack_bf16x2(o[db * 16 + rr * 4 + 2] * inv, o[db * 16 + rr * 4 + 3] * inv);
            *reinterpret_cast<u32x2_t *>(orow + db * 32 + rr * 8) = w;
        }
}

// prefill_merge_store for np <= NPMAX pieces known at run time of NW-wave workgroups (two heads at NW = 4, one at
// NW = 2), laid out NW * PART_WAVE_FLOATS apart from `base`.  The
// pieces' (m, l) are read at once; then each piece's 64 accumulator values are read together (64 loads in flight)
// and folded into the running sums, piece by piece in order, as prefill_merge_store combines them.  The loop over
// the pieces stays a loop: unrolled over NPMAX with a branch per load, its code outgrew the instruction cache.
template <int NPMAX, int NW = 4>
__device__ __forceinline__ void prefill_merge_store_n(bf16_t *__restrict__ out, const int *__restrict__ cu_q,
                                                      const int *__restrict__ tile_seq,
                                                      const int *__restrict__ tile_q0, int n_tiles, int nq, int nkv,
                                                      int G, int head_groups, int bid, const float *base, int np) {
    const int kvh = bid % nkv, rest = bid / nkv, hg = rest % head_groups;
    const int tile = n_tiles - 1 - rest / head_groups;
    const int s = tile_seq[tile], q0 = tile_q0[tile];
    const int q_beg = cu_q[s], q_len = cu_q[s + 1] - q_beg;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int head = kvh * G + hg * (NW / 2) + (wave >> 1);
    const int r0 = q0 + (wave & 1) * 32, l32 = lane & 31, hh = lane >> 5;
    if (r0 >= q_len) return;  // an inactive wave left no partial
    auto ld = [&](const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    constexpr int PSTRIDE = NW * PART_WAVE_FLOATS;  // floats per piece
    const float *pw = base + wave * PART_WAVE_FLOATS + lane;
    float mv[NPMAX], lv[NPMAX];
#pragma unroll
    for (int p = 0; p < NPMAX; ++p) {
        const int pp = min(p, np - 1);  // no branch: pieces past np reread the last one and are not used
        mv[p] = ld(pw + (long)pp * PSTRIDE + 64 * 64);
        lv[p] = ld(pw + (long)pp * PSTRIDE + 65 * 64);
    }
    float M = -INFINITY;
#pragma unroll
    for (int p = 0; p < NPMAX; ++p)
        if (p < np) M = fmaxf(M, mv[p]);
    const float Mu = M == -INFINITY ? 0.f : M;
    float o[64], l = 0.f;
#pragma unroll
    for (int v = 0; v < 64; ++v) o[v] = 0.f;
    for (int p = 0; p < np; ++p) {
        float c = 0.f, lp = 0.f;
#pragma unroll
        for (int i = 0; i < NPMAX; ++i)
            if (i == p) {
                c = fast_exp2(mv[i] - Mu);
                lp = lv[i];
            }
        l += lp * c;
        const float *src = pw + (long)p * PSTRIDE;
        float x[64];
#pragma unroll
        for (int v = 0; v < 64; ++v) x[v] = ld(src + v * 64);
#pragma unroll
        for (int v = 0; v < 64; ++v) o[v] += x[v] * c;
    }
    const float l_tot = l + lane_xor(l, 32);
    const int my_row = r0 + l32;
    if (my_row >= q_len) return;
    const float inv = 1.f / l_tot;
    bf16_t *orow = out + ((long)(q_beg + my_row) * nq + head) * HD + hh * 4;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            u32x2_t w;
            w[0] = pack_bf16x2(o[db * 16 + rr * 4 + 0] * inv, o[db * 16 + rr * 4 + 1] * inv);
            w[1] = pack_bf16x2(o[db * 16 + rr * 4 + 2] * inv, o[db * 16 + rr * 4 + 3] * inv);
            *reinterpret_cast<u32x2_t *>(orow + db * 32 + rr * 8) = w;
        }
}

}  // namespace llmgen_prefill
