// mixed.hip -- one launch for a mixed chunked-prefill + decode step (gfx950).
//
// A mixed step holds two kinds of work that want different parts of the chip: query tiles of prefill chunks
// (MFMA-bound, prefill_kernel.h) and decode rows, segments with one query row (HBM-bound, decode_kernel.h).  Run
// as two kernels on two streams, they hardly overlap: the command processor dispatches one kernel's workgroups
// before the other's, the decode-row grid must cover every tile of the list (which tiles are single rows is
// device data), and the cross-stream fork and join cost 12-17 us per step on MI355X.  This kernel gives each of
// its workgroups one of the two roles instead, so a step is one launch on one stream and the grid order decides
// how the dispatcher hands out the work.
//
// Roles come in groups of nkv workgroups (one per KV head, so every workgroup of one KV head lands on the same
// XCD, as in the separate kernels), in a repeating pattern of nine prefill groups then twenty-three decode-row
// groups while both kinds last, then whatever is left.  An XCD hands consecutive workgroups to its CUs in turn,
// so a pattern whose period divides the XCD's 32 CUs gives each CU one role: 9 of every 32 CUs run prefill units
// (two per CU, as the prefill kernel alone) and the rest stream decode rows, which need the memory system more
// than compute units.  On c4 (8 chunks of 512 rows beside 248 decode rows) per-workgroup timelines show both roles
// ending within a few microseconds of each other: 188.6 us, against 227 us for the two-kernel form, 165 us for
// the decode rows alone and 54 us for the chunks alone.  Measured alternatives: prefill first (its units fill
// every CU and the decode rows wait: 229 us), one-to-one alternation (201 us), blocks of 32 groups so that every
// CU holds one workgroup of each role (200 us: a decode row beside a prefill unit streams slower than two decode
// rows), and other prefill shares (same box: 1:3 190.4 us, 5:11 190.0 us, 3:5 190.8 us).  Within each role the work goes
// heaviest first: prefill units from the end of the multi-row part of the list (the executor lists tiles lightest
// first) and decode rows longest context first.
//
// The host passes the number of single-row segments and lists them first (llmgen_fill_meta does), which sizes
// the two parts of the grid.  The roles still check each tile: a multi-row tile found in the decode part runs
// the prefill work and a single-row tile found in the prefill part runs the decode work, so a list in another
// order gives the same result, only later.
#include "decode_kernel.h"
#include "hip_common.h"
#include "prefill_kernel.h"

#include <algorithm>

namespace {

using llmgen_decode::decode_split_body;
using llmgen_decode::DecodeLds;
using llmgen_prefill::prefill_body;
using llmgen_prefill::PrefillLds;

constexpr int MIX_NW = 4;  // waves per workgroup, both roles: prefill units of two heads, decode rows of 64-token
                           // wave rounds
constexpr int MIX_NT = 4;
constexpr int MIX_PF = 9, MIX_DEC = 23;  // role pattern: prefill groups, then decode-row groups, per period
constexpr int MIX_PIECES_MAX = 8, MIX_PIECE_TILES = 16;  // prefill units split over pieces (few long units)

template <int G>
constexpr size_t mixed_lds_bytes() {
    return sizeof(DecodeLds<G, MIX_NT, MIX_NW>) > sizeof(PrefillLds<MIX_NW, 1>) ? sizeof(DecodeLds<G, MIX_NT, MIX_NW>)
                                                                                : sizeof(PrefillLds<MIX_NW, 1>);
}

// G = query heads per KV head (2 or 4); POW2 = power-of-two block size (decode rows); MODE = prefill DMA mode.
// n_pf = number of multi-row tiles, at the end of the list (tiles [n_rows, n_rows + n_pf)); n_rows = number of
// single-row tiles at its front.  Grid: n_pf * nkv * (G / 2) prefill workgroups and n_rows * nkv decode ones,
// interleaved as described at the top.
template <int G, bool POW2, int MODE>
__global__ void __launch_bounds__(64 * MIX_NW) __attribute__((amdgpu_waves_per_eu(2)))
    attn_mixed_kernel(bf16_t *__restrict__ out, const bf16_t *__restrict__ q, const bf16_t *__restrict__ kc,
                      const bf16_t *__restrict__ vc, const int *__restrict__ block_tables,
                      const int *__restrict__ ctx_lens, const int *__restrict__ cu_q,
                      const int *__restrict__ tile_seq, const int *__restrict__ tile_q0, int n_rows, int n_pf,
                      int nq, int nkv, int max_blocks, int block_size, int bs_shift, float scale_log2, int P,
                      float *__restrict__ part, int *__restrict__ counters) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[mixed_lds_bytes<G>()];
    __shared__ int s_last;
    constexpr int HG = G / 2;  // prefill head groups of two heads
    const long n_units = (long)n_pf * nkv * HG;
    const long n_pf_wg = n_units * P;
    // role and index of this workgroup: groups of nkv, periods of MIX_PF prefill groups then MIX_DEC decode groups
    // while both last
    long b;
    {
        const long pg = n_pf_wg / nkv, dg = n_rows, g = blockIdx.x / nkv, j = blockIdx.x % nkv;
        const long periods = min(pg / MIX_PF, dg / MIX_DEC);
        constexpr int PER = MIX_PF + MIX_DEC;
        long pf_idx = -1, dec_idx = -1;  // group index within the role
        if (g < periods * PER) {
            const long k = g / PER, r = g % PER;
            if (r < MIX_PF) pf_idx = k * MIX_PF + r;
            else dec_idx = k * MIX_DEC + (r - MIX_PF);
        } else {
            const long rest = g - periods * PER, pf_left = pg - periods * MIX_PF;
            if (rest < pf_left) pf_idx = periods * MIX_PF + rest;
            else dec_idx = periods * MIX_DEC + (rest - pf_left);
        }
        b = pf_idx >= 0 ? pf_idx * nkv + j : n_pf_wg + dec_idx * nkv + j;
    }
    auto prefill = [&](const int *ts, const int *tq, int n_list, int bid) {
        prefill_body<MIX_NW, MODE, 1>(out, q, kc, vc, block_tables, ctx_lens, cu_q, ts, tq, n_list, nq, nkv, G, HG,
                                      max_blocks, block_size, bs_shift, scale_log2, bid, lds);
    };
    auto decode = [&](const int *ts, int n_list, int kvh, int by) {
        decode_split_body<G, MIX_NT, POW2, false, MIX_NW>(out, nullptr, nullptr, q, kc, vc, block_tables, ctx_lens,
                                                          nq, nkv, max_blocks, block_size, bs_shift, scale_log2,
                                                          1 << 30, 1, 1, nullptr, cu_q, ts, nullptr, nullptr,
                                                          nullptr, nullptr, nullptr, kvh, by, 0, n_list, lds);
    };
    if (b < n_pf_wg) {
        // prefill part: piece `piece` of unit `bid` of the list's multi-row tiles, walked from the end
        const int *ts = tile_seq + n_rows, *tq = tile_q0 + n_rows;
        const int bid = (int)(b % n_units), piece = (int)(b / n_units), kvh = bid % nkv, rest = bid / nkv;
        const int t = n_pf - 1 - rest / HG;
        const int s = ts[t];
        const int q_len = cu_q[s + 1] - cu_q[s];
        if (q_len == 1) {  // a single-row tile out of place: the decode work, once per KV head
            if (piece == 0 && rest % HG == 0) decode(ts, n_pf, kvh, rest / HG);
            return;
        }
        // A launch with few prefill units (P > 1) splits each long unit's key tiles: a unit of n key tiles keeps
        // min(P, n / 16) pieces, each a contiguous equal share, and the last piece to finish merges them in piece
        // order from the library's scratch (the pieces kernel's scheme); shorter units run whole, as P = 1 does.
        const int ctx = ctx_lens[s];
        const int n = ctx >= q_len ? (ctx - q_len + min(tq[t] + llmgen_prefill::BQ, q_len) + llmgen_prefill::BK - 1) /
                                         llmgen_prefill::BK
                                   : 0;
        const int pe = P > 1 ? max(1, min(P, n / MIX_PIECE_TILES)) : 1;
        if (piece >= pe) return;
        if (pe == 1) {
            prefill(ts, tq, n_pf, bid);
            return;
        }
        const int j0 = (int)((long)piece * n / pe), j1 = (int)((long)(piece + 1) * n / pe);
        float *base = part + (long)bid * P * llmgen_prefill::PART_FLOATS;
        prefill_body<MIX_NW, MODE, 1, true>(out, q, kc, vc, block_tables, ctx_lens, cu_q, ts, tq, n_pf, nq, nkv, G,
                                            HG, max_blocks, block_size, bs_shift, scale_log2, bid, lds, j0, j1,
                                            base + (long)piece * llmgen_prefill::PART_FLOATS);
        __builtin_amdgcn_s_waitcnt(0);  // the partial's device-coherent stores complete before the ticket
        __syncthreads();
        if (threadIdx.x == 0)
            s_last = __hip_atomic_fetch_add(counters + bid, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == pe - 1;
        __syncthreads();
        if (!s_last) return;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        llmgen_prefill::prefill_merge_store_n<MIX_PIECES_MAX>(out, cu_q, ts, tq, n_pf, nq, nkv, G, HG, bid, base, pe);
        if (threadIdx.x == 0) __hip_atomic_store(counters + bid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // decode part: (row, kv head), longest context first
    const int d = (int)(b - n_pf_wg), kvh = d % nkv, by = d / nkv;
    const int s = tile_seq[n_rows - 1 - by];
    if (cu_q[s + 1] - cu_q[s] != 1) {  // a multi-row tile out of place: its prefill units, one head group at a time
        for (int h = 0; h < HG; ++h) {
            prefill(tile_seq, tile_q0, n_rows, (by * HG + h) * nkv + kvh);
            __syncthreads();  // the next unit reuses the LDS stages
        }
        return;
    }
    decode(tile_seq, n_rows, kvh, by);
}

template <int G>
void launch_mixed_g(int mode, bool pow2, long grid, bf16_t *out, const bf16_t *q, const bf16_t *kc, const bf16_t *vc,
                    const int *bt, const int *ctx, const int *cu_q, const int *tile_seq, const int *tile_q0,
                    int n_rows, int n_pf, int nq, int nkv, int max_blocks, int block_size, int bs_shift, float sl2,
                    int P, float *part, int *counters) {
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * MIX_NW), 0, g_llmgen_stream, out, q, kc, vc, bt, ctx,
                           cu_q, tile_seq, tile_q0, n_rows, n_pf, nq, nkv, max_blocks, block_size, bs_shift, sl2, P,
                           part, counters);
    };
    using namespace llmgen_prefill;
    if (pow2) {
        if (mode == DMA_BLOCK) go(attn_mixed_kernel<G, true, DMA_BLOCK>);
        else if (mode == DMA_ROW4) go(attn_mixed_kernel<G, true, DMA_ROW4>);
        else go(attn_mixed_kernel<G, true, DMA_FLAT>);
    } else {
        if (mode == DMA_ROW4) go(attn_mixed_kernel<G, false, DMA_ROW4>);
        else go(attn_mixed_kernel<G, false, DMA_FLAT>);
    }
}

}  // namespace

// Called by hip_attn_prefill_rows for a mixed step at G = 2 or 4 whose caller passed its single-row count (> 0):
// the whole step in one launch.  Returns false (nothing launched) for shapes this kernel does not take.
bool llmgen_mixed_step(bf16_t *out, const bf16_t *q, const bf16_t *k_cache, const bf16_t *v_cache,
                       const int *block_tables, const int *ctx_lens, const int *cu_q, const int *tile_seq,
                       const int *tile_q0, int n_tiles, int single_rows, int nq, int nkv, int max_blocks,
                       int block_size, float scale, int dma_mode) {
    const int G = nq / nkv;
    if ((G != 2 && G != 4) || single_rows <= 0 || single_rows > n_tiles) return false;
    const int bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
    const int n_pf = n_tiles - single_rows;
    // few prefill units (at most half a unit per CU): up to MIX_PIECES_MAX pieces each
    const long units = (long)n_pf * (G / 2) * nkv;
    float *part = nullptr;
    int *counters = nullptr;
    int P = 1;
    if (units > 0 && units * 2 <= llmgen_num_cus() && llmgen_prefill_scratch(&part, &counters, units))
        P = (int)std::min<long>({(long)MIX_PIECES_MAX, 2L * llmgen_num_cus() / units, 512L / units});
    if (P < 2) P = 1;
    const long grid = ((long)n_pf * (G / 2) * P + single_rows) * nkv;
    const float sl2 = scale * LLMGEN_LOG2E;
    if (G == 2)
        launch_mixed_g<2>(dma_mode, bs_shift >= 0, grid, out, q, k_cache, v_cache, block_tables, ctx_lens, cu_q,
                          tile_seq, tile_q0, single_rows, n_pf, nq, nkv, max_blocks, block_size, bs_shift, sl2, P,
                          part, counters);
    else
        launch_mixed_g<4>(dma_mode, bs_shift >= 0, grid, out, q, k_cache, v_cache, block_tables, ctx_lens, cu_q,
                          tile_seq, tile_q0, single_rows, n_pf, nq, nkv, max_blocks, block_size, bs_shift, sl2, P,
                          part, counters);
    return true;
}
