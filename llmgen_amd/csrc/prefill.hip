// prefill.hip -- FA2-style causal varlen attention over the paged KV cache on bf16 MFMA (gfx950, wave64).
//
// Contract: src/backend/cuda/attention/attention_v1.zig:30-48 (cuda_attn_prefill argument list) with the
// semantics of src/backend/cpu/attention.zig:64-118: sequence s owns query rows [cu_q[s], cu_q[s+1]) of q
// [T, nq, 128]; after this step it has ctx[s] keys; query j of the segment sits at position ctx - q_len + j
// and sees keys 0..pos; output bf16(softmax(scale q K^T) V); a sequence with ctx < q_len is padding and
// writes zeros.  The host tiles each segment into hip_attn_prefill_tile() rows (tile_seq, tile_q0).
//
// Design (one workgroup = one query tile x one KV head x a group of its G query heads):
//   * K and V tiles of 64 keys move HBM -> LDS with buffer_load_dwordx4 ... lds (no register staging, no VALU
//     work): each wave instruction fills four 256-byte key rows through a buffer descriptor whose base is the
//     rows' cache block.  Buffer (MUBUF) rather than FLAT-encoded global_load_lds: a FLAT load that writes LDS
//     makes the compiler wait for every LDS read in flight (lgkmcnt(0)) wherever it waits for one, which
//     serialises the fragment reads below.  Two LDS stages: tile t+1 streams in while tile t is computed, one
//     barrier per tile (one stage for the 2-wave workgroups of G = 1, so that four share a CU and hide each other's
//     DMA).  Rows are stored as 16 chunks of 16 bytes with the chunk index XOR-swizzled by the row
//     (K: row & 15, V: 4*row & 15) so the fragment reads below are bank-conflict free;
//   * each wave owns 32 query rows of one head and computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16: K
//     (ds_read_b128 from LDS, issued KPF MFMA pairs ahead of use) is the A operand, Q (registers, loaded once)
//     the B operand.  In the S^T
//     accumulator layout every lane holds 32 keys of ONE query row, so the online softmax is lane-local except
//     one exchange between the two half-waves;
//   * the probabilities are rounded to bf16 in registers and used directly as the B operand of O^T = V^T P^T
//     (the MFMA's k-slots are assigned to keys in the order the S^T accumulator holds them).  The V^T A operand
//     comes straight from the row-major V tile through ds_read_b64_tr_b16: a 16-lane group whose lane 4j+m
//     addresses four dims of key j receives, in lane i, key j's value of dim i -- the transpose happens in the
//     LDS read.  The first VPF of these reads are issued before the softmax (they do not depend on P) and the
//     rest stay VPF MFMAs ahead; scheduling barriers keep the compiler from sinking the reads back next to
//     their uses;
//   * online softmax in base 2 with scale * log2 e folded in and fp32 row state.  The first tile sets each row's
//     reference from its row max; later tiles take their probabilities against that reference without a row
//     max (a VALU chain and a half-wave exchange per tile saved) and move it only when a tile's row sum passes
//     2^64, recomputing that tile against its row max.  Causal masking only on tiles that cross a wave's
//     diagonal; tiles wholly above a wave's diagonal are skipped by that wave;
//   * grid is 1-D with the KV head fastest, so every workgroup of one KV head lands on the same XCD (8 XCDs,
//     round-robin dispatch) and its K/V tiles stay in that XCD's L2; later tiles of the list go first (the
//     executor lists tiles lightest first, so dispatch is heaviest first across sequences).
#include "hip_common.h"
#include "prefill_kernel.h"

#include <math.h>

#include <algorithm>
#include <stdlib.h>
#include <type_traits>

namespace {

using namespace llmgen_prefill;

// NW = waves per workgroup; MODE = DmaMode; KS = key groups.  One workgroup per (query tile, KV head, head group).
template <int NW, int MODE, int KS>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2)))
    attn_prefill_kernel(bf16_t *__restrict__ out, const bf16_t *__restrict__ q, const bf16_t *__restrict__ kc,
                        const bf16_t *__restrict__ vc, const int *__restrict__ block_tables,
                        const int *__restrict__ ctx_lens, const int *__restrict__ cu_q,
                        const int *__restrict__ tile_seq, const int *__restrict__ tile_q0, int n_tiles, int nq,
                        int nkv, int G, int head_groups, int max_blocks, int block_size, int bs_shift,
                        float scale_log2) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[sizeof(PrefillLds<NW, KS>)];
    prefill_body<NW, MODE, KS>(out, q, kc, vc, block_tables, ctx_lens, cu_q, tile_seq, tile_q0, n_tiles, nq, nkv, G,
                               head_groups, max_blocks, block_size, bs_shift, scale_log2, blockIdx.x, lds);
}

template <int NW, int MODE, int KS>
void launch_prefill_mode(long grid, bf16_t *out, const bf16_t *q, const bf16_t *kc, const bf16_t *vc, const int *bt,
                         const int *ctx, const int *cu_q, const int *tile_seq, const int *tile_q0, int n_tiles, int nq,
                         int nkv, int G, int head_groups, int max_blocks, int block_size, int bs_shift, float sl2) {
    hipLaunchKernelGGL((attn_prefill_kernel<NW, MODE, KS>), dim3((unsigned)grid), dim3(64 * NW), 0, g_llmgen_stream, out, q,
                       kc, vc, bt, ctx, cu_q, tile_seq, tile_q0, n_tiles, nq, nkv, G, head_groups, max_blocks,
                       block_size, bs_shift, sl2);
}

template <int NW, int KS = 1>
void launch_prefill(int mode, int head_groups, bf16_t *out, const bf16_t *q, const bf16_t *kc, const bf16_t *vc,
                    const int *bt, const int *ctx, const int *cu_q, const int *tile_seq, const int *tile_q0,
                    int n_tiles, int nq, int nkv, int G, int max_blocks, int block_size, int bs_shift, float sl2) {
    const long grid = (long)n_tiles * nkv * head_groups;
    auto go = [&](auto m) {
        launch_prefill_mode<NW, decltype(m)::value, KS>(grid, out, q, kc, vc, bt, ctx, cu_q, tile_seq, tile_q0, n_tiles,
                                                    nq, nkv, G, head_groups, max_blocks, block_size, bs_shift, sl2);
    };
    if (mode == DMA_BLOCK) go(std::integral_constant<int, DMA_BLOCK>{});
    else if (mode == DMA_ROW4) go(std::integral_constant<int, DMA_ROW4>{});
    else go(std::integral_constant<int, DMA_FLAT>{});
}

// ---- pure prefill with the heaviest units split over two workgroups ----
//
// A pure prefill step at G = 2 too large for the key-split kernel is as long as its heaviest unit: the last tiles
// of a long prompt need every key tile before them, one after another (c3: 56 key tiles).  Here the units of the
// n_heavy heaviest tiles (the end of the executor's lightest-first list) each get two 4-wave workgroups, one per
// half of the unit's key tiles; both leave their partial (O, m, l) in the library's scratch array and the one that
// finishes second merges the two in a fixed order (piece 0, then piece 1: bit-reproducible) and stores the rows.
// Every other unit is one workgroup as in the 4-wave kernel.  The grid keeps the KV head fastest, so a KV head
// stays on its XCD.
constexpr int SPLIT_MAX_UNITS = 256;  // heavy units (tile x KV head x head group) one launch can split
__device__ __align__(256) float g_split_part[(size_t)SPLIT_MAX_UNITS * 2 * PART_FLOATS];
__device__ int g_split_counters[SPLIT_MAX_UNITS];

template <int MODE>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
    attn_prefill_split_kernel(bf16_t *__restrict__ out, const bf16_t *__restrict__ q, const bf16_t *__restrict__ kc,
                              const bf16_t *__restrict__ vc, const int *__restrict__ block_tables,
                              const int *__restrict__ ctx_lens, const int *__restrict__ cu_q,
                              const int *__restrict__ tile_seq, const int *__restrict__ tile_q0, int n_tiles, int nq,
                              int nkv, int G, int head_groups, int max_blocks, int block_size, int bs_shift,
                              float scale_log2, int n_heavy, float *__restrict__ part, int *__restrict__ counters) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[sizeof(PrefillLds<4, 1>)];
    __shared__ int s_last;
    const int Q = nkv * head_groups;  // units per tile
    const long b = blockIdx.x;
    auto body = [&](int bid, int j0, int j1, float *dst) {
        prefill_body<4, MODE, 1, true>(out, q, kc, vc, block_tables, ctx_lens, cu_q, tile_seq, tile_q0, n_tiles, nq,
                                      nkv, G, head_groups, max_blocks, block_size, bs_shift, scale_log2, bid, lds, j0,
                                      j1, dst);
    };
    // Grid order, longest first over all pieces: the halves of heavy tile k (2 groups of Q workgroups), then the
    // unsplit tile n_heavy + k, whose units are about as long as those halves, for k < periods; then what is left
    // of either kind.  t = the tile's position from the end of the list; half = -1 for an unsplit unit.
    const int n_light = n_tiles - n_heavy, periods = min(n_heavy, n_light);
    const long g = b / Q;
    const int within = (int)(b % Q);
    int t, half;
    if (g < 3L * periods) {
        const int k = (int)(g / 3), r = (int)(g % 3);
        t = r < 2 ? k : n_heavy + k;
        half = r < 2 ? r : -1;
    } else if (n_heavy > periods) {  // heavy tiles left over (fewer light tiles than heavy ones)
        const long r = g - 3L * periods;
        if (r < 2L * (n_heavy - periods)) {
            t = periods + (int)(r / 2);
            half = (int)(r % 2);
        } else {
            t = n_heavy + periods + (int)(r - 2L * (n_heavy - periods));
            half = -1;
        }
    } else {
        t = n_heavy + (int)(g - 2L * periods);  // light tiles from n_heavy + periods on
        half = -1;
    }
    const int bid = t * Q + within;  // the unit, numbered as in the one-unit-per-workgroup grid
    if (half < 0) {  // one workgroup, all its key tiles
        body(bid, 0, -1, nullptr);
        return;
    }
    const int tile = n_tiles - 1 - t;
    const int s = tile_seq[tile], q_len = cu_q[s + 1] - cu_q[s], ctx = ctx_lens[s];
    const int n = q_len > 1 && ctx >= q_len ? (ctx - q_len + min(tile_q0[tile] + BQ, q_len) + BK - 1) / BK : 0;
    if (n < 4) {  // not worth a merge (a unit under four key tiles, a padding or single-row segment): the first
                  // half runs it whole (64 prompts of 128 tokens: 37.1 -> 35.2 us)
        if (half == 0) body(bid, 0, -1, nullptr);
        return;
    }
    float *mine = part + ((long)bid * 2 + half) * PART_FLOATS;
    body(bid, half ? n / 2 : 0, half ? -1 : n / 2, mine);
    // publish, then draw a ticket: the second half to arrive merges (the partials are device-coherent stores,
    // complete before the barrier; the merger reads them with device-coherent loads after an acquire fence)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(counters + bid, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 1;
    __syncthreads();
    if (!s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const float *const pieces[2] = {part + (long)bid * 2 * PART_FLOATS, part + ((long)bid * 2 + 1) * PART_FLOATS};
    prefill_merge_store<2>(out, cu_q, tile_seq, tile_q0, n_tiles, nq, nkv, G, head_groups, bid, pieces);
    if (threadIdx.x == 0) __hip_atomic_store(counters + bid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- prefill of few units: each unit's key tiles over several workgroups ----
//
// A pure prefill step of few units -- a chunk of a long prompt against its cached keys, a short prompt -- leaves
// most of the chip idle with one workgroup per unit: a 512-row chunk at GQA 2 against 32K cached keys is 64 units
// of 520 key tiles, one chain each on 64 of 256 CUs (455 us).  Units are (tile x KV head x head pair) for 4-wave
// workgroups, or (tile x head) for 2-wave ones at G = 1; a step qualifies with at most half a 4-wave unit (one
// 2-wave unit) per CU.  Each unit gets P workgroups (P = min(8, the CUs' workgroup slots / units), so all are
// resident at once); a unit of n key tiles uses min(P, ceil(n / 4)) of them, each a contiguous equal share of its
// key tiles, and the others exit.  A unit with one piece stores its rows directly; otherwise every piece leaves
// its partial (O, m, l) in the library's scratch array (shared with the heavy-tile split) and the last to finish,
// by a ticket on a per-unit counter, merges them in piece order, so the output is bit-reproducible.  The unit
// index runs fastest in the grid, so a KV head's workgroups stay on one XCD.  A mixed step at G = 1, 8 or 16 runs
// its prefill tiles here beside the decode-row launch: the list's leading single-row tiles (n_front) are only
// checked, a few hundred units per workgroup, and not split.
constexpr int PIECES_MAX = 8, PIECE_MIN_TILES = 4;

template <int MODE, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2)))
    attn_prefill_pieces_kernel(bf16_t *__restrict__ out, const bf16_t *__restrict__ q, const bf16_t *__restrict__ kc,
                               const bf16_t *__restrict__ vc, const int *__restrict__ block_tables,
                               const int *__restrict__ ctx_lens, const int *__restrict__ cu_q,
                               const int *__restrict__ tile_seq, const int *__restrict__ tile_q0, int n_tiles, int nq,
                               int nkv, int G, int head_groups, int max_blocks, int block_size, int bs_shift,
                               float scale_log2, int n_front, int n_units, int P, float *__restrict__ part,
                               int *__restrict__ counters) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[sizeof(PrefillLds<NW, 1>)];
    __shared__ int s_last;
    constexpr int PSTRIDE = NW * PART_WAVE_FLOATS;  // scratch floats per piece
    // The list's first n_front tiles (a mixed step's single-row segments, streamed by the decode-row launch) are
    // checked 64 * NW units per workgroup, one per thread; a multi-row tile found there (a list out of order) runs
    // whole.  The rest of the list is split into pieces.
    constexpr int FRONT = 64 * NW;
    const long front_units = (long)n_front * nkv * head_groups;
    const long front_wg = (front_units + FRONT - 1) / FRONT;
    if (blockIdx.x < front_wg) {
        __shared__ int s_multi[FRONT];
        const long u = (long)blockIdx.x * FRONT + threadIdx.x;
        int multi = 0;
        if (u < front_units) {
            const int s = tile_seq[n_front - 1 - (int)(u / (nkv * head_groups))];
            multi = cu_q[s + 1] - cu_q[s] > 1;
        }
        s_multi[threadIdx.x] = multi;
        __syncthreads();
        for (int i = 0; i < FRONT; ++i) {
            if (!s_multi[i]) continue;  // uniform: every thread reads the same flag
            prefill_body<NW, MODE, 1, true>(out, q, kc, vc, block_tables, ctx_lens, cu_q, tile_seq, tile_q0, n_front,
                                            nq, nkv, G, head_groups, max_blocks, block_size, bs_shift, scale_log2,
                                            (int)((long)blockIdx.x * FRONT + i), lds, 0, -1, nullptr);
            __syncthreads();  // the next unit reuses the LDS stages
        }
        return;
    }
    tile_seq += n_front;
    tile_q0 += n_front;
    n_tiles -= n_front;
    const long b = blockIdx.x - front_wg;
    const int unit = (int)(b % n_units), piece = (int)(b / n_units);
    auto body = [&](int j0, int j1, float *dst) {
        prefill_body<NW, MODE, 1, true>(out, q, kc, vc, block_tables, ctx_lens, cu_q, tile_seq, tile_q0, n_tiles, nq,
                                      nkv, G, head_groups, max_blocks, block_size, bs_shift, scale_log2, unit, lds,
                                      j0, j1, dst);
    };
    const int tile = n_tiles - 1 - unit / (nkv * head_groups);
    const int s = tile_seq[tile], q_len = cu_q[s + 1] - cu_q[s], ctx = ctx_lens[s];
    const int n = q_len > 1 && ctx >= q_len ? (ctx - q_len + min(tile_q0[tile] + BQ, q_len) + BK - 1) / BK : 0;
    const int pe = n < 2 ? 1 : min(P, (n + PIECE_MIN_TILES - 1) / PIECE_MIN_TILES);
    if (piece >= pe) return;
    if (pe == 1) {  // one piece (also padding and single-row segments): the whole unit, rows stored directly
        body(0, -1, nullptr);
        return;
    }
    const int j0 = (int)((long)piece * n / pe), j1 = (int)((long)(piece + 1) * n / pe);
    float *mine = part + ((long)unit * P + piece) * PSTRIDE;
    body(j0, j1, mine);
    // publish (device-coherent stores, complete before the barrier), then draw a ticket: the last piece merges
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(counters + unit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == pe - 1;
    __syncthreads();
    if (!s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    prefill_merge_store_n<PIECES_MAX, NW>(out, cu_q, tile_seq, tile_q0, n_tiles, nq, nkv, G, head_groups, unit,
                                          part + (long)unit * P * PSTRIDE, pe);
    if (threadIdx.x == 0) __hip_atomic_store(counters + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
T *symbol_address(const T &sym) {
    static T *ptr[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    if (!ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, sym) != hipSuccess) return nullptr;
        ptr[dev] = (T *)p;
    }
    return ptr[dev];
}

// Heavy tiles to split for a pure prefill step of two-head units (0 = do not split).  Automatic: half a CU's worth
// of units, n_heavy * nkv * head_groups = CUs / 2, on steps of at most 5 units per CU; steps with more are bound by
// throughput, not by their heaviest units.  Measured on c3 (99 tiles x 8 KV heads), interleaved grid, same box:
// 0 tiles 78.7 us, 6: 74.2, 10: 71.9, 14: 67.3, 16: 66.8, 20: 68.5, 22: 78.4 (the unsplit tiles beside the halves
// then outlast them), 32: 78.6 us; two other draws of c3's prompt lengths 79.7 -> 70.5 and 79.0 -> 68.7 us at 16;
// single prompts of 5632 / 8192 tokens 137.9 -> 139.0 / 272.3 -> 267.0 us, 16384 tokens (8 units per CU, so not
// split) 985.9 against 995.1 us when split.  LLMGEN_OPT_PREFILL_SPLIT_TILES overrides the count (0 = off).
int split_heavy_tiles(int n_tiles, int nkv, int head_groups) {
    const int Q = nkv * head_groups;
    const int opt = llmgen_opt(LLMGEN_OPT_PREFILL_SPLIT_TILES);
    int h;
    if (opt >= 0) {
        h = opt;
    } else {
        const int cus = llmgen_num_cus();
        if ((long)n_tiles * Q > 5L * cus) return 0;
        h = std::max(1, cus / (2 * Q));
    }
    h = std::min(h, n_tiles);
    h = std::min(h, SPLIT_MAX_UNITS / Q);
    return h > 0 ? h : 0;
}

bool launch_prefill_split(int mode, bf16_t *out, const bf16_t *q, const bf16_t *kc, const bf16_t *vc, const int *bt,
                          const int *ctx, const int *cu_q, const int *tile_seq, const int *tile_q0, int n_tiles,
                          int nq, int nkv, int G, int max_blocks, int block_size, int bs_shift, float sl2) {
    const int head_groups = G / 2;
    const int h = split_heavy_tiles(n_tiles, nkv, head_groups);
    if (h <= 0) return false;
    float *part = reinterpret_cast<float *>(symbol_address(HIP_SYMBOL(g_split_part)));
    int *counters = reinterpret_cast<int *>(symbol_address(HIP_SYMBOL(g_split_counters)));
    if (!part || !counters) return false;
    const long grid = ((long)n_tiles + h) * nkv * head_groups;
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), 0, g_llmgen_stream, out, q, kc, vc, bt, ctx, cu_q,
                           tile_seq, tile_q0, n_tiles, nq, nkv, G, head_groups, max_blocks, block_size, bs_shift,
                           sl2, h, part, counters);
    };
    if (mode == DMA_BLOCK) go(attn_prefill_split_kernel<DMA_BLOCK>);
    else if (mode == DMA_ROW4) go(attn_prefill_split_kernel<DMA_ROW4>);
    else go(attn_prefill_split_kernel<DMA_FLAT>);
    return true;
}

// Pieces per unit for a pure prefill step of `units` units of nw-wave workgroups (0: too many units for this
// launch).  The CUs hold 8 / nw such workgroups each; a step qualifies when every unit can have at least 4.
int prefill_pieces(long units, int nw) {
    const long slots = (long)llmgen_num_cus() * (8 / nw);
    const long capacity = 2L * SPLIT_MAX_UNITS * 4 / nw;  // pieces the scratch array holds
    if (units <= 0 || units * 4 > slots || units > SPLIT_MAX_UNITS) return 0;
    const long p = std::min<long>({(long)PIECES_MAX, slots / units, capacity / units});
    return p >= 2 ? (int)p : 0;
}

// n_front: tiles at the front of the list not to split (a mixed step's single-row segments), 0 for a pure step.
bool launch_prefill_pieces(int mode, bf16_t *out, const bf16_t *q, const bf16_t *kc, const bf16_t *vc,
                           const int *bt, const int *ctx, const int *cu_q, const int *tile_seq, const int *tile_q0,
                           int n_tiles, int nq, int nkv, int G, int max_blocks, int block_size, int bs_shift,
                           float sl2, int n_front) {
    const int nw = G == 1 ? 2 : 4;  // one head per 2-wave workgroup at G = 1, else two per 4-wave workgroup
    const int head_groups = G / (nw / 2);
    const long units = (long)(n_tiles - n_front) * nkv * head_groups;
    const long front_wg = ((long)n_front * nkv * head_groups + 64 * nw - 1) / (64 * nw);  // as the kernel counts
    const int P = prefill_pieces(units, nw);
    if (P <= 0) return false;
    float *part = reinterpret_cast<float *>(symbol_address(HIP_SYMBOL(g_split_part)));
    int *counters = reinterpret_cast<int *>(symbol_address(HIP_SYMBOL(g_split_counters)));
    if (!part || !counters) return false;
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3((unsigned)(front_wg + units * P)), dim3(64 * nw), 0, g_llmgen_stream, out, q,
                           kc, vc, bt, ctx, cu_q, tile_seq, tile_q0, n_tiles, nq, nkv, G, head_groups, max_blocks,
                           block_size, bs_shift, sl2, n_front, (int)units, P, part, counters);
    };
    if (nw == 2) {
        if (mode == DMA_BLOCK) go(attn_prefill_pieces_kernel<DMA_BLOCK, 2>);
        else if (mode == DMA_ROW4) go(attn_prefill_pieces_kernel<DMA_ROW4, 2>);
        else go(attn_prefill_pieces_kernel<DMA_FLAT, 2>);
    } else {
        if (mode == DMA_BLOCK) go(attn_prefill_pieces_kernel<DMA_BLOCK, 4>);
        else if (mode == DMA_ROW4) go(attn_prefill_pieces_kernel<DMA_ROW4, 4>);
        else go(attn_prefill_pieces_kernel<DMA_FLAT, 4>);
    }
    return true;
}

}  // namespace

bool llmgen_prefill_scratch(float **part, int **counters, long units) {
    if (units > SPLIT_MAX_UNITS) return false;
    *part = reinterpret_cast<float *>(symbol_address(HIP_SYMBOL(g_split_part)));
    *counters = reinterpret_cast<int *>(symbol_address(HIP_SYMBOL(g_split_counters)));
    return *part && *counters;
}

extern "C" int hip_attn_prefill_tile(void) { return BQ; }

namespace {

// The launch hip_attn_prefill_rows makes for a step of this shape (hip_attn_prefill_plan reports it).
struct PrefillPlan {
    int kernel = 0;          // LLMGEN_PREFILL_* of llmgen_attn.h; 0 = nothing to launch
    int heads_per_wg = 0;    // query heads per prefill workgroup (two waves each)
    bool rows_launch = false;  // a separate decode-row launch on the side stream
};

PrefillPlan plan_prefill(int n_tiles, int G, int nkv, int single_rows) {
    PrefillPlan p;
    if (n_tiles <= 0) return p;
    // A mixed step whose single-row count the caller knows runs as one launch (mixed.hip) at G = 2 and 4.
    if (single_rows > 0 && (G == 2 || G == 4) && single_rows <= n_tiles) {
        p.kernel = LLMGEN_PREFILL_MIXED;
        p.heads_per_wg = 2;
        return p;
    }
    // two waves per head; at most 8 waves (4 heads) per workgroup, the rest of the group in further workgroups
    p.heads_per_wg = G < 4 ? G : 4;
    // A small pure-prefill step at G >= 4 runs as G / 2 two-head groups so that it can take the key-split
    // workgroups below (single G = 4 prompt of 2048 tokens: 47 against 57 us; at 3584 tokens, 896 units, the
    // 8-wave four-head workgroups stay faster: 105 against 112-122 us)
    if (single_rows == 0 && G >= 4 && (long)n_tiles * nkv * (G / 2) * 2 <= 5L * llmgen_num_cus()) p.heads_per_wg = 2;
    const int head_groups = G / p.heads_per_wg;
    // Decode rows (q_len == 1) of other mixed steps go to the bandwidth-oriented decode kernel on the side stream,
    // concurrently with the MFMA kernel (which skips them).  Its grid covers every tile (which tiles are single rows
    // is device data), so it is skipped when the caller knows there are none.
    p.rows_launch = single_rows != 0;
    // A mixed step at other G whose prefill tiles (after its single rows) are few units: the pieces kernel for them,
    // beside the decode-row launch
    if (single_rows > 0 && single_rows < n_tiles) {
        const int nw = G == 1 ? 2 : 4;
        if (prefill_pieces((long)(n_tiles - single_rows) * nkv * (G / (nw / 2)), nw) > 0) {
            p.kernel = LLMGEN_PREFILL_PIECES;
            return p;
        }
    }
    if (p.heads_per_wg == 1) {
        // a pure prefill step of at most one one-head unit per CU: the pieces kernel's 2-wave form
        p.kernel = single_rows == 0 && prefill_pieces((long)n_tiles * nkv * head_groups, 2) > 0 ? LLMGEN_PREFILL_PIECES
                                                                                              : LLMGEN_PREFILL_W2;
    } else if (p.heads_per_wg == 2) {
        // Pure prefill of up to 2.5 units per CU: 8-wave workgroups whose two key groups split each unit's key
        // tiles, so the heaviest units (a long prompt's last tiles) take half as many iterations (measured on
        // single prompts: 64 against 75 us at 3584 tokens, even at 4608).  Larger steps are bound by throughput,
        // where the 4-wave workgroups (two per CU) are faster (5632 tokens: 137 against 148 us; 16384: 986 against
        // 1069 us).  With decode rows beside it a 128 KB workgroup finds no room next to the decode kernel's waves.
        p.kernel = single_rows == 0 && prefill_pieces((long)n_tiles * nkv * head_groups, 4) > 0
                       ? LLMGEN_PREFILL_PIECES
                   : single_rows == 0 && (long)n_tiles * nkv * head_groups * 2 <= 5L * llmgen_num_cus()
                       ? LLMGEN_PREFILL_KEYSPLIT
                       : (single_rows == 0 && G == 2 && split_heavy_tiles(n_tiles, nkv, head_groups) > 0
                              ? LLMGEN_PREFILL_SPLIT
                              : LLMGEN_PREFILL_W4);
    } else {
        p.kernel = LLMGEN_PREFILL_W8;
    }
    return p;
}

}  // namespace

extern "C" int hip_attn_prefill_plan(int n_tiles, int nq, int nkv, int hd, int block_size, int single_rows) {
    if (hd != HD || nkv <= 0 || nq <= 0 || nq % nkv != 0 || block_size <= 0) return -1;
    const int G = nq / nkv;
    if (G != 1 && G != 2 && G != 4 && G != 8 && G != 16) return -1;
    const PrefillPlan p = plan_prefill(n_tiles, G, nkv, single_rows);
    return p.kernel | (p.rows_launch ? LLMGEN_PREFILL_ROWS_LAUNCH : 0);
}

extern "C" void hip_attn_prefill_rows(bf16_t *out, const bf16_t *q, const bf16_t *k_cache,
                                      const bf16_t *v_cache, const int *block_tables, const int *ctx_lens,
                                      const int *cu_q, const int *tile_seq, const int *tile_q0, int n_tiles, int nq,
                                      int nkv, int hd, int max_blocks, int block_size, float scale,
                                      int single_rows) {
    if (n_tiles <= 0) return;
    if (hd != HD) {
        fprintf(stderr, "[llmgen-hip] attn_prefill: only head_dim=128 is supported (got %d)\n", hd);
        return;
    }
    if (nkv <= 0 || nq <= 0 || nq % nkv != 0 || block_size <= 0) {
        fprintf(stderr, "[llmgen-hip] attn_prefill: bad shape nq=%d nkv=%d block_size=%d\n", nq, nkv, block_size);
        return;
    }
    const int G = nq / nkv;
    if (G != 1 && G != 2 && G != 4 && G != 8 && G != 16) {
        fprintf(stderr, "[llmgen-hip] attn_prefill: unsupported GQA group size %d\n", G);
        return;
    }
    const int bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
    const int mode = (bs_shift >= 0 && block_size % BK == 0) ? DMA_BLOCK : (block_size % 4 == 0 ? DMA_ROW4 : DMA_FLAT);
    const float sl2 = scale * LLMGEN_LOG2E;
    const PrefillPlan plan = plan_prefill(n_tiles, G, nkv, single_rows);
    if (plan.kernel == LLMGEN_PREFILL_MIXED) {
        llmgen_mixed_step(out, q, k_cache, v_cache, block_tables, ctx_lens, cu_q, tile_seq, tile_q0, n_tiles,
                          single_rows, nq, nkv, max_blocks, block_size, scale, mode);
        return;
    }
    const int head_groups = G / plan.heads_per_wg;
    hipStream_t side = g_llmgen_stream;
    if (plan.rows_launch) {
        side = llmgen_fork_side_stream();
        llmgen_decode_rows_of_prefill(out, q, k_cache, v_cache, block_tables, ctx_lens, cu_q, tile_seq, n_tiles, nq,
                                      nkv, max_blocks, block_size, scale, side);
    }
    PrefillPlan run = plan;
    if (plan.kernel == LLMGEN_PREFILL_PIECES &&
        !launch_prefill_pieces(mode, out, q, k_cache, v_cache, block_tables, ctx_lens, cu_q, tile_seq, tile_q0,
                               n_tiles, nq, nkv, G, max_blocks, block_size, bs_shift, sl2,
                               single_rows > 0 ? single_rows : 0))
        run.kernel = G == 1 ? LLMGEN_PREFILL_W2 : single_rows > 0 ? LLMGEN_PREFILL_W8 : LLMGEN_PREFILL_KEYSPLIT;
    if (plan.kernel == LLMGEN_PREFILL_SPLIT &&
        !launch_prefill_split(mode, out, q, k_cache, v_cache, block_tables, ctx_lens, cu_q, tile_seq, tile_q0,
                              n_tiles, nq, nkv, G, max_blocks, block_size, bs_shift, sl2))
        run.kernel = LLMGEN_PREFILL_W4;
    switch (run.kernel) {
        case LLMGEN_PREFILL_SPLIT:
        case LLMGEN_PREFILL_PIECES:
            break;
        case LLMGEN_PREFILL_W2:
            launch_prefill<2>(mode, head_groups, out, q, k_cache, v_cache, block_tables, ctx_lens, cu_q, tile_seq,
                              tile_q0, n_tiles, nq, nkv, G, max_blocks, block_size, bs_shift, sl2);
            break;
        case LLMGEN_PREFILL_KEYSPLIT:
            launch_prefill<8, 2>(mode, head_groups, out, q, k_cache, v_cache, block_tables, ctx_lens, cu_q, tile_seq,
                                 tile_q0, n_tiles, nq, nkv, G, max_blocks, block_size, bs_shift, sl2);
            break;
        case LLMGEN_PREFILL_W4:
            launch_prefill<4>(mode, head_groups, out, q, k_cache, v_cache, block_tables, ctx_lens, cu_q, tile_seq,
                              tile_q0, n_tiles, nq, nkv, G, max_blocks, block_size, bs_shift, sl2);
            break;
        default:
            launch_prefill<8>(mode, head_groups, out, q, k_cache, v_cache, block_tables, ctx_lens, cu_q, tile_seq,
                              tile_q0, n_tiles, nq, nkv, G, max_blocks, block_size, bs_shift, sl2);
            break;
    }
    llmgen_join_side_stream(side);
}

extern "C" void hip_attn_prefill(bf16_t *out, const bf16_t *q, const bf16_t *k_cache, const bf16_t *v_cache,
                                 const int *block_tables, const int *ctx_lens, const int *cu_q, const int *tile_seq,
                                 const int *tile_q0, int n_tiles, int nq, int nkv, int hd, int max_blocks,
                                 int block_size, float scale) {
    hip_attn_prefill_rows(out, q, k_cache, v_cache, block_tables, ctx_lens, cu_q, tile_seq, tile_q0, n_tiles, nq, nkv,
                          hd, max_blocks, block_size, scale, -1);
}
