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
#include "decode_kernel.h"
#include "hip_common.h"

#include <math.h>
#include <stdlib.h>

#include <algorithm>

namespace {

using namespace llmgen_decode;

// G = query heads per KV head (1..16); NT = 16-token tiles per wave per round; W = waves per workgroup (4 or 8);
// FUSE = also write the step's token into the cache.  One workgroup per (kv head, sequence, span).
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
    __shared__ __attribute__((aligned(16))) unsigned char lds[sizeof(DecodeLds<G, NT, W>)];
    decode_split_body<G, NT, POW2, FUSE, W>(out, part_o, part_ml, q, kc, vc, block_tables, ctx_lens, nq, nkv,
                                            max_blocks, block_size, bs_shift, scale_log2, span, max_parts, nparts,
                                            counters, cu_q, tile_seq, k_new, v_new, slots, kc_w, vc_w, blockIdx.x,
                                            blockIdx.y, blockIdx.z, gridDim.y, lds);
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

