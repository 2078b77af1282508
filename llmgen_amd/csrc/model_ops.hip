// model_ops.hip -- the non-attention ops of the Qwen3 forward (embedding, RMSNorm, linear, NEOX RoPE, SiLU,
// add, mul, gather_last, sampling) for the end-to-end greedy-token check, and the fused q/k norm + RoPE + KV
// write that replaces five of them before attention.
//
// These kernels trade speed for reproducibility: every output is computed in the order the reference CPU
// backend uses (src/backend/cpu/*.zig), with one IEEE rounding per f32 multiply / add / divide / sqrt and one
// RNE rounding to bf16 per stored value, so a forward built from them matches the CPU backend bit for bit
// outside attention.  Contraction into FMAs is switched off for the whole file for that reason.  They are not
// part of the measured hot path.
#include "hip_common.h"

#include <math.h>

#pragma clang fp contract(off)

namespace {

__device__ __forceinline__ float bf2f(bf16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }
__device__ __forceinline__ bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// ---------------------------------------------------------------------------------------------- embedding
__global__ void embedding_kernel(bf16_t *out, const int *ids, const bf16_t *w, int T, int H) {
    const int chunks = H >> 3;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)T * chunks) return;
    const int t = (int)(i / chunks), c = (int)(i % chunks);
    const long row = ids[t];
    *reinterpret_cast<u32x4_t *>(out + (long)t * H + c * 8) = ld16(w + row * H + c * 8);
}

// ---------------------------------------------------------------------------------------------- RMSNorm
// One wave per row.  The row is staged in LDS as f32; lane 0 forms the sum of squares in index order (the
// reference's order), the wave then writes bf16(bf16(x * scale) * w).
constexpr int NORM_MAX_D = 8192;
__global__ void __launch_bounds__(64) rmsnorm_kernel(bf16_t *out, const bf16_t *x, const float *w, int D,
                                                      float eps) {
    __shared__ float row[NORM_MAX_D];
    __shared__ float scale_s;
    const long r = blockIdx.x;
    const bf16_t *xr = x + r * D;
    for (int c = threadIdx.x; c < (D >> 3); c += 64) {
        float f[8];
        unpack_bf16x8(ld16(xr + c * 8), f);
#pragma unroll
        for (int j = 0; j < 8; ++j) row[c * 8 + j] = f[j];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float ss = 0.0f;
        for (int h = 0; h < D; ++h) ss += row[h] * row[h];
        scale_s = 1.0f / sqrtf(ss / (float)D + eps);
    }
    __syncthreads();
    const float scale = scale_s;
    for (int h = threadIdx.x; h < D; h += 64) {
        const float normed = bf2f(f2bf(row[h] * scale));
        out[r * D + h] = f2bf(normed * w[h]);
    }
}

// ---------------------------------------------------------------------------------------------- linear
// y[m][n] = sum_k x[m][k] * w[n][k], k ascending.  A workgroup owns 256 output columns (one per thread) and
// LIN_MB rows; K advances in tiles of LIN_KT: the W tile (256 x LIN_KT bf16) and the x tile (LIN_MB x LIN_KT,
// as f32) are staged in LDS with coalesced 16-byte loads.  W rows are padded to an odd number of dwords so the
// 64 lanes of a wave read 64 different banks.  Each thread keeps LIN_MB independent chains.
constexpr int LIN_N = 256, LIN_MB = 8, LIN_KT = 32;
constexpr int LIN_WSTRIDE = LIN_KT / 2 + 1;  // dwords per padded W row (17)

__global__ void __launch_bounds__(LIN_N) linear_kernel(void *y, int y_f32, const bf16_t *x, const bf16_t *w, int M,
                                                       int N, int K) {
    __shared__ uint32_t ws[LIN_N * LIN_WSTRIDE];
    __shared__ float xs[LIN_MB][LIN_KT];
    const int tid = threadIdx.x;
    const int n0 = blockIdx.x * LIN_N, m0 = blockIdx.y * LIN_MB;
    const int n = n0 + tid;
    const int mrows = min(LIN_MB, M - m0);
    float acc[LIN_MB];
#pragma unroll
    for (int m = 0; m < LIN_MB; ++m) acc[m] = 0.0f;

    for (int k0 = 0; k0 < K; k0 += LIN_KT) {
        const int kt = min(LIN_KT, K - k0);  // multiple of 8
        // W tile: 256 rows x (kt / 8) chunks of 16 bytes
        for (int i = tid; i < LIN_N * (LIN_KT / 8); i += LIN_N) {
            const int r = i / (LIN_KT / 8), c = i % (LIN_KT / 8);
            u32x4_t v = {0u, 0u, 0u, 0u};
            if (n0 + r < N && c * 8 < kt) v = ld16(w + (long)(n0 + r) * K + k0 + c * 8);
#pragma unroll
            for (int j = 0; j < 4; ++j) ws[r * LIN_WSTRIDE + c * 4 + j] = v[j];
        }
        // x tile: mrows x (kt / 8) chunks
        for (int i = tid; i < LIN_MB * (LIN_KT / 8); i += LIN_N) {
            const int r = i / (LIN_KT / 8), c = i % (LIN_KT / 8);
            float f[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (r < mrows && c * 8 < kt) unpack_bf16x8(ld16(x + (long)(m0 + r) * K + k0 + c * 8), f);
#pragma unroll
            for (int j = 0; j < 8; ++j) xs[r][c * 8 + j] = f[j];
        }
        __syncthreads();
        for (int kk = 0; kk < kt; kk += 2) {
            const uint32_t wp = ws[tid * LIN_WSTRIDE + (kk >> 1)];
            const float w0 = bf16lo_to_f32(wp), w1 = bf16hi_to_f32(wp);
#pragma unroll
            for (int m = 0; m < LIN_MB; ++m) {
                acc[m] = acc[m] + xs[m][kk] * w0;
                acc[m] = acc[m] + xs[m][kk + 1] * w1;
            }
        }
        __syncthreads();
    }
    if (n >= N) return;
    for (int m = 0; m < mrows; ++m) {
        const long o = (long)(m0 + m) * N + n;
        if (y_f32)
            static_cast<float *>(y)[o] = acc[m];
        else
            static_cast<bf16_t *>(y)[o] = f2bf(acc[m]);
    }
}

// ---------------------------------------------------------------------------------------------- RoPE
__global__ void rope_kernel(bf16_t *out, const bf16_t *x, const float *cos_t, const float *sin_t, const int *pos,
                            int T, int n_head, int hd) {
    const int half = hd >> 1;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)T * n_head * half) return;
    const int d = (int)(i % half);
    const long th = i / half;  // t * n_head + h
    const int t = (int)(th / n_head);
    const long b = th * hd;
    const long p = pos[t];
    const float c = cos_t[p * hd + d], s = sin_t[p * hd + d];
    const float x0 = bf2f(x[b + d]), x1 = bf2f(x[b + d + half]);
    out[b + d] = f2bf(x0 * c - x1 * s);
    out[b + d + half] = f2bf(x1 * c + x0 * s);
}

// ---------------------------------------------------------------------------------------------- elementwise
// exp in double, rounded once to f32: the correctly rounded f32 exp except in vanishingly rare double-rounding
// cases, which is what a correctly rounded host expf returns.
__global__ void silu_kernel(bf16_t *out, const bf16_t *x, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = bf2f(x[i]);
    const float e = (float)exp(-(double)v);
    out[i] = f2bf(v / (1.0f + e));
}

__global__ void add_kernel(bf16_t *out, const bf16_t *a, const bf16_t *b, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f2bf(bf2f(a[i]) + bf2f(b[i]));
}

__global__ void mul_kernel(bf16_t *out, const bf16_t *a, const bf16_t *b, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f2bf(bf2f(a[i]) * bf2f(b[i]));
}

__global__ void gather_rows_kernel(bf16_t *out, const bf16_t *x, const int *idx, int S, int H) {
    const int chunks = H >> 3;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)S * chunks) return;
    const int s = (int)(i / chunks), c = (int)(i % chunks);
    *reinterpret_cast<u32x4_t *>(out + (long)s * H + c * 8) = ld16(x + (long)idx[s] * H + c * 8);
}

// ---------------------------------------------------------------------------------------------- sampling
// Greedy / Gumbel-max token choice (cpu/sample.zig:17-45 semantics): one workgroup of ROW_THREADS lanes owns one
// row and the whole choice is made in that workgroup, so no partial results leave it and no scratch is needed.
// Every candidate (value v, index i) becomes one 64-bit key: the high word is v's bits mapped so that unsigned
// order is float order, the low word is ~i.  The largest key is then the largest value and, among equal values,
// the smallest index -- exactly what the reference's strictly-greater scan keeps -- so the reduction is a plain
// unsigned max with no tie logic.  NaN and -inf never win that scan (no comparison with them is true), so they
// are not candidates; key 0 means "no candidate" and yields index 0, the scan's starting index.
// What bit parity with the CPU backend fixes is kept as it is: the splitmix64 stream per (seed, row, index), the
// uniform from its top 24 bits and the Gumbel value v / t - log(-log u), each f32 operation rounded once.
constexpr int ROW_THREADS = 1024;

__device__ __forceinline__ uint64_t mix64(uint64_t x) {  // SplitMix64 finaliser, as cpu/sample.zig:7-12
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

__device__ __forceinline__ uint64_t cand_key(float v, int i) {
    if (!(v > -INFINITY)) return 0;  // NaN, -inf
    if (v == 0.f) v = 0.f;           // -0 == +0 for the scan: equal keys, so the smaller index wins
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint32_t)~(uint32_t)i;
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t x, int m) {
    const int lane = __lane_id();
    const int lo = __builtin_amdgcn_ds_bpermute((lane ^ m) << 2, (int)(uint32_t)x);
    const int hi = __builtin_amdgcn_ds_bpermute((lane ^ m) << 2, (int)(uint32_t)(x >> 32));
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

template <bool GUMBEL>
__device__ __forceinline__ uint64_t scan_row(const bf16_t *row, int V, float temp, uint64_t rs) {
    uint64_t best = 0;
    auto take = [&](float x, int i) {
        if (GUMBEL) {
            const uint64_t r = mix64(rs + (uint64_t)i);
            const float u = ((float)(r >> 40) + 0.5f) * (1.0f / 16777216.0f);
            x = x / temp - logf(-logf(u));
        }
        const uint64_t k = cand_key(x, i);
        best = k > best ? k : best;
    };
    // eight consecutive logits per lane per step: one 16-byte load when the row is 16-byte aligned
    const bool vec = ((uintptr_t)row & 15) == 0;
    for (int i0 = threadIdx.x * 8; i0 < V; i0 += ROW_THREADS * 8) {
        if (vec && i0 + 8 <= V) {
            float f[8];
            unpack_bf16x8(ld16(row + i0), f);
#pragma unroll
            for (int e = 0; e < 8; ++e) take(f[e], i0 + e);
        } else {
            for (int i = i0; i < min(i0 + 8, V); ++i) take(bf2f(row[i]), i);
        }
    }
    return best;
}

__global__ void __launch_bounds__(ROW_THREADS) sample_rows_kernel(int *out, const bf16_t *logits, const float *temps,
                                                                   const uint64_t *seed, int V) {
    const int s = blockIdx.x;
    const bf16_t *row = logits + (long)s * V;
    const float temp = temps[s];
    uint64_t best = temp > 0.0f ? scan_row<true>(row, V, temp, mix64(*seed ^ ((uint64_t)s << 40)))
                                : scan_row<false>(row, V, temp, 0);
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const uint64_t o = shfl_xor64(best, m);
        best = o > best ? o : best;
    }
    __shared__ uint64_t wave_best[ROW_THREADS / 64];
    if ((threadIdx.x & 63) == 0) wave_best[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < ROW_THREADS / 64; ++w) best = wave_best[w] > best ? wave_best[w] : best;
        out[s] = best == 0 ? 0 : (int)~(uint32_t)best;
    }
}

bool reject(const char *what) {
    fprintf(stderr, "llmgen: %s\n", what);
    return true;
}

unsigned blocks_for(size_t n, unsigned per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

extern "C" {

void hip_embedding(uint16_t *out, const int32_t *ids, const uint16_t *weight, int T, int H) {
    if (T <= 0) return;
    if (H <= 0 || H % 8 != 0) {
        reject("hip_embedding: H must be a positive multiple of 8");
        return;
    }
    const size_t n = (size_t)T * (H / 8);
    embedding_kernel<<<blocks_for(n, 256), 256, 0, g_llmgen_stream>>>(out, ids, weight, T, H);
}

void hip_rmsnorm(uint16_t *out, const uint16_t *x, const float *w, long rows, int D, float eps) {
    if (rows <= 0) return;
    if (D <= 0 || D % 8 != 0 || D > NORM_MAX_D) {
        reject("hip_rmsnorm: D must be a positive multiple of 8, at most 8192");
        return;
    }
    rmsnorm_kernel<<<(unsigned)rows, 64, 0, g_llmgen_stream>>>(out, x, w, D, eps);
}

void hip_linear(void *y, int y_f32, const uint16_t *x, const uint16_t *w, int M, int N, int K) {
    if (M <= 0 || N <= 0) return;
    if (K <= 0 || K % 8 != 0) {
        reject("hip_linear: K must be a positive multiple of 8");
        return;
    }
    const dim3 grid((N + LIN_N - 1) / LIN_N, (M + LIN_MB - 1) / LIN_MB);
    linear_kernel<<<grid, LIN_N, 0, g_llmgen_stream>>>(y, y_f32, x, w, M, N, K);
}

void hip_rope(uint16_t *out, const uint16_t *x, const float *cos_tab, const float *sin_tab, const int32_t *positions,
              int T, int n_head, int hd) {
    if (T <= 0 || n_head <= 0) return;
    if (hd <= 0 || hd % 2 != 0) {
        reject("hip_rope: hd must be positive and even");
        return;
    }
    const size_t n = (size_t)T * n_head * (hd / 2);
    rope_kernel<<<blocks_for(n, 256), 256, 0, g_llmgen_stream>>>(out, x, cos_tab, sin_tab, positions, T, n_head, hd);
}

void hip_silu(uint16_t *out, const uint16_t *x, size_t n) {
    if (n == 0) return;
    silu_kernel<<<blocks_for(n, 256), 256, 0, g_llmgen_stream>>>(out, x, n);
}

void hip_add(uint16_t *out, const uint16_t *a, const uint16_t *b, size_t n) {
    if (n == 0) return;
    add_kernel<<<blocks_for(n, 256), 256, 0, g_llmgen_stream>>>(out, a, b, n);
}

void hip_mul(uint16_t *out, const uint16_t *a, const uint16_t *b, size_t n) {
    if (n == 0) return;
    mul_kernel<<<blocks_for(n, 256), 256, 0, g_llmgen_stream>>>(out, a, b, n);
}

void hip_gather_rows(uint16_t *out, const uint16_t *x, const int32_t *idx, int S, int H) {
    if (S <= 0) return;
    if (H <= 0 || H % 8 != 0) {
        reject("hip_gather_rows: H must be a positive multiple of 8");
        return;
    }
    const size_t n = (size_t)S * (H / 8);
    gather_rows_kernel<<<blocks_for(n, 256), 256, 0, g_llmgen_stream>>>(out, x, idx, S, H);
}

// The choice is made inside one workgroup per row: no scratch is needed (the argument stays for the reference's
// argument list, sample.zig:4-14, and may be null).
size_t hip_sample_scratch_bytes(int max_S) {
    (void)max_S;
    return 0;
}

void hip_sample(int32_t *out_ids, const uint16_t *logits, const float *temps, const uint64_t *seed, int S, int V,
                void *scratch) {
    (void)scratch;
    if (S <= 0) return;
    if (V <= 0) {
        reject("hip_sample: V must be positive");
        return;
    }
    sample_rows_kernel<<<S, ROW_THREADS, 0, g_llmgen_stream>>>(out_ids, logits, temps, seed, V);
}

}  // extern "C"

// ------------------------------------------------------------------------------------------------------------
// Fused per-head q/k RMSNorm + NEOX RoPE + paged KV write (one launch for what the unfused graph does in five:
// rmsnorm(q), rmsnorm(k), rope(q), rope(k), store_kv).  Eight lanes own one 128-wide head row, 16 elements each
// (two 16-byte loads, coalesced), and the row stays in registers from load to store.  Every value is rounded
// exactly where the unfused ops round it, and the sum of squares is formed in index order: lane j of the row
// continues the running sum it receives from lane j-1 (a DPP shift per step, eight steps), so the outputs are
// bit-identical to the unfused sequence.  RoPE partners (i, i + 64) sit in lanes j and j ^ 4.  Rows
// [0, T*nq) are q rows (written to q_out, which may alias q); rows [T*nq, T*(nq+nkv)) are k rows, written into
// the paged cache together with the v row of the same (token, KV head).  Slot < 0 skips the cache write.
namespace {
constexpr int QK_HD = 128;
constexpr int QK_LPR = 8;  // lanes per row

__global__ void __launch_bounds__(256) qk_norm_rope_store_kernel(
    bf16_t *q_out, bf16_t *k_cache, bf16_t *v_cache, const bf16_t *q, const bf16_t *k, const bf16_t *v,
    const float *q_w, const float *k_w, float eps, const float *cos_t, const float *sin_t, const int *pos,
    const int *slots, int T, int nq, int nkv, int block_size) {
    const long gt = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int sub = threadIdx.x & (QK_LPR - 1);
    const long rows_q = (long)T * nq, rows = rows_q + (long)T * nkv;
    const bool valid = gt / QK_LPR < rows;
    const long r = valid ? gt / QK_LPR : rows - 1;  // out-of-range lanes still take part in the exchanges
    const bool is_q = r < rows_q;
    const long rk = r - rows_q;
    const int t = is_q ? (int)(r / nq) : (int)(rk / nkv);
    const int h = is_q ? 0 : (int)(rk % nkv);
    const bf16_t *src = (is_q ? q + r * QK_HD : k + rk * QK_HD) + sub * 16;
    const float *w = (is_q ? q_w : k_w) + sub * 16;

    u32x4_t xv[2] = {ld16(src), ld16(src + 8)};
    float x[16];
    unpack_bf16x8(xv[0], x);
    unpack_bf16x8(xv[1], x + 8);
    // running sum of squares in index order across the row's eight lanes
    float in = 0.0f, cand = 0.0f;
#pragma unroll
    for (int step = 0; step < QK_LPR; ++step) {
        cand = in;
#pragma unroll
        for (int e = 0; e < 16; ++e) cand += x[e] * x[e];
        // row_shr:1 -- lane j receives lane j-1's running sum (lane 0 of each row starts from 0)
        const float prev = __builtin_bit_cast(
            float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, cand), 0x111, 0xF, 0xF, false));
        in = sub ? prev : 0.0f;
    }
    // the last lane of the row holds the complete sum
    const int last_lane = (__lane_id() & ~(QK_LPR - 1)) | (QK_LPR - 1);
    const float ss = __builtin_bit_cast(
        float, __builtin_amdgcn_ds_bpermute(last_lane << 2, __builtin_bit_cast(int, cand)));
    const float scale = 1.0f / sqrtf(ss / (float)QK_HD + eps);
    float n[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) n[e] = bf2f(f2bf(bf2f(f2bf(x[e] * scale)) * w[e]));
    // RoPE: lanes 0-3 hold dims i < 64 (x0), lanes 4-7 their partners i + 64 (x1); cos/sin rows repeat per half
    float other[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) other[e] = lane_xor(n[e], 4);
    const int dim0 = sub * 16;
    const float *cr = cos_t + (long)pos[t] * QK_HD + dim0;
    const float *sr = sin_t + (long)pos[t] * QK_HD + dim0;
    const bool low = sub < 4;
    u32x4_t ov[2];
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
        float o2[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const float c = cr[e + u], s = sr[e + u];
            o2[u] = low ? n[e + u] * c - other[e + u] * s : n[e + u] * c + other[e + u] * s;
        }
        ov[e >> 3][(e & 7) >> 1] = pack_bf16x2(o2[0], o2[1]);
    }
    if (!valid) return;
    if (is_q) {
        bf16_t *dst = q_out + r * QK_HD + dim0;
        *reinterpret_cast<u32x4_t *>(dst) = ov[0];
        *reinterpret_cast<u32x4_t *>(dst + 8) = ov[1];
        return;
    }
    const int slot = slots[t];
    if (slot < 0) return;
    const long off = (((long)(slot / block_size) * nkv + h) * block_size + slot % block_size) * QK_HD + dim0;
    const bf16_t *vsrc = v + rk * QK_HD + dim0;
    const u32x4_t v0 = ld16(vsrc), v1 = ld16(vsrc + 8);
    *reinterpret_cast<u32x4_t *>(k_cache + off) = ov[0];
    *reinterpret_cast<u32x4_t *>(k_cache + off + 8) = ov[1];
    *reinterpret_cast<u32x4_t *>(v_cache + off) = v0;
    *reinterpret_cast<u32x4_t *>(v_cache + off + 8) = v1;
}
}  // namespace

extern "C" void hip_qk_norm_rope_store_kv(uint16_t *q_out, uint16_t *k_cache, uint16_t *v_cache, const uint16_t *q,
                                          const uint16_t *k, const uint16_t *v, const float *q_norm_w,
                                          const float *k_norm_w, float eps, const float *cos_tab,
                                          const float *sin_tab, const int32_t *positions,
                                          const int32_t *slot_mapping, int T, int nq, int nkv, int hd,
                                          int block_size) {
    if (T <= 0) return;
    if (hd != QK_HD || nq <= 0 || nkv <= 0 || block_size <= 0) {
        reject("hip_qk_norm_rope_store_kv: needs hd == 128 and positive nq, nkv, block_size");
        return;
    }
    const size_t threads = (size_t)T * (nq + nkv) * QK_LPR;
    qk_norm_rope_store_kernel<<<blocks_for(threads, 256), 256, 0, g_llmgen_stream>>>(
        q_out, k_cache, v_cache, q, k, v, q_norm_w, k_norm_w, eps, cos_tab, sin_tab, positions, slot_mapping, T, nq,
        nkv, block_size);
}
