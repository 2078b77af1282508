// store_kv.hip -- paged-KV write: this step's k, v [T, nkv, hd] into the layer's paged cache at slots[t].
//
// Semantics: src/backend/cpu/attention.zig:31-44 (storeKv) and the launcher contract of
// src/backend/cuda/attention/attention.cu:35-44 (cuda_store_kv).  Cache layout per block is
// [kv_head][slot_in_block][hd]; slot < 0 rows are skipped; bit-exact copy.
//
// gfx950 design: a pure HBM copy.  One lane moves one 16-byte chunk; the flat thread index is laid out as
// (K or V, token, kv head, chunk) with the chunk fastest, so a wave reads 1 KB of contiguous source and writes
// four 256-byte rows of the destination.  No LDS, no atomics; every access is a 16-byte vector op.
#include "hip_common.h"

__global__ void __launch_bounds__(256) store_kv_kernel(const bf16_t *__restrict__ k, const bf16_t *__restrict__ v,
                                                       const int *__restrict__ slots, bf16_t *__restrict__ kc,
                                                       bf16_t *__restrict__ vc, long rows, int nkv, int chunks,
                                                       int block_size) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long per_tensor = rows * chunks;  // rows = T * nkv
    if (idx >= 2 * per_tensor) return;
    const int which = idx >= per_tensor;  // 0 = K, 1 = V
    const long r = idx - which * per_tensor;
    const long row = r / chunks;  // t * nkv + h
    const int c = (int)(r - row * chunks);
    const long t = row / nkv;
    const int h = (int)(row - t * nkv);
    const int slot = slots[t];
    if (slot < 0) return;
    const long blk = slot / block_size, off = slot % block_size;
    const long hd = (long)chunks * 8;
    const long dst = ((blk * nkv + h) * block_size + off) * hd + c * 8;
    const long src = row * hd + c * 8;
    const bf16_t *s = which ? v : k;
    bf16_t *d = which ? vc : kc;
    *reinterpret_cast<u32x4_t *>(d + dst) = *reinterpret_cast<const u32x4_t *>(s + src);
}

extern "C" void hip_store_kv(const bf16_t *k, const bf16_t *v, const int *slot_mapping, bf16_t *k_cache,
                             bf16_t *v_cache, int T, int nkv, int hd, int block_size) {
    if (T <= 0) return;
    // The copy works for any head size that is a multiple of 8 (16-byte rows); the attention kernels need 128.
    if (hd <= 0 || hd % 8 != 0 || nkv <= 0 || block_size <= 0) {
        fprintf(stderr, "[llmgen-hip] store_kv: unsupported shape hd=%d nkv=%d block_size=%d\n", hd, nkv,
                block_size);
        return;
    }
    const long rows = (long)T * nkv;
    const int chunks = hd / 8;
    const long total = 2 * rows * chunks;
    const long blocks = (total + 255) / 256;
    hipLaunchKernelGGL(store_kv_kernel, dim3((unsigned)blocks), dim3(256), 0, g_llmgen_stream, k, v, slot_mapping,
                       k_cache, v_cache, rows, nkv, chunks, block_size);
}
