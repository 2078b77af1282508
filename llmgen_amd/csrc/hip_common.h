// hip_common.h -- shared device helpers for the gfx950 attention kernels.
//
// Vector types for 16-byte bf16x8 loads, bf16 <-> f32 bit conversions (bf16 is the high half of an f32; the
// round to bf16 uses the hardware's round-to-nearest-even conversion), wave64 DPP row reductions and the
// process-global stream every launcher enqueues on.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "llmgen_attn.h"

typedef uint16_t bf16_t;  // bf16 bit pattern as stored in memory
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// The stream all launchers use; created by hip_init, replaceable with hip_set_stream.
extern hipStream_t g_llmgen_stream;

#define LLMGEN_LOG2E 1.4426950408889634f

// ---- bf16 <-> f32 ----
__device__ __forceinline__ float bf16lo_to_f32(uint32_t packed) { return __builtin_bit_cast(float, packed << 16); }
__device__ __forceinline__ float bf16hi_to_f32(uint32_t packed) {
    return __builtin_bit_cast(float, packed & 0xFFFF0000u);
}
// Unpack 8 bf16 (one 16-byte vector) into f32.
__device__ __forceinline__ void unpack_bf16x8(const u32x4_t v, float *f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = bf16lo_to_f32(v[i]);
        f[2 * i + 1] = bf16hi_to_f32(v[i]);
    }
}
// Round two f32 to bf16 (RNE, v_cvt_pk_bf16_f32) and pack lo | hi << 16.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2_t r;
    r[0] = (__bf16)lo;
    r[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, r);
}

// ---- wave64 row (16-lane) reductions through DPP ----
// DPP controls: quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E, row_half_mirror = 0x141,
// row_mirror = 0x140.  After the two quad steps each quad holds its result; the half-mirror pairs quad 0 with
// quad 1 (and 2 with 3); the mirror pairs the two halves of the 16-lane row.  All 16 lanes end with the result.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp_f<0xB1>(x));
    x = fmaxf(x, dpp_f<0x4E>(x));
    x = fmaxf(x, dpp_f<0x141>(x));
    x = fmaxf(x, dpp_f<0x140>(x));
    return x;
}
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_f<0xB1>(x);
    x += dpp_f<0x4E>(x);
    x += dpp_f<0x141>(x);
    x += dpp_f<0x140>(x);
    return x;
}

// Lane exchange across the whole wave (ds_bpermute; no LDS memory is touched).
__device__ __forceinline__ float lane_xor(float x, int mask) {
    const int lane = __lane_id();
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __builtin_bit_cast(int, x)));
}

// s_waitcnt immediate that waits until at most n vector-memory operations of this wave are outstanding
// (vmcnt, 6 bits split over [3:0] and [15:14]) and leaves the export and LDS counters unconstrained.
#define LLMGEN_WAIT_VMCNT(n) (0x0f70 | ((n) & 15) | ((((n) >> 4) & 3) << 14))
// cache-policy operand of the LDS-DMA builtins: nontemporal (the rows are read once)
#define LLMGEN_CPOL_NT 2

// 16-byte global load as four dwords.
__device__ __forceinline__ u32x4_t ld16(const void *p) { return *reinterpret_cast<const u32x4_t *>(p); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Internal: the library's prefill scratch (partial results of key-range pieces, 512 slots of PART_FLOATS floats,
// and one ticket counter per unit, zero between launches), shared by the heavy-tile split, the pieces kernel and the
// mixed-step kernel's split prefill units; false if its address cannot be taken or `units` exceeds its counters.
__attribute__((visibility("hidden"))) bool llmgen_prefill_scratch(float **part, int **counters, long units);

// Internal (not exported): decode rows (segments with q_len == 1) of a prefill / mixed step, streamed by the
// split-K decode kernel; defined in decode.hip, launched by hip_attn_prefill.
__attribute__((visibility("hidden"))) void llmgen_decode_rows_of_prefill(
    bf16_t *out, const bf16_t *q, const bf16_t *k_cache, const bf16_t *v_cache,
                                   const int *block_tables, const int *ctx_lens, const int *cu_q,
                                   const int *tile_seq, int n_tiles, int nq, int nkv, int max_blocks,
                                   int block_size, float scale, hipStream_t stream);

// Internal: a mixed step (single_rows > 0 single-row segments listed first, then prefill tiles) as one launch of
// the mixed-step kernel (mixed.hip); false if the shape is not one it takes (then nothing is launched).
__attribute__((visibility("hidden"))) bool llmgen_mixed_step(
    bf16_t *out, const bf16_t *q, const bf16_t *k_cache, const bf16_t *v_cache, const int *block_tables,
    const int *ctx_lens, const int *cu_q, const int *tile_seq, const int *tile_q0, int n_tiles, int single_rows,
    int nq, int nkv, int max_blocks, int block_size, float scale, int dma_mode);

// Internal: fork onto / join back from the library's side stream (hip_context.hip).  Used to run independent
// kernels of one launcher concurrently; legal inside stream capture.
__attribute__((visibility("hidden"))) hipStream_t llmgen_fork_side_stream();
__attribute__((visibility("hidden"))) void llmgen_join_side_stream(hipStream_t side);

// Internal: the value of a launcher option (LLMGEN_OPT_* of llmgen_attn.h), set by hip_attn_set_option.
__attribute__((visibility("hidden"))) int llmgen_opt(int which);

// Internal: compute units of the current device (256 if the query fails); cached after the first call.
__attribute__((visibility("hidden"))) int llmgen_num_cus();

// Internal: record an error of the library's own (a launch rejected on the host) for hip_last_error to return;
// the first recorded error is kept until hip_last_error reads it.
__attribute__((visibility("hidden"))) void llmgen_record_error(hipError_t e);
