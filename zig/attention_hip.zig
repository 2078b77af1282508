//! attention_hip.zig -- PagedAttentionImpl for the MI355X attention library (libllmgen_attn.so, gfx950).
//!
//! Drop-in for src/backend/cuda/attention/attention_v1.zig: the engine finds `PagedAttentionImpl` (and the
//! `FlashAttentionImpl` alias, attention_v1.zig:123) by name in the backend module (src/ops.zig:31-37, 63-65), so
//! this file takes that file's place in src/backend/cuda/ when the engine is built with -Dhip=true (see
//! build_hip.zig).  Every per-step value comes from `common.g_step` and the layer's KV pools from
//! `common.kvOf(out.layer_id)`, exactly as the CUDA implementation reads them; the externs below are the C-ABI of
//! include/llmgen_attn.h, each the hip_ counterpart of one cuda_ extern of attention_v1.zig:10-48.
//!
//! Prefill and mixed steps call hip_attn_prefill_rows (hip_attn_prefill plus the step's single-row count, which
//! the executor records with step_hints.zig).  One more difference in what is issued: a decode step (one query token per sequence) calls
//! hip_attn_decode_store_kv, which writes the step's K/V into the cache and attends in one launch; the CUDA path
//! issues cuda_store_kv and then cuda_attn_decode.  Outputs and cache contents are the same.
//! Not compiled in this repository (no Zig toolchain here); tests/test_zig_binding.py checks every extern
//! against the C header.
const Tensor = @import("../../../Tensor.zig");
const common = @import("../../cpu/common.zig");

// ---- attention launchers (include/llmgen_attn.h) ----
pub extern fn hip_store_kv(
    k: ?*const anyopaque,
    v: ?*const anyopaque,
    slot_mapping: ?*const anyopaque,
    k_cache: ?*anyopaque,
    v_cache: ?*anyopaque,
    T: c_int,
    nkv: c_int,
    hd: c_int,
    block_size: c_int,
) void;

pub extern fn hip_attn_decode(
    out: ?*anyopaque,
    q: ?*const anyopaque,
    k_cache: ?*const anyopaque,
    v_cache: ?*const anyopaque,
    block_tables: ?*const anyopaque,
    ctx_lens: ?*const anyopaque,
    S: c_int,
    nq: c_int,
    nkv: c_int,
    hd: c_int,
    max_blocks: c_int,
    block_size: c_int,
    scale: f32,
    part_o: ?*anyopaque,
    part_ml: ?*anyopaque,
    part_size: c_int,
    max_parts: c_int,
) void;

pub extern fn hip_attn_decode_store_kv(
    out: ?*anyopaque,
    q: ?*const anyopaque,
    k: ?*const anyopaque,
    v: ?*const anyopaque,
    slot_mapping: ?*const anyopaque,
    k_cache: ?*anyopaque,
    v_cache: ?*anyopaque,
    block_tables: ?*const anyopaque,
    ctx_lens: ?*const anyopaque,
    S: c_int,
    nq: c_int,
    nkv: c_int,
    hd: c_int,
    max_blocks: c_int,
    block_size: c_int,
    scale: f32,
    part_o: ?*anyopaque,
    part_ml: ?*anyopaque,
    part_size: c_int,
    max_parts: c_int,
) void;

pub extern fn hip_attn_decode_noalloc(
    out: ?*anyopaque,
    q: ?*const anyopaque,
    k_cache: ?*const anyopaque,
    v_cache: ?*const anyopaque,
    block_tables: ?*const anyopaque,
    ctx_lens: ?*const anyopaque,
    S: c_int,
    nq: c_int,
    nkv: c_int,
    hd: c_int,
    max_blocks: c_int,
    block_size: c_int,
    scale: f32,
    part_size: c_int,
    max_parts: c_int,
) void;

pub extern fn hip_attn_prefill(
    out: ?*anyopaque,
    q: ?*const anyopaque,
    k_cache: ?*const anyopaque,
    v_cache: ?*const anyopaque,
    block_tables: ?*const anyopaque,
    ctx_lens: ?*const anyopaque,
    cu_q: ?*const anyopaque,
    tile_seq: ?*const anyopaque,
    tile_q0: ?*const anyopaque,
    n_tiles: c_int,
    nq: c_int,
    nkv: c_int,
    hd: c_int,
    max_blocks: c_int,
    block_size: c_int,
    scale: f32,
) void;

pub extern fn hip_attn_prefill_rows(
    out: ?*anyopaque,
    q: ?*const anyopaque,
    k_cache: ?*const anyopaque,
    v_cache: ?*const anyopaque,
    block_tables: ?*const anyopaque,
    ctx_lens: ?*const anyopaque,
    cu_q: ?*const anyopaque,
    tile_seq: ?*const anyopaque,
    tile_q0: ?*const anyopaque,
    n_tiles: c_int,
    nq: c_int,
    nkv: c_int,
    hd: c_int,
    max_blocks: c_int,
    block_size: c_int,
    scale: f32,
    single_rows: c_int,
) void;

pub extern fn hip_attn_prefill_tile() c_int;

/// The launch hip_attn_prefill_rows makes for a step of this shape (tests and tuning; no cuda_ counterpart).
pub extern fn hip_attn_prefill_plan(n_tiles: c_int, nq: c_int, nkv: c_int, hd: c_int, block_size: c_int,
    single_rows: c_int) c_int;

pub extern fn hip_attn_set_option(option: c_int, value: c_int) c_int;

/// Split-K part length and part count the engine sizes its scratch with (attention_v1.zig:51-57, unchanged:
/// executor.zig:92-102 sizes part_o / part_ml from them and the launcher accepts them as they are).
pub fn partSize(s: usize) usize {
    if (s >= 64) return 512;
    if (s >= 16) return 256;
    if (s >= 4) return 128;
    return 64;
}

pub fn maxParts(s: usize, max_model_len: usize) usize {
    const ps = partSize(s);
    return (max_model_len + ps - 1) / ps;
}

/// The step's count of single-row segments, if the engine's StepState carries it (a `single_rows: c_int = -1`
/// field added to common.zig's StepState, set by bindStep from step_hints.singleRows), else -1.
fn singleRowsOf(st: anytype) c_int {
    if (@hasField(@TypeOf(st.*), "single_rows")) return st.single_rows;
    return -1;
}

/// src[0] = q [1, T, nq, hd], src[1] = k [1, T, nkv, hd], src[2] = v [1, T, nkv, hd]; out.data = [1, T, nq, hd],
/// all bf16.  Errors as the CUDA implementation: error.NoAttentionManager / error.LayerNotActive from kvOf.
pub const PagedAttentionImpl = struct {
    pub fn execute(_: i32, out: *Tensor) !void {
        const st = &common.g_step;
        const layer = try common.kvOf(out.layer_id);
        const q = out.src[0].?.data;
        const k = out.src[1].?.data;
        const v = out.src[2].?.data;

        if (!st.decode) {
            // prefill or mixed step: write the step's rows into the paged cache, then causal varlen attention with
            // the step's single-row count (step_hints.zig; -1 = unknown when the executor does not record it)
            hip_store_kv(k, v, st.slots, layer.k, layer.v, st.n_tok, st.n_kv_head, st.head_dim, st.block_size);
            hip_attn_prefill_rows(out.data, q, layer.k, layer.v, st.block_tables, st.ctx, st.cu_q, st.tile_seq,
                st.tile_q0, st.n_tiles, st.n_head, st.n_kv_head, st.head_dim, st.max_blocks, st.block_size,
                st.attn_scale, singleRowsOf(st));
            return;
        }
        // decode step (also the body of a captured graph bucket): KV write and split-K decode in one launch
        const s: usize = @intCast(st.n_seq);
        hip_attn_decode_store_kv(out.data, q, k, v, st.slots, layer.k, layer.v, st.block_tables, st.ctx, st.n_seq,
            st.n_head, st.n_kv_head, st.head_dim, st.max_blocks, st.block_size, st.attn_scale, st.part_o, st.part_ml,
            @intCast(partSize(s)), @intCast(maxParts(s, st.max_model_len)));
    }
};

/// The FLASH_ATTN graph node (LLMGEN_FLASH=1) runs the same implementation (attention_v1.zig:123).
pub const FlashAttentionImpl = PagedAttentionImpl;
