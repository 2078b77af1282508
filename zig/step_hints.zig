//! step_hints.zig -- the two facts about a step that the HIP prefill launcher uses and the engine's executor
//! knows while it packs the step (src/executor.zig:772-861 fillMeta), written for that executor:
//!
//!   * singleRows: how many segments of the step have one query row (decode rows of a mixed step, and graph
//!     padding rows).  hip_attn_prefill_rows takes it: 0 skips the launch that streams such rows (a grid of
//!     workgroups that would find nothing to do) and lets small pure-prefill steps take the key-split kernel.
//!   * sortTilesLightestFirst: reorder the packed prefill tiles: single-row tiles first, then the multi-row ones,
//!     each part lightest first (by the number of keys a tile needs) and stable.  The launcher sizes the two parts
//!     of the mixed-step grid from singleRows, and the kernels walk each part from its end, so the longest decode
//!     rows and the heaviest prefill tiles (a long prompt's last ones) start first.  Any order is valid for the
//!     kernels; this one is faster.
//! Both are the C++ executor slice's behaviour (llmgen_amd/csrc/executor.cpp llmgen_fill_meta /
//! llmgen_single_rows), restated for the Zig executor.  Neither allocates.  Not compiled in this repository (no Zig
//! toolchain here).

/// Segments with one query row: entries with q_len == 1, plus the seq_num - entries.len padding rows of a graph
/// bucket.  `entries` is any slice whose elements have a `q_len` field (executor.zig's Entry).
pub fn singleRows(entries: anytype, seq_num: usize) c_int {
    var n: usize = if (seq_num > entries.len) seq_num - entries.len else 0;
    for (entries) |e| {
        if (e.q_len == 1) n += 1;
    }
    return @intCast(n);
}

/// Ordering key of tile i: single-row tiles before multi-row ones, then the keys the tile needs (its sequence's
/// context minus the rows after the tile).
fn tileKey(tseq: [*]const i32, tq0: [*]const i32, cu_q: [*]const i32, ctx: [*]const i32, pf_tile: usize, i: usize) i64 {
    const s: usize = @intCast(tseq[i]);
    const q_len = cu_q[s + 1] - cu_q[s];
    const tile_end = @min(tq0[i] + @as(i32, @intCast(pf_tile)), q_len);
    const keys: i64 = ctx[s] - q_len + tile_end;
    const multi: i64 = if (q_len > 1) 1 else 0;
    return (multi << 32) + keys;
}

/// Stable insertion sort of the n_tiles packed tiles (tile_seq / tile_q0 segments of the metadata) by tileKey.
/// Tiles of one sequence are already in increasing order, so the sort only interleaves sequences; a step has at
/// most max_tokens / pf_tile + max_seqs tiles.
pub fn sortTilesLightestFirst(tseq: [*]i32, tq0: [*]i32, n_tiles: usize, cu_q: [*]const i32, ctx: [*]const i32,
    pf_tile: usize) void {
    var i: usize = 1;
    while (i < n_tiles) : (i += 1) {
        const key = tileKey(tseq, tq0, cu_q, ctx, pf_tile, i);
        const s = tseq[i];
        const q0 = tq0[i];
        var j = i;
        while (j > 0 and tileKey(tseq, tq0, cu_q, ctx, pf_tile, j - 1) > key) : (j -= 1) {
            tseq[j] = tseq[j - 1];
            tq0[j] = tq0[j - 1];
        }
        tseq[j] = s;
        tq0[j] = q0;
    }
}
