"""The C++ executor slice (include/llmgen_host.h) -- host logic on the CPU, no GPU calls.

Pinned against the reference's own worked example of the metadata layout (the comment at
src/executor.zig:776-797: T=6, S=3, n_tiles=3, max_blocks=4 -> total 204 bytes), against the independent Python
restatement in llmgen_amd/step.py (fill_meta, decode_buckets, workspace_bytes), and against hand-computed pass
splits of src/executor.zig:986-1043.
"""
from __future__ import annotations

import numpy as np
import pytest

from llmgen_amd import host as H
from llmgen_amd import step as S


def test_layout_matches_reference_worked_example():
    lay = H.layout(6, 3, 3, 4).as_dict()
    assert lay == {"seed": 0, "ids": 8, "pos": 32, "slots": 56, "cu_q": 80, "ctx": 96, "last": 108, "temps": 120,
                   "tile_seq": 132, "tile_q0": 144, "bt": 156, "total": 204}


def _mixed():
    rng = np.random.default_rng(0)
    seqs = [H.Sequence_(rng.integers(0, 1000, 130).tolist(), [3, 1, 4, 0, 2, 7, 5, 6, 8], 0.7),
            H.Sequence_(rng.integers(0, 1000, 41).tolist(), [9, 10, 11], 0.0),
            H.Sequence_(rng.integers(0, 1000, 64).tolist(), [12, 13, 14, 15], 1.0)]
    # seq0 prefills positions 60..129 (chunk, emits), seq1 decodes position 40, seq2 prefills 0..63 (emits)
    entries = [(0, 60, 70), (1, 40, 1), (2, 0, 64)]
    return seqs, entries


def test_fill_meta_matches_python_restatement_mixed_step():
    seqs, entries = _mixed()
    bs, mb, tile = 16, 10, 64
    n_tiles = sum((e[2] + tile - 1) // tile for e in entries)
    buf, lay, seed, _ = H.fill_meta(seqs, entries, len(entries), n_tiles, tile, bs, mb, step_seed=5)
    n_tok = sum(e[2] for e in entries)
    seg = H.segments(buf, lay, n_tok, len(entries), n_tiles, mb)
    py = S.fill_meta([S.Entry(e[1], e[2], seqs[e[0]].block_table) for e in entries], bs, mb, tile,
                     decode=False)
    for name in ("slots", "cu_q", "ctx", "last", "tile_seq", "tile_q0", "pos"):
        np.testing.assert_array_equal(seg[name], getattr(py, name), err_msg=name)
    np.testing.assert_array_equal(seg["block_tables"], py.block_tables)
    # ids / temps / seed (not in the attention-only Python restatement)
    expect_ids = np.concatenate([np.asarray(seqs[s].token_ids)[q0:q0 + ql] for s, q0, ql in entries])
    np.testing.assert_array_equal(seg["ids"], expect_ids)
    np.testing.assert_array_equal(seg["temps"], np.float32([0.7, 0.0, 1.0]))
    assert seed == (5 + 0x9E3779B97F4A7C15) % 2 ** 64 and seg["seed"] == seed


def test_fill_meta_decode_bucket_padding():
    seqs = [H.Sequence_(list(range(100)), [2, 0], 0.0), H.Sequence_(list(range(11)), [1], 0.0)]
    entries = [(0, 99, 1), (1, 10, 1)]
    buf, lay, _, single = H.fill_meta(seqs, entries, 4, 0, 64, 64, 2)
    assert single == 4
    seg = H.segments(buf, lay, 4, 4, 0, 2)
    py = S.fill_meta([S.Entry(99, 1, [2, 0]), S.Entry(10, 1, [1])], 64, 2, 64, seq_num=4)
    for name in ("slots", "cu_q", "ctx", "last"):
        np.testing.assert_array_equal(seg[name], getattr(py, name), err_msg=name)
    assert list(seg["slots"]) == [0 * 64 + 35, 1 * 64 + 10, -1, -1]
    assert list(seg["ids"]) == [99, 10, 0, 0] and not seg["block_tables"][2:].any()
    # the bucket layout does not depend on the entries: a step with fewer sequences reuses it
    buf2, lay2, _, _ = H.fill_meta([], [], 4, 0, 64, 64, 2)
    assert lay2.as_dict() == lay.as_dict()


def test_fill_meta_rejects_bad_steps():
    seqs = [H.Sequence_(list(range(10)), [0], 0.0)]
    with pytest.raises(ValueError):
        H.fill_meta(seqs, [(0, 5, 10)], 1, 1, 64, 16, 1)  # runs past the sequence's tokens
    with pytest.raises(ValueError):
        H.fill_meta(seqs, [(0, 9, 1), (0, 9, 1)], 1, 0, 64, 16, 1)  # seq_num < entries


def test_decode_step_rule_and_emits():
    seqs = [H.Sequence_(list(range(10)), [0], 0.0), H.Sequence_(list(range(5)), [1], 0.0)]
    L = H.L()
    sa = H._SeqArray(seqs)
    dec = H._entries([(0, 9, 1), (1, 4, 1)])
    assert L.llmgen_step_is_decode(sa.arr, dec, 2) == 1
    not_last = H._entries([(0, 8, 1)])  # a one-token chunk that does not reach the end: not a decode step
    assert L.llmgen_step_is_decode(sa.arr, not_last, 1) == 0
    assert L.llmgen_entry_emits(sa.arr, not_last) == 0
    assert L.llmgen_step_tiles(H._entries([(0, 0, 65), (1, 0, 5)]), 2, 64) == 3


def test_plan_passes_splits_at_max_tokens():
    entries = [(0, 0, 100), (1, 40, 1), (2, 0, 300)]
    got = H.plan_passes(entries, 128)
    # pass 0: e0 [0,100) + e1 [40,41) + e2 [0,27); pass 1: e2 [27,155); pass 2: e2 [155,283); pass 3: e2 [283,300)
    assert got == [(0, 0, (0, 0, 100)), (0, 1, (1, 40, 1)), (0, 2, (2, 0, 27)), (1, 2, (2, 27, 128)),
                   (2, 2, (2, 155, 128)), (3, 2, (2, 283, 17))]
    assert H.plan_passes(entries, 10_000) == [(0, i, e) for i, e in enumerate(entries)]


def test_buckets_and_workspace_match_python():
    for m in (1, 3, 8, 40, 64, 100):
        assert H.decode_buckets(m) == S.decode_buckets(m)
    w = H.workspace(16, 128, 32, 2048, 4096, 16)
    po, pml = S.workspace_bytes(16, 128, 32, 4096)
    assert (w["part_o"], w["part_ml"]) == (po, pml)
    assert w["meta"] == H.layout(2048, 32, 2048 // 64 + 32, 4096 // 16).total
    assert H.L().llmgen_part_size(16) == S.part_size(16) and H.L().llmgen_max_parts(5, 1000) == S.max_parts(5, 1000)


def test_single_rows_counts_one_row_segments():
    """llmgen_single_rows (the count hip_attn_prefill_rows takes) equals the one-row segments of the packed
    cu_q, for a mixed step and for a padded decode bucket."""
    seqs, entries = _mixed()
    tile, bs, mb = 64, 16, 10
    n_tiles = sum((e[2] + tile - 1) // tile for e in entries)
    buf, lay, _, single = H.fill_meta(seqs, entries, len(entries), n_tiles, tile, bs, mb)
    seg = H.segments(buf, lay, sum(e[2] for e in entries), len(entries), n_tiles, mb)
    expect = int(np.count_nonzero(np.diff(seg["cu_q"]) == 1))
    assert H.single_rows(entries, len(entries)) == expect == single
    py = S.fill_meta([S.Entry(e[1], e[2], seqs[e[0]].block_table) for e in entries], bs, mb, tile, decode=False)
    assert py.single_rows() == expect
    # padding rows of a bucket are one-row segments too
    assert H.single_rows([(0, 99, 1), (1, 10, 1)], 4) == 4
    assert H.single_rows([(0, 0, 70)], 1) == 0


def test_fill_meta_prefill_padding_rows_get_tiles():
    """A prefill step with padding rows (not an engine step, but legal): each padding row gets a tile, the tile
    list (lightest first, padding rows first) equals the Python restatement's, and the single-row count covers
    the padding rows; a tile count without room for them is rejected."""
    seqs, entries = _mixed()
    tile, bs, mb = 64, 16, 10
    n_pad = 2
    n_tiles = sum((e[2] + tile - 1) // tile for e in entries) + n_pad
    seq_num = len(entries) + n_pad
    buf, lay, _, single = H.fill_meta(seqs, entries, seq_num, n_tiles, tile, bs, mb)
    n_tok = sum(e[2] for e in entries) + n_pad
    seg = H.segments(buf, lay, n_tok, seq_num, n_tiles, mb)
    py = S.fill_meta([S.Entry(e[1], e[2], seqs[e[0]].block_table) for e in entries], bs, mb, tile,
                     seq_num=seq_num, decode=False)
    for name in ("slots", "cu_q", "ctx", "last", "tile_seq", "tile_q0"):
        np.testing.assert_array_equal(seg[name], getattr(py, name), err_msg=name)
    assert single == py.single_rows() == H.single_rows(entries, seq_num)
    assert set(seg["tile_seq"][:n_pad]) == {len(entries), len(entries) + 1}
    with pytest.raises(ValueError):
        H.fill_meta(seqs, entries, seq_num, n_tiles - 1, tile, bs, mb)
