"""Per-step metadata the attention path consumes, restated from the reference executor in Python.

The product path builds this metadata in C++ (``llmgen_fill_meta``, include/llmgen_host.h); this module is an
independent restatement that the tests hold the C++ one against and that feeds the CPU oracle's inputs.

* :func:`part_size` / :func:`max_parts` -- split-K part length and count (``attention_v1.zig:51-57``).
* :func:`workspace_bytes` -- split-K scratch sizing (``executor.zig:92-102``).
* :func:`slot_of` -- logical position -> KV slot (``runner/batching.zig:74-77``).
* :class:`Entry`, :func:`fill_meta` -- the packed step metadata (``executor.zig:139-202`` Layout,
  ``executor.zig:772-861`` fillMeta): token slots, ``cu_q``, ``ctx``, ``last``, prefill tiles and the block
  table, with CUDA-graph padding rows (``ctx = 0``, ``slot = -1``).
* :func:`decode_buckets` -- the graph bucket sizes of ``executor.zig:609-632``.

All arrays are numpy int32 so they can be uploaded with one host-to-device copy.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np


def part_size(n_seq: int) -> int:
    """attention_v1.zig:51-53: finer split-K parts for small batches so the grid fills the GPU."""
    if n_seq >= 64:
        return 512
    if n_seq >= 16:
        return 256
    if n_seq >= 4:
        return 128
    return 64


def max_parts(n_seq: int, max_model_len: int) -> int:
    """attention_v1.zig:54-57."""
    ps = part_size(n_seq)
    return (max_model_len + ps - 1) // ps


def workspace_bytes(nq: int, hd: int, max_seqs: int, max_model_len: int):
    """executor.zig:92-102: part_o / part_ml bytes sized for the worst S x max_parts(S) over 1..max_seqs."""
    cap = max(s * max_parts(s, max_model_len) for s in range(1, max_seqs + 1))
    return cap * nq * hd * 4, cap * nq * 2 * 4


def slot_of(block_table: Sequence[int], pos: int, block_size: int) -> int:
    """runner/batching.zig:74-77: slot = block_table[pos / bs] * bs + pos % bs."""
    return int(block_table[pos // block_size]) * block_size + pos % block_size


def decode_buckets(max_seqs: int) -> List[int]:
    """executor.zig:614-632: 1, 2, 4, 8, then multiples of 16 up to max_seqs, plus max_seqs itself."""
    out = [b for b in (1, 2, 4, 8) if b <= max_seqs]
    b = 16
    while b <= max_seqs:
        out.append(b)
        b += 16
    if not out or out[-1] != max_seqs:
        out.append(max_seqs)
    return out


@dataclass
class Entry:
    """One sequence's share of a step (runner/batching.zig:93-103): this step computes positions
    [q_start, q_start + q_len) and afterwards the sequence holds q_start + q_len keys."""

    q_start: int
    q_len: int
    block_table: List[int]
    emits: bool = True


@dataclass
class StepMeta:
    n_tok: int
    n_seq: int
    n_tiles: int
    decode: bool
    slots: np.ndarray
    cu_q: np.ndarray
    ctx: np.ndarray
    last: np.ndarray
    tile_seq: np.ndarray
    tile_q0: np.ndarray
    block_tables: np.ndarray  # [n_seq, max_blocks]
    pos: Optional[np.ndarray] = None  # [n_tok] position of each token in its sequence (padding rows: 0)
    offsets: dict = field(default_factory=dict)

    def single_rows(self) -> int:
        """Segments with one query row (decode rows of a mixed step, padding rows)."""
        return int(np.count_nonzero(np.diff(self.cu_q[:self.n_seq + 1]) == 1))

    def packed(self) -> np.ndarray:
        """One contiguous int32 buffer in Layout order (executor.zig:139-202, without ids/temps/seed, which
        attention does not read); offsets (in int32 elements) are recorded in ``self.offsets``."""
        pos = self.pos if self.pos is not None else np.zeros(self.n_tok, np.int32)
        parts = [("pos", pos), ("slots", self.slots), ("cu_q", self.cu_q), ("ctx", self.ctx), ("last", self.last),
                 ("tile_seq", self.tile_seq), ("tile_q0", self.tile_q0),
                 ("block_tables", self.block_tables.reshape(-1))]
        off = 0
        for name, arr in parts:
            self.offsets[name] = off
            off += arr.size
        buf = np.zeros(max(off, 1), np.int32)
        for name, arr in parts:
            buf[self.offsets[name]:self.offsets[name] + arr.size] = arr
        return buf


def fill_meta(entries: Sequence[Entry], block_size: int, max_blocks: int, pf_tile: int,
              seq_num: Optional[int] = None, decode: Optional[bool] = None) -> StepMeta:
    """executor.zig:530-552 + 772-861, except that prefill tiles are listed single-row tiles first, then multi-row
    ones, each part lightest first (stable), rather than in entry order, so that the kernels' last-first dispatch is
    longest / heaviest first.

    ``decode`` defaults to the engine's rule (every entry has q_len == 1 and emits).  ``seq_num`` >= len(entries)
    adds padding rows (one token each, ctx = 0, slot = -1, zero block-table row) as for a graph bucket.  Prefill
    tiles are produced only for non-decode steps.
    """
    if decode is None:
        decode = all(e.q_len == 1 and e.emits for e in entries)
    n_seq = len(entries) if seq_num is None else seq_num
    assert n_seq >= len(entries)
    n_tok_real = sum(e.q_len for e in entries)
    n_tok = n_tok_real + (n_seq - len(entries))
    n_pad = n_seq - len(entries)
    # padding rows of a prefill step get a tile of their own so the kernel writes their zero rows (the CPU
    # backend writes zeros for every row with ctx < q_len); the engine only pads decode steps
    n_tiles = 0 if decode else sum((e.q_len + pf_tile - 1) // pf_tile for e in entries) + n_pad

    slots = np.empty(n_tok, np.int32)
    posv = np.zeros(n_tok, np.int32)
    cu_q = np.zeros(n_seq + 1, np.int32)
    ctx = np.zeros(n_seq, np.int32)
    last = np.zeros(n_seq, np.int32)
    tile_seq = np.zeros(n_tiles, np.int32)
    tile_q0 = np.zeros(n_tiles, np.int32)
    bt = np.zeros((n_seq, max_blocks), np.int32)

    t = 0
    tile = 0
    for si, e in enumerate(entries):
        nb = len(e.block_table)
        assert nb <= max_blocks, "block table longer than max_blocks"
        pos = np.arange(e.q_start, e.q_start + e.q_len)
        table = np.asarray(e.block_table, np.int64)
        slots[t:t + e.q_len] = table[pos // block_size] * block_size + pos % block_size
        posv[t:t + e.q_len] = pos
        t += e.q_len
        cu_q[si + 1] = t
        ctx[si] = e.q_start + e.q_len
        last[si] = t - 1
        bt[si, :nb] = e.block_table
        if n_tiles > 0:
            for q0 in range(0, e.q_len, pf_tile):
                tile_seq[tile] = si
                tile_q0[tile] = q0
                tile += 1
    for si in range(len(entries), n_seq):  # padding rows
        slots[t] = -1
        if n_tiles > 0:
            tile_seq[tile] = si
            tile_q0[tile] = 0
            tile += 1
        t += 1
        cu_q[si + 1] = t
        ctx[si] = 0
        last[si] = t - 1
    if n_tiles > 1:
        # single-row tiles first, then multi-row ones, each part lightest first by the keys a tile needs (stable);
        # the kernels walk each part from its end
        q_lens = np.diff(cu_q)[tile_seq]
        kend = ctx[tile_seq] - q_lens + np.minimum(tile_q0 + pf_tile, q_lens)
        order = np.lexsort((kend, q_lens > 1))
        tile_seq, tile_q0 = tile_seq[order].copy(), tile_q0[order].copy()
    return StepMeta(n_tok=n_tok, n_seq=n_seq, n_tiles=n_tiles, decode=decode, slots=slots, cu_q=cu_q, ctx=ctx,
                    last=last, tile_seq=tile_seq, tile_q0=tile_q0, block_tables=bt, pos=posv)
