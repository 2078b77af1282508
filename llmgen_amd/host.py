"""ctypes front end of the C++ executor slice (include/llmgen_host.h, llmgen_amd/csrc/executor.cpp).

The engine's executor (``src/executor.zig``) packs each step's metadata, binds it for the kernels, dispatches
attention per layer, splits oversized batches into passes and replays decode steps from graph buckets.  That
slice is implemented in C++ inside libllmgen_attn.so; this module exposes it to Python with the same names:

* :func:`layout`, :func:`fill_meta` -- ``Layout.init`` and ``fillMeta`` (executor.zig:139-202, 772-861);
* :class:`StepState`, :func:`bind_step`, :func:`paged_attention` -- ``bindStep`` and
  ``PagedAttentionImpl.execute`` (executor.zig:864-895, attention_v1.zig:60-120);
* :func:`plan_passes`, :func:`decode_buckets`, :func:`workspace` -- ``execute``/``flushPass``, ``captureGraphs``
  bucket sizes and ``Workspace.of`` (executor.zig:986-1043, 609-632, 92-102);
* :class:`Graphs` -- decode graph buckets (captureGraphs + forward's replay path).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Sequence

import numpy as np

from ._lib import lib

_sz = ctypes.c_size_t
_i32 = ctypes.c_int32
_P = ctypes.c_void_p


class Layout(ctypes.Structure):
    _fields_ = [(n, _sz) for n in ("seed", "ids", "pos", "slots", "cu_q", "ctx", "last", "temps", "tile_seq",
                                   "tile_q0", "bt", "total")]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


class Seq(ctypes.Structure):
    _fields_ = [("token_ids", _P), ("n_tokens", _i32), ("block_table", _P), ("n_blocks", _i32),
                ("temperature", ctypes.c_float)]


class Entry(ctypes.Structure):
    _fields_ = [("seq", _i32), ("q_start", _i32), ("q_len", _i32)]


class StepState(ctypes.Structure):
    """common.zig:10-41."""
    _fields_ = ([(n, _i32) for n in ("n_tok", "n_seq", "n_tiles", "decode", "hidden", "n_head", "n_kv_head",
                                     "head_dim")]
                + [("attn_scale", ctypes.c_float), ("block_size", _i32), ("max_blocks", _i32),
                   ("max_model_len", _sz)]
                + [(n, _P) for n in ("seed", "pos", "slots", "cu_q", "ctx", "last", "temps", "tile_seq", "tile_q0",
                                     "block_tables", "cos_sin", "part_o", "part_ml", "sample_scratch")]
                + [("single_rows", _i32)])


HOST_SIGNATURES = {
    "llmgen_layout_init": (Layout, [_sz, _sz, _sz, _sz]),
    "llmgen_entry_emits": (ctypes.c_int, [ctypes.POINTER(Seq), ctypes.POINTER(Entry)]),
    "llmgen_step_is_decode": (ctypes.c_int, [ctypes.POINTER(Seq), ctypes.POINTER(Entry), ctypes.c_int]),
    "llmgen_step_tiles": (ctypes.c_int, [ctypes.POINTER(Entry), ctypes.c_int, ctypes.c_int]),
    "llmgen_single_rows": (ctypes.c_int, [ctypes.POINTER(Entry), ctypes.c_int, ctypes.c_int]),
    "llmgen_fill_meta": (ctypes.c_int, [_P, Layout, ctypes.POINTER(Seq), ctypes.POINTER(Entry), ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.POINTER(ctypes.c_uint64)]),
    "llmgen_bind_step": (None, [ctypes.POINTER(StepState), _P, Layout] + [ctypes.c_int] * 10
                         + [_sz, _P, _P, _P, ctypes.c_int]),
    "llmgen_paged_attention": (ctypes.c_int, [ctypes.POINTER(StepState), _P, _P, _P, _P, _P, _P, ctypes.c_int]),
    "llmgen_part_size": (ctypes.c_int, [ctypes.c_int]),
    "llmgen_max_parts": (ctypes.c_int, [ctypes.c_int, _sz]),
    "llmgen_workspace": (None, [ctypes.c_int, ctypes.c_int, ctypes.c_int, _sz, _sz, ctypes.c_int, ctypes.c_int,
                                ctypes.POINTER(_sz)]),
    "llmgen_decode_buckets": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.c_int]),
    "llmgen_plan_passes": (ctypes.c_int, [ctypes.POINTER(Entry), ctypes.c_int, _sz, ctypes.POINTER(Entry),
                                          ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int), ctypes.c_int]),
    "llmgen_graphs_create": (_P, [ctypes.c_int, ctypes.POINTER(_P), ctypes.POINTER(_P)] + [ctypes.c_int] * 4
                             + [_sz, ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.c_int]),
    "llmgen_graphs_step": (ctypes.c_int, [_P, ctypes.POINTER(Seq), ctypes.POINTER(Entry), ctypes.c_int, _P, _P, _P,
                                          _P]),
    "llmgen_graphs_replay": (ctypes.c_int, [_P]),
    "llmgen_graphs_destroy": (None, [_P]),
}

_bound = False


def L():
    """The library with the host-slice signatures attached."""
    global _bound
    h = lib()
    if not _bound:
        for name, (res, args) in HOST_SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _bound = True
    return h


@dataclass
class Sequence_:
    """A sequence: all token ids so far (prompt + generated), its block table, sampling temperature."""

    token_ids: List[int]
    block_table: List[int]
    temperature: float = 0.0


class _SeqArray:
    """Keeps the numpy buffers alive while the C structs point at them."""

    def __init__(self, seqs: Sequence[Sequence_]):
        self.bufs = []
        arr = (Seq * max(len(seqs), 1))()
        for i, s in enumerate(seqs):
            ids = np.ascontiguousarray(s.token_ids, np.int32)
            bt = np.ascontiguousarray(s.block_table, np.int32)
            self.bufs += [ids, bt]
            arr[i] = Seq(ids.ctypes.data, ids.size, bt.ctypes.data, bt.size, float(s.temperature))
        self.arr = arr


def _entries(entries) -> ctypes.Array:
    arr = (Entry * max(len(entries), 1))()
    for i, e in enumerate(entries):
        arr[i] = Entry(*e) if isinstance(e, tuple) else e
    return arr


def layout(n_tok: int, n_seq: int, n_tiles: int, max_blocks: int) -> Layout:
    return L().llmgen_layout_init(n_tok, n_seq, n_tiles, max_blocks)


def fill_meta(seqs: Sequence[Sequence_], entries, seq_num: int, n_tiles: int, pf_tile: int, block_size: int,
              max_blocks: int, step_seed: int = 0):
    """Returns (packed bytes as a uint8 array, layout, new step seed, the step's single-row count)."""
    n_tok = sum(e[2] for e in entries) + (seq_num - len(entries))  # padding rows carry one token each
    lay = layout(n_tok, seq_num, n_tiles, max_blocks)
    buf = np.zeros(lay.total, np.uint8)
    sa = _SeqArray(seqs)
    seed = ctypes.c_uint64(step_seed)
    rc = L().llmgen_fill_meta(buf.ctypes.data, lay, sa.arr, _entries(entries), len(entries), seq_num, n_tiles,
                              pf_tile, block_size, max_blocks, ctypes.byref(seed))
    if rc < 0:
        raise ValueError(f"llmgen_fill_meta rejected the step (rc={rc})")
    return buf, lay, seed.value, rc


def single_rows(entries, seq_num: int) -> int:
    """Segments of the step with one query row (entries with q_len == 1, plus padding rows)."""
    return L().llmgen_single_rows(_entries(entries), len(entries), seq_num)


def segments(buf: np.ndarray, lay: Layout, n_tok: int, n_seq: int, n_tiles: int, max_blocks: int) -> dict:
    """Views of the packed metadata's segments."""
    def i32(off, n):
        return buf[off:off + 4 * n].view(np.int32)
    return {"seed": int(buf[:8].view(np.uint64)[0]), "ids": i32(lay.ids, n_tok), "pos": i32(lay.pos, n_tok),
            "slots": i32(lay.slots, n_tok), "cu_q": i32(lay.cu_q, n_seq + 1), "ctx": i32(lay.ctx, n_seq),
            "last": i32(lay.last, n_seq), "temps": buf[lay.temps:lay.temps + 4 * n_seq].view(np.float32),
            "tile_seq": i32(lay.tile_seq, n_tiles), "tile_q0": i32(lay.tile_q0, n_tiles),
            "block_tables": i32(lay.bt, n_seq * max_blocks).reshape(n_seq, max_blocks)}


def plan_passes(entries, max_tokens: int):
    """Returns [(pass, owner, (seq, q_start, q_len))...] in order."""
    cap = sum(e[2] for e in entries) // max(max_tokens, 1) + len(entries) + 2
    pieces, owner, pas = (Entry * cap)(), (ctypes.c_int * cap)(), (ctypes.c_int * cap)()
    n = L().llmgen_plan_passes(_entries(entries), len(entries), max_tokens, pieces, owner, pas, cap)
    if n < 0:
        raise ValueError("plan_passes failed")
    return [(pas[i], owner[i], (pieces[i].seq, pieces[i].q_start, pieces[i].q_len)) for i in range(n)]


def decode_buckets(max_seqs: int) -> List[int]:
    out = (ctypes.c_int * 256)()
    n = L().llmgen_decode_buckets(max_seqs, out, 256)
    return list(out[:n])


def workspace(n_head, head_dim, max_seqs, max_tokens, max_model_len, block_size, pf_tile=64):
    out = (_sz * 4)()
    L().llmgen_workspace(n_head, head_dim, max_seqs, max_tokens, max_model_len, block_size, pf_tile, out)
    return {"meta": out[0], "part_o": out[1], "part_ml": out[2], "sample": out[3]}


def bind_step(meta_dev_ptr: int, lay: Layout, n_tok, n_seq, n_tiles, decode, n_head, n_kv_head, head_dim,
              block_size, max_blocks, max_model_len, part_o=0, part_ml=0, sample_scratch=0,
              hidden: int = 0, single_rows: int = -1) -> StepState:
    """``single_rows``: llmgen_fill_meta's return value for this step (-1 if unknown)."""
    st = StepState()
    L().llmgen_bind_step(ctypes.byref(st), meta_dev_ptr, lay, n_tok, n_seq, n_tiles, int(decode), hidden, n_head,
                         n_kv_head, head_dim, block_size, max_blocks, max_model_len, part_o, part_ml, sample_scratch,
                         single_rows)
    return st


def paged_attention(st: StepState, out, q, k, v, k_cache, v_cache, store_kv: bool = True) -> None:
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    rc = L().llmgen_paged_attention(ctypes.byref(st), p(out), p(q), p(k), p(v), p(k_cache), p(v_cache),
                                    int(store_kv))
    if rc != 0:
        raise ValueError(f"llmgen_paged_attention rejected its arguments (rc={rc})")


class Graphs:
    """Decode graph buckets over a list of layers' KV pools (C++: llmgen_graphs_*)."""

    def __init__(self, k_caches, v_caches, n_head, n_kv_head, head_dim, block_size, max_model_len, max_seqs,
                 buckets=None):
        n = len(k_caches)
        kp = (_P * n)(*[t.data_ptr() for t in k_caches])
        vp = (_P * n)(*[t.data_ptr() for t in v_caches])
        b = None if buckets is None else (ctypes.c_int * len(buckets))(*buckets)
        self._keep = (k_caches, v_caches)
        self.h = L().llmgen_graphs_create(n, kp, vp, n_head, n_kv_head, head_dim, block_size, max_model_len,
                                          max_seqs, b, 0 if buckets is None else len(buckets))
        if not self.h:
            raise RuntimeError("llmgen_graphs_create failed")

    def step(self, seqs: Sequence[Sequence_], entries, q, k, v, out) -> int:
        sa = _SeqArray(seqs)
        rc = L().llmgen_graphs_step(self.h, sa.arr, _entries(entries), len(entries), q.data_ptr(), k.data_ptr(),
                                    v.data_ptr(), None if out is None else out.data_ptr())
        if rc < 0:
            raise ValueError(f"llmgen_graphs_step failed (rc={rc})")
        self._sa = sa  # the pinned upload was issued from host memory owned by the library; keep ids alive anyway
        return rc

    def replay(self) -> int:
        return L().llmgen_graphs_replay(self.h)

    def destroy(self) -> None:
        if self.h:
            L().llmgen_graphs_destroy(self.h)
            self.h = None
