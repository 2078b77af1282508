"""hipGraph decode buckets for the attention step, mirroring the engine's captureGraphs / forward replay.

``executor.zig:609-660`` records one graph per decode batch-size bucket (1, 2, 4, 8, 16, 32, ...): it fills the
step metadata with padding rows only (ctx = 0, slot = -1), runs the nodes once eagerly to warm up, then
captures them on the global stream.  ``executor.zig:541-575`` picks the smallest bucket >= S, rewrites the
metadata in place (same layout, so the recorded pointers stay valid) with one host-to-device copy, and replays.

Here the recorded nodes are the attention steps (store_kv + split-K decode) of one or more layers -- the engine
records all decoder layers of a step in one graph, each layer with its own KV pools -- with buffers owned by
the bucket (q / k / v / out of ``bucket`` rows, the packed metadata and the split-K scratch), exactly the fixed
pointers the engine's activation pool gives the captured kernels.
"""
from __future__ import annotations

import bisect
from dataclasses import dataclass
from typing import Dict, List, Sequence

import torch

from . import attention as A
from . import step as stepmod
from ._lib import lib


@dataclass
class Bucket:
    size: int
    graph: int
    meta: stepmod.StepMeta
    meta_dev: torch.Tensor
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    out: torch.Tensor
    ws: A.Workspace


class DecodeGraphs:
    """Captured store_kv + decode steps, one per bucket size, over one layer's KV pools."""

    def __init__(self, layer, nq: int, nkv: int, hd: int, block_size: int, max_blocks: int,
                 max_model_len: int, max_seqs: int, buckets: Sequence[int] = None):
        """``layer``: one LayerState, or a list of them (one per decoder layer, recorded in order)."""
        A.init_device()
        self.layers = list(layer) if isinstance(layer, (list, tuple)) else [layer]
        self.layer, self.nq, self.nkv, self.hd = self.layers[0], nq, nkv, hd
        self.block_size, self.max_blocks, self.max_model_len = block_size, max_blocks, max_model_len
        sizes = list(buckets) if buckets is not None else stepmod.decode_buckets(max_seqs)
        self.buckets: Dict[int, Bucket] = {}
        for bs in sizes:
            self.buckets[bs] = self._capture(bs)
        self.sizes: List[int] = sorted(self.buckets)

    def _run_nodes(self, b: Bucket) -> None:
        mgr = A.PagedAttentionManager()
        for i, st in enumerate(self.layers):
            mgr.layers[i] = st
        A.g_attn_mgr = mgr
        for i in range(len(self.layers)):
            A.PagedAttentionImpl.execute(0, A.AttnNode(b.out, [b.q, b.k, b.v], layer_id=i))

    def _capture(self, size: int) -> Bucket:
        dev = self.layer.k.device
        meta = stepmod.fill_meta([], self.block_size, self.max_blocks, 64, seq_num=size, decode=True)
        buf = meta.packed()
        ws = A.Workspace.allocate(self.nq, self.hd, size, self.max_model_len, meta_elems=buf.size, device=dev)
        bf = torch.bfloat16
        b = Bucket(size=size, graph=0, meta=meta, meta_dev=ws.meta,
                   q=torch.zeros(size, self.nq, self.hd, dtype=bf, device=dev),
                   k=torch.zeros(size, self.nkv, self.hd, dtype=bf, device=dev),
                   v=torch.zeros(size, self.nkv, self.hd, dtype=bf, device=dev),
                   out=torch.zeros(size, self.nq, self.hd, dtype=bf, device=dev), ws=ws)
        A.bind_step(meta, ws, self.nq, self.nkv, self.hd, self.block_size, self.max_blocks, self.max_model_len)
        self._run_nodes(b)  # warm-up with padding rows only: no KV is read or written
        torch.cuda.synchronize()
        L = lib()
        if L.hip_graph_begin() != 0:
            raise RuntimeError("hip_graph_begin failed")
        self._run_nodes(b)  # recorded, not executed
        g = L.hip_graph_end()
        if not g:
            raise RuntimeError("hip_graph_end failed")
        b.graph = g
        return b

    def bucket_for(self, n_seq: int) -> Bucket:
        i = bisect.bisect_left(self.sizes, n_seq)
        if i == len(self.sizes):
            raise ValueError(f"no decode bucket for {n_seq} sequences")
        return self.buckets[self.sizes[i]]

    def prepare(self, entries: Sequence[stepmod.Entry], q: torch.Tensor, k: torch.Tensor,
                v: torch.Tensor) -> Bucket:
        """fillMeta + uploadMeta for a decode step, and copy this step's q / k / v into the bucket's buffers."""
        b = self.bucket_for(len(entries))
        meta = stepmod.fill_meta(entries, self.block_size, self.max_blocks, 64, seq_num=b.size, decode=True)
        buf = meta.packed()
        assert meta.offsets == b.meta.offsets, "bucket layout changed"
        b.meta_dev[:buf.size].copy_(torch.from_numpy(buf))
        n = len(entries)
        b.q[:n].copy_(q)
        b.k[:n].copy_(k)
        b.v[:n].copy_(v)
        if n < b.size:
            b.k[n:].zero_()
            b.v[n:].zero_()
            b.q[n:].zero_()
        return b

    def launch(self, b: Bucket) -> None:
        lib().hip_graph_launch(b.graph)

    def destroy(self) -> None:
        for b in self.buckets.values():
            lib().hip_graph_destroy(b.graph)
        self.buckets.clear()
