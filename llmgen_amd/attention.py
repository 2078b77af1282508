"""Host-side mirror of the engine's attention operator for the HIP backend.

The reference engine dispatches the ``OP_TYPE_PAGED_ATTN`` node to ``PagedAttentionImpl(device).execute(device_id,
out)`` (``src/ops.zig:63-65, 197-209``), which reads every per-step value from the global ``g_step``
(``src/backend/cpu/common.zig:10-43``) and the layer's KV pools from ``kvOf(layer_id)`` (``common.zig:46-52``).
This module keeps those names, argument meanings and error behaviour, and drives ``libllmgen_attn.so``:

* :class:`StepState` / :data:`g_step` -- the attention fields of ``common.StepState`` (device pointers as ints).
* :class:`PagedAttentionManager` / :func:`kv_of` -- per-layer K/V pools (``memory/page_atten.zig:15-28``).
* :class:`PagedAttentionImpl` -- ``attention_v1.zig:60-120``: store_kv, then decode (split-K) or prefill.
* :func:`bind_step` -- ``executor.zig:864-895`` bindStep: uploads the packed metadata and fills ``g_step``.

Tensors are torch tensors on the GPU (torch is used for device memory only); bf16 tensors may be
``torch.bfloat16`` or ``torch.int16``/``uint16`` views of the same bits.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np
import torch

from . import step as stepmod
from ._lib import lib


class AttentionNeedsBf16(TypeError):
    """cpu/attention.zig:123 error.AttentionNeedsBf16."""


class NoAttentionManager(RuntimeError):
    """common.zig:50 error.NoAttentionManager."""


class LayerNotActive(KeyError):
    """common.zig:51 error.LayerNotActive."""


@dataclass
class StepState:
    """common.zig:10-41 (the fields attention reads). Pointers are device addresses (int)."""

    n_tok: int = 0
    n_seq: int = 0
    n_tiles: int = 0
    decode: bool = False
    n_head: int = 0
    n_kv_head: int = 0
    head_dim: int = 0
    attn_scale: float = 0.0
    block_size: int = 0
    max_blocks: int = 0
    max_model_len: int = 0
    pos: int = 0
    slots: int = 0
    cu_q: int = 0
    ctx: int = 0
    last: int = 0
    tile_seq: int = 0
    tile_q0: int = 0
    block_tables: int = 0
    part_o: int = 0
    part_ml: int = 0
    single_rows: int = -1  # segments with one query row (-1 unknown); not in the reference's StepState


g_step = StepState()


@dataclass
class LayerState:
    """memory/page_atten.zig:15-28: one contiguous K pool and one V pool of
    num_blocks x [nkv][block_size][hd] bf16 per layer."""

    k: torch.Tensor
    v: torch.Tensor


@dataclass
class PagedAttentionManager:
    layers: Dict[int, LayerState] = field(default_factory=dict)

    def reserve_layer(self, layer_id: int, num_blocks: int, nkv: int, block_size: int, hd: int,
                      device="cuda") -> LayerState:
        shape = (num_blocks, nkv, block_size, hd)
        st = LayerState(torch.zeros(shape, dtype=torch.bfloat16, device=device),
                        torch.zeros(shape, dtype=torch.bfloat16, device=device))
        self.layers[layer_id] = st
        return st

    def get_layer(self, layer_id: int) -> Optional[LayerState]:
        return self.layers.get(layer_id)


g_attn_mgr: Optional[PagedAttentionManager] = None


def kv_of(layer_id: int) -> LayerState:
    """common.zig:49-52."""
    if g_attn_mgr is None:
        raise NoAttentionManager("no paged attention manager")
    st = g_attn_mgr.get_layer(layer_id)
    if st is None:
        raise LayerNotActive(f"layer {layer_id} has no KV pools")
    return st


@dataclass
class AttnNode:
    """The slice of the engine's Tensor that PagedAttentionImpl reads: out.data [1,T,nq,hd], out.src[0..2] =
    q [1,T,nq,hd], k / v [1,T,nkv,hd], out.layer_id, out.data_type (module/attention.zig:66-112)."""

    data: torch.Tensor
    src: List[torch.Tensor]
    layer_id: int = 0


_BF16_LIKE = (torch.bfloat16, torch.int16, torch.uint16)


def _ptr(t: torch.Tensor) -> int:
    assert t.is_cuda and t.is_contiguous(), "attention tensors must be contiguous device tensors"
    return t.data_ptr()


class PagedAttentionImpl:
    """attention_v1.zig:60-120 for the HIP backend.  Decode steps issue store_kv and split-K decode as one fused
    launch (hip_attn_decode_store_kv); prefill / mixed steps issue store_kv, then prefill, as the reference does."""

    @staticmethod
    def execute(device_id: int, out: AttnNode, store_kv: bool = True) -> None:
        """``store_kv=False`` when this step's k / v are already in the cache (written by the fused
        hip_qk_norm_rope_store_kv); ``out.src[1:]`` are then not read."""
        if out.data.dtype not in _BF16_LIKE:
            raise AttentionNeedsBf16(f"attention needs bf16, got {out.data.dtype}")
        s = g_step
        kv = kv_of(out.layer_id)
        L = lib()
        q, k, v = out.src
        if s.decode and store_kv:
            # store_kv fused into the decode launch (one kernel per decode step)
            L.hip_attn_decode_store_kv(_ptr(out.data), _ptr(q), _ptr(k), _ptr(v), s.slots, _ptr(kv.k), _ptr(kv.v),
                                       s.block_tables, s.ctx, s.n_seq, s.n_head, s.n_kv_head, s.head_dim,
                                       s.max_blocks, s.block_size, s.attn_scale, s.part_o, s.part_ml,
                                       stepmod.part_size(s.n_seq), stepmod.max_parts(s.n_seq, s.max_model_len))
            return
        if store_kv:
            L.hip_store_kv(_ptr(k), _ptr(v), s.slots, _ptr(kv.k), _ptr(kv.v), s.n_tok, s.n_kv_head, s.head_dim,
                           s.block_size)
        if s.decode:
            L.hip_attn_decode(_ptr(out.data), _ptr(q), _ptr(kv.k), _ptr(kv.v), s.block_tables, s.ctx, s.n_seq,
                              s.n_head, s.n_kv_head, s.head_dim, s.max_blocks, s.block_size, s.attn_scale,
                              s.part_o, s.part_ml, stepmod.part_size(s.n_seq),
                              stepmod.max_parts(s.n_seq, s.max_model_len))
        else:
            L.hip_attn_prefill_rows(_ptr(out.data), _ptr(q), _ptr(kv.k), _ptr(kv.v), s.block_tables, s.ctx,
                                    s.cu_q, s.tile_seq, s.tile_q0, s.n_tiles, s.n_head, s.n_kv_head, s.head_dim,
                                    s.max_blocks, s.block_size, s.attn_scale, s.single_rows)


# attention_v1.zig:123: the legacy FLASH_ATTN node runs the same implementation
FlashAttentionImpl = PagedAttentionImpl


@dataclass
class Workspace:
    """Device buffers the executor owns for attention: packed step metadata and split-K scratch
    (executor.zig:81-112)."""

    meta: torch.Tensor
    part_o: torch.Tensor
    part_ml: torch.Tensor

    @staticmethod
    def allocate(nq: int, hd: int, max_seqs: int, max_model_len: int, meta_elems: int,
                 device="cuda") -> "Workspace":
        po, pml = stepmod.workspace_bytes(nq, hd, max_seqs, max_model_len)
        return Workspace(meta=torch.zeros(meta_elems, dtype=torch.int32, device=device),
                         part_o=torch.empty(po // 4, dtype=torch.float32, device=device),
                         part_ml=torch.empty(pml // 4, dtype=torch.float32, device=device))


def bind_step(meta: "stepmod.StepMeta", ws: Workspace, nq: int, nkv: int, hd: int, block_size: int,
              max_blocks: int, max_model_len: int, upload: bool = True) -> StepState:
    """executor.zig:864-895: upload the packed metadata (one host-to-device copy) and publish its device
    addresses in g_step."""
    buf = meta.packed()
    if buf.size > ws.meta.numel():
        raise ValueError("step metadata does not fit the workspace")
    if upload:
        ws.meta[:buf.size].copy_(torch.from_numpy(buf), non_blocking=False)
    base = ws.meta.data_ptr()
    off = meta.offsets
    g = g_step
    g.n_tok, g.n_seq, g.n_tiles, g.decode = meta.n_tok, meta.n_seq, meta.n_tiles, meta.decode
    g.n_head, g.n_kv_head, g.head_dim = nq, nkv, hd
    g.attn_scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))  # f32, as executor.zig:877
    g.block_size, g.max_blocks, g.max_model_len = block_size, max_blocks, max_model_len
    for name in ("pos", "slots", "cu_q", "ctx", "last", "tile_seq", "tile_q0", "block_tables"):
        setattr(g, name, base + 4 * off[name])
    g.part_o, g.part_ml = ws.part_o.data_ptr(), ws.part_ml.data_ptr()
    g.single_rows = meta.single_rows()
    return g


_inited = False


def init_device() -> None:
    """cuda_init equivalent.  Creates one stream, makes it PyTorch's current stream and routes the library's
    launches onto it, so torch-owned buffers and the kernels are ordered on one stream (and can be captured)."""
    global _inited
    if _inited:
        return
    L = lib()
    if L.hip_init(0) != 0:
        raise RuntimeError("hip_init failed: no HIP device")
    # a dedicated (default-priority) stream: capturable, unlike the legacy null stream
    global _stream
    _stream = torch.cuda.Stream()
    torch.cuda.set_stream(_stream)
    L.hip_set_stream(_stream.cuda_stream)
    _inited = True


_stream = None
