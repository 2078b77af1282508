"""Host-side mirror of the engine's attention operator for the HIP backend.

The reference engine dispatches the ``OP_TYPE_PAGED_ATTN`` node to ``PagedAttentionImpl(device).execute(device_id,
out)`` (``src/ops.zig:63-65, 197-209``), which reads every per-step value from the global ``g_step``
(``src/backend/cpu/common.zig:10-43``) and the layer's KV pools from ``kvOf(layer_id)`` (``common.zig:46-52``).
This module keeps those names, argument meanings and error behaviour.  It holds no host logic of its own: the
step metadata, the StepState and the per-layer dispatch are the C++ executor slice in ``libllmgen_attn.so``
(``include/llmgen_host.h``), reached through :mod:`llmgen_amd.host`:

* :data:`g_step` -- the C++ ``llmgen_step_state`` (``common.StepState``) of the bound step.
* :class:`PagedAttentionManager` / :func:`kv_of` -- per-layer K/V pools (``memory/page_atten.zig:15-28``).
* :class:`PagedAttentionImpl` -- ``attention_v1.zig:60-120``: checks as the Zig operator does, then
  ``llmgen_paged_attention`` (store_kv, then decode or prefill).
* :func:`bind_step` -- ``executor.zig:772-895`` fillMeta + bindStep: ``llmgen_fill_meta`` packs the step, one
  host-to-device copy uploads it, ``llmgen_bind_step`` fills ``g_step``.

Tensors are torch tensors on the GPU (torch is used for device memory only); bf16 tensors may be
``torch.bfloat16`` or ``torch.int16``/``uint16`` views of the same bits.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np
import torch

from . import host as H
from . import step as stepmod
from ._lib import lib


class AttentionNeedsBf16(TypeError):
    """cpu/attention.zig:123 error.AttentionNeedsBf16."""


class NoAttentionManager(RuntimeError):
    """common.zig:50 error.NoAttentionManager."""


class LayerNotActive(KeyError):
    """common.zig:51 error.LayerNotActive."""


g_step = H.StepState()  # the bound step (C++ llmgen_step_state)


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
    """attention_v1.zig:60-120 for the HIP backend: the checks of the Zig operator, then the C++
    ``llmgen_paged_attention``.  Decode steps issue store_kv and split-K decode as one fused launch
    (hip_attn_decode_store_kv); prefill / mixed steps issue store_kv, then prefill with the step's single-row
    count, as the reference issues store_kv then prefill."""

    @staticmethod
    def execute(device_id: int, out: AttnNode, store_kv: bool = True) -> None:
        """``store_kv=False`` when this step's k / v are already in the cache (written by the fused
        hip_qk_norm_rope_store_kv); ``out.src[1:]`` are then not read."""
        if out.data.dtype not in _BF16_LIKE:
            raise AttentionNeedsBf16(f"attention needs bf16, got {out.data.dtype}")
        kv = kv_of(out.layer_id)
        q, k, v = out.src
        for t in (out.data, q, kv.k, kv.v) + ((k, v) if store_kv else ()):
            _ptr(t)
        H.paged_attention(g_step, out.data, q, k if store_kv else None, v if store_kv else None, kv.k, kv.v,
                          store_kv=store_kv)


# attention_v1.zig:123: the legacy FLASH_ATTN node runs the same implementation
FlashAttentionImpl = PagedAttentionImpl


@dataclass
class Workspace:
    """Device buffers the executor owns for attention: packed step metadata and split-K scratch
    (executor.zig:81-112)."""

    meta: torch.Tensor  # uint8, at least the packed layout's bytes
    part_o: torch.Tensor
    part_ml: torch.Tensor

    @staticmethod
    def allocate(nq: int, hd: int, max_seqs: int, max_model_len: int, meta_bytes: int,
                 device="cuda") -> "Workspace":
        po, pml = stepmod.workspace_bytes(nq, hd, max_seqs, max_model_len)
        return Workspace(meta=torch.zeros(meta_bytes, dtype=torch.uint8, device=device),
                         part_o=torch.empty(po // 4, dtype=torch.float32, device=device),
                         part_ml=torch.empty(pml // 4, dtype=torch.float32, device=device))


def _step_shape(entries, seq_num, decode, pf_tile):
    n_pad = seq_num - len(entries)
    if n_pad < 0:
        raise ValueError("seq_num < number of entries")
    if decode is None:  # the engine's rule (executor.zig:530-552)
        decode = all(e.q_len == 1 and e.emits for e in entries)
    n_tok = sum(e.q_len for e in entries) + n_pad
    n_tiles = 0 if decode else sum((e.q_len + pf_tile - 1) // pf_tile for e in entries) + n_pad
    return bool(decode), n_tok, n_tiles


def meta_bytes(entries, max_blocks: int, seq_num: Optional[int] = None, decode: Optional[bool] = None) -> int:
    """Bytes of the packed metadata of this step (the C++ layout, executor.zig:139-202)."""
    seq_num = len(entries) if seq_num is None else seq_num
    _, n_tok, n_tiles = _step_shape(entries, seq_num, decode, lib().hip_attn_prefill_tile())
    return H.layout(n_tok, seq_num, n_tiles, max_blocks).total


def bind_step(entries, ws: Workspace, nq: int, nkv: int, hd: int, block_size: int, max_blocks: int,
              max_model_len: int, seq_num: Optional[int] = None, decode: Optional[bool] = None,
              upload: bool = True) -> "H.StepState":
    """executor.zig:772-895 for one step: ``llmgen_fill_meta`` packs the step (slots, cu_q, ctx, prefill tiles
    lightest first, block tables, padding rows up to ``seq_num``), one host-to-device copy uploads it, and
    ``llmgen_bind_step`` publishes its device addresses and the single-row count in :data:`g_step`.

    ``entries``: :class:`~llmgen_amd.step.Entry` (q_start, q_len, block_table, emits).  ``decode`` defaults to
    the engine's rule (every entry has q_len == 1 and emits).  Attention reads no token ids, so the sequences
    handed to fillMeta carry zeros."""
    global g_step
    seq_num = len(entries) if seq_num is None else seq_num
    pf = lib().hip_attn_prefill_tile()
    decode, n_tok, n_tiles = _step_shape(entries, seq_num, decode, pf)
    seqs = [H.Sequence_([0] * (e.q_start + e.q_len + (0 if e.emits else 1)), list(e.block_table))
            for e in entries]
    ents = [(i, e.q_start, e.q_len) for i, e in enumerate(entries)]
    buf, lay, _, single = H.fill_meta(seqs, ents, seq_num, n_tiles, pf, block_size, max_blocks)
    if buf.size > ws.meta.numel():
        raise ValueError("step metadata does not fit the workspace")
    if upload:
        ws.meta[:buf.size].copy_(torch.from_numpy(buf), non_blocking=False)
    g_step = H.bind_step(ws.meta.data_ptr(), lay, n_tok, seq_num, n_tiles, decode, nq, nkv, hd, block_size,
                         max_blocks, max_model_len, ws.part_o.data_ptr(), ws.part_ml.data_ptr(),
                         single_rows=single)
    return g_step


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
