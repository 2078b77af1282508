"""Shared test harness: run one attention step of a workload on the GPU (through the C-ABI, exactly as the
engine's operator does) and on the CPU oracle, and compare."""
from __future__ import annotations

import numpy as np
import torch

import oracle
from llmgen_amd import attention as A
from llmgen_amd._lib import lib
from llmgen_amd.workloads import Workload, to_u16

MAX_ABS = 2e-2  # bf16 output tolerance against the f32 result before rounding (with REL_L2)
REL_L2 = 1e-2


def check_hip_error(what: str) -> None:
    err = lib().hip_last_error()
    assert err == 0, f"{what}: HIP error {err}"


def run_gpu(wl: Workload, t: dict):
    """store_kv + attention on the GPU via PagedAttentionImpl (the C++ executor slice: fillMeta, bindStep,
    llmgen_paged_attention).  t: dict of bf16 device tensors (not modified).
    Returns (out [T,nq,hd] bf16 device, kc, vc after the step)."""
    A.init_device()
    ws = wl.workspace()
    mgr = A.PagedAttentionManager()
    mgr.layers[0] = A.LayerState(t["kc"].clone(), t["vc"].clone())
    A.g_attn_mgr = mgr
    wl.bind(ws)
    out = torch.full((wl.n_tok, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device=t["q"].device)
    A.PagedAttentionImpl.execute(0, A.AttnNode(out, [t["q"], t["k"], t["v"]], layer_id=0))
    torch.cuda.synchronize()
    check_hip_error(wl.name)
    return out, mgr.layers[0].k, mgr.layers[0].v


def run_oracle(wl: Workload, t: dict, rows=None, threads: int = 1):
    """The CPU oracle on host copies: store_kv then attend (all rows, or only ``rows``).
    Returns (kc, vc, out_bf16 u16, out_f32) -- outputs for ``rows`` only when given."""
    meta = wl.meta(64)
    kc = to_u16(t["kc"]).copy()
    vc = to_u16(t["vc"]).copy()
    oracle.store_kv(to_u16(t["k"]), to_u16(t["v"]), meta.slots, kc, vc, wl.nkv, wl.hd, wl.block_size)
    args = (to_u16(t["q"]), kc, vc, meta.block_tables, meta.ctx, meta.cu_q, wl.nq, wl.nkv, wl.hd, wl.max_blocks,
            wl.block_size, wl.scale)
    if rows is None:
        ob, of = oracle.attend(*args)
    else:
        ob, of = oracle.attend_rows(*args, rows=rows, threads=threads)
    return kc, vc, ob, of


def assert_cache_equal(got: np.ndarray, ref: np.ndarray, what: str) -> None:
    """Bit-exact paged-cache comparison; on mismatch name the (block, head, slot) rows that differ."""
    if np.array_equal(got, ref):
        return
    bad = np.argwhere((got != ref).any(axis=-1))
    raise AssertionError(f"{what}: {len(bad)} cache rows differ, first (block, head, slot): {bad[:8].tolist()}")


def compare(got_bf16_u16: np.ndarray, ref_f32: np.ndarray, what: str, max_abs=MAX_ABS, rel_l2=REL_L2):
    g = oracle.bf16_to_f32(got_bf16_u16).astype(np.float64)
    r = ref_f32.astype(np.float64)
    assert np.isfinite(g).all(), f"{what}: non-finite outputs"
    err = np.abs(g - r)
    mx = float(err.max()) if err.size else 0.0
    den = float(np.linalg.norm(r))
    rel = float(np.linalg.norm(g - r) / den) if den > 0 else float(np.linalg.norm(g - r))
    assert mx <= max_abs, f"{what}: max abs err {mx:.4g} > {max_abs} (at {np.unravel_index(err.argmax(), err.shape)})"
    assert rel <= rel_l2, f"{what}: rel-L2 {rel:.4g} > {rel_l2}"
    return mx, rel
