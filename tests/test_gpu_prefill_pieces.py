"""Prefill steps of few units (at most half a unit -- query tile x KV head x head pair -- per CU), which
run the pieces kernel: each unit's key tiles split over up to 8 workgroups whose partial results the last one to
finish merges in piece order.  Chunks of one sequence against long cached contexts reach the full 8 pieces;
sampled rows against the oracle (max-abs 2e-2, rel-L2 1e-2), the KV cache bit for bit, and two runs of the same
step bit-identical.  A mixed step whose prefill part is such a chunk (beside decode rows) splits it the same way
inside the mixed-step kernel (GQA 2, 4) or in the pieces kernel beside the decode-row launch (GQA 1, 8)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from harness import assert_cache_equal, compare, run_gpu, run_oracle
from llmgen_amd._lib import lib
from llmgen_amd.step import Entry
from llmgen_amd.workloads import Workload, _tables, to_u16

PIECES = 7  # LLMGEN_PREFILL_PIECES

# (q heads, kv heads, block size, [(cached keys, chunk rows), ...])
SHAPES = {
    "g2_512_on_32k": (16, 8, 256, [(32256, 512)]),
    "g2_200_on_5k_bs48": (4, 2, 48, [(4800, 200)]),
    "g4_256_on_8k": (32, 8, 256, [(7936, 256)]),
    "g2_two_chunks_bs16": (16, 8, 16, [(3000, 130), (900, 64)]),
    "g1_512_on_16k": (16, 16, 256, [(15872, 512)]),  # GQA 1: one head per 2-wave workgroup
}


def _workload(name):
    nq, nkv, bs, spec = SHAPES[name]
    rng = np.random.default_rng(len(name))
    ctxs = [a + b for a, b in spec]
    tables, nb = _tables(rng, ctxs, bs, permute=True, extra_blocks=2)
    mb = max(len(t) for t in tables)
    return Workload(name, nq, nkv, 128, bs, nb, mb, mb * bs, [Entry(a, b, t) for (a, b), t in zip(spec, tables)],
                    std=1.0, seed=len(name) + 100, decode=False)


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(SHAPES))
def test_pieces_prefill_matches_oracle(gpu, name):
    wl = _workload(name)
    print(f"[gpu-test] pieces {name}", flush=True)
    m = wl.meta(lib().hip_attn_prefill_tile())
    assert m.single_rows() == 0
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert lib().hip_attn_prefill_plan(m.n_tiles, wl.nq, wl.nkv, wl.hd, wl.block_size, 0) == PIECES
    t = wl.tensors(device="cuda")
    out, kc, vc = run_gpu(wl, t)
    out2, _, _ = run_gpu(wl, t)
    np.testing.assert_array_equal(to_u16(out2), to_u16(out), err_msg=f"{name}: two runs differ")
    n = m.n_tok
    rows = np.arange(n, dtype=np.int32)
    if n > 96:  # the first and last rows of every tile plus a seeded sample
        picks = set(np.random.default_rng(7).integers(0, n, size=48).tolist())
        for q0 in range(0, n, 64):
            picks.update((q0, min(q0 + 63, n - 1)))
        rows = np.array(sorted(picks), dtype=np.int32)
    okc, ovc, _, of = run_oracle(wl, t, rows=rows, threads=16)
    assert_cache_equal(to_u16(kc), okc, f"{name} K")
    assert_cache_equal(to_u16(vc), ovc, f"{name} V")
    compare(to_u16(out)[rows], of, name)


# one chunk against a long cached context beside decode rows: (q heads, kv heads, cached, chunk, decode contexts)
MIXED_SHAPES = {
    "g2_512_on_16k_with_63_rows": (16, 8, 15872, 512, 63),
    "g4_192_on_6k_with_20_rows": (32, 8, 6000, 192, 20),
    "g1_512_on_16k_with_31_rows": (16, 16, 15872, 512, 31),  # GQA 1 and 8: the pieces kernel beside the rows
    "g8_256_on_8k_with_15_rows": (64, 8, 7936, 256, 15),
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(MIXED_SHAPES))
def test_mixed_step_with_a_long_chunk_matches_oracle(gpu, name):
    nq, nkv, cached, chunk, nd = MIXED_SHAPES[name]
    rng = np.random.default_rng(nd)
    dctx = [int(c) for c in rng.integers(100, 3000, size=nd)]
    ctxs = [cached + chunk] + dctx
    tables, nb = _tables(rng, ctxs, 256, permute=True, extra_blocks=2)
    mb = max(len(t) for t in tables)
    ents = [Entry(cached, chunk, tables[0])] + [Entry(c - 1, 1, t) for c, t in zip(dctx, tables[1:])]
    wl = Workload(name, nq, nkv, 128, 256, nb, mb, mb * 256, ents, std=1.0, seed=nd, decode=False)
    print(f"[gpu-test] mixed long chunk {name}", flush=True)
    m = wl.meta(lib().hip_attn_prefill_tile())
    assert m.single_rows() == nd
    want = 1 if nq // nkv in (2, 4) else PIECES | 16  # MIXED, or PIECES + the decode-row launch
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert lib().hip_attn_prefill_plan(m.n_tiles, wl.nq, wl.nkv, wl.hd, wl.block_size, nd) == want
    t = wl.tensors(device="cuda")
    out, kc, vc = run_gpu(wl, t)
    out2, _, _ = run_gpu(wl, t)
    np.testing.assert_array_equal(to_u16(out2), to_u16(out), err_msg=f"{name}: two runs differ")
    n = m.n_tok
    picks = set(range(n - nd, n)) | set(np.random.default_rng(3).integers(0, n - nd, size=40).tolist())
    for q0 in range(0, chunk, 64):
        picks.update((q0, min(q0 + 63, chunk - 1)))
    rows = np.array(sorted(picks), dtype=np.int32)
    okc, ovc, _, of = run_oracle(wl, t, rows=rows, threads=16)
    assert_cache_equal(to_u16(kc), okc, f"{name} K")
    assert_cache_equal(to_u16(vc), ovc, f"{name} V")
    compare(to_u16(out)[rows], of, name)


@pytest.mark.gpu
def test_pieces_prefill_graph_replay(gpu):
    """The 8-piece step captured into a graph: three replays with eager torch work between them each equal the
    eager step bit for bit (the per-unit ticket counters are back at 0 after every launch)."""
    from harness import check_hip_error
    from llmgen_amd import attention as A

    wl = _workload("g2_512_on_32k")
    print("[gpu-test] pieces graph replay", flush=True)
    t = wl.tensors(device="cuda")
    A.init_device()
    L = lib()
    ws = wl.workspace()
    mgr = A.PagedAttentionManager()
    mgr.layers[0] = A.LayerState(t["kc"].clone(), t["vc"].clone())
    A.g_attn_mgr = mgr
    wl.bind(ws)
    node_out = torch.full((wl.n_tok, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device="cuda")
    node = A.AttnNode(node_out, [t["q"], t["k"], t["v"]], layer_id=0)
    A.PagedAttentionImpl.execute(0, node)
    torch.cuda.synchronize()
    check_hip_error("pieces eager")
    ref = to_u16(node_out).copy()
    assert L.hip_graph_begin() == 0
    A.PagedAttentionImpl.execute(0, node)
    g = L.hip_graph_end()
    assert g
    try:
        for i in range(3):
            node_out.fill_(float("nan"))
            junk = torch.randn(1 << 20, device="cuda").sum()  # eager work between the replays
            torch.cuda.synchronize()
            L.hip_graph_launch(g)
            torch.cuda.synchronize()
            check_hip_error(f"pieces replay {i}")
            np.testing.assert_array_equal(to_u16(node_out), ref)
            del junk
    finally:
        L.hip_graph_destroy(g)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["gqa8", "gqa1"])
def test_pieces_beside_rows_any_tile_order(gpu, name):
    """A mixed step at GQA 8 / 1 with a known single-row count runs its prefill tiles in the pieces kernel beside the
    decode-row launch, expecting the single rows first; a seeded shuffle of the tile list (multi-row tiles among
    the leading single-row part, single rows among the rest) must still give every row: against the oracle."""
    from harness import check_hip_error
    from llmgen_amd.workloads import make
    import oracle

    wl = make(name)
    print(f"[gpu-test] pieces any order {name}", flush=True)
    t = wl.tensors(device="cuda")
    L = lib()
    meta = wl.meta(L.hip_attn_prefill_tile())
    assert not meta.decode and meta.single_rows() > 0
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert L.hip_attn_prefill_plan(meta.n_tiles, wl.nq, wl.nkv, wl.hd, wl.block_size, meta.single_rows()) == \
            PIECES | 16
    kc, vc = t["kc"].clone(), t["vc"].clone()
    buf = meta.packed().copy()
    perm = np.random.default_rng(9).permutation(meta.n_tiles)
    o_s, o_q = meta.offsets["tile_seq"], meta.offsets["tile_q0"]
    buf[o_s:o_s + meta.n_tiles] = meta.tile_seq[perm]
    buf[o_q:o_q + meta.n_tiles] = meta.tile_q0[perm]
    moved = np.diff(meta.cu_q)[meta.tile_seq[perm]][:meta.single_rows()]
    assert (moved > 1).any(), "the shuffle must put multi-row tiles into the leading part"
    seg = torch.from_numpy(buf).to("cuda")
    off = {k: seg.data_ptr() + 4 * v for k, v in meta.offsets.items()}
    L.hip_store_kv(t["k"].data_ptr(), t["v"].data_ptr(), off["slots"], kc.data_ptr(), vc.data_ptr(), wl.n_tok,
                   wl.nkv, wl.hd, wl.block_size)
    out = torch.full((wl.n_tok, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device="cuda")
    L.hip_attn_prefill_rows(out.data_ptr(), t["q"].data_ptr(), kc.data_ptr(), vc.data_ptr(), off["block_tables"],
                            off["ctx"], off["cu_q"], off["tile_seq"], off["tile_q0"], meta.n_tiles, wl.nq, wl.nkv,
                            wl.hd, wl.max_blocks, wl.block_size, wl.scale, meta.single_rows())
    torch.cuda.synchronize()
    check_hip_error(f"{name} shuffled")
    got = to_u16(out)
    assert not np.isnan(oracle.bf16_to_f32(got)).any()
    _, _, _, of = run_oracle(wl, t)
    compare(got, of, f"{name} shuffled")
