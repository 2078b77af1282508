"""GPU parity: the HIP path (through the C-ABI) against the CPU oracle on the same seeded inputs.

Bars: store_kv bit-exact; attention within max-abs 2e-2 and rel-L2 1e-2 of the oracle's f32 result before bf16
rounding, and padding rows exactly 0.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from harness import assert_cache_equal, check_hip_error, compare, run_gpu, run_oracle
from llmgen_amd import attention as A
from llmgen_amd._lib import lib
from llmgen_amd.workloads import make, to_u16

pytestmark = pytest.mark.gpu


def _sample_rows(wl, meta, n_random=48, seed=0):
    """First and last row of every prefill tile and sequence, plus seeded random rows."""
    rows = set()
    tile = lib().hip_attn_prefill_tile()
    for s in range(meta.n_seq):
        b, e = int(meta.cu_q[s]), int(meta.cu_q[s + 1])
        for q0 in range(b, e, tile):
            rows.add(q0)
            rows.add(min(q0 + tile, e) - 1)
    rng = np.random.default_rng(seed)
    rows.update(int(x) for x in rng.integers(0, meta.n_tok, size=n_random))
    return np.array(sorted(rows), np.int32)


@pytest.mark.parametrize("name", ["kt_prefill", "cpu_mixed", "c1", "c2", "gqa1", "gqa8", "gqa16",
                                  "gqa1d", "gqa8d", "gqa16d", "bs48", "bs48d", "bs6", "bs6d", "gqa2",
                                  "g1bs6", "g1bs256"])
def test_step_matches_oracle_all_rows(gpu, name):
    wl = make(name)
    print(f"[gpu-test] {name}", flush=True)
    t = wl.tensors(device="cuda")
    out, kc, vc = run_gpu(wl, t)
    okc, ovc, ob, of = run_oracle(wl, t)
    assert_cache_equal(to_u16(kc), okc, f"{name} store_kv K")
    assert_cache_equal(to_u16(vc), ovc, f"{name} store_kv V")
    got = to_u16(out)
    compare(got, of, name)
    # padding rows (ctx < q_len) are exactly zero
    meta = wl.meta(lib().hip_attn_prefill_tile())
    for s in range(meta.n_seq):
        if meta.ctx[s] < meta.cu_q[s + 1] - meta.cu_q[s]:
            assert not got[meta.cu_q[s]:meta.cu_q[s + 1]].any(), "padding row not zero"


@pytest.mark.parametrize("part_size", [64, 128, 256, 512])
def test_decode_part_size_sweep(gpu, part_size):
    """kernel_test.zig:212-231: decode of the last row of ctx=150 for several split-K part sizes."""
    wl = make("kt_decode")
    print(f"[gpu-test] kt_decode part_size={part_size}", flush=True)
    t = wl.tensors(device="cuda")
    _, _, _, of = run_oracle(wl, t)
    # write this step's K/V through the library, then call the decode launcher directly
    meta = wl.meta(64)
    dev = t["q"].device
    kc, vc = t["kc"].clone(), t["vc"].clone()
    slots = torch.from_numpy(meta.slots).to(dev)
    L = lib()
    L.hip_store_kv(t["k"].data_ptr(), t["v"].data_ptr(), slots.data_ptr(), kc.data_ptr(), vc.data_ptr(), 1, wl.nkv,
                   wl.hd, wl.block_size)
    max_parts = (4096 + part_size - 1) // part_size
    po = torch.empty(wl.nq * max_parts * wl.hd, dtype=torch.float32, device=dev)
    pml = torch.empty(wl.nq * max_parts * 2, dtype=torch.float32, device=dev)
    bt = torch.from_numpy(meta.block_tables).to(dev)
    ctx = torch.from_numpy(meta.ctx).to(dev)
    out = torch.full((1, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device=dev)
    L.hip_attn_decode(out.data_ptr(), t["q"].data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(),
                      ctx.data_ptr(), 1, wl.nq, wl.nkv, wl.hd, wl.max_blocks, wl.block_size, wl.scale,
                      po.data_ptr(), pml.data_ptr(), part_size, max_parts)
    torch.cuda.synchronize()
    check_hip_error("decode")
    compare(to_u16(out), of, f"kt_decode ps={part_size}")


@pytest.mark.parametrize("name,pad", [("c2", 0), ("c2", 5), ("kt_decode", 0), ("gqa8d", 3), ("c1", 0)])
def test_fused_decode_store_kv_equals_unfused(gpu, name, pad):
    """hip_attn_decode_store_kv == hip_store_kv then hip_attn_decode, bit for bit (output and both caches),
    including graph-bucket padding rows (ctx 0, slot -1)."""
    import copy as _copy
    from llmgen_amd import step as S

    wl = _copy.copy(make(name))
    wl.pad_rows = pad
    print(f"[gpu-test] fused decode {name} pad={pad}", flush=True)
    t = wl.tensors(device="cuda")
    meta = wl.meta(64)
    assert meta.decode
    dev = t["q"].device
    n = meta.n_tok
    q = torch.zeros((n, wl.nq, wl.hd), dtype=torch.bfloat16, device=dev)
    k = torch.zeros((n, wl.nkv, wl.hd), dtype=torch.bfloat16, device=dev)
    v = torch.zeros_like(k)
    m = t["q"].shape[0]
    q[:m], k[:m], v[:m] = t["q"], t["k"], t["v"]
    d = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    slots, bt, ctx = d(meta.slots), d(meta.block_tables), d(meta.ctx)
    ps, mp = S.part_size(n), S.max_parts(n, wl.max_model_len)
    L = lib()
    outs, caches = [], []
    for fused in (False, True):
        kc, vc = t["kc"].clone(), t["vc"].clone()
        po = torch.empty(n * wl.nq * mp * wl.hd, dtype=torch.float32, device=dev)
        pml = torch.empty(n * wl.nq * mp * 2, dtype=torch.float32, device=dev)
        out = torch.full((n, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device=dev)
        common = (bt.data_ptr(), ctx.data_ptr(), n, wl.nq, wl.nkv, wl.hd, wl.max_blocks, wl.block_size, wl.scale,
                  po.data_ptr(), pml.data_ptr(), ps, mp)
        if fused:
            L.hip_attn_decode_store_kv(out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), slots.data_ptr(),
                                       kc.data_ptr(), vc.data_ptr(), *common)
        else:
            L.hip_store_kv(k.data_ptr(), v.data_ptr(), slots.data_ptr(), kc.data_ptr(), vc.data_ptr(), n, wl.nkv,
                           wl.hd, wl.block_size)
            L.hip_attn_decode(out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), *common)
        torch.cuda.synchronize()
        check_hip_error(f"fused={fused}")
        outs.append(to_u16(out))
        caches.append((to_u16(kc), to_u16(vc)))
    np.testing.assert_array_equal(outs[1], outs[0])
    assert_cache_equal(caches[1][0], caches[0][0], "fused K cache")
    assert_cache_equal(caches[1][1], caches[0][1], "fused V cache")
    if pad:
        assert not outs[1][m:].any(), "padding rows not zero"


@pytest.mark.parametrize("name", ["c3", "c4", "c5d", "c5p"])
def test_step_matches_oracle_sampled_rows(gpu, name):
    wl = make(name)
    print(f"[gpu-test] {name}", flush=True)
    t = wl.tensors(device="cuda")
    out, kc, vc = run_gpu(wl, t)
    meta = wl.meta(lib().hip_attn_prefill_tile())
    rows = _sample_rows(wl, meta)
    okc, ovc, ob, of = run_oracle(wl, t, rows=rows, threads=16)
    assert_cache_equal(to_u16(kc), okc, f"{name} store_kv K")
    assert_cache_equal(to_u16(vc), ovc, f"{name} store_kv V")
    compare(to_u16(out)[rows], of, name)


def test_golden_vectors(gpu):
    """The committed golden step (oracle outputs) through the C-ABI: store_kv + prefill launcher."""
    import os

    print("[gpu-test] golden", flush=True)
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "paged_attention_golden.npz"))
    nq, nkv, hd, bs, mb = (int(x) for x in g["shape"])

    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16) if a.dtype == np.uint16 else a).to("cuda")

    kc, vc = dev(g["kc"]), dev(g["vc"])
    q, k, v = dev(g["q"]), dev(g["k"]), dev(g["v"])
    slots, bt, cu_q, ctx = dev(g["slots"]), dev(g["block_tables"]), dev(g["cu_q"]), dev(g["ctx"])
    tile = lib().hip_attn_prefill_tile()
    tseq, tq0 = [], []
    cq = g["cu_q"]
    for s in range(3):
        for q0 in range(0, int(cq[s + 1] - cq[s]), tile):
            tseq.append(s)
            tq0.append(q0)
    tseq = torch.tensor(tseq, dtype=torch.int32, device="cuda")
    tq0 = torch.tensor(tq0, dtype=torch.int32, device="cuda")
    out = torch.full((32, nq, hd), -1, dtype=torch.int16, device="cuda")
    L = lib()
    L.hip_store_kv(k.data_ptr(), v.data_ptr(), slots.data_ptr(), kc.data_ptr(), vc.data_ptr(), 32, nkv, hd, bs)
    L.hip_attn_prefill(out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), ctx.data_ptr(),
                       cu_q.data_ptr(), tseq.data_ptr(), tq0.data_ptr(), len(tseq), nq, nkv, hd, mb, bs,
                       1 / math.sqrt(hd))
    torch.cuda.synchronize()
    check_hip_error("golden")
    got = out.cpu().numpy().view(np.uint16)
    compare(got, g["out_f32"], "golden")
    assert not got[31].any(), "padding row not zero"


def test_decode_graph_replays(gpu):
    """executor.zig:541-575 replay semantics through the C++ graph buckets: one captured store_kv + decode bucket
    replayed with different batches (all rows real, then 20 real + 12 padding rows, then all real again), with
    eager launches in between; every replay is checked against the oracle and padding rows are zero."""
    from llmgen_amd import host as H

    print("[gpu-test] decode graph replays", flush=True)
    wl = make("c2")
    t = wl.tensors(device="cuda")
    kc, vc = t["kc"].clone(), t["vc"].clone()
    graphs = H.Graphs([kc], [vc], wl.nq, wl.nkv, wl.hd, wl.block_size, wl.max_model_len, max_seqs=32, buckets=[32])
    seqs = [H.Sequence_([0] * (e.q_start + e.q_len), list(e.block_table)) for e in wl.entries]
    try:
        for n in (32, 20, 32):
            ents = [(i, e.q_start, e.q_len) for i, e in enumerate(wl.entries[:n])]
            sub = type(wl)(**{**wl.__dict__, "entries": wl.entries[:n]})
            kc.copy_(t["kc"])
            vc.copy_(t["vc"])
            out = torch.full((32, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device="cuda")
            used = graphs.step(seqs, ents, t["q"][:n], t["k"][:n], t["v"][:n], out)
            assert used == 32
            torch.cuda.synchronize()
            check_hip_error(f"graph replay n={n}")
            ts = {"q": t["q"][:n], "k": t["k"][:n], "v": t["v"][:n], "kc": t["kc"], "vc": t["vc"]}
            okc, _, _, of = run_oracle(sub, ts)
            compare(to_u16(out[:n]), of, f"graph replay n={n}")
            assert_cache_equal(to_u16(kc), okc, f"graph replay K n={n}")
            assert np.isnan(out[n:].float().cpu().numpy()).all(), "only the real rows are copied out"
            # eager work between replays (a different step through the same library)
            run_gpu(make("kt_decode"), make("kt_decode").tensors(device="cuda"))
    finally:
        graphs.destroy()


def test_mixed_step_graph_capture(gpu):
    """A mixed prefill + decode-row step (two kernels on two streams, joined by events) recorded into a hip graph
    and replayed three times with eager work in between; every replay matches the oracle."""
    print("[gpu-test] mixed step graph capture", flush=True)
    wl = make("gqa8")
    t = wl.tensors(device="cuda")
    pf = lib().hip_attn_prefill_tile()
    meta = wl.meta(pf)
    ws = wl.workspace()
    mgr = A.PagedAttentionManager()
    mgr.layers[0] = A.LayerState(t["kc"].clone(), t["vc"].clone())
    A.g_attn_mgr = mgr
    wl.bind(ws)
    out = torch.zeros((wl.n_tok, wl.nq, wl.hd), dtype=torch.bfloat16, device="cuda")
    node = A.AttnNode(out, [t["q"], t["k"], t["v"]], layer_id=0)
    A.PagedAttentionImpl.execute(0, node)  # warm-up (module load) outside capture
    torch.cuda.synchronize()
    L = lib()
    assert L.hip_graph_begin() == 0
    A.PagedAttentionImpl.execute(0, node)
    g = L.hip_graph_end()
    assert g, "capture failed"
    _, _, _, of = run_oracle(wl, t)
    try:
        for i in range(3):
            out.zero_()
            L.hip_graph_launch(g)
            torch.cuda.synchronize()
            check_hip_error(f"mixed replay {i}")
            compare(to_u16(out), of, f"mixed replay {i}")
            run_gpu(make("kt_prefill"), make("kt_prefill").tensors(device="cuda"))  # eager work in between
            A.g_attn_mgr = mgr
    finally:
        L.hip_graph_destroy(g)


# ---------------------------------------------------------------- full-size properties
def _step(wl, t):
    """store_kv + attention of wl through PagedAttentionImpl on tensors t (not modified); returns out, kc, vc."""
    return run_gpu(wl, t)


def test_c5d_block_permutation_invariance(gpu):
    """Full c5d (16 x 32768 keys): relabelling the physical blocks (pool rows moved, tables mapped the same way)
    leaves the decode output bit-identical and moves the written KV rows with it."""
    import copy as _copy

    from llmgen_amd.step import Entry

    wl = make("c5d")
    print("[gpu-test] c5d permutation", flush=True)
    t = wl.tensors(device="cuda")
    out0, kc0, vc0 = _step(wl, t)
    perm = np.random.default_rng(9).permutation(wl.num_blocks)  # physical block b -> perm[b]
    inv = torch.from_numpy(np.argsort(perm)).to("cuda")
    t2 = dict(t)
    t2["kc"], t2["vc"] = t["kc"][inv], t["vc"][inv]  # new pool row perm[b] holds old block b
    wl2 = _copy.copy(wl)
    wl2.entries = [Entry(e.q_start, e.q_len, [int(perm[b]) for b in e.block_table]) for e in wl.entries]
    out1, kc1, vc1 = _step(wl2, t2)
    np.testing.assert_array_equal(to_u16(out1), to_u16(out0))
    assert_cache_equal(to_u16(kc1), to_u16(kc0[inv]), "permuted K cache")
    assert_cache_equal(to_u16(vc1), to_u16(vc0[inv]), "permuted V cache")


def test_c5p_chunked_prefill_equals_tail(gpu):
    """Full c5p (16384-token prompt): prefilling the last 4096 tokens as a chunk against the cached first 12288
    gives exactly the last 4096 rows of the full prefill (each row's keys, order and arithmetic are the same)."""
    import copy as _copy

    from llmgen_amd.step import Entry

    wl = make("c5p")
    print("[gpu-test] c5p chunk", flush=True)
    t = wl.tensors(device="cuda")
    out_full, kc, vc = _step(wl, t)
    L, tail = wl.entries[0].q_len, 4096
    wl2 = _copy.copy(wl)
    wl2.entries = [Entry(L - tail, tail, wl.entries[0].block_table)]
    t2 = {"q": t["q"][L - tail:].contiguous(), "k": t["k"][L - tail:].contiguous(),
          "v": t["v"][L - tail:].contiguous(), "kc": kc, "vc": vc}
    out_chunk, _, _ = _step(wl2, t2)
    np.testing.assert_array_equal(to_u16(out_chunk), to_u16(out_full)[L - tail:])


@pytest.mark.parametrize("tail", [2048, 2000])
def test_c3_chunked_prefill_equals_tail(gpu, tail):
    """c3's 3584-token prompt alone (GQA 2, a pure prefill step: the key-split kernel), then its last `tail` tokens
    as a chunk against the cached rest (256 units: the key-split kernel again): bit-identical to the tail of the full
    prefill.  Key tiles sit at absolute positions, so each tile goes to the same key group in both runs and every
    row sums the same keys in the same order; 2000 is not a multiple of the 64-row tile, so the chunk's tiles start
    mid-tile of the full prefill.  (A chunk of at most 128 units runs the pieces kernel, whose piece boundaries
    follow the chunk: its rows match the full prefill within tolerance, not bit for bit.)"""
    import copy as _copy

    from llmgen_amd.step import Entry

    wl = _copy.copy(make("c3"))
    wl.entries = wl.entries[:1]
    L = wl.entries[0].q_len
    print(f"[gpu-test] c3 chunk tail={tail}", flush=True)
    t = wl.tensors(device="cuda")
    t = {k: (v[:L].contiguous() if k in ("q", "k", "v") else v) for k, v in t.items()}
    assert wl.meta(lib().hip_attn_prefill_tile()).single_rows() == 0
    out_full, kc, vc = _step(wl, t)
    wl2 = _copy.copy(wl)
    wl2.entries = [Entry(L - tail, tail, wl.entries[0].block_table)]
    t2 = {"q": t["q"][L - tail:].contiguous(), "k": t["k"][L - tail:].contiguous(),
          "v": t["v"][L - tail:].contiguous(), "kc": kc, "vc": vc}
    m2 = wl2.meta(lib().hip_attn_prefill_tile())
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert lib().hip_attn_prefill_plan(m2.n_tiles, wl.nq, wl.nkv, wl.hd, wl.block_size, 0) == 2  # KEYSPLIT
    out_chunk, _, _ = _step(wl2, t2)
    np.testing.assert_array_equal(to_u16(out_chunk), to_u16(out_full)[L - tail:])


def test_zero_sized_launches_are_noops(gpu):
    """T <= 0, S <= 0 and n_tiles <= 0 launch nothing (the reference's degenerate-input contract), also for the
    fused entry points; the output buffer is untouched and no error is raised."""
    L = lib()
    out = torch.full((4, 4, 128), 7.0, dtype=torch.bfloat16, device="cuda")
    before = to_u16(out).copy()
    dummy = torch.zeros(1 << 16, dtype=torch.int32, device="cuda").data_ptr()
    p = out.data_ptr()
    for n in (0, -3):
        L.hip_store_kv(dummy, dummy, dummy, dummy, dummy, n, 2, 128, 16)
        L.hip_attn_decode(p, dummy, dummy, dummy, dummy, dummy, n, 4, 2, 128, 4, 16, 0.1, dummy, dummy, 64, 4)
        L.hip_attn_decode_store_kv(p, dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, n, 4, 2, 128, 4, 16,
                                   0.1, dummy, dummy, 64, 4)
        L.hip_attn_prefill(p, dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, n, 4, 2, 128, 4, 16, 0.1)
        L.hip_qk_norm_rope_store_kv(p, dummy, dummy, dummy, dummy, dummy, dummy, dummy, 1e-6, dummy, dummy, dummy,
                                    dummy, n, 4, 2, 128, 16)
    torch.cuda.synchronize()
    check_hip_error("zero-sized launches")
    np.testing.assert_array_equal(to_u16(out), before)



@pytest.mark.parametrize("name", ["cpu_mixed", "bs48", "bs6", "gqa8", "c4", "c3", "kt_prefill"])
def test_prefill_rows_hint_matches_unknown_count(gpu, name):
    """hip_attn_prefill_rows with the step's single-row segment count against hip_attn_prefill (count unknown).
    With a count > 0 the step runs as one launch of the mixed-step kernel at GQA 2 and 4 (cpu_mixed, bs48, bs6, c4),
    bit-identical since every workgroup role computes its rows as the separate kernels do (their prefill units are
    too short to be split).  Otherwise a known count or 0 (a pure prefill step: no decode-row launch) can select
    another prefill kernel (the pieces kernel for gqa8's few units, the key-split or pieces kernel for small pure
    steps), which sums the keys in another order: then both outputs are checked against the oracle (sampled
    rows)."""
    wl = make(name)
    print(f"[gpu-test] {name}", flush=True)
    t = wl.tensors(device="cuda")
    meta = wl.meta(lib().hip_attn_prefill_tile())
    assert not meta.decode
    L = lib()
    kc, vc = t["kc"].clone(), t["vc"].clone()
    seg = torch.from_numpy(meta.packed()).to("cuda")
    off = {k: seg.data_ptr() + 4 * v for k, v in meta.offsets.items()}
    L.hip_store_kv(t["k"].data_ptr(), t["v"].data_ptr(), off["slots"], kc.data_ptr(), vc.data_ptr(), wl.n_tok,
                   wl.nkv, wl.hd, wl.block_size)
    outs = []
    for hint in (None, meta.single_rows()):
        out = torch.full((wl.n_tok, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device="cuda")
        args = (out.data_ptr(), t["q"].data_ptr(), kc.data_ptr(), vc.data_ptr(), off["block_tables"], off["ctx"],
                off["cu_q"], off["tile_seq"], off["tile_q0"], meta.n_tiles, wl.nq, wl.nkv, wl.hd, wl.max_blocks,
                wl.block_size, wl.scale)
        if hint is None:
            L.hip_attn_prefill(*args)
        else:
            L.hip_attn_prefill_rows(*args, hint)
        torch.cuda.synchronize()
        check_hip_error(name)
        outs.append(to_u16(out))
    plans = [L.hip_attn_prefill_plan(meta.n_tiles, wl.nq, wl.nkv, wl.hd, wl.block_size, h)
             for h in (-1, meta.single_rows())]
    if (plans[1] & 15) not in (1, plans[0] & 15):  # another kernel than the mixed one or the unknown count's
        rows = _sample_rows(wl, meta)
        _, _, _, of = run_oracle(wl, t, rows=rows, threads=16)
        for o, what in zip(outs, ("unknown", "hint 0")):
            compare(o[rows], of, f"{name} {what}")
    else:
        np.testing.assert_array_equal(outs[1], outs[0])


def test_prefill_plan_names_the_kernel_each_config_runs(gpu):
    """hip_attn_prefill_plan reports the launch hip_attn_prefill_rows makes, from the same rule: mixed steps at
    GQA 2 / 4 with a known single-row count run one mixed-step launch, c3 (99 tiles x 8 KV heads = 792 units of two
    heads, above 2.5 per CU) the 4-wave kernel, c5p (GQA 4, 256 tiles) the 8-wave four-head kernel, pure prefills
    of at most half a unit per CU (kt_prefill) the pieces kernel, larger small ones the key-split kernel, and an
    unknown count adds the separate decode-row launch; c3 (792 two-head units, 3.1 per CU) splits its heaviest
    tiles' units over two workgroups each."""
    L = lib()
    pf = L.hip_attn_prefill_tile()
    plan = {}
    for name in ("c3", "c4", "c5p", "kt_prefill", "gqa8", "gqa1", "cpu_mixed", "bs48"):
        wl = make(name)
        m = wl.meta(pf)
        plan[name] = (L.hip_attn_prefill_plan(m.n_tiles, wl.nq, wl.nkv, wl.hd, wl.block_size, m.single_rows()),
                      L.hip_attn_prefill_plan(m.n_tiles, wl.nq, wl.nkv, wl.hd, wl.block_size, -1))
    MIXED, KEYSPLIT, W2, W4, W8, SPLIT, PIECES, ROWS = 1, 2, 3, 4, 5, 6, 7, 16
    assert plan["c3"] == (SPLIT, W4 | ROWS)
    assert plan["c4"] == (MIXED, W4 | ROWS)
    assert plan["c5p"] == (W8, W8 | ROWS)
    assert plan["kt_prefill"] == (PIECES, W4 | ROWS)
    # pure prefill at GQA 2, 8 KV heads, 256 CUs: up to 128 units the pieces kernel, then the key split
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert L.hip_attn_prefill_plan(16, 16, 8, 128, 256, 0) == PIECES
        assert L.hip_attn_prefill_plan(17, 16, 8, 128, 256, 0) == KEYSPLIT
        assert L.hip_attn_prefill_plan(20, 16, 8, 128, 256, 0) == KEYSPLIT
    # GQA 8 and 1 mixed steps with a known count: their few prefill units take the pieces kernel beside the rows
    assert plan["gqa8"] == (PIECES | ROWS, W8 | ROWS)
    assert plan["gqa1"] == (PIECES | ROWS, W2 | ROWS)
    assert plan["cpu_mixed"][0] == MIXED and plan["bs48"][0] == MIXED
    assert L.hip_attn_prefill_plan(0, 16, 8, 128, 256, 0) == 0
    assert L.hip_attn_prefill_plan(4, 16, 8, 64, 256, 0) == -1 and L.hip_attn_prefill_plan(4, 24, 8, 128, 256, 0) == -1


@pytest.mark.parametrize("name", ["c4", "bs48", "cpu_mixed"])
def test_mixed_kernel_gives_the_same_rows_for_any_tile_order(gpu, name):
    """The mixed-step kernel sizes its two parts from the single-row count and expects the single-row tiles first;
    a list in any other order (here a seeded shuffle, which puts multi-row tiles in the decode part and single-row
    tiles in the prefill part) must give the same output bit for bit, every role running whatever tile it finds."""
    wl = make(name)
    print(f"[gpu-test] mixed any order {name}", flush=True)
    t = wl.tensors(device="cuda")
    L = lib()
    meta = wl.meta(L.hip_attn_prefill_tile())
    assert not meta.decode and meta.single_rows() > 0
    assert L.hip_attn_prefill_plan(meta.n_tiles, wl.nq, wl.nkv, wl.hd, wl.block_size, meta.single_rows()) == 1
    kc, vc = t["kc"].clone(), t["vc"].clone()
    outs = []
    for shuffle in (False, True):
        buf = meta.packed().copy()
        if shuffle:
            perm = np.random.default_rng(9).permutation(meta.n_tiles)
            o_s, o_q = meta.offsets["tile_seq"], meta.offsets["tile_q0"]
            buf[o_s:o_s + meta.n_tiles] = meta.tile_seq[perm]
            buf[o_q:o_q + meta.n_tiles] = meta.tile_q0[perm]
            moved = np.diff(meta.cu_q)[meta.tile_seq[perm]][:meta.single_rows()]
            assert (moved > 1).any(), "the shuffle must put multi-row tiles into the decode part"
        seg = torch.from_numpy(buf).to("cuda")
        off = {k: seg.data_ptr() + 4 * v for k, v in meta.offsets.items()}
        if not shuffle:
            L.hip_store_kv(t["k"].data_ptr(), t["v"].data_ptr(), off["slots"], kc.data_ptr(), vc.data_ptr(),
                           wl.n_tok, wl.nkv, wl.hd, wl.block_size)
        out = torch.full((wl.n_tok, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device="cuda")
        L.hip_attn_prefill_rows(out.data_ptr(), t["q"].data_ptr(), kc.data_ptr(), vc.data_ptr(), off["block_tables"],
                                off["ctx"], off["cu_q"], off["tile_seq"], off["tile_q0"], meta.n_tiles, wl.nq, wl.nkv,
                                wl.hd, wl.max_blocks, wl.block_size, wl.scale, meta.single_rows())
        torch.cuda.synchronize()
        check_hip_error(f"{name} shuffle={shuffle}")
        outs.append(to_u16(out))
    assert not np.isnan(oracle.bf16_to_f32(outs[0])).any()
    np.testing.assert_array_equal(outs[1], outs[0])
    if name != "c4":  # small steps: every row against the oracle as well
        _, _, _, of = run_oracle(wl, t)
        compare(outs[1], of, f"{name} shuffled")


@pytest.mark.parametrize("name", ["kt_prefill", "cpu_mixed", "c2", "gqa8d", "bs48", "bs6", "c3"])
def test_uniform_scores_give_mean_v(gpu, name):
    """Closed form, independent of the oracle: with q = 0 every score is 0, so each output row is the plain mean
    of V over the keys its position sees (0..pos), and padding rows are 0.  Checks the decode and prefill kernels'
    key ranges, causal masks, block-table walks and normalisation against numpy on the post-step cache."""
    wl = make(name)
    print(f"[gpu-test] {name}", flush=True)
    t = wl.tensors(device="cuda")
    t["q"] = torch.zeros_like(t["q"])
    out, _, vc = run_gpu(wl, t)
    got = oracle.bf16_to_f32(to_u16(out)).astype(np.float64)
    v = oracle.bf16_to_f32(to_u16(vc)).astype(np.float64)  # [blocks, nkv, bs, hd]
    meta = wl.meta(lib().hip_attn_prefill_tile())
    G = wl.nq // wl.nkv
    for s in range(meta.n_seq):
        b, e, ctx = int(meta.cu_q[s]), int(meta.cu_q[s + 1]), int(meta.ctx[s])
        q_len = e - b
        if q_len == 0:
            continue
        if ctx < q_len:
            assert not got[b:e].any(), f"{name}: padding rows of sequence {s} not zero"
            continue
        keys = np.arange(ctx)
        blk = meta.block_tables[s][keys // wl.block_size]
        vs = v[blk, :, keys % wl.block_size, :]  # [ctx, nkv, hd]
        mean = np.cumsum(vs, axis=0) / (keys + 1)[:, None, None]
        want = mean[ctx - q_len:ctx]  # [q_len, nkv, hd]
        want = np.repeat(want, G, axis=1)  # heads kvh*G .. kvh*G+G-1 share kv head kvh
        np.testing.assert_allclose(got[b:e], want, rtol=8e-3, atol=2e-3, err_msg=f"{name} sequence {s}")


@pytest.mark.parametrize("name", ["kt_prefill", "kt_decode", "gqa8"])
def test_scores_growing_along_the_keys(gpu, name):
    """Scores that grow by ~1.6 (log2 units) per key, to ~245 at the last key: every later key tile exceeds the
    running softmax reference by far more than 2^64, so the kernels must move their reference (and rescale the
    accumulated output) again and again.  q = 1, key at position p = 0.1 p in every dim, both in the cache
    history and in this step's k."""
    wl = make(name)
    print(f"[gpu-test] {name}", flush=True)
    t = wl.tensors(device="cpu")
    meta = wl.meta(lib().hip_attn_prefill_tile())
    t["q"] = torch.ones_like(t["q"])
    kc, k = t["kc"].float(), t["k"].float()
    for s in range(meta.n_seq):
        b, e, ctx = int(meta.cu_q[s]), int(meta.cu_q[s + 1]), int(meta.ctx[s])
        for p in range(ctx):
            val = 0.1 * p
            if p < ctx - (e - b):  # history: in the cache at the block table's slot
                kc[meta.block_tables[s][p // wl.block_size], :, p % wl.block_size, :] = val
            else:
                k[b + p - (ctx - (e - b))] = val
    t["kc"], t["k"] = kc.to(torch.bfloat16), k.to(torch.bfloat16)
    td = {n: x.to("cuda") for n, x in t.items()}
    out, _, _ = run_gpu(wl, td)
    _, _, _, of = run_oracle(wl, t)
    compare(to_u16(out), of, f"{name} growing scores")



@pytest.mark.parametrize("name", ["c2", "gqa8d", "c1", "cpu_mixed", "c3"])
def test_step_output_is_bit_reproducible(gpu, name):
    """The same step run twice gives the same bits: each wave's token set and every merge order are fixed (no
    dynamic work distribution, no atomics on values), for split-K decode with its cross-workgroup merge (c1,
    gqa8d), batched decode (c2), a mixed step (cpu_mixed) and prefill (c3)."""
    wl = make(name)
    print(f"[gpu-test] {name}", flush=True)
    t = wl.tensors(device="cuda")
    outs = [to_u16(run_gpu(wl, t)[0]) for _ in range(3)]
    np.testing.assert_array_equal(outs[1], outs[0])
    np.testing.assert_array_equal(outs[2], outs[0])


@pytest.mark.parametrize("name", ["cpu_mixed", "gqa8", "c4"])
def test_mixed_step_graph_replay(gpu, name):
    """A whole mixed step captured into a graph: store_kv, the MFMA prefill kernel, and the decode rows forked to
    the library's side stream and joined back inside the capture.  Three replays, with eager torch work and
    synchronisations between them, each give the eager step's output bit for bit."""
    wl = make(name)
    print(f"[gpu-test] {name}", flush=True)
    t = wl.tensors(device="cuda")
    A.init_device()
    L = lib()
    meta = wl.meta(L.hip_attn_prefill_tile())
    assert not meta.decode and meta.single_rows() > 0
    ws = wl.workspace()
    mgr = A.PagedAttentionManager()
    mgr.layers[0] = A.LayerState(t["kc"].clone(), t["vc"].clone())
    A.g_attn_mgr = mgr
    wl.bind(ws)
    node_out = torch.full((wl.n_tok, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device="cuda")
    node = A.AttnNode(node_out, [t["q"], t["k"], t["v"]], layer_id=0)
    A.PagedAttentionImpl.execute(0, node)
    torch.cuda.synchronize()
    check_hip_error(name)
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
            check_hip_error(f"{name} replay {i}")
            np.testing.assert_array_equal(to_u16(node_out), ref)
            del junk
    finally:
        L.hip_graph_destroy(g)


@pytest.mark.parametrize("name", ["c3", "kt_prefill"])
def test_pure_prefill_graph_replay(gpu, name):
    """A pure prefill step at GQA 2 (no decode-row launch) captured into a graph: three replays with eager torch
    work between them each give the eager step's output bit for bit.  c3 (792 two-head units, above the key-split
    rule's 2.5 per CU) runs the 4-wave kernel with its heaviest units split over two workgroups (halves merged
    through the library's scratch, their ticket counters back at 0 after every launch), kt_prefill (2 tiles, 4
    units) the pieces kernel."""
    wl = make(name)
    print(f"[gpu-test] pure prefill graph {name}", flush=True)
    t = wl.tensors(device="cuda")
    A.init_device()
    L = lib()
    meta = wl.meta(L.hip_attn_prefill_tile())
    assert not meta.decode and meta.single_rows() == 0 and wl.nq // wl.nkv == 2
    want = {"c3": 6, "kt_prefill": 7}[name]  # LLMGEN_PREFILL_SPLIT, LLMGEN_PREFILL_PIECES
    assert L.hip_attn_prefill_plan(meta.n_tiles, wl.nq, wl.nkv, wl.hd, wl.block_size, 0) == want
    ws = wl.workspace()
    mgr = A.PagedAttentionManager()
    mgr.layers[0] = A.LayerState(t["kc"].clone(), t["vc"].clone())
    A.g_attn_mgr = mgr
    wl.bind(ws)
    node_out = torch.full((wl.n_tok, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device="cuda")
    node = A.AttnNode(node_out, [t["q"], t["k"], t["v"]], layer_id=0)
    A.PagedAttentionImpl.execute(0, node)
    torch.cuda.synchronize()
    check_hip_error(name)
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
            check_hip_error(f"{name} replay {i}")
            np.testing.assert_array_equal(to_u16(node_out), ref)
            del junk
    finally:
        L.hip_graph_destroy(g)
