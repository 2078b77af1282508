"""GPU: hip_attn_decode_noalloc (split-K partials in the library's own device array, no caller scratch, no
allocation) gives bit for bit what hip_attn_decode gives with caller-owned scratch, on consecutive calls whose
inputs shrink (so the second call finds the first call's partials in the shared array), runs single-part launches
of any size without the array, and rejects a launch whose partials exceed the array without launching anything,
reporting it through hip_last_error()."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from harness import check_hip_error
from llmgen_amd import step as S
from llmgen_amd._lib import lib
from llmgen_amd.workloads import make, to_u16

pytestmark = pytest.mark.gpu


def _decode_inputs(name, n_seq=None):
    wl = make(name)
    if n_seq is not None:
        wl.entries = wl.entries[:n_seq]
    t = wl.tensors(device="cuda")
    meta = wl.meta(64)
    assert meta.decode
    n = meta.n_tok
    d = lambda a: torch.from_numpy(a).to("cuda")  # noqa: E731
    kc, vc = t["kc"].clone(), t["vc"].clone()
    lib().hip_store_kv(t["k"].data_ptr(), t["v"].data_ptr(), d(meta.slots).data_ptr(), kc.data_ptr(),
                       vc.data_ptr(), n, wl.nkv, wl.hd, wl.block_size)
    return wl, n, t["q"][:n].contiguous(), kc, vc, d(meta.block_tables), d(meta.ctx)


def _both(wl, n, q, kc, vc, bt, ctx):
    L = lib()
    ps, mp = S.part_size(n), S.max_parts(n, wl.max_model_len)
    common = (q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), ctx.data_ptr(), n, wl.nq, wl.nkv, wl.hd,
              wl.max_blocks, wl.block_size, wl.scale)
    po = torch.empty(n * wl.nq * mp * wl.hd, dtype=torch.float32, device="cuda")
    pml = torch.empty(n * wl.nq * mp * 2, dtype=torch.float32, device="cuda")
    ref = torch.full((n, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device="cuda")
    L.hip_attn_decode(ref.data_ptr(), *common, po.data_ptr(), pml.data_ptr(), ps, mp)
    got = torch.full_like(ref, float("nan"))
    L.hip_attn_decode_noalloc(got.data_ptr(), *common, ps, mp)
    torch.cuda.synchronize()
    check_hip_error(f"noalloc {wl.name}")
    return to_u16(ref), to_u16(got)


def test_noalloc_decode_equals_caller_scratch_on_shrinking_calls(gpu):
    # c5d: 16 x 32K keys, split into several partials per (sequence, head); then smaller launches that reuse
    # the same array: c1 (1 sequence, 4-wave workgroups, partials merged in the kernel), kt_decode, c2 subset
    for name, n_seq in (("c5d", None), ("c1", None), ("kt_decode", None), ("c2", 20)):
        print(f"[gpu-test] noalloc {name} n_seq={n_seq}", flush=True)
        ref, got = _both(*_decode_inputs(name, n_seq))
        assert np.isfinite(ref.view(np.int16).astype(np.float32)).all()
        np.testing.assert_array_equal(got, ref, err_msg=f"noalloc != hip_attn_decode on {name}")


def _custom(name, nq, nkv, bs, ctxs, seed):
    """A decode step of len(ctxs) sequences with contiguous per-sequence blocks, as a named Workload."""
    from llmgen_amd.workloads import Workload, _decode_entries, _tables

    rng = np.random.default_rng(seed)
    tables, nb = _tables(rng, ctxs, bs, permute=True)
    mb = max(len(t) for t in tables)
    return Workload(name, nq, nkv, 128, bs, nb, mb, mb * bs, _decode_entries(ctxs, tables), std=1.0, seed=seed)


def _inputs_of(wl):
    t = wl.tensors(device="cuda")
    meta = wl.meta(64)
    n = meta.n_tok
    d = lambda a: torch.from_numpy(a).to("cuda")  # noqa: E731
    kc, vc = t["kc"], t["vc"]
    lib().hip_store_kv(t["k"].data_ptr(), t["v"].data_ptr(), d(meta.slots).data_ptr(), kc.data_ptr(),
                       vc.data_ptr(), n, wl.nkv, wl.hd, wl.block_size)
    return n, t["q"][:n].contiguous(), kc, vc, d(meta.block_tables), d(meta.ctx)


def test_noalloc_decode_large_single_part_batch(gpu):
    """512 sequences at 32 heads: one part per (sequence, head), so no partial is stored and the launch runs
    whatever S * nq is (its partials at max_parts would exceed the array); equal to hip_attn_decode bit for bit."""
    print("[gpu-test] noalloc 512x32 single part", flush=True)
    rng = np.random.default_rng(61)
    wl = _custom("big", 32, 8, 16, [int(c) for c in rng.integers(1, 120, size=512)], 61)
    n, q, kc, vc, bt, ctx = _inputs_of(wl)
    assert lib().hip_last_error() == 0
    ref, got = _both(wl, n, q, kc, vc, bt, ctx)
    np.testing.assert_array_equal(got, ref)


def test_noalloc_decode_rejects_oversized_launch(gpu):
    """One sequence of 65280 keys at GQA 16 (nkv 1) with 64-token parts and max_parts 1020: the launcher keeps
    1020 parts (a 1-pair launch is far below one generation of workgroups), whose partials need
    16 x 1020 x 520 B > 8 MiB.  The call prints one line, launches nothing (the output keeps its sentinel) and
    hip_last_error() reports the rejection; hip_attn_decode with caller scratch runs the same launch.  All
    buffers are real and sized for the launch, so a launch accepted by mistake stays in bounds."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the part count of this launch is derived for 256 compute units")
    print("[gpu-test] noalloc oversized", flush=True)
    L = lib()
    wl = _custom("over", 16, 1, 256, [65280], 62)
    n, q, kc, vc, bt, ctx = _inputs_of(wl)
    ps, mp = 64, 1020
    assert wl.max_blocks * wl.block_size >= ps * mp
    common = (q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), ctx.data_ptr(), n, wl.nq, wl.nkv, wl.hd,
              wl.max_blocks, wl.block_size, wl.scale)
    torch.cuda.synchronize()
    assert L.hip_last_error() == 0
    out = torch.full((n, wl.nq, wl.hd), 3.0, dtype=torch.bfloat16, device="cuda")
    before = to_u16(out).copy()
    L.hip_attn_decode_noalloc(out.data_ptr(), *common, ps, mp)
    torch.cuda.synchronize()
    assert L.hip_last_error() != 0, "the rejected launch must be reported"
    assert L.hip_last_error() == 0, "the report is cleared by the read"
    np.testing.assert_array_equal(to_u16(out), before)
    po = torch.empty(n * wl.nq * mp * wl.hd, dtype=torch.float32, device="cuda")
    pml = torch.empty(n * wl.nq * mp * 2, dtype=torch.float32, device="cuda")
    L.hip_attn_decode(out.data_ptr(), *common, po.data_ptr(), pml.data_ptr(), ps, mp)
    torch.cuda.synchronize()
    check_hip_error("decode of the launch noalloc rejects")
    assert not np.array_equal(to_u16(out), before)


def test_noalloc_decode_replays_from_a_graph(gpu):
    """The allocation-free decode recorded into a graph (the use it exists for) and replayed three times with eager
    calls of other sizes between the replays (which rewrite the shared array): every replay equals
    hip_attn_decode with caller scratch, bit for bit."""
    from llmgen_amd.attention import init_device

    print("[gpu-test] noalloc graph", flush=True)
    init_device()
    L = lib()
    wl, n, q, kc, vc, bt, ctx = _decode_inputs("c1")  # 4 partial parts per (sequence, head): the array is used
    ref, got = _both(wl, n, q, kc, vc, bt, ctx)  # eager first call (takes the array's address outside capture)
    np.testing.assert_array_equal(got, ref)
    ps, mp = S.part_size(n), S.max_parts(n, wl.max_model_len)
    out = torch.full((n, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device="cuda")
    args = (out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), ctx.data_ptr(), n, wl.nq,
            wl.nkv, wl.hd, wl.max_blocks, wl.block_size, wl.scale, ps, mp)
    assert L.hip_graph_begin() == 0
    L.hip_attn_decode_noalloc(*args)
    g = L.hip_graph_end()
    assert g
    try:
        other = _decode_inputs("kt_decode")
        for i in range(3):
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            L.hip_graph_launch(g)
            torch.cuda.synchronize()
            check_hip_error(f"noalloc graph replay {i}")
            np.testing.assert_array_equal(to_u16(out), ref)
            _both(*other)  # eager calls of another shape between the replays
    finally:
        L.hip_graph_destroy(g)
