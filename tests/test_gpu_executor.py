"""GPU: the C++ executor slice drives the kernels (include/llmgen_host.h).

fill_meta + one upload + bind_step + llmgen_paged_attention (the C++ PagedAttentionImpl) on the reference's
test steps and c2, checked against the oracle; and the C++ decode graph buckets replayed with changing batches
(eager steps in between), checked against the eager C++ path bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from harness import assert_cache_equal, check_hip_error, compare, run_oracle
from llmgen_amd import host as H
from llmgen_amd import step as S
from llmgen_amd.workloads import make, to_u16

pytestmark = pytest.mark.gpu


def _seqs_entries(wl, rng):
    seqs, entries = [], []
    for i, e in enumerate(wl.entries):
        n = e.q_start + e.q_len
        seqs.append(H.Sequence_(rng.integers(0, 1000, n).tolist(), list(e.block_table), 0.0))
        entries.append((i, e.q_start, e.q_len))
    return seqs, entries


def _run_cpp(wl, t, seqs, entries, pf_tile, seq_num=None, max_blocks=None):
    """One eager step through the C++ slice.  seq_num > len(entries) adds decode padding rows (zero q/k/v)."""
    decode = all(e[2] == 1 for e in entries)
    n_tiles = 0 if decode else sum((e[2] + pf_tile - 1) // pf_tile for e in entries)
    n = len(entries)
    seq_num = n if seq_num is None else seq_num
    mb = wl.max_blocks if max_blocks is None else max_blocks
    buf, lay, _, single = H.fill_meta(seqs, entries, seq_num, n_tiles, pf_tile, wl.block_size, mb)
    dev = t["q"].device
    meta_dev = torch.from_numpy(buf).to(dev)
    n_real = sum(e[2] for e in entries)
    n_tok = n_real + (seq_num - n)
    ws = H.workspace(wl.nq, wl.hd, max(seq_num, 1), n_tok, wl.max_model_len, wl.block_size)
    po = torch.empty(ws["part_o"] // 4 + 1, dtype=torch.float32, device=dev)
    pml = torch.empty(ws["part_ml"] // 4 + 1, dtype=torch.float32, device=dev)
    st = H.bind_step(meta_dev.data_ptr(), lay, n_tok, seq_num, n_tiles, decode, wl.nq, wl.nkv, wl.hd,
                     wl.block_size, mb, wl.max_model_len, po.data_ptr(), pml.data_ptr(), single_rows=single)
    assert st.single_rows == H.single_rows(entries, seq_num)
    kc, vc = t["kc"].clone(), t["vc"].clone()

    def rows(x):
        y = torch.zeros((n_tok,) + tuple(x.shape[1:]), dtype=x.dtype, device=dev)
        y[:n_real] = x[:n_real]
        return y

    q, k, v = rows(t["q"]), rows(t["k"]), rows(t["v"])
    out = torch.full((n_tok, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device=dev)
    H.paged_attention(st, out, q, k, v, kc, vc)
    torch.cuda.synchronize()
    check_hip_error(wl.name)
    return out[:n_real], kc, vc


@pytest.mark.parametrize("name", ["kt_prefill", "kt_decode", "c1", "c2", "gqa8"])
def test_cpp_executor_step_matches_oracle(gpu, name):
    wl = make(name)
    wl.pad_rows = 0  # the engine pads decode graph buckets only; eager steps carry their real rows
    print(f"[gpu-test] C++ executor {name}", flush=True)
    t = wl.tensors(device="cuda")
    seqs, entries = _seqs_entries(wl, np.random.default_rng(1))
    out, kc, vc = _run_cpp(wl, t, seqs, entries, H.L().hip_attn_prefill_tile())
    okc, ovc, ob, of = run_oracle(wl, t)
    assert_cache_equal(to_u16(kc), okc, f"{name} K")
    assert_cache_equal(to_u16(vc), ovc, f"{name} V")
    meta = wl.meta(64)
    real = np.ones(meta.n_tok, bool)
    for s in range(meta.n_seq):  # padding sequences (ctx < q_len) are zero rows in both
        if meta.ctx[s] < meta.cu_q[s + 1] - meta.cu_q[s]:
            real[meta.cu_q[s]:meta.cu_q[s + 1]] = False
    compare(to_u16(out)[real], of[real], f"C++ {name}")


def test_cpp_decode_graph_buckets(gpu):
    """captureGraphs / forward replay in C++: buckets {8, 32}; steps of 32, 20 (padded to 32), 5 (padded to 8)
    and 32 sequences, eager C++ steps in between; each replay equals the eager C++ step with the same padding
    rows bit for bit (output and KV caches).  (Without the same padding the split-K partition, which depends
    on the row count, differs and so does the last bit of a few outputs.)"""
    wl = make("c2")
    print("[gpu-test] C++ decode graphs", flush=True)
    t = wl.tensors(device="cuda")
    rng = np.random.default_rng(2)
    seqs, entries = _seqs_entries(wl, rng)
    kc_g, vc_g = t["kc"].clone(), t["vc"].clone()
    graphs = H.Graphs([kc_g], [vc_g], wl.nq, wl.nkv, wl.hd, wl.block_size, wl.max_model_len, max_seqs=32,
                      buckets=[8, 32])
    try:
        for n in (32, 20, 5, 32):
            ents = entries[:n]
            out_g = torch.full((n, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device="cuda")
            kc_g.copy_(t["kc"])
            vc_g.copy_(t["vc"])
            used = graphs.step(seqs, ents, t["q"][:n], t["k"][:n], t["v"][:n], out_g)
            assert used == (8 if n <= 8 else 32)
            torch.cuda.synchronize()
            check_hip_error(f"graph n={n}")
            sub = type(wl)(**{**wl.__dict__, "entries": wl.entries[:n]})
            mb = (wl.max_model_len + wl.block_size - 1) // wl.block_size  # the bucket's block-table width
            out_e, kc_e, vc_e = _run_cpp(sub, t, seqs, ents, 64, seq_num=used, max_blocks=mb)
            np.testing.assert_array_equal(to_u16(out_g), to_u16(out_e))
            assert_cache_equal(to_u16(kc_g), to_u16(kc_e), f"graph K n={n}")
            assert_cache_equal(to_u16(vc_g), to_u16(vc_e), f"graph V n={n}")
    finally:
        graphs.destroy()


@pytest.mark.parametrize("name", ["c3", "c4", "c5d", "c5p"])
def test_cpp_executor_full_configs_sampled_rows(gpu, name):
    """The full-size configs through the C++ PagedAttentionImpl (llmgen_paged_attention), the entry non-Zig hosts
    use: store_kv bit-exact over the whole cache, sampled rows (first and last of every tile and sequence plus
    48 seeded random rows) against the oracle, and the C++ step bit-identical to the Python operator's."""
    from harness import run_gpu
    from test_gpu_attention import _sample_rows

    wl = make(name)
    wl.pad_rows = 0
    print(f"[gpu-test] C++ executor {name}", flush=True)
    t = wl.tensors(device="cuda")
    seqs, entries = _seqs_entries(wl, np.random.default_rng(3))
    out, kc, vc = _run_cpp(wl, t, seqs, entries, H.L().hip_attn_prefill_tile())
    meta = wl.meta(64)
    rows = _sample_rows(wl, meta)
    okc, ovc, _, of = run_oracle(wl, t, rows=rows, threads=16)
    assert_cache_equal(to_u16(kc), okc, f"{name} K")
    assert_cache_equal(to_u16(vc), ovc, f"{name} V")
    compare(to_u16(out)[rows], of, f"C++ {name}")
    out_py, _, _ = run_gpu(wl, t)
    np.testing.assert_array_equal(to_u16(out), to_u16(out_py))


def test_cpp_executor_equals_python_operator_on_wide_steps(gpu):
    """The wide random steps (block sizes 1-512, GQA 1-16, decode-only, prefill-only and mixed) through the C++
    slice and through the Python operator: outputs and written caches bit for bit (steps with graph-bucket padding
    rows are left to the graph tests)."""
    from harness import run_gpu
    from test_gpu_random_shapes import WIDE_CASES, _wide_workload

    checked = 0
    for case in WIDE_CASES:
        wl = _wide_workload(case)
        if wl.pad_rows:
            continue
        print(f"[gpu-test] C++ vs Python {wl.name}: {wl.note}", flush=True)
        t = wl.tensors(device="cuda")
        out_py, kc_py, vc_py = run_gpu(wl, t)
        seqs, entries = _seqs_entries(wl, np.random.default_rng(case))
        assert (wl.decode is None) == all(e[2] == 1 for e in entries)  # both hosts pick the same launch
        out_c, kc_c, vc_c = _run_cpp(wl, t, seqs, entries, H.L().hip_attn_prefill_tile())
        assert_cache_equal(to_u16(kc_c), to_u16(kc_py), f"{wl.name} K")
        assert_cache_equal(to_u16(vc_c), to_u16(vc_py), f"{wl.name} V")
        np.testing.assert_array_equal(to_u16(out_c), to_u16(out_py), err_msg=wl.name)
        checked += 1
    assert checked >= 12
