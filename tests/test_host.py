"""Host-side logic and the C-ABI library, CPU only (no kernel is launched).

* step metadata restated from the executor (executor.zig:139-202, 609-632, 772-861; attention_v1.zig:51-57),
* algorithmic work of the BASELINE configurations (the metric definitions),
* libllmgen_attn.so loads and exports every symbol include/*.h declares,
* launcher argument checks that return before any device call (stderr message, no launch),
* operator error behaviour (AttentionNeedsBf16, NoAttentionManager, LayerNotActive).
"""
from __future__ import annotations

import glob
import os
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

from llmgen_amd import step as S
from llmgen_amd.workloads import BASELINE_CONFIGS, make

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


# ---------------------------------------------------------------- executor restatements
def test_part_size_and_max_parts():
    assert [S.part_size(s) for s in (1, 3, 4, 15, 16, 63, 64, 256)] == [64, 64, 128, 128, 256, 256, 512, 512]
    assert S.max_parts(16, 32768) == 128
    assert S.max_parts(1, 100) == 2
    assert S.max_parts(64, 4096) == 8


def test_workspace_bytes_takes_worst_bucket():
    nq, hd = 16, 128
    po, pml = S.workspace_bytes(nq, hd, 20, 4096)
    cap = max(s * S.max_parts(s, 4096) for s in range(1, 21))
    assert cap == 15 * 32  # S=15 with 128-token parts beats S=20 with 256-token parts and S=3 with 64
    assert po == cap * nq * hd * 4 and pml == cap * nq * 2 * 4


def test_decode_buckets():
    assert S.decode_buckets(1) == [1]
    assert S.decode_buckets(5) == [1, 2, 4, 5]
    assert S.decode_buckets(48) == [1, 2, 4, 8, 16, 32, 48]
    assert S.decode_buckets(50) == [1, 2, 4, 8, 16, 32, 48, 50]


def test_fill_meta_prefill_and_padding():
    ents = [S.Entry(0, 70, [3, 1, 4, 0, 2]), S.Entry(40, 1, [5, 6, 7])]
    m = S.fill_meta(ents, block_size=16, max_blocks=6, pf_tile=64, seq_num=3)
    assert not m.decode  # entry 0 has q_len 70
    assert m.n_tok == 72 and m.n_seq == 3
    assert list(m.cu_q) == [0, 70, 71, 72]
    assert list(m.ctx) == [70, 41, 0]
    assert list(m.last) == [69, 70, 71]
    # slot = bt[pos / bs] * bs + pos % bs (runner/batching.zig:74-77)
    for j in range(70):
        assert m.slots[j] == S.slot_of(ents[0].block_table, j, 16)
    assert m.slots[70] == 7 * 16 + 40 % 16  # position 40 lies in logical block 2 -> physical 7
    assert m.slots[71] == -1  # padding row never writes KV
    # tiles: 70 rows -> 2 tiles, decode entry -> 1, padding -> 1; listed lightest first by the keys each needs
    # (padding 0, decode row 41, rows 0-63 of entry 0: 64, rows 64-69: 70)
    assert list(m.tile_seq) == [2, 1, 0, 0] and list(m.tile_q0) == [0, 0, 0, 64]
    assert list(m.block_tables[0]) == [3, 1, 4, 0, 2, 0] and not m.block_tables[2].any()


def test_fill_meta_decode_bucket_and_packing():
    ents = [S.Entry(99, 1, [2, 0]), S.Entry(10, 1, [1])]
    m = S.fill_meta(ents, block_size=64, max_blocks=2, pf_tile=64, seq_num=4)
    assert m.decode and m.n_tiles == 0
    assert list(m.ctx) == [100, 11, 0, 0] and list(m.slots) == [0 * 64 + 35, 1 * 64 + 10, -1, -1]
    buf = m.packed()
    o = m.offsets
    assert list(buf[o["cu_q"]:o["cu_q"] + 5]) == [0, 1, 2, 3, 4]
    assert list(buf[o["block_tables"]:o["block_tables"] + 8]) == [2, 0, 1, 0, 0, 0, 0, 0]
    # layout is fixed per (T, S, tiles, max_blocks): the graph bucket can be refilled in place
    m2 = S.fill_meta([], 64, 2, 64, seq_num=4, decode=True)
    m2.packed()
    assert m2.offsets == o


# ---------------------------------------------------------------- metric definitions
def test_baseline_algorithmic_work():
    c5d = make("c5d")
    assert c5d.decode_bytes() == 2147483648 + 2 * 16 * 32 * 128 * 2
    c5p = make("c5p")
    assert c5p.attention_flops() == 4 * 128 * 32 * 16384 * 16385 // 2  # 2.199 TFLOP
    c3 = make("c3")
    prompt = 4 * 128 * 16 * 3584 * 3585 // 2
    assert abs(prompt / 1e9 - 52.6) < 0.1
    assert c3.attention_flops() > prompt
    c1 = make("c1")
    assert c1.decode_bytes() == 2097152 + 8192
    for name in BASELINE_CONFIGS:
        wl = make(name)
        m = wl.meta(64)
        assert m.n_tok == wl.n_tok and m.block_tables.shape == (len(wl.entries), wl.max_blocks)
        assert (m.ctx <= wl.max_model_len).all()
        # every block id of a table is a distinct physical block
        used = np.concatenate([np.asarray(e.block_table) for e in wl.entries])
        assert len(np.unique(used)) == len(used) and used.max() < wl.num_blocks


def test_c4_mixed_shape():
    wl = make("c4")
    qls = sorted(e.q_len for e in wl.entries)
    assert qls.count(512) == 8 and qls.count(1) == 248
    assert all(100 <= e.q_start + e.q_len <= 2048 for e in wl.entries if e.q_len == 1)


# ---------------------------------------------------------------- C-ABI library
def _declared_symbols():
    names = set()
    for header in sorted(glob.glob(os.path.join(ROOT, "include", "*.h"))):
        with open(header) as f:
            text = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
        names.update(re.findall(r"\b((?:hip|llmgen)_\w+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    from llmgen_amd._lib import SIGNATURES, lib

    from llmgen_amd.host import HOST_SIGNATURES

    declared = _declared_symbols()
    assert len(declared) >= 25
    assert sorted(list(SIGNATURES) + list(HOST_SIGNATURES)) == declared, "ctypes signatures out of sync with headers"
    L = lib()  # loads without a GPU
    for name in declared:
        assert hasattr(L, name), f"{name} not exported"


def test_prefill_tile_size():
    from llmgen_amd._lib import lib

    assert lib().hip_attn_prefill_tile() == 64


_BAD_SHAPES = r"""
import ctypes, sys
sys.path.insert(0, {root!r})
from llmgen_amd._lib import lib
L = lib()
# every call below is rejected on the host before any device call
L.hip_attn_decode(None, None, None, None, None, None, 1, 16, 8, 64, 4, 256, 0.1, None, None, 64, 8)
L.hip_attn_decode(None, None, None, None, None, None, 1, 24, 8, 128, 4, 256, 0.1, None, None, 64, 8)
L.hip_attn_prefill(None, None, None, None, None, None, None, None, None, 1, 16, 8, 96, 4, 256, 0.1)
L.hip_attn_prefill(None, None, None, None, None, None, None, None, None, 1, 12, 8, 128, 4, 256, 0.1)
L.hip_store_kv(None, None, None, None, None, 3, 8, 100, 256)
# degenerate sizes are no-ops
L.hip_attn_decode(None, None, None, None, None, None, 0, 16, 8, 128, 4, 256, 0.1, None, None, 64, 8)
L.hip_attn_prefill(None, None, None, None, None, None, None, None, None, 0, 16, 8, 128, 4, 256, 0.1)
L.hip_store_kv(None, None, None, None, None, 0, 8, 128, 256)
print("survived")
"""


def test_launchers_reject_bad_shapes_without_launching():
    r = subprocess.run([sys.executable, "-c", _BAD_SHAPES.format(root=ROOT)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0 and "survived" in r.stdout, r.stderr
    err = r.stderr
    assert "attn_decode: only head_dim=128" in err
    assert "attn_decode: unsupported GQA group size 3" in err
    assert "attn_prefill: only head_dim=128" in err
    assert "attn_prefill: bad shape" in err or "unsupported GQA" in err
    assert "store_kv: unsupported shape" in err
    assert err.count("[llmgen-hip]") == 5  # the degenerate calls print nothing


# ---------------------------------------------------------------- operator error behaviour
def test_operator_errors():
    from llmgen_amd import attention as A

    out32 = torch.zeros(1, 4, 128, dtype=torch.float32)
    with pytest.raises(A.AttentionNeedsBf16):
        A.PagedAttentionImpl.execute(0, A.AttnNode(out32, [out32, out32, out32]))
    out = torch.zeros(1, 4, 128, dtype=torch.bfloat16)
    A.g_attn_mgr = None
    with pytest.raises(A.NoAttentionManager):
        A.PagedAttentionImpl.execute(0, A.AttnNode(out, [out, out, out]))
    A.g_attn_mgr = A.PagedAttentionManager()
    with pytest.raises(A.LayerNotActive):
        A.PagedAttentionImpl.execute(0, A.AttnNode(out, [out, out, out], layer_id=3))
    A.g_attn_mgr = None
    assert A.FlashAttentionImpl is A.PagedAttentionImpl


def test_workload_slots_are_unique():
    """No two tokens of a step write the same KV slot (a racing pair would make store_kv order-dependent)."""
    from llmgen_amd.workloads import make

    for name in ("kt_prefill", "cpu_mixed", "c1", "c2", "c3", "c4", "gqa1", "gqa8", "gqa16", "gqa1d", "gqa8d"):
        m = make(name).meta(64)
        s = m.slots[m.slots >= 0]
        assert len(np.unique(s)) == len(s), name


def test_bench_kernel_names_follow_the_header():
    """bench.py names the prefill kernel of each config from hip_attn_prefill_plan's value; its table must cover
    exactly the LLMGEN_PREFILL_* kernel values that include/llmgen_attn.h declares."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    hdr = open(os.path.join(root, "include", "llmgen_attn.h")).read()
    vals = {int(v) for name, v in re.findall(r"LLMGEN_PREFILL_(\w+)\s*=\s*(\d+)", hdr) if name != "ROWS_LAUNCH"}
    assert vals == {1, 2, 3, 4, 5, 6, 7}
    sys.path.insert(0, root)
    import bench

    assert set(bench.PREFILL_KERNELS) == vals
    assert "split" in bench.PREFILL_KERNELS[int(re.search(r"LLMGEN_PREFILL_SPLIT\s*=\s*(\d+)", hdr).group(1))]
    assert "mixed" in bench.PREFILL_KERNELS[int(re.search(r"LLMGEN_PREFILL_MIXED\s*=\s*(\d+)", hdr).group(1))]


def test_prefill_plan_rules():
    """hip_attn_prefill_plan's choice is integer arithmetic on the step's shape and the CU count (256 without a GPU,
    as on MI355X): pure prefill steps of at most half a two-head unit per CU (one one-head unit at GQA 1) take the
    pieces kernel, up to 2.5 units per CU the key split, c3's 792 units the heavy-tile split, c5p's GQA 4 the 8-wave
    kernel; mixed steps with a known count the mixed-step kernel at GQA 2 / 4, else (few prefill units) the pieces
    kernel beside the decode-row launch; an unknown count the 4-wave kernel beside the decode-row launch."""
    from llmgen_amd._lib import lib

    L = lib()
    MIXED, KEYSPLIT, W2, W4, W8, SPLIT, PIECES, ROWS = 1, 2, 3, 4, 5, 6, 7, 16
    plan = lambda n, nq, nkv, rows: L.hip_attn_prefill_plan(n, nq, nkv, 128, 256, rows)  # noqa: E731
    assert plan(8, 16, 8, 0) == PIECES and plan(16, 16, 8, 0) == PIECES
    assert plan(17, 16, 8, 0) == KEYSPLIT and plan(80, 16, 8, 0) == KEYSPLIT
    assert plan(99, 16, 8, 0) == SPLIT
    assert plan(256, 32, 8, 0) == W8
    assert plan(16, 16, 16, 0) == PIECES and plan(17, 16, 16, 0) == W2
    assert plan(71, 16, 8, 63) == MIXED and plan(71, 32, 8, 63) == MIXED
    assert plan(71, 16, 16, 63) == PIECES | ROWS and plan(71, 64, 8, 67) == PIECES | ROWS
    assert plan(400, 16, 16, 63) == W2 | ROWS
    assert plan(8, 16, 8, -1) == W4 | ROWS
    assert plan(0, 16, 8, 0) == 0 and plan(4, 24, 8, 0) == -1
