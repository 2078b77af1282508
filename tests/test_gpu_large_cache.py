"""Caches past the int32 element range: a layer's K (or V) pool of 8256 blocks x 8 heads x 256 slots x 128 dims
holds 2.16e9 bf16 elements (4.3 GB), and the steps below read and write only blocks 8192..8255, whose element
offsets all exceed 2^31.  A 288 GB device keeps pools far larger than that, so every cache address in store_kv,
decode (split and fused), the mixed-step decode rows and both prefill kernels must be computed in 64 bits.

Each case runs the step on the large pools and, on the CPU oracle, on a compact copy of the same step whose block
tables are the large ones minus 8192; outputs must agree within the usual tolerance (max-abs <= 2e-2,
rel-L2 <= 1e-2) and the written cache blocks bit for bit."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from harness import assert_cache_equal, compare, run_gpu, run_oracle
from llmgen_amd.step import Entry
from llmgen_amd.workloads import Workload, to_u16

BASE = 8192  # first physical block used: offsets from block BASE on are >= BASE * 8 * 256 * 128 = 2^31 elements
NB = 64      # blocks actually used
BS = 256


def _case(kind: str, G: int):
    rng = np.random.default_rng({"mixed": 1, "decode": 2, "prefill": 3}[kind] * 10 + G)
    if kind == "decode":
        spec = [(int(c) - 1, 1) for c in rng.integers(300, 2300, size=6)]
    elif kind == "prefill":
        spec = [(0, 700), (500, 300), (0, 65)]
    else:
        spec = [(999, 1), (0, 200), (500, 300), (1500, 1)]
    perm = rng.permutation(NB)
    tables, used = [], 0
    for a, b in spec:
        n = -(-(a + b) // BS)
        tables.append([int(x) for x in perm[used:used + n]])
        used += n
    assert used <= NB
    nkv = 8
    mb = max(len(t) for t in tables)
    compact = Workload(f"large_{kind}_g{G}", G * nkv, nkv, 128, BS, NB, mb, mb * BS,
                       [Entry(a, b, t) for (a, b), t in zip(spec, tables)], std=1.0, seed=90 + G,
                       decode=None if kind == "decode" else False)
    large = Workload(compact.name + "_big", G * nkv, nkv, 128, BS, BASE + NB, mb, mb * BS,
                     [Entry(a, b, [x + BASE for x in t]) for (a, b), t in zip(spec, tables)], std=1.0,
                     seed=90 + G, decode=compact.decode)
    return compact, large


CASES = [("decode", 2), ("decode", 4), ("mixed", 2), ("prefill", 2), ("prefill", 4)]


@pytest.mark.gpu
@pytest.mark.parametrize("kind,G", CASES)
def test_cache_beyond_int32_elements(gpu, kind, G):
    compact, large = _case(kind, G)
    print(f"[gpu-test] {large.name}: pools of {large.num_blocks} blocks, blocks {BASE}..{BASE + NB - 1} used",
          flush=True)
    assert BASE * large.nkv * BS * 128 >= 2 ** 31
    tc = compact.tensors(device="cuda")
    pool = (large.num_blocks, large.nkv, BS, 128)
    kc = torch.empty(pool, dtype=torch.bfloat16, device="cuda")
    vc = torch.empty(pool, dtype=torch.bfloat16, device="cuda")
    kc[BASE:] = tc["kc"]
    vc[BASE:] = tc["vc"]
    tl = {"q": tc["q"], "k": tc["k"], "v": tc["v"], "kc": kc, "vc": vc}
    out, kco, vco = run_gpu(large, tl)
    got_k, got_v = to_u16(kco[BASE:]), to_u16(vco[BASE:])
    del kc, vc, kco, vco, tl
    torch.cuda.empty_cache()
    okc, ovc, _, of = run_oracle(compact, tc, threads=16)
    assert_cache_equal(got_k, okc, f"{large.name} store_kv K")
    assert_cache_equal(got_v, ovc, f"{large.name} store_kv V")
    compare(to_u16(out), of, large.name)


def test_large_cases_reach_past_int32():
    """CPU check of the case builder: every case uses only blocks >= BASE, whose first element offset is past 2^31,
    and the compact twin's tables are the same tables shifted by BASE."""
    for kind, G in CASES:
        compact, large = _case(kind, G)
        for ec, el in zip(compact.entries, large.entries):
            assert [x + BASE for x in ec.block_table] == el.block_table
            assert min(el.block_table) >= BASE and max(el.block_table) < BASE + NB
        assert BASE * large.nkv * BS * 128 >= 2 ** 31
        meta = large.meta(64)
        assert int(meta.slots.max()) < 2 ** 31
