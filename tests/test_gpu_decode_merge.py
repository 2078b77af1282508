"""The split-K merge of a long single sequence against the oracle: one decode row of 1500, 20000 and 65000 keys at
GQA 2 (one KV head), whose (sequence, head) pairs are cut into 12, 157 and 508 parts.  The merging workgroup takes
three routes by part count -- all parts' (m, l, o) loaded at once (up to 16), (m, l) staged in LDS with o read 32
parts at a time (up to 256 at four waves), part by part beyond that -- and each must give the oracle's result.
Every row against the oracle (max-abs 2e-2, rel-L2 1e-2); the KV cache written by the step bit for bit."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from harness import assert_cache_equal, compare, run_gpu, run_oracle
from llmgen_amd import step as S
from llmgen_amd.step import Entry
from llmgen_amd.workloads import Workload, _tables, to_u16

MAX_MODEL_LEN = 65536


def _parts(ctx: int, n_seq: int, nkv: int) -> int:
    """Parts per (sequence, head) under the launcher's span rule for a 4-wave launch (few pairs): k parts of
    part_size tokens per workgroup, k = max(nkv * S * max_parts / (2 * CUs), one 128-token round)."""
    ps, mp = S.part_size(n_seq), S.max_parts(n_seq, MAX_MODEL_LEN)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    total, target = nkv * n_seq * mp, 2 * cus
    k = max(total // target if total > target else 1, -(-128 // ps))
    return -(-ctx // (k * ps))


@pytest.mark.gpu
@pytest.mark.parametrize("ctx", [1500, 20000, 65000])
def test_long_sequence_decode_merge_matches_oracle(gpu, ctx):
    parts = _parts(ctx, 1, 1)
    print(f"[gpu-test] decode merge ctx={ctx} parts={parts}", flush=True)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert parts == {1500: 12, 20000: 157, 65000: 508}[ctx]
    rng = np.random.default_rng(ctx)
    tables, nb = _tables(rng, [ctx], 256, permute=True, extra_blocks=2)
    mb = max(len(t) for t in tables)
    wl = Workload(f"merge{ctx}", 2, 1, 128, 256, nb, mb, MAX_MODEL_LEN, [Entry(ctx - 1, 1, tables[0])], std=1.0,
                  seed=ctx, decode=True)
    t = wl.tensors(device="cuda")
    out, kc, vc = run_gpu(wl, t)
    okc, ovc, _, of = run_oracle(wl, t)
    assert_cache_equal(to_u16(kc), okc, "K")
    assert_cache_equal(to_u16(vc), ovc, "V")
    compare(to_u16(out), of, f"merge ctx={ctx}")
