"""GPU: the launcher paths that hip_attn_set_option selects, each against the CPU oracle.

- LLMGEN_OPT_DECODE_MERGE_KERNEL = 1: split-K partials merged by the separate merge kernel (the path that
  launches with more than 2^18 (sequence, KV head) pairs take) instead of inside the decode kernel;
- LLMGEN_OPT_DECODE_ROW_WAVES = 8: 8-wave workgroups for the decode rows of mixed steps;
- LLMGEN_OPT_ATTN_PART_MIN (the reference's SV_ATTN_PART, attention.cu:219-229): longer split-K parts, down to
  one part per sequence;
- LLMGEN_OPT_PREFILL_SPLIT_TILES: how many of a pure prefill step's heaviest tiles have their units split over two
  workgroups (0 = none, the 4-wave kernel; more tiles than the step has = all of them).
Every option is restored after its test.
"""
from __future__ import annotations

import contextlib

import numpy as np
import pytest

from harness import compare, run_gpu, run_oracle
from llmgen_amd._lib import lib
from llmgen_amd.workloads import make, to_u16

pytestmark = pytest.mark.gpu

OPT_ATTN_PART_MIN, OPT_DECODE_ROW_WAVES, OPT_DECODE_MERGE_KERNEL, OPT_PREFILL_SPLIT_TILES = 0, 1, 2, 3


@contextlib.contextmanager
def option(which, value):
    prev = lib().hip_attn_set_option(which, value)
    assert prev >= 0 or which == OPT_PREFILL_SPLIT_TILES, f"option {which}={value} refused"
    try:
        yield
    finally:
        assert lib().hip_attn_set_option(which, prev) == value


def _check(name, sampled=False):
    wl = make(name)
    t = wl.tensors(device="cuda")
    out, _, _ = run_gpu(wl, t)
    if sampled:
        from test_gpu_attention import _sample_rows

        rows = _sample_rows(wl, wl.meta(64))
        _, _, _, of = run_oracle(wl, t, rows=rows, threads=16)
        compare(to_u16(out)[rows], of, name)
    else:
        _, _, _, of = run_oracle(wl, t)
        compare(to_u16(out), of, name)
    return to_u16(out)


@pytest.mark.parametrize("name", ["c1", "kt_decode", "gqa8d", "gqa16d", "bs6d", "c5d"])
def test_separate_merge_kernel(gpu, name):
    print(f"[gpu-test] merge kernel {name}", flush=True)
    with option(OPT_DECODE_MERGE_KERNEL, 1):
        _check(name, sampled=name == "c5d")


def _check_unknown_count(name, sampled=False):
    """store_kv + hip_attn_prefill (single-row count unknown: the decode rows run as a separate launch on the side
    stream, the path whose workgroup size LLMGEN_OPT_DECODE_ROW_WAVES selects) against the oracle."""
    import torch

    wl = make(name)
    t = wl.tensors(device="cuda")
    L = lib()
    meta = wl.meta(L.hip_attn_prefill_tile())
    kc, vc = t["kc"].clone(), t["vc"].clone()
    seg = torch.from_numpy(meta.packed()).to("cuda")
    off = {k: seg.data_ptr() + 4 * v for k, v in meta.offsets.items()}
    L.hip_store_kv(t["k"].data_ptr(), t["v"].data_ptr(), off["slots"], kc.data_ptr(), vc.data_ptr(), wl.n_tok,
                   wl.nkv, wl.hd, wl.block_size)
    out = torch.full((wl.n_tok, wl.nq, wl.hd), float("nan"), dtype=torch.bfloat16, device="cuda")
    L.hip_attn_prefill(out.data_ptr(), t["q"].data_ptr(), kc.data_ptr(), vc.data_ptr(), off["block_tables"],
                       off["ctx"], off["cu_q"], off["tile_seq"], off["tile_q0"], meta.n_tiles, wl.nq, wl.nkv, wl.hd,
                       wl.max_blocks, wl.block_size, wl.scale)
    torch.cuda.synchronize()
    assert L.hip_last_error() == 0
    if sampled:
        from test_gpu_attention import _sample_rows

        rows = _sample_rows(wl, meta)
        _, _, _, of = run_oracle(wl, t, rows=rows, threads=16)
        compare(to_u16(out)[rows], of, name)
    else:
        _, _, _, of = run_oracle(wl, t)
        compare(to_u16(out), of, name)


@pytest.mark.parametrize("name", ["cpu_mixed", "gqa8", "bs6", "c4"])
def test_eight_wave_decode_rows(gpu, name):
    """Mixed steps at G = 2 and 4 with a known count run the mixed-step kernel, which has its own 4-wave decode
    role; the option applies to the separate decode-row launch, reached here with the count unknown."""
    print(f"[gpu-test] 8-wave decode rows {name}", flush=True)
    with option(OPT_DECODE_ROW_WAVES, 8):
        _check_unknown_count(name, sampled=name == "c4")


def _split_workload(name):
    """Pure prefill steps at G = 2 above the key-split kernel's 2.5 units per CU: c3, and four 1500-token prompts
    (one a chunked tail) at block sizes 48 (one DMA descriptor per 4 rows) and 6 (per-lane DMA)."""
    from llmgen_amd.step import Entry
    from llmgen_amd.workloads import Workload, _tables

    if name == "c3":
        return make("c3")
    bs = {"split_bs48": 48, "split_bs6": 6}[name]
    rng = np.random.default_rng(bs)
    spec = [(0, 1500), (0, 1437), (200, 1300), (0, 1501)]
    ctxs = [a + b for a, b in spec]
    tables, nb = _tables(rng, ctxs, bs, permute=True, extra_blocks=2)
    mb = max(len(t) for t in tables)
    ents = [Entry(a, b, t) for (a, b), t in zip(spec, tables)]
    return Workload(name, 16, 8, 128, bs, nb, mb, mb * bs, ents, std=1.0, seed=bs, decode=False,
                    note=f"pure prefill G=2, 4 x ~1500 tokens, block size {bs}")


@pytest.mark.parametrize("tiles", [0, 1, 16, 1000])
@pytest.mark.parametrize("name", ["c3", "split_bs48", "split_bs6"])
def test_prefill_split_tiles(gpu, name, tiles):
    """Any number of split heavy tiles, including none and all (then the step has more heavy tiles than light ones
    to pair them with): sampled rows against the oracle, and two runs bit-identical (the halves merge in a fixed
    order whichever finishes last)."""
    from test_gpu_attention import _sample_rows

    wl = _split_workload(name)
    print(f"[gpu-test] prefill split {name} tiles={tiles}", flush=True)
    L = lib()
    m = wl.meta(L.hip_attn_prefill_tile())
    assert m.single_rows() == 0 and m.n_tiles * wl.nkv * 2 > 5 * 256
    t = wl.tensors(device="cuda")
    with option(OPT_PREFILL_SPLIT_TILES, tiles):
        plan = L.hip_attn_prefill_plan(m.n_tiles, wl.nq, wl.nkv, wl.hd, wl.block_size, 0)
        assert plan == (4 if tiles == 0 else 6), plan  # LLMGEN_PREFILL_W4 / LLMGEN_PREFILL_SPLIT
        outs = [to_u16(run_gpu(wl, t)[0]) for _ in range(2)]
    np.testing.assert_array_equal(outs[1], outs[0])
    rows = _sample_rows(wl, m)
    _, _, _, of = run_oracle(wl, t, rows=rows, threads=16)
    compare(outs[0][rows], of, f"{name} split {tiles}")


@pytest.mark.parametrize("part_min", [256, 100000])
@pytest.mark.parametrize("name", ["c1", "kt_decode", "c2"])
def test_attn_part_min(gpu, name, part_min):
    print(f"[gpu-test] SV_ATTN_PART={part_min} {name}", flush=True)
    with option(OPT_ATTN_PART_MIN, part_min):
        _check(name)


def test_option_rejects_bad_values(gpu):
    L = lib()
    assert L.hip_attn_set_option(7, 1) == -1
    assert L.hip_attn_set_option(OPT_DECODE_ROW_WAVES, 6) == -1
    assert L.hip_attn_set_option(OPT_ATTN_PART_MIN, -5) == -1
    assert L.hip_attn_set_option(OPT_PREFILL_SPLIT_TILES, -2) == -1
