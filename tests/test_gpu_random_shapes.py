"""Seeded random steps against the oracle: batch size, contexts, block size, GQA group size and the mix of decode
rows, fresh prompts and chunked-prefill tails are drawn from a fixed seed per case, so every run checks the same
cases.  The shapes stay small enough for the CPU oracle (a few seconds per case) while crossing the kernels'
structural boundaries: spans shorter and longer than one decode round, several split-K parts, prefill tiles that
straddle blocks, block sizes that are not powers of two, and 1-key contexts.

Tolerance (all rows): max-abs <= 2e-2 and rel-L2 <= 1e-2 against the oracle's f32 output (the wide cases scale the
element bound with the output, see their test); the KV cache written by
the step is compared bit for bit."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from harness import assert_cache_equal, compare, run_gpu, run_oracle
from llmgen_amd._lib import lib
from llmgen_amd.step import Entry
from llmgen_amd.workloads import Workload, _tables, to_u16

CASES = list(range(12))


def _random_workload(case: int) -> Workload:
    rng = np.random.default_rng(1000 + case)
    G = int(rng.choice([1, 2, 4, 8, 16]))
    nkv = int(rng.choice([1, 2, 4])) if G >= 8 else int(rng.choice([2, 4, 8]))
    bs = int(rng.choice([6, 16, 32, 48, 64, 256]))
    decode_only = case % 3 == 0
    S = int(rng.integers(1, 24))
    spec = []
    for _ in range(S):
        ctx = int(rng.integers(1, 1800))
        if decode_only:
            spec.append((ctx - 1, 1))
        else:
            kind = rng.integers(0, 3)  # 0: decode row, 1: fresh prompt, 2: chunked tail
            if kind == 0:
                spec.append((ctx - 1, 1))
            elif kind == 1:
                q = min(ctx, int(rng.integers(2, 300)))
                spec.append((0, q))
            else:
                q = int(rng.integers(2, 200))
                spec.append((ctx, q))
    ctxs = [a + b for a, b in spec]
    tables, nb = _tables(rng, ctxs, bs, permute=True, extra_blocks=2)
    mb = max(len(t) for t in tables)
    mml = mb * bs
    ents = [Entry(a, b, t) for (a, b), t in zip(spec, tables)]
    return Workload(f"rand{case}", G * nkv, nkv, 128, bs, nb, mb, mml, ents, std=1.0, seed=50 + case,
                    decode=None if decode_only else False,
                    note=f"random: G={G} nkv={nkv} bs={bs} S={S} {'decode' if decode_only else 'mixed'}")


PREFILL_CASES = list(range(8))


def _random_prefill_workload(case: int) -> Workload:
    """Pure prefill steps (fresh prompts and chunked tails, no decode rows) at GQA 2: the paths of the pieces and
    key-split kernels.
    Prompt lengths cross 1, 2 and many key tiles, odd and even tile counts, and tiles that straddle blocks."""
    rng = np.random.default_rng(2000 + case)
    nkv = int(rng.choice([1, 2, 4, 8]))
    bs = int(rng.choice([6, 16, 48, 64, 256]))
    S = int(rng.integers(1, 7))
    spec = []
    for _ in range(S):
        q = int(rng.integers(2, 700))
        prev = 0 if rng.integers(0, 2) == 0 else int(rng.integers(1, 900))
        spec.append((prev, q))
    ctxs = [a + b for a, b in spec]
    tables, nb = _tables(rng, ctxs, bs, permute=True, extra_blocks=2)
    mb = max(len(t) for t in tables)
    ents = [Entry(a, b, t) for (a, b), t in zip(spec, tables)]
    return Workload(f"rprefill{case}", 2 * nkv, nkv, 128, bs, nb, mb, mb * bs, ents, std=1.0, seed=80 + case,
                    decode=False, note=f"random prefill: G=2 nkv={nkv} bs={bs} S={S}")


@pytest.mark.gpu
@pytest.mark.parametrize("case", PREFILL_CASES)
def test_random_gqa2_prefill_matches_oracle(gpu, case):
    wl = _random_prefill_workload(case)
    print(f"[gpu-test] {wl.name}: {wl.note}", flush=True)
    m = wl.meta(64)
    # a pure prefill step: up to half a unit (tile x KV head) per CU the pieces kernel (LLMGEN_PREFILL_PIECES,
    # every case but 3 on 256 CUs), else the key-split kernel (LLMGEN_PREFILL_KEYSPLIT, case 3)
    assert m.single_rows() == 0
    units, cus = m.n_tiles * wl.nkv, torch.cuda.get_device_properties(0).multi_processor_count
    want = 7 if units * 2 <= cus else 2
    assert lib().hip_attn_prefill_plan(m.n_tiles, wl.nq, wl.nkv, wl.hd, wl.block_size, 0) == want
    t = wl.tensors(device="cuda")
    out, kc, vc = run_gpu(wl, t)
    okc, ovc, _, of = run_oracle(wl, t, threads=16)
    assert_cache_equal(to_u16(kc), okc, f"{wl.name} store_kv K")
    assert_cache_equal(to_u16(vc), ovc, f"{wl.name} store_kv V")
    compare(to_u16(out), of, wl.name)


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES)
def test_random_step_matches_oracle(gpu, case):
    wl = _random_workload(case)
    print(f"[gpu-test] {wl.name}: {wl.note}", flush=True)
    t = wl.tensors(device="cuda")
    out, kc, vc = run_gpu(wl, t)
    okc, ovc, _, of = run_oracle(wl, t, threads=16)
    assert_cache_equal(to_u16(kc), okc, f"{wl.name} store_kv K")
    assert_cache_equal(to_u16(vc), ovc, f"{wl.name} store_kv V")
    compare(to_u16(out), of, wl.name)


WIDE_CASES = list(range(24))


def _wide_workload(case: int) -> Workload:
    """A wider net: block sizes down to 1 and up to 512 (odd ones take the per-lane DMA path), GQA 1-16, 1-4 KV
    heads up to 8, contexts up to 5000, graph-bucket padding rows on decode steps, and input scales 0.5-2."""
    rng = np.random.default_rng(5000 + case)
    G = int(rng.choice([1, 2, 4, 8, 16]))
    nkv = int(rng.choice([1, 2, 4, 8]))
    bs = int(rng.choice([1, 2, 3, 5, 8, 16, 24, 32, 64, 100, 128, 256, 512]))
    kind = int(rng.integers(0, 3))  # 0 decode-only, 1 prefill-only, 2 mixed
    S = int(rng.integers(1, 12))
    spec = []
    for _ in range(S):
        ctx = int(rng.integers(1, 5000))
        k = kind if kind < 2 else int(rng.integers(0, 3))
        if k == 0:
            spec.append((ctx - 1, 1))
        elif k == 1:
            spec.append((0, min(ctx, int(rng.integers(2, 700)))))
        else:
            spec.append((ctx, int(rng.integers(2, 300))))
    ctxs = [a + b for a, b in spec]
    tables, nb = _tables(rng, ctxs, bs, permute=True, extra_blocks=3)
    mb = max(len(t) for t in tables)
    pad = int(rng.integers(0, 3)) if kind == 0 else 0
    return Workload(f"wide{case}", G * nkv, nkv, 128, bs, nb, mb, mb * bs,
                    [Entry(a, b, t) for (a, b), t in zip(spec, tables)], std=float(rng.choice([0.5, 1.0, 2.0])),
                    seed=7000 + case, decode=None if kind == 0 else False, pad_rows=pad,
                    note=f"wide: G={G} nkv={nkv} bs={bs} S={S} kind={kind} pad={pad}")


@pytest.mark.gpu
@pytest.mark.parametrize("case", WIDE_CASES)
def test_wide_random_step_matches_oracle(gpu, case):
    """As above on the wider net.  At input scale 2 the outputs reach |o| of 5-8, whose own bf16 rounding is up to
    2^-9 |o|, so the element bound is 2e-2 + 2^-6 |o| (2e-2 flat at the configs' scales); rel-L2 <= 1e-2 as
    everywhere.  Steps of more than 400 rows are checked on 200 seeded rows."""
    import oracle

    wl = _wide_workload(case)
    print(f"[gpu-test] {wl.name}: {wl.note} std={wl.std}", flush=True)
    t = wl.tensors(device="cuda")
    out, kc, vc = run_gpu(wl, t)
    n = wl.n_tok
    rows = None
    if n > 400:
        rows = np.array(sorted(set(np.random.default_rng(case).integers(0, n, size=200).tolist())), np.int32)
    okc, ovc, _, of = run_oracle(wl, t, rows=rows, threads=16)
    assert_cache_equal(to_u16(kc), okc, f"{wl.name} store_kv K")
    assert_cache_equal(to_u16(vc), ovc, f"{wl.name} store_kv V")
    got = to_u16(out) if rows is None else to_u16(out)[rows]
    g = oracle.bf16_to_f32(got).astype(np.float64)
    r = of.astype(np.float64)
    assert np.isfinite(g).all(), f"{wl.name}: non-finite outputs"
    err = np.abs(g - r)
    bound = 2e-2 + np.abs(r) * 2.0 ** -6
    worst = np.unravel_index(int((err - bound).argmax()), err.shape)
    assert (err <= bound).all(), f"{wl.name}: error {err[worst]:.4g} beyond {bound[worst]:.4g} at {worst}"
    rel = float(np.linalg.norm(g - r) / max(float(np.linalg.norm(r)), 1e-30))
    assert rel <= 1e-2, f"{wl.name}: rel-L2 {rel:.4g}"


def test_random_shapes_are_valid():
    """CPU check of the generator: every case builds step metadata, and the cases cover both step kinds, several
    group sizes and block sizes."""
    seen_g, seen_bs, kinds = set(), set(), set()
    for case in CASES:
        wl = _random_workload(case)
        meta = wl.meta(64)
        assert meta.n_tok == wl.n_tok
        seen_g.add(wl.nq // wl.nkv)
        seen_bs.add(wl.block_size)
        kinds.add(wl.decode is None)
    assert len(seen_g) >= 3 and len(seen_bs) >= 3 and kinds == {True, False}
    bss = set()
    for case in PREFILL_CASES:
        wl = _random_prefill_workload(case)
        meta = wl.meta(64)
        assert meta.single_rows() == 0 and not meta.decode
        bss.add(wl.block_size)
    assert len(bss) >= 3
    wide_bs = {_wide_workload(c).block_size for c in WIDE_CASES}
    assert len(wide_bs) >= 6 and min(wide_bs) <= 3
