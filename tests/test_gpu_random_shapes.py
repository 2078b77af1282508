"""Seeded random steps against the oracle: batch size, contexts, block size, GQA group size and the mix of decode
rows, fresh prompts and chunked-prefill tails are drawn from a fixed seed per case, so every run checks the same
cases.  The shapes stay small enough for the CPU oracle (a few seconds per case) while crossing the kernels'
structural boundaries: spans shorter and longer than one decode round, several split-K parts, prefill tiles that
straddle blocks, block sizes that are not powers of two, and 1-key contexts.

Tolerance (all rows): max-abs <= 2e-2 and rel-L2 <= 1e-2 against the oracle's f32 output; the KV cache written by
the step is compared bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

from harness import assert_cache_equal, compare, run_gpu, run_oracle
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
    """Pure prefill steps (fresh prompts and chunked tails, no decode rows) at GQA 2: the key-split kernel's path.
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
    assert wl.meta(64).single_rows() == 0  # a pure prefill step: the key-split kernel runs
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
