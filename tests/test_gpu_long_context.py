"""Long contexts against the oracle: decode rows at 131072 keys (the split-K launch at its largest part counts:
2048 parts of 64 tokens per sequence for a 2-sequence batch) and a mixed step whose 512-token chunk follows 65280
cached keys beside decode rows of 98304 and 131071 keys.  Block tables are seeded permutations; tolerance as
everywhere (max-abs <= 2e-2, rel-L2 <= 1e-2 of the oracle's f32 result), and the written cache bit for bit.  The
mixed step is checked on sampled rows (first and last row of every tile and sequence plus 48 seeded rows)."""
from __future__ import annotations

import numpy as np
import pytest

from harness import assert_cache_equal, compare, run_gpu, run_oracle
from llmgen_amd._lib import lib
from llmgen_amd.step import Entry
from llmgen_amd.workloads import Workload, _tables, to_u16

BS = 256


def _workload(kind: str) -> Workload:
    if kind == "decode128k":
        rng = np.random.default_rng(128)
        spec = [(131071, 1), (100002, 1)]
        G, nkv, seed = 4, 8, 128
    else:
        rng = np.random.default_rng(64)
        spec = [(65280, 512), (98303, 1), (131070, 1)]
        G, nkv, seed = 2, 8, 64
    ctxs = [a + b for a, b in spec]
    tables, nb = _tables(rng, ctxs, BS, permute=True, extra_blocks=2)
    mb = max(len(t) for t in tables)
    return Workload(kind, G * nkv, nkv, 128, BS, nb, mb, mb * BS,
                    [Entry(a, b, t) for (a, b), t in zip(spec, tables)], std=1.0, seed=seed,
                    decode=None if kind == "decode128k" else False, note=kind)


def _rows(meta, n_random=48, seed=0):
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


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["decode128k", "mixed64k"])
def test_long_context_matches_oracle(gpu, kind):
    wl = _workload(kind)
    print(f"[gpu-test] {kind}: contexts {wl.ctx_lens.tolist()}", flush=True)
    t = wl.tensors(device="cuda")
    out, kc, vc = run_gpu(wl, t)
    if kind == "decode128k":
        okc, ovc, _, of = run_oracle(wl, t, threads=16)
        got = to_u16(out)
    else:
        rows = _rows(wl.meta(lib().hip_attn_prefill_tile()))
        okc, ovc, _, of = run_oracle(wl, t, rows=rows, threads=16)
        got = to_u16(out)[rows]
    assert_cache_equal(to_u16(kc), okc, f"{kind} store_kv K")
    assert_cache_equal(to_u16(vc), ovc, f"{kind} store_kv V")
    compare(got, of, kind)


def test_long_context_shapes():
    """CPU check of the builder: the decode case is a decode step with 131072 keys in its longest row, the mixed case
    a prefill-path step with a 512-row chunk after 65280 keys."""
    d = _workload("decode128k")
    md = d.meta(64)
    assert md.decode and int(d.ctx_lens.max()) == 131072
    m = _workload("mixed64k")
    mm = m.meta(64)
    assert not mm.decode and mm.single_rows() == 2 and int(m.ctx_lens[0]) == 65792
