"""Seeded synthetic workloads: the five BASELINE configurations and the reference's own attention test cases.

A :class:`Workload` is one attention step of one layer: the sequences of the step (:class:`~llmgen_amd.step.Entry`
with a physical block table each), the paged K/V pools as they are before the step (random bf16 history), and
this step's q / k / v.  The step runs as the engine runs it: store_kv of this step's k / v, then decode or
prefill attention.  Inputs are drawn N(0,1)*std from a seeded generator and rounded to bf16 (RNE).

Configurations (shape Qwen3-0.6B unless stated: 16 Q heads, 8 KV heads, head_dim 128, block size 256):
  c1  single-sequence decode, ctx 512, contiguous blocks {0, 1}, std 0.5
  c2  batched decode, 32 sequences, ctx ~ U[128, 1024], permuted blocks, std 1
  c3  causal prefill of one 3584-token prompt + 8 prompts of U[128, 512] tokens, std 0.5
  c4  mixed step: 256 sequences with ctx ~ U[100, 2048]; 8 prefill a 512-token chunk, 248 decode one token
  c5d decode, 32 Q / 8 KV heads (GQA 4), 16 sequences at ctx 32768, permuted blocks, std 1
  c5p prefill, 32 Q / 8 KV heads, one 16384-token causal prompt, permuted blocks, std 1
Outside BASELINE, ``chunk32k`` (one 512-row chunk against 32256 cached keys) and ``chunkmix`` (a 512-row chunk on
16384 keys beside 63 decode rows) are chunked-prefill steps of few, long units.
Reference test cases (src/backend/cuda/kernel_test.zig:151-232, src/backend/cpu/attention.zig:188-251) are
``kt_prefill``, ``kt_decode`` and ``cpu_mixed``, with U(-1, 1) inputs from a seeded generator.  Further small
steps cover other GQA group sizes (``gqa*``), block sizes 48 and 6 (``bs48*``, ``bs6*``) and G = 1 at block sizes 6
and 256 (``g1bs*``).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np
import torch

from .step import Entry, StepMeta, fill_meta


@dataclass
class Workload:
    name: str
    nq: int
    nkv: int
    hd: int
    block_size: int
    num_blocks: int
    max_blocks: int
    max_model_len: int
    entries: List[Entry]
    std: float = 1.0
    uniform: bool = False  # U(-1, 1) instead of N(0, 1) * std
    seed: int = 0
    decode: Optional[bool] = None  # None = the engine's rule
    pad_rows: int = 0  # graph-bucket style padding sequences appended (1 token, ctx = 0, slot = -1)
    note: str = ""

    @property
    def scale(self) -> float:
        return 1.0 / float(np.sqrt(self.hd))

    def meta(self, pf_tile: int) -> StepMeta:
        return fill_meta(self.entries, self.block_size, self.max_blocks, pf_tile,
                         seq_num=len(self.entries) + self.pad_rows, decode=self.decode)

    @property
    def seq_num(self) -> int:
        return len(self.entries) + self.pad_rows

    def workspace(self, device="cuda"):
        """The executor's attention workspace for this step (metadata buffer + split-K scratch)."""
        from . import attention as A

        return A.Workspace.allocate(self.nq, self.hd, max(self.seq_num, 1), self.max_model_len,
                                    A.meta_bytes(self.entries, self.max_blocks, self.seq_num, self.decode),
                                    device=device)

    def bind(self, ws):
        """fillMeta + upload + bindStep of this step through the C++ executor slice; returns (and publishes as
        ``attention.g_step``) the bound StepState."""
        from . import attention as A

        return A.bind_step(self.entries, ws, self.nq, self.nkv, self.hd, self.block_size, self.max_blocks,
                           self.max_model_len, seq_num=self.seq_num, decode=self.decode)

    @property
    def n_tok(self) -> int:
        return sum(e.q_len for e in self.entries) + self.pad_rows

    @property
    def ctx_lens(self) -> np.ndarray:
        return np.array([e.q_start + e.q_len for e in self.entries], np.int64)

    # ---- algorithmic work (the metric definitions) ----
    def decode_bytes(self) -> int:
        """K+V bytes of every attended key plus q and out: sum ctx * nkv * hd * 2 B * 2 + 2 * S * nq * hd * 2 B."""
        ctx = self.ctx_lens
        return int(ctx.sum()) * self.nkv * self.hd * 2 * 2 + 2 * len(self.entries) * self.nq * self.hd * 2

    def attention_flops(self) -> int:
        """4 * hd * nq * sum over query rows of the keys it attends (ctx - q_len + j + 1)."""
        pairs = 0
        for e in self.entries:
            ctx, ql = e.q_start + e.q_len, e.q_len
            # sum_{j<ql} (ctx - ql + j + 1)
            pairs += ql * (ctx - ql) + ql * (ql + 1) // 2
        return 4 * self.hd * self.nq * pairs

    def store_kv_bytes(self) -> int:
        return 2 * 2 * self.n_tok * self.nkv * self.hd * 2  # read + write, K and V

    # ---- tensors ----
    def tensors(self, device="cpu"):
        """q [T,nq,hd], k / v [T,nkv,hd] and the pools kc / vc [num_blocks,nkv,bs,hd], all torch.bfloat16 on
        ``device``.  Deterministic for a given (seed, device type)."""
        gen = torch.Generator(device=device)
        gen.manual_seed(self.seed)

        def draw(*shape):
            if self.uniform:
                x = torch.rand(*shape, generator=gen, device=device, dtype=torch.float32) * 2 - 1
            else:
                x = torch.randn(*shape, generator=gen, device=device, dtype=torch.float32) * self.std
            return x.to(torch.bfloat16)

        T = self.n_tok
        pool = (self.num_blocks, self.nkv, self.block_size, self.hd)
        kc = draw(*pool)
        vc = draw(*pool)
        k = draw(T, self.nkv, self.hd)
        v = draw(T, self.nkv, self.hd)
        q = draw(T, self.nq, self.hd)
        return {"q": q, "k": k, "v": v, "kc": kc, "vc": vc}


def to_u16(t: torch.Tensor) -> np.ndarray:
    """bf16 torch tensor -> numpy uint16 bit patterns (host copy)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _tables(rng: np.random.Generator, ctxs, bs: int, permute: bool, extra_blocks: int = 0):
    nbs = [(int(c) + bs - 1) // bs for c in ctxs]
    total = sum(nbs) + extra_blocks
    ids = rng.permutation(total) if permute else np.arange(total)
    out, o = [], 0
    for nb in nbs:
        out.append([int(x) for x in ids[o:o + nb]])
        o += nb
    return out, total


def _decode_entries(ctxs, tables):
    return [Entry(q_start=int(c) - 1, q_len=1, block_table=t) for c, t in zip(ctxs, tables)]


def make(name: str, seed: Optional[int] = None) -> Workload:
    """Build a named workload (see the module docstring)."""
    bs = 256
    if name == "c1":
        s = 1 if seed is None else seed
        ctxs = [512]
        tables = [[0, 1]]
        return Workload("c1", 16, 8, 128, bs, 2, 2, 512, _decode_entries(ctxs, tables), std=0.5, seed=s,
                        note="decode S=1 ctx=512 contiguous blocks")
    if name == "c2":
        s = 2 if seed is None else seed
        rng = np.random.default_rng(s)
        ctxs = rng.integers(128, 1025, size=32)
        tables, nb = _tables(rng, ctxs, bs, permute=True)
        return Workload("c2", 16, 8, 128, bs, nb, 4, 1024, _decode_entries(ctxs, tables), std=1.0, seed=s,
                        note="decode S=32 ctx~U[128,1024] permuted blocks")
    if name == "c3":
        s = 3 if seed is None else seed
        rng = np.random.default_rng(s)
        lens = [3584] + [int(x) for x in rng.integers(128, 513, size=8)]
        tables, nb = _tables(rng, lens, bs, permute=True)
        ents = [Entry(0, L, t) for L, t in zip(lens, tables)]
        return Workload("c3", 16, 8, 128, bs, nb, 14, 4096, ents, std=0.5, seed=s,
                        note="causal prefill 3584 + 8 x U[128,512]")
    if name == "c4":
        s = 4 if seed is None else seed
        rng = np.random.default_rng(s)
        n = 256
        chunk_ids = set(int(x) for x in rng.choice(n, size=8, replace=False))
        ents_spec = []
        for i in range(n):
            if i in chunk_ids:
                prev = int(rng.integers(100, 2048 - 512 + 1))
                ents_spec.append((prev, 512))
            else:
                ctx = int(rng.integers(100, 2049))
                ents_spec.append((ctx - 1, 1))
        ctxs = [a + b for a, b in ents_spec]
        tables, nb = _tables(rng, ctxs, bs, permute=True)
        ents = [Entry(a, b, t) for (a, b), t in zip(ents_spec, tables)]
        return Workload("c4", 16, 8, 128, bs, nb, 8, 2048, ents, std=1.0, seed=s, decode=False,
                        note="mixed: 8 x 512-token chunks + 248 decodes, ctx~U[100,2048]")
    if name == "c5d":
        s = 5 if seed is None else seed
        rng = np.random.default_rng(s)
        ctxs = [32768] * 16
        tables, nb = _tables(rng, ctxs, bs, permute=True)
        return Workload("c5d", 32, 8, 128, bs, nb, 128, 32768, _decode_entries(ctxs, tables), std=1.0, seed=s,
                        note="decode GQA4 S=16 ctx=32768 permuted blocks")
    if name == "c5p":
        s = 6 if seed is None else seed
        rng = np.random.default_rng(s)
        lens = [16384]
        tables, nb = _tables(rng, lens, bs, permute=True)
        return Workload("c5p", 32, 8, 128, bs, nb, 64, 32768, [Entry(0, 16384, tables[0])], std=1.0, seed=s,
                        note="causal prefill GQA4 T=16384 permuted blocks")
    # ---- chunked prefill against a long cached context (outside BASELINE: the pieces kernels' case) ----
    if name == "chunk32k":
        s = 8 if seed is None else seed
        rng = np.random.default_rng(s)
        tables, nb = _tables(rng, [32768], bs, permute=True)
        return Workload("chunk32k", 16, 8, 128, bs, nb, 128, 32768, [Entry(32256, 512, tables[0])], std=1.0, seed=s,
                        decode=False, note="512-row chunk of a 32768-token prompt, 32256 keys cached")
    if name == "chunkmix":
        s = 9 if seed is None else seed
        rng = np.random.default_rng(s)
        dctx = [int(x) for x in rng.integers(1024, 3073, size=63)]
        tables, nb = _tables(rng, [16384] + dctx, bs, permute=True)
        ents = [Entry(15872, 512, tables[0])] + [Entry(c - 1, 1, t) for c, t in zip(dctx, tables[1:])]
        return Workload("chunkmix", 16, 8, 128, bs, nb, 64, 16384, ents, std=1.0, seed=s, decode=False,
                        note="512-row chunk on 16384 keys + 63 decodes, ctx~U[1024,3072]")
    # ---- reference test cases ----
    if name in ("kt_prefill", "kt_decode"):
        # kernel_test.zig:151-232: nq=4, nkv=2, hd=128, bs=16, 32 blocks, ctx=150, bt[i]=(i*7+3)%32 (16 columns)
        s = 7 if seed is None else seed
        table = [(i * 7 + 3) % 32 for i in range(16)]
        if name == "kt_prefill":
            ents = [Entry(50, 100, table)]  # the last q_len=100 positions of ctx=150 (chunked-prefill tail)
            return Workload(name, 4, 2, 128, 16, 32, 16, 4096, ents, uniform=True, seed=s,
                            note="kernel_test prefill: ctx=150, q_len=100")
        ents = [Entry(149, 1, table)]
        return Workload(name, 4, 2, 128, 16, 32, 16, 4096, ents, uniform=True, seed=s,
                        note="kernel_test decode: last row of ctx=150")
    if name == "cpu_mixed":
        # cpu/attention.zig:188-251 with head_dim 128 (the kernels' head size): nq=4, nkv=2, bs=16, 24 blocks,
        # max_blocks=8; seq0 ctx=70 q_len=30, seq1 decode ctx=41, seq2 padding ctx=0.  The reference test only
        # attends, and its second table (i*7+2)%24 shares physical block 16 with the first; this step also writes
        # this step's K/V, so seq1 uses (i*7+3)%24 and no two tokens write one slot.
        s = 11 if seed is None else seed
        t0 = [(i * 5 + 1) % 24 for i in range(8)]
        t1 = [(i * 7 + 3) % 24 for i in range(8)]
        ents = [Entry(40, 30, t0), Entry(40, 1, t1)]
        return Workload(name, 4, 2, 128, 16, 24, 8, 128, ents, uniform=True, seed=s, decode=False, pad_rows=1,
                        note="cpu test: chunked tail + decode + padding row")
    if name in ("gqa1", "gqa2", "gqa8", "gqa16"):
        # small mixed steps at other group sizes: chunked tail + fresh prompt + decode rows, bs 32, permuted blocks
        s = {"gqa1": 21, "gqa2": 24, "gqa8": 22, "gqa16": 23}[name] if seed is None else seed
        nq, nkv = {"gqa1": (8, 8), "gqa2": (8, 4), "gqa8": (16, 2), "gqa16": (32, 2)}[name]
        rng = np.random.default_rng(s)
        spec = [(200, 90), (0, 150), (333, 1), (64, 1), (0, 1)]
        ctxs = [a + b for a, b in spec]
        tables, nb = _tables(rng, ctxs, 32, permute=True, extra_blocks=3)
        ents = [Entry(a, b, t) for (a, b), t in zip(spec, tables)]
        return Workload(name, nq, nkv, 128, 32, nb, 12, 512, ents, std=1.0, seed=s, decode=False,
                        note=f"mixed step at GQA {nq // nkv}")
    if name in ("gqa1d", "gqa8d", "gqa16d"):
        # decode-only steps at other group sizes (ragged contexts, one of them a single key), bs 32
        s = {"gqa1d": 31, "gqa8d": 32, "gqa16d": 33}[name] if seed is None else seed
        nq, nkv = {"gqa1d": (8, 8), "gqa8d": (16, 2), "gqa16d": (32, 2)}[name]
        rng = np.random.default_rng(s)
        ctxs = [290, 1500, 64, 700, 1]
        tables, nb = _tables(rng, ctxs, 32, permute=True, extra_blocks=3)
        return Workload(name, nq, nkv, 128, 32, nb, 48, 1536, _decode_entries(ctxs, tables), std=1.0, seed=s,
                        note=f"decode step at GQA {nq // nkv}")
    if name in ("bs48", "bs48d"):
        # a block size that is not a power of two (the kernels' generic block-table path), GQA 4
        s = 41 if seed is None else seed
        rng = np.random.default_rng(s)
        if name == "bs48":
            spec = [(100, 170), (0, 97), (47, 1), (0, 1)]
        else:
            spec = [(c - 1, 1) for c in (48, 49, 1000, 2, 385)]
        ctxs = [a + b for a, b in spec]
        tables, nb = _tables(rng, ctxs, 48, permute=True, extra_blocks=2)
        ents = [Entry(a, b, t) for (a, b), t in zip(spec, tables)]
        return Workload(name, 16, 4, 128, 48, nb, 24, 1152, ents, std=1.0, seed=s,
                        decode=None if name == "bs48d" else False,
                        note=f"block size 48, GQA 4 ({'decode' if name == 'bs48d' else 'mixed'})")
    if name in ("bs6", "bs6d"):
        # a block size that is not a multiple of 4 (the prefill kernel's per-lane DMA path), GQA 2
        s = 43 if seed is None else seed
        rng = np.random.default_rng(s)
        if name == "bs6":
            spec = [(50, 70), (0, 33), (11, 1), (0, 1)]
        else:
            spec = [(c - 1, 1) for c in (6, 7, 120, 1, 61)]
        ctxs = [a + b for a, b in spec]
        tables, nb = _tables(rng, ctxs, 6, permute=True, extra_blocks=2)
        ents = [Entry(a, b, t) for (a, b), t in zip(spec, tables)]
        return Workload(name, 8, 4, 128, 6, nb, 24, 144, ents, std=1.0, seed=s,
                        decode=None if name == "bs6d" else False,
                        note=f"block size 6, GQA 2 ({'decode' if name == 'bs6d' else 'mixed'})")
    if name in ("g1bs6", "g1bs256"):
        # G = 1 (the one-LDS-stage prefill kernel) with the per-lane DMA path (bs 6) and the one-descriptor-per-
        # tile path (bs 256): prompts long enough for many key tiles, a chunked tail, decode rows
        s = {"g1bs6": 51, "g1bs256": 52}[name] if seed is None else seed
        bs = 6 if name == "g1bs6" else 256
        rng = np.random.default_rng(s)
        spec = [(0, 700), (300, 333), (521, 1), (0, 1)]
        ctxs = [a + b for a, b in spec]
        tables, nb = _tables(rng, ctxs, bs, permute=True, extra_blocks=2)
        ents = [Entry(a, b, t) for (a, b), t in zip(spec, tables)]
        mb = max(len(t) for t in tables)
        return Workload(name, 4, 4, 128, bs, nb, mb, mb * bs, ents, std=1.0, seed=s, decode=False,
                        note=f"GQA 1, block size {bs}, 700-token prompt + chunked tail + decode rows")
    raise KeyError(name)


BASELINE_CONFIGS = ("c1", "c2", "c3", "c4", "c5d", "c5p")
