#!/usr/bin/env python3
"""Benchmark of the MI355X attention path on BASELINE's configurations (1 GPU).

A step is one layer's attention step of configuration c2 (32-sequence batched decode, the configuration the
metric is quoted on): store_kv of the step's K/V plus split-K paged decode (one fused launch).  As in the engine,
the decode step is a hipGraph bucket holding every decoder layer (28 for Qwen3-0.6B, each with its own KV pools),
captured by the C++ executor slice; the bench replays it and reports graph time / 28 per step.  ``value`` = algorithmic decode bytes (sum ctx * nkv * hd * 2 B * 2 + q + out)
per step / step time, in GB/s.  The other configurations are reported under ``extra``: decode GB/s for c1 and
c5d, prefill TFLOP/s (4 * hd * nq * causal pairs / time) for c3 and c5p, and the mixed step c4.

All timings use HIP events recorded on the stream the kernels run on, and every launch reads KV pools that no
recent launch read (the graph walks 28 layers' pools; eager launches rotate over pool copies), as in the engine.  ``roofline`` is for the dominant kernel
launch (hip_attn_decode on c2).  ``cpu_baseline`` times the CPU oracle (a C restatement of the reference CPU
backend's attention, single-threaded like the reference) on a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--no-extra] [--only c2|c5d|c3|...]
"""
from __future__ import annotations

import argparse
import copy
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
ROOT = os.path.dirname(os.path.abspath(__file__))
N_LAYERS = 28  # Qwen3-0.6B decoder layers: the decode graph replays this many attention steps
# Eager launches rotate over KV pool copies totalling at least this many bytes, so that no launch finds its pages in
# the 256 MB memory-side Infinity Cache (MALL) left warm by the launch before it: as in the engine, where each of
# the layers a step walks reads its own pools.  A 90 MB pool re-read every launch runs 20 % faster than a cold one.
COLD_POOL_BYTES = 1 << 30


def _timer_pair():
    from llmgen_amd._lib import lib

    L = lib()
    return L.hip_timer_create(), L.hip_timer_create()


def time_launches(fn, iters: int, warmup: int) -> float:
    """Average ms per call of fn() over ``iters`` back-to-back calls, HIP events on the launch stream."""
    import torch
    from llmgen_amd._lib import lib

    L = lib()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = _timer_pair()
    L.hip_timer_record(e0)
    for _ in range(iters):
        fn()
    L.hip_timer_record(e1)
    ms = L.hip_timer_elapsed_ms(e0, e1)
    torch.cuda.synchronize()
    L.hip_timer_destroy(e0)
    L.hip_timer_destroy(e1)
    return ms / iters


WARM_S = 0.5


def warm(fn, seconds: float = None) -> None:
    """Run fn() back to back for about ``seconds``: the GPU's clocks rise and every rotating pool copy has been
    touched once (its pages mapped) before anything is timed."""
    import torch

    t_end = time.perf_counter() + (WARM_S if seconds is None else seconds)
    while time.perf_counter() < t_end:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()


class Step:
    """One workload's attention step wired to the library (eager launchers + optional decode graph)."""

    def __init__(self, name: str):
        import torch
        from llmgen_amd import attention as A
        from llmgen_amd import host as H
        from llmgen_amd._lib import lib
        from llmgen_amd.workloads import make

        self.L = lib()
        self.wl = wl = make(name)
        self.t = wl.tensors(device="cuda")
        self.meta = wl.meta(self.L.hip_attn_prefill_tile())  # the Python restatement: the CPU baseline's input
        self.ws = wl.workspace()
        self.layer = A.LayerState(self.t["kc"].clone(), self.t["vc"].clone())
        mgr = A.PagedAttentionManager()
        mgr.layers[0] = self.layer
        A.g_attn_mgr = mgr
        # the StepState the C++ executor slice binds (fillMeta + bindStep); a private copy, since later binds
        # rewrite the global g_step
        self.g = H.StepState.from_buffer_copy(wl.bind(self.ws))
        self.out = torch.zeros(wl.n_tok, wl.nq, wl.hd, dtype=torch.bfloat16, device="cuda")
        self.node = A.AttnNode(self.out, [self.t["q"], self.t["k"], self.t["v"]], layer_id=0)
        self.A = A
        self.H = H
        # write this step's K/V once so attention-only launches see the full context
        self.store_kv()
        pool_bytes = 2 * self.layer.k.numel() * self.layer.k.element_size()
        n_pools = max(1, -(-COLD_POOL_BYTES // pool_bytes))
        self.pools = [(self.layer.k, self.layer.v)] + [(self.layer.k.clone(), self.layer.v.clone())
                                                       for _ in range(n_pools - 1)]
        self._turn = 0
        torch.cuda.synchronize()

    def store_kv(self):
        g, wl = self.g, self.wl
        self.L.hip_store_kv(self.t["k"].data_ptr(), self.t["v"].data_ptr(), g.slots, self.layer.k.data_ptr(),
                            self.layer.v.data_ptr(), g.n_tok, wl.nkv, wl.hd, wl.block_size)

    def attn(self):
        """The attention launch alone, exactly as the engine's operator issues it after store_kv: the C++
        llmgen_paged_attention with the StepState the C++ bind produced (hip_attn_decode for a decode step,
        hip_attn_prefill_rows with the step's single-row count otherwise).  Successive calls read successive
        copies of the KV pools (cold in every cache)."""
        kc, vc = self.pools[self._turn % len(self.pools)]
        self._turn += 1
        self.H.paged_attention(self.g, self.out, self.t["q"], None, None, kc, vc, store_kv=False)

    def full_step(self):
        self.A.PagedAttentionImpl.execute(0, self.node)


def bench_extra(name: str, iters: int) -> dict:
    st = Step(name)
    wl = st.wl
    warm(st.attn)
    ms = time_launches(st.attn, iters, warmup=2)
    ms_kv = time_launches(st.store_kv, iters, warmup=1)
    r = {"config": name, "note": wl.note, "attn_us": round(ms * 1e3, 2), "store_kv_us": round(ms_kv * 1e3, 2),
         "store_kv_GBs": round(wl.store_kv_bytes() / (ms_kv * 1e-3) / 1e9, 1)}
    if st.meta.decode:
        gbs = wl.decode_bytes() / (ms * 1e-3) / 1e9
        r.update(decode_GBs=round(gbs, 1), hbm_frac=round(gbs / HBM_PEAK_GBS, 4))
    else:
        tf = wl.attention_flops() / (ms * 1e-3) / 1e12
        gbs = wl.decode_bytes() / (ms * 1e-3) / 1e9
        r.update(prefill_TFLOPs=round(tf, 1), mfma_frac=round(tf / BF16_PEAK_TFLOPS, 4), kv_GBs=round(gbs, 1))
        # which kernel the launcher ran for this step (the launcher's own record, hip_attn_prefill_plan)
        plan = st.L.hip_attn_prefill_plan(st.g.n_tiles, wl.nq, wl.nkv, wl.hd, wl.block_size, st.g.single_rows)
        r["kernel"] = PREFILL_KERNELS.get(plan & 15, f"plan {plan}") + (
            " + decode rows on the side stream" if plan >= 0 and plan & 16 else "")
    return r


PREFILL_KERNELS = {1: "attn_mixed_kernel (prefill units and decode rows as workgroup roles)",
                   2: "attn_prefill_kernel<8, *, 2> (key split in the workgroup)",
                   3: "attn_prefill_kernel<2, *, 1>", 4: "attn_prefill_kernel<4, *, 1>",
                   5: "attn_prefill_kernel<8, *, 1>",
                   6: "attn_prefill_split_kernel (heaviest tiles' units over two workgroups)",
                   7: "attn_prefill_pieces_kernel (each unit's key tiles over up to 8 workgroups)"}


def bench_qk_fused(name: str, iters: int) -> dict:
    """The pre-attention step of one layer for a config's token shape: q/k RMSNorm + RoPE + KV write as one
    fused launch (hip_qk_norm_rope_store_kv) against the unfused graph's five launches (2 x rmsnorm, 2 x rope,
    store_kv).  Bytes = q, k, v read + q, K, V written (2 * T * (nq + 2 nkv) * hd * 2 B)."""
    import torch
    from llmgen_amd.qwen3 import rope_tables

    st = Step(name)
    wl, g, L = st.wl, st.g, st.L
    T = g.n_tok
    P = lambda t: t.data_ptr()  # noqa: E731
    gen = torch.Generator(device="cuda").manual_seed(0)
    qw = 1 + 0.1 * torch.randn(wl.hd, device="cuda", generator=gen)
    kw = 1 + 0.1 * torch.randn(wl.hd, device="cuda", generator=gen)
    c, s = (torch.from_numpy(a).cuda() for a in rope_tables(wl.max_model_len, wl.hd, 1e6))
    pos = torch.from_numpy(st.meta.pos).cuda()
    q, k, v = st.t["q"], st.t["k"], st.t["v"]
    qo, k2 = torch.empty_like(q), torch.empty_like(k)
    kc, vc = st.layer.k, st.layer.v

    def fused():
        L.hip_qk_norm_rope_store_kv(P(qo), P(kc), P(vc), P(q), P(k), P(v), P(qw), P(kw), 1e-6, P(c), P(s), P(pos),
                                    g.slots, T, wl.nq, wl.nkv, wl.hd, wl.block_size)

    def unfused():
        L.hip_rmsnorm(P(qo), P(q), P(qw), T * wl.nq, wl.hd, 1e-6)
        L.hip_rmsnorm(P(k2), P(k), P(kw), T * wl.nkv, wl.hd, 1e-6)
        L.hip_rope(P(qo), P(qo), P(c), P(s), P(pos), T, wl.nq, wl.hd)
        L.hip_rope(P(k2), P(k2), P(c), P(s), P(pos), T, wl.nkv, wl.hd)
        L.hip_store_kv(P(k2), P(v), g.slots, P(kc), P(vc), T, wl.nkv, wl.hd, wl.block_size)

    ms_f = time_launches(fused, iters, warmup=2)
    ms_u = time_launches(unfused, iters, warmup=2)
    nbytes = 2 * T * (wl.nq + 2 * wl.nkv) * wl.hd * 2
    return {"config": name, "tokens": T, "fused_us": round(ms_f * 1e3, 2), "unfused_us": round(ms_u * 1e3, 2),
            "speedup": round(ms_u / ms_f, 2), "fused_GBs": round(nbytes / (ms_f * 1e-3) / 1e9, 1)}


def cpu_baseline(st: "Step", budget_s: float = 10.0) -> dict:
    """The CPU oracle (single thread, like the reference's scalar loop) on full c2 steps, repeated until
    ``budget_s`` seconds of CPU work; value in the metric's unit (GB/s of algorithmic decode bytes)."""
    sys.path.insert(0, ROOT)
    import oracle
    from llmgen_amd.workloads import to_u16

    wl, meta = st.wl, st.meta
    q = to_u16(st.t["q"])
    kc = to_u16(st.layer.k)
    vc = to_u16(st.layer.v)
    args = (q, kc, vc, meta.block_tables, meta.ctx, meta.cu_q, wl.nq, wl.nkv, wl.hd, wl.max_blocks, wl.block_size,
            wl.scale)
    reps, t0 = 0, time.perf_counter()
    while True:
        ob, of = oracle.attend(*args)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    per = el / reps
    # the same step on all host cores the box gives this job (OpenMP over (token, head)), for scale
    n_thr = min(16, os.cpu_count() or 1)
    rows = np.arange(int(meta.cu_q[-1]), dtype=np.int32)
    reps_mt, t1 = 0, time.perf_counter()
    while True:
        oracle.attend_rows(*args, rows=rows, threads=n_thr)
        reps_mt += 1
        el_mt = time.perf_counter() - t1
        if el_mt >= budget_s / 4:
            break
    per_mt = el_mt / reps_mt
    # parity of the GPU output of the same step (already computed by the benchmark's warm-up)
    got = oracle.bf16_to_f32(to_u16(st.out)).astype(np.float64)
    err = float(np.abs(got - of).max())
    rel = float(np.linalg.norm(got - of) / np.linalg.norm(of))
    return {
        "value": round(wl.decode_bytes() / per / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"full c2 decode step (32 seqs, all heads) x{reps} reps, {per * 1e3:.1f} ms/step, oracle/attend",
        "gpu_vs_oracle": {"max_abs": round(err, 5), "rel_l2": round(rel, 5)},
        "multicore": {"value": round(wl.decode_bytes() / per_mt / 1e9, 4), "unit": "GB/s", "cores": n_thr,
                      "sample": f"same step x{reps_mt} reps, {per_mt * 1e3:.1f} ms/step, OpenMP over (token, head)"},
    }


def load_traffic(kernel_key: str):
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        d = json.load(f)
    v = d.get(kernel_key)
    return None if v is None else v.get("hbm_bytes_per_launch")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--warm-s", type=float, default=0.5,
                    help="seconds of untimed launches before each timed loop (clocks up, pool copies touched)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--only", default=None, help="time only this config's attention launcher (for profiling)")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="run only a plain device copy of this many MiB (calibrates rocprofv3 FETCH/WRITE_SIZE)")
    args = ap.parse_args()
    global WARM_S
    WARM_S = args.warm_s

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (the attention kernel on one GPU's share); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        return 2

    import torch
    from llmgen_amd.attention import init_device

    init_device()

    if args.copy_mb:
        n = args.copy_mb << 20
        src = torch.ones(n // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": n, "launches": args.steps}), flush=True)
        return 0

    if args.only and args.only.startswith("qk_fused_"):
        print(json.dumps(bench_qk_fused(args.only[len("qk_fused_"):], args.steps)), flush=True)
        return 0
    if args.only:
        st = Step(args.only)
        warm(st.attn)  # a few milliseconds of launches leave the clocks low
        ms = time_launches(st.attn, args.steps, args.warmup)
        print(json.dumps({"config": args.only, "attn_us": round(ms * 1e3, 2)}), flush=True)
        return 0

    # ---- the metric step: c2 decode (store_kv fused into split-K decode), replayed from a hipGraph bucket
    #      captured by the C++ executor slice (llmgen_graphs_*, the engine's captureGraphs / replay) ----
    from llmgen_amd import host as H
    from llmgen_amd._lib import loaded_library

    st = Step("c2")
    wl = st.wl
    # the engine's decode graph holds every decoder layer: N_LAYERS attention steps, each with its own KV pools
    kcs = [st.layer.k] + [st.t["kc"].clone() for _ in range(N_LAYERS - 1)]
    vcs = [st.layer.v] + [st.t["vc"].clone() for _ in range(N_LAYERS - 1)]
    graphs = H.Graphs(kcs, vcs, wl.nq, wl.nkv, wl.hd, wl.block_size, wl.max_model_len, max_seqs=len(wl.entries),
                      buckets=[len(wl.entries)])
    rng = np.random.default_rng(0)
    seqs = [H.Sequence_(rng.integers(0, 1000, e.q_start + e.q_len).tolist(), list(e.block_table))
            for e in wl.entries]
    ents = [(i, e.q_start, e.q_len) for i, e in enumerate(wl.entries)]
    graphs.step(seqs, ents, st.t["q"], st.t["k"], st.t["v"], st.out)  # metadata upload + q/k/v + one replay
    warm(graphs.replay)  # steady state: clocks up, every layer's pools touched
    for _ in range(args.warmup):
        graphs.replay()
    torch.cuda.synchronize()
    L = st.L
    e0, e1 = _timer_pair()
    torch.cuda.synchronize()  # barrier (one rank) + synchronize
    L.hip_timer_record(e0)
    for _ in range(args.steps):
        graphs.replay()
    L.hip_timer_record(e1)
    graph_ms = L.hip_timer_elapsed_ms(e0, e1) / args.steps
    torch.cuda.synchronize()
    step_ms = graph_ms / N_LAYERS  # one layer's attention step
    value = wl.decode_bytes() / (step_ms * 1e-3) / 1e9

    # ---- dominant kernel launch: hip_attn_decode alone (split-K partials + merge), events on its stream ----
    warm(st.attn)
    kern_ms = time_launches(st.attn, max(args.steps, 50), warmup=3)
    achieved = wl.decode_bytes() / (kern_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": load_traffic("decode_c2"),
                "kernel": "hip_attn_decode (attn_decode_split_kernel + attn_decode_reduce_kernel)",
                "launch_us": round(kern_ms * 1e3, 2), "bytes_per_launch": wl.decode_bytes()}

    extra = {}
    if not args.no_extra:
        for name in ("c1", "c5d", "c3", "c5p", "c4", "chunk32k", "chunkmix"):
            try:
                extra[name] = bench_extra(name, iters=20 if name != "c5p" else 5)
            except Exception as e:  # report, keep the headline line
                extra[name] = {"error": repr(e)}
            torch.cuda.empty_cache()
        for name in ("c2", "c5p"):
            try:
                extra["qk_fused_" + name] = bench_qk_fused(name, iters=20)
            except Exception as e:
                extra["qk_fused_" + name] = {"error": repr(e)}
            torch.cuda.empty_cache()

    line = {
        "metric": "decode attn HBM GB/s (% of peak) + prefill attn TFLOP/s (% MFMA peak), 1 GPU",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded N(0,1) bf16 q/k/v and KV history, random block tables)",
        "config": {"workload": "c2: batched decode, 32 seqs, ctx~U[128,1024], 16q/8kv/hd128, block 256; step = one "
                               "layer's store_kv + split-K decode (one fused launch), timed inside a 28-layer "
                               "hipGraph decode bucket captured by the C++ executor slice (graph time / 28)",
                   "graph_ms": round(graph_ms, 4), "layers_per_graph": N_LAYERS,
                   "hbm_frac": round(value / HBM_PEAK_GBS, 4), "parallelism": "single GPU"},
        "roofline": roofline,
        "library": loaded_library(),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(st)
    line["extra"] = extra
    graphs.destroy()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
