"""Pinning the CPU oracle (oracle/attention_oracle.c) -- CPU only.

Every oracle function is checked against something other than its own formula:
  * the reference's literal test cases (src/backend/cpu/attention.zig:253-274 storeKv; :188-251 mixed batch),
  * an independent float64 numpy softmax attention (vectorised, gathers K/V through the block table itself),
  * closed forms and invariants that a dropped term, swapped index or wrong sign would break:
    one key -> v exactly, q = 0 -> mean of V, block-table permutation invariance, padding rows -> 0,
    chunked prefill == tail of the full prefill, GQA with replicated KV heads == MHA,
  * torch's bf16 conversion (round-to-nearest-even) for f32 -> bf16.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle


# ---------------------------------------------------------------- helpers
def bf16(x) -> np.ndarray:
    """f32 -> bf16 bits via torch (an independent RNE implementation)."""
    t = torch.tensor(np.asarray(x, np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def rand_bf16(rng, shape, lo=-1.0, hi=1.0):
    return bf16(rng.uniform(lo, hi, size=shape).astype(np.float32))


def numpy_attention(q, kc, vc, bt, ctx, cu_q, nq, nkv, hd, bs, scale):
    """Independent float64 reference: gather each sequence's K/V through its block table, full softmax."""
    T = int(cu_q[-1])
    out = np.zeros((T, nq, hd), np.float64)
    qf = oracle.bf16_to_f32(q).astype(np.float64).reshape(T, nq, hd)
    kf = oracle.bf16_to_f32(kc).astype(np.float64)
    vf = oracle.bf16_to_f32(vc).astype(np.float64)
    G = nq // nkv
    for s in range(len(ctx)):
        b, e, c = int(cu_q[s]), int(cu_q[s + 1]), int(ctx[s])
        ql = e - b
        if c < ql:
            continue
        pos = np.arange(c)
        blocks = np.asarray(bt[s])[pos // bs]
        K = kf[blocks, :, pos % bs, :]  # [c, nkv, hd]
        V = vf[blocks, :, pos % bs, :]
        for j in range(ql):
            nk = c - ql + j + 1
            for h in range(nq):
                sc = K[:nk, h // G, :] @ qf[b + j, h] * scale
                w = np.exp(sc - sc.max())
                out[b + j, h] = (w[:, None] * V[:nk, h // G, :]).sum(0) / w.sum()
    return out


def mixed_case(hd=64, seed=11):
    """attention.zig:188-251: nq=4, nkv=2, bs=16, 24 blocks, max_blocks=8; seq0 ctx=70 q_len=30, seq1 decode
    ctx=41, seq2 padding ctx=0; permuted tables (i*5+1)%24 and (i*7+2)%24."""
    rng = np.random.default_rng(seed)
    nq, nkv, bs, nb, mb = 4, 2, 16, 24, 8
    kc = rand_bf16(rng, (nb, nkv, bs, hd))
    vc = rand_bf16(rng, (nb, nkv, bs, hd))
    bt = np.zeros((3, mb), np.int32)
    for i in range(mb):
        bt[0, i] = (i * 5 + 1) % nb
        bt[1, i] = (i * 7 + 2) % nb
    cu_q = np.array([0, 30, 31, 32], np.int32)
    ctx = np.array([70, 41, 0], np.int32)
    q = rand_bf16(rng, (32, nq, hd))
    return dict(q=q, kc=kc, vc=vc, bt=bt, ctx=ctx, cu_q=cu_q, nq=nq, nkv=nkv, hd=hd, mb=mb, bs=bs,
                scale=1.0 / np.sqrt(hd))


def run_attend(c, **over):
    d = dict(c)
    d.update(over)
    return oracle.attend(d["q"], d["kc"], d["vc"], d["bt"], d["ctx"], d["cu_q"], d["nq"], d["nkv"], d["hd"],
                         d["mb"], d["bs"], d["scale"])


# ---------------------------------------------------------------- bf16 conversion (common.zig:55-65)
def test_bf16_rne_known_values():
    f = oracle.f32_to_bf16
    assert f(np.float32(1.0)) == 0x3F80
    assert f(np.float32(1.0 + 2 ** -8)) == 0x3F80  # tie -> even (down)
    assert f(np.float32(1.0 + 3 * 2 ** -8)) == 0x3F82  # tie -> even (up)
    assert f(np.float32(1.0 + 2 ** -8 + 2 ** -20)) == 0x3F81  # above the tie -> up
    assert f(np.float32(-0.0)) == 0x8000
    assert f(np.float32(np.inf)) == 0x7F80
    assert f(np.float32(np.nan)) == 0x7FC0
    assert f(np.float32(3.4e38)) == 0x7F80  # rounds past the largest bf16 -> inf


def test_bf16_matches_torch_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
                        rng.uniform(-2, 2, 10000).astype(np.float32)]).astype(np.float32)
    assert np.array_equal(oracle.f32_to_bf16(x), bf16(x))
    b = bf16(x)
    assert np.array_equal(oracle.bf16_to_f32(b), torch.tensor(b.view(np.int16)).view(torch.bfloat16).float().numpy())


# ---------------------------------------------------------------- storeKv (attention.zig:31-44, test :253-274)
def test_store_kv_reference_literal_case():
    nkv, hd, bs = 2, 4, 2
    k = bf16(np.arange(3 * nkv * hd, dtype=np.float32))
    v = bf16(100 + np.arange(3 * nkv * hd, dtype=np.float32))
    kc = np.zeros(3 * nkv * bs * hd, np.uint16)
    vc = np.zeros(3 * nkv * bs * hd, np.uint16)
    slots = np.array([5, -1, 0], np.int32)  # token0 -> block 2 offset 1; token1 skipped; token2 -> block 0
    oracle.store_kv(k, v, slots, kc, vc, nkv, hd, bs)
    assert kc[44] == k[1 * hd]  # token0, kv head 1: ((2*2+1)*2+1)*4 = 44
    assert vc[47] == v[1 * hd + 3]
    assert kc[0] == k[2 * nkv * hd]  # token2, kv head 0
    assert not kc[16:32].any()  # block 1 untouched (token1 skipped)


def test_store_kv_full_placement():
    rng = np.random.default_rng(3)
    T, nkv, hd, bs, nb = 37, 3, 16, 8, 12
    k = rand_bf16(rng, (T, nkv, hd))
    v = rand_bf16(rng, (T, nkv, hd))
    slots = rng.permutation(nb * bs)[:T].astype(np.int32)
    slots[[3, 17]] = -1
    kc = np.zeros((nb, nkv, bs, hd), np.uint16)
    vc = np.zeros_like(kc)
    oracle.store_kv(k, v, slots, kc, vc, nkv, hd, bs)
    exp_k = np.zeros_like(kc)
    exp_v = np.zeros_like(vc)
    for t, sl in enumerate(slots):
        if sl >= 0:
            exp_k[sl // bs, :, sl % bs, :] = k[t]
            exp_v[sl // bs, :, sl % bs, :] = v[t]
    assert np.array_equal(kc, exp_k) and np.array_equal(vc, exp_v)


# ---------------------------------------------------------------- attend (attention.zig:64-118)
@pytest.mark.parametrize("hd", [64, 128])
def test_attend_reference_mixed_batch(hd):
    """attention.zig:188-251 re-expressed: mixed batch within abs 1e-2 of an f32 reference, padding row 0; here
    against an independent float64 reference (much tighter than the reference test's 1e-2)."""
    c = mixed_case(hd)
    ob, of = run_attend(c)
    ref = numpy_attention(c["q"], c["kc"], c["vc"], c["bt"], c["ctx"], c["cu_q"], c["nq"], c["nkv"], hd, c["bs"],
                          c["scale"])
    assert np.abs(of - ref).max() < 2e-6
    assert np.abs(oracle.bf16_to_f32(ob) - ref).max() < 1e-2
    assert not ob[31].any() and not of[31].any()  # padding row exactly 0
    # the bf16 output is the RNE rounding of the f32 value
    assert np.array_equal(ob, oracle.f32_to_bf16(of))


def test_attend_matches_two_pass_reference():
    c = mixed_case(128, seed=5)
    _, of = run_attend(c)
    ref = oracle.ref_two_pass(c["q"], c["kc"], c["vc"], c["bt"], c["ctx"], c["cu_q"], c["nq"], c["nkv"], 128,
                              c["mb"], c["bs"], c["scale"])
    assert np.abs(of - ref).max() < 1e-6


def test_single_key_returns_v_exactly():
    rng = np.random.default_rng(1)
    nq, nkv, hd, bs = 4, 2, 128, 16
    kc = rand_bf16(rng, (2, nkv, bs, hd))
    vc = rand_bf16(rng, (2, nkv, bs, hd))
    q = rand_bf16(rng, (1, nq, hd), -4, 4)
    bt = np.array([[1, 0]], np.int32)
    ob, of = oracle.attend(q, kc, vc, bt, np.array([1], np.int32), np.array([0, 1], np.int32), nq, nkv, hd, 2, bs,
                           0.1)
    for h in range(nq):
        assert np.array_equal(ob[0, h], vc[1, h // 2, 0])


def test_zero_query_gives_mean_of_v():
    rng = np.random.default_rng(2)
    nq, nkv, hd, bs, ctx = 2, 1, 128, 16, 45
    kc = rand_bf16(rng, (4, nkv, bs, hd))
    vc = rand_bf16(rng, (4, nkv, bs, hd))
    q = np.zeros((1, nq, hd), np.uint16)
    bt = np.array([[2, 0, 3, 1]], np.int32)
    _, of = oracle.attend(q, kc, vc, bt, np.array([ctx], np.int32), np.array([0, 1], np.int32), nq, nkv, hd, 4, bs,
                          0.3)
    pos = np.arange(ctx)
    mean = oracle.bf16_to_f32(vc).astype(np.float64)[bt[0][pos // bs], 0, pos % bs].mean(0)
    assert np.abs(of[0, 0] - mean).max() < 1e-6 and np.abs(of[0, 1] - mean).max() < 1e-6


def test_block_permutation_invariance():
    c = mixed_case(128, seed=7)
    ob, of = run_attend(c)
    perm = np.random.default_rng(9).permutation(24)  # physical block b moves to perm[b]
    kc2 = np.zeros_like(c["kc"])
    vc2 = np.zeros_like(c["vc"])
    kc2[perm] = c["kc"]
    vc2[perm] = c["vc"]
    bt2 = perm[c["bt"]].astype(np.int32)
    ob2, of2 = run_attend(c, kc=kc2, vc=vc2, bt=bt2)
    assert np.array_equal(ob, ob2) and np.array_equal(of, of2)


def test_chunked_prefill_equals_tail_of_full_prefill():
    rng = np.random.default_rng(4)
    nq, nkv, hd, bs, L, chunk = 4, 2, 128, 16, 90, 35
    kc = rand_bf16(rng, (8, nkv, bs, hd))
    vc = rand_bf16(rng, (8, nkv, bs, hd))
    q = rand_bf16(rng, (L, nq, hd))
    bt = np.array([[5, 2, 7, 0, 1, 6, 3, 4]], np.int32)
    full_b, full_f = oracle.attend(q, kc, vc, bt, np.array([L], np.int32), np.array([0, L], np.int32), nq, nkv, hd,
                                   8, bs, 0.088)
    tail_b, tail_f = oracle.attend(q[L - chunk:], kc, vc, bt, np.array([L], np.int32), np.array([0, chunk], np.int32),
                                   nq, nkv, hd, 8, bs, 0.088)
    assert np.array_equal(full_b[L - chunk:], tail_b) and np.array_equal(full_f[L - chunk:], tail_f)


def test_gqa_equals_mha_with_replicated_kv():
    c = mixed_case(128, seed=13)
    ob, of = run_attend(c)
    kc4 = np.repeat(c["kc"], 2, axis=1)  # kv head h -> heads 2h, 2h+1
    vc4 = np.repeat(c["vc"], 2, axis=1)
    ob4, of4 = run_attend(c, kc=kc4, vc=vc4, nkv=4)
    assert np.array_equal(ob, ob4) and np.array_equal(of, of4)


def test_rows_and_threads_agree_with_full_attend():
    c = mixed_case(128, seed=17)
    ob, of = run_attend(c)
    rows = np.array([0, 7, 29, 30, 31], np.int32)
    args = (c["q"], c["kc"], c["vc"], c["bt"], c["ctx"], c["cu_q"], c["nq"], c["nkv"], 128, c["mb"], c["bs"],
            c["scale"])
    rb, rf = oracle.attend_rows(*args, rows=rows)
    assert np.array_equal(rb, ob[rows]) and np.array_equal(rf, of[rows])
    tb, tf = oracle.attend_rows(*args, rows=rows, threads=4)
    assert np.array_equal(tb, ob[rows]) and np.array_equal(tf, of[rows])


def test_rejects_bad_shapes():
    c = mixed_case(128)
    with pytest.raises(ValueError):
        run_attend(c, nkv=3)  # nq % nkv != 0
    with pytest.raises(ValueError):
        run_attend(c, hd=512)  # > MAX_HD (attention.zig:12)


# ---------------------------------------------------------------- committed golden vectors
def test_oracle_reproduces_golden_vectors():
    import os

    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "paged_attention_golden.npz"))
    nq, nkv, hd, bs, mb = (int(x) for x in g["shape"])
    kc, vc = g["kc"].copy(), g["vc"].copy()
    oracle.store_kv(g["k"], g["v"], g["slots"], kc, vc, nkv, hd, bs)
    ob, of = oracle.attend(g["q"], kc, vc, g["block_tables"], g["ctx"], g["cu_q"], nq, nkv, hd, mb, bs,
                           1 / np.sqrt(hd))
    assert np.array_equal(ob, g["out_bf16"]) and np.array_equal(of, g["out_f32"])
    ref = numpy_attention(g["q"], kc, vc, g["block_tables"], g["ctx"], g["cu_q"], nq, nkv, hd, bs, 1 / np.sqrt(hd))
    assert np.abs(g["out_f32"] - ref).max() < 2e-6
