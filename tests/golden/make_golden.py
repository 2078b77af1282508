"""Write tests/golden/paged_attention_golden.npz: small seeded inputs and the CPU oracle's outputs.

The oracle (oracle/attention_oracle.c) restates src/backend/cpu/attention.zig:31-118; the reference engine itself
cannot run here (Zig toolchain absent), so these vectors are the oracle's, pinned by tests/test_oracle.py.
Case: nq=4, nkv=2, hd=128, bs=16, 12 physical blocks, permuted block tables; a step with a chunked-prefill tail
(ctx=70, q_len=30, tokens written by store_kv this step), a decode row (ctx=41) and a padding row (ctx=0,
slot=-1) -- the shape of attention.zig:188-251 at the kernels' head size.  Inputs U(-1, 1) rounded to bf16.
Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402


def main():
    rng = np.random.default_rng(20260101)
    nq, nkv, hd, bs, nb, mb = 4, 2, 128, 16, 12, 8
    kc = oracle.f32_to_bf16(rng.uniform(-1, 1, (nb, nkv, bs, hd)))
    vc = oracle.f32_to_bf16(rng.uniform(-1, 1, (nb, nkv, bs, hd)))
    bt = np.zeros((3, mb), np.int32)
    bt[0, :5] = [7, 2, 10, 0, 5]  # ctx 70 -> 5 blocks
    bt[1, :3] = [11, 4, 8]  # ctx 41 -> 3 blocks
    cu_q = np.array([0, 30, 31, 32], np.int32)
    ctx = np.array([70, 41, 0], np.int32)
    T = 32
    q = oracle.f32_to_bf16(rng.uniform(-1, 1, (T, nq, hd)))
    k = oracle.f32_to_bf16(rng.uniform(-1, 1, (T, nkv, hd)))
    v = oracle.f32_to_bf16(rng.uniform(-1, 1, (T, nkv, hd)))
    slots = np.empty(T, np.int32)
    for j in range(30):
        p = 40 + j
        slots[j] = bt[0, p // bs] * bs + p % bs
    slots[30] = bt[1, 40 // bs] * bs + 40 % bs
    slots[31] = -1
    kc_after, vc_after = kc.copy(), vc.copy()
    oracle.store_kv(k, v, slots, kc_after, vc_after, nkv, hd, bs)
    out_bf16, out_f32 = oracle.attend(q, kc_after, vc_after, bt, ctx, cu_q, nq, nkv, hd, mb, bs, 1 / np.sqrt(hd))
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "paged_attention_golden.npz")
    np.savez_compressed(path, q=q, k=k, v=v, kc=kc, vc=vc, slots=slots, block_tables=bt, cu_q=cu_q, ctx=ctx,
                        out_bf16=out_bf16, out_f32=out_f32,
                        shape=np.array([nq, nkv, hd, bs, mb], np.int32))
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
