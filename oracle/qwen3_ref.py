"""CPU Qwen3 forward built from the oracle's restated CPU-backend ops -- TEST INFRASTRUCTURE ONLY.

The graph is the reference's ``src/models/qwen3.zig:165-330`` (Qwen3Attention, Qwen3DecoderLayer, Qwen3Model
forward), executed op by op as the CPU backend executes it: embedding, RMSNorm, linear, per-head q/k RMSNorm,
NEOX RoPE at the step's positions, paged attention (``storeKv`` then ``attend``,
``src/backend/cpu/attention.zig:31-118``), residual adds, SwiGLU, final RMSNorm, gather of each sequence's last
row, tied LM head and sampling.  Activations are bf16 (the weights' dtype), so every op rounds its output to bf16.

Weights come in as the dict of GGUF-named numpy arrays that the GPU side uploads (uint16 bf16 bits for matrices,
f32 gains); the step metadata is the same :class:`StepMeta` the GPU step binds.
"""
from __future__ import annotations

import numpy as np

import oracle as O


class Qwen3Ref:
    def __init__(self, cfg, weights, num_blocks: int, rope_tables=None, attention: str = "online"):
        """``attention`` = "online" runs the CPU backend's attend (cpu/attention.zig:64-118); "two_pass" runs the
        reference's two-pass f32 test reference (kernel_test.zig:117-149) rounded to bf16 instead -- an equally
        exact summation order, used to measure how far two valid orderings drift apart through the model."""
        assert attention in ("online", "two_pass")
        self.attention = attention
        self.cfg, self.w = cfg, weights
        shape = (num_blocks, cfg.n_kv_head, cfg.block_size, cfg.head_dim)
        self.kc = [np.zeros(shape, np.uint16) for _ in range(cfg.n_layers)]
        self.vc = [np.zeros(shape, np.uint16) for _ in range(cfg.n_layers)]
        self.cos, self.sin = rope_tables if rope_tables is not None else O.rope_table(
            cfg.max_model_len, cfg.head_dim, cfg.rope_theta)

    def forward(self, meta, ids, max_blocks: int, temps=None, seed: int = 0, return_logits: bool = False):
        """One engine step for the packed step metadata ``meta`` (fill_meta output) and token ids ``ids``."""
        cfg, W = self.cfg, self.w
        T = meta.n_tok
        nq, nkv, hd, H = cfg.n_head, cfg.n_kv_head, cfg.head_dim, cfg.hidden
        scale = np.float32(1.0 / np.sqrt(np.float32(hd)))  # module/attention.zig:95 (f32 sqrt)
        eps = cfg.rms_eps
        x = O.embedding(np.asarray(ids, np.int32), W["token_embd.weight"])
        for i in range(cfg.n_layers):
            b = f"blk.{i}."
            xn = O.rmsnorm(x, W[b + "attn_norm.weight"], eps)
            q = O.linear(xn, W[b + "attn_q.weight"]).reshape(T, nq, hd)
            k = O.linear(xn, W[b + "attn_k.weight"]).reshape(T, nkv, hd)
            v = O.linear(xn, W[b + "attn_v.weight"]).reshape(T, nkv, hd)
            q = O.rmsnorm(q, W[b + "attn_q_norm.weight"], eps)
            k = O.rmsnorm(k, W[b + "attn_k_norm.weight"], eps)
            q = O.rope(q, meta.pos, self.cos, self.sin)
            k = O.rope(k, meta.pos, self.cos, self.sin)
            O.store_kv(k, v, meta.slots, self.kc[i], self.vc[i], nkv, hd, cfg.block_size)
            args = (q, self.kc[i], self.vc[i], meta.block_tables, meta.ctx, meta.cu_q, nq, nkv, hd, max_blocks,
                    cfg.block_size, float(scale))
            if self.attention == "online":
                attn, _ = O.attend(*args)
            else:
                attn = O.f32_to_bf16(O.ref_two_pass(*args))
            o = O.linear(attn.reshape(T, nq * hd), W[b + "attn_output.weight"])
            x = O.add(x, o)
            fn = O.rmsnorm(x, W[b + "ffn_norm.weight"], eps)
            gate = O.linear(fn, W[b + "ffn_gate.weight"])
            up = O.linear(fn, W[b + "ffn_up.weight"])
            down = O.linear(O.mul(O.silu(gate), up), W[b + "ffn_down.weight"])
            x = O.add(x, down)
        fx = O.rmsnorm(x, W["output_norm.weight"], eps)
        last = O.gather(fx, meta.last)
        logits = O.linear(last, W["token_embd.weight"])
        ids_out = O.sample(logits, temps, seed)
        return (ids_out, logits) if return_logits else ids_out
