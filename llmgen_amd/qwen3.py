"""Qwen3 forward on the GPU around the HIP attention path -- the end-to-end greedy-token check.

Mirrors the reference model graph (``src/models/qwen3.zig:165-330``): per layer RMSNorm -> q/k/v projections ->
head split -> per-head q/k RMSNorm -> NEOX RoPE at ``g_step.pos`` -> paged attention (store_kv, then split-K
decode or causal varlen prefill) -> output projection -> residual add; RMSNorm -> SwiGLU MLP -> residual add;
then the final RMSNorm, gather of each sequence's last row, the tied LM head and sampling.

Each step is prepared and dispatched by the C++ executor slice (``include/llmgen_host.h``): ``llmgen_fill_meta``
packs the step's metadata (token ids, positions, slots, ``cu_q``, ``ctx``, ``last``, temperatures, prefill tiles,
block tables, step seed) into one buffer uploaded with one copy, ``llmgen_bind_step`` publishes its device
addresses, and ``llmgen_paged_attention`` runs each layer's attention.  Every other op is an
``include/llmgen_model.h`` kernel that computes each value in the reference CPU backend's order and rounding, so a
forward here differs from the CPU backend's only through the attention kernels.

Weights are random (no checkpoint is available offline): :func:`random_weights` draws a seeded Qwen3-0.6B-shaped
set in GGUF tensor naming, bf16 for matrices and f32 for norm gains as GGUF stores them.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, List, Sequence

import numpy as np
import torch

from . import attention as A
from . import host as Hx
from . import step as stepmod
from ._lib import lib


@dataclass(frozen=True)
class Qwen3Config:
    """Qwen3-0.6B: 28 layers, hidden 1024, 16 Q / 8 KV heads of 128, MLP 3072, vocab 151936, tied LM head."""

    vocab: int = 151936
    hidden: int = 1024
    n_layers: int = 28
    n_head: int = 16
    n_kv_head: int = 8
    head_dim: int = 128
    ffn: int = 3072
    rms_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    max_model_len: int = 1024
    block_size: int = 16  # memory/page_atten.zig:12 PAGE_BLOCK_SIZE


def weight_shapes(cfg: Qwen3Config) -> Dict[str, tuple]:
    """GGUF tensor names and shapes ([out, in] for matrices)."""
    H, hd = cfg.hidden, cfg.head_dim
    shapes = {"token_embd.weight": (cfg.vocab, H), "output_norm.weight": (H,)}
    for i in range(cfg.n_layers):
        b = f"blk.{i}."
        shapes.update({
            b + "attn_norm.weight": (H,),
            b + "attn_q.weight": (cfg.n_head * hd, H),
            b + "attn_k.weight": (cfg.n_kv_head * hd, H),
            b + "attn_v.weight": (cfg.n_kv_head * hd, H),
            b + "attn_q_norm.weight": (hd,),
            b + "attn_k_norm.weight": (hd,),
            b + "attn_output.weight": (H, cfg.n_head * hd),
            b + "ffn_norm.weight": (H,),
            b + "ffn_gate.weight": (cfg.ffn, H),
            b + "ffn_up.weight": (cfg.ffn, H),
            b + "ffn_down.weight": (H, cfg.ffn),
        })
    return shapes


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round f32 to bf16 (nearest even) and return the bit patterns (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def random_weights(cfg: Qwen3Config, seed: int = 0, std: float = 0.02,
                   embd_row_sigma: float = 0.0) -> Dict[str, np.ndarray]:
    """Seeded random weights: matrices N(0, std) as bf16 bits (uint16), norm gains 1 + N(0, 0.1) as f32.
    ``embd_row_sigma`` > 0 scales each row of the (tied) token embedding by exp(N(0, sigma)), giving the
    log-normal spread of row norms trained embeddings have."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in weight_shapes(cfg).items():
        if len(shape) == 1:
            out[name] = (1.0 + 0.1 * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)
            continue
        w = std * rng.standard_normal(shape, dtype=np.float32)
        if name == "token_embd.weight" and embd_row_sigma > 0:
            w *= np.exp(embd_row_sigma * rng.standard_normal((shape[0], 1))).astype(np.float32)
        out[name] = f32_to_bf16_bits(w)
    return out


def rope_tables(max_seq: int, head_dim: int, theta: float):
    """cpu/rope.zig:38-68 RopeCache: inv_freq = 1 / theta^(2i/hd) and angle = pos * inv_freq in double, cos / sin
    rounded to f32 and stored in both halves of each row.  Computed with the C library's pow / cos / sin."""
    half = head_dim // 2
    inv = [1.0 / math.pow(theta, (2.0 * i) / head_dim) for i in range(half)]
    c = np.empty((max_seq, head_dim), np.float32)
    s = np.empty((max_seq, head_dim), np.float32)
    for p in range(max_seq):
        ang = [p * f for f in inv]
        c[p, :half] = c[p, half:] = np.array([math.cos(a) for a in ang], np.float64)
        s[p, :half] = s[p, half:] = np.array([math.sin(a) for a in ang], np.float64)
    return c, s


def _bits(t: np.ndarray, device) -> torch.Tensor:
    """Upload a uint16 (bf16 bits) or float32 numpy array."""
    if t.dtype == np.uint16:
        return torch.from_numpy(t.view(np.int16)).to(device)
    return torch.from_numpy(np.ascontiguousarray(t)).to(device)


class Qwen3:
    """A Qwen3 model resident on one GPU with its paged KV cache.  :meth:`forward` runs one engine step
    (``executor.zig`` forward: bind the step metadata, run the graph, sample) for a list of
    :class:`~llmgen_amd.step.Entry` and their input token ids, and returns the sampled id per sequence."""

    def __init__(self, cfg: Qwen3Config, weights: Dict[str, np.ndarray], num_blocks: int, max_seqs: int = 8,
                 max_tokens: int = 1024, device: str = "cuda"):
        A.init_device()
        self.cfg, self.device = cfg, device
        self.L = lib()
        self.w = {k: _bits(v, device) for k, v in weights.items()}
        cos_t, sin_t = rope_tables(cfg.max_model_len, cfg.head_dim, cfg.rope_theta)
        self.cos, self.sin = _bits(cos_t, device), _bits(sin_t, device)
        self.max_blocks = (cfg.max_model_len + cfg.block_size - 1) // cfg.block_size
        # paged KV pools, one pair per layer (memory/page_atten.zig:15-28)
        self.kv = [A.PagedAttentionManager().reserve_layer(i, num_blocks, cfg.n_kv_head, cfg.block_size,
                                                           cfg.head_dim, device) for i in range(cfg.n_layers)]
        self.pf_tile = self.L.hip_attn_prefill_tile()
        # executor.zig:92-102 Workspace.of: metadata, split-K scratch, sampling scratch
        ws = Hx.workspace(cfg.n_head, cfg.head_dim, max_seqs, max_tokens, cfg.max_model_len, cfg.block_size,
                          self.pf_tile)
        u8 = torch.uint8
        self.meta_dev = torch.zeros(ws["meta"], dtype=u8, device=device)
        self.part_o = torch.empty(max(ws["part_o"], 4), dtype=u8, device=device)
        self.part_ml = torch.empty(max(ws["part_ml"], 4), dtype=u8, device=device)
        self.sample_scratch = torch.empty(max(ws["sample"], 4), dtype=u8, device=device)
        self.max_seqs, self.max_tokens = max_seqs, max_tokens
        self.step_seed = 0

    def execute(self, entries: Sequence[stepmod.Entry], ids: Sequence[int], temps=None) -> List[int]:
        """executor.zig:986-1043: a step larger than max_tokens runs as several passes (an entry's query range may
        be cut); the sampled id of an entry comes from the pass that reaches its end."""
        total = sum(e.q_len for e in entries)
        if total <= self.max_tokens:
            return self.forward(entries, ids, temps)
        starts = np.cumsum([0] + [e.q_len for e in entries])
        pieces = Hx.plan_passes([(i, e.q_start, e.q_len) for i, e in enumerate(entries)], self.max_tokens)
        out = [0] * len(entries)
        by_pass = {}
        for pas, owner, piece in pieces:
            by_pass.setdefault(pas, []).append((owner, piece))
        for pas in sorted(by_pass):
            group = by_pass[pas]
            ents, pids, ptemps = [], [], []
            for owner, (_, q_start, q_len) in group:
                e = entries[owner]
                ents.append(stepmod.Entry(q_start, q_len, e.block_table))
                off = starts[owner] + (q_start - e.q_start)
                pids.extend(ids[off:off + q_len])
                ptemps.append(0.0 if temps is None else temps[owner])
            toks = self.forward(ents, pids, ptemps)
            for (owner, (_, q_start, q_len)), tk in zip(group, toks):
                e = entries[owner]
                if q_start + q_len == e.q_start + e.q_len:
                    out[owner] = tk
        return out

    # -- buffers of one step
    def _empty(self, *shape, dtype=torch.int16):
        return torch.empty(shape, dtype=dtype, device=self.device)

    def forward(self, entries: Sequence[stepmod.Entry], ids: Sequence[int], temps=None, seed=None,
                fused_qk: bool = True) -> List[int]:
        """One step: entries[i] computes positions [q_start, q_start + q_len) of sequence i with this step's
        token ids (concatenated in entry order).  ``temps[i]`` > 0 samples sequence i (Gumbel-max), else greedy.
        ``seed`` resets the step-seed state (executor.zig:773 advances it every step).  ``fused_qk`` runs q/k norm
        + RoPE + the KV write as one kernel (hip_qk_norm_rope_store_kv); the unfused path runs the reference
        graph's five launches.  Both give identical values."""
        cfg, L = self.cfg, self.L
        T, S = sum(e.q_len for e in entries), len(entries)
        if len(ids) != T or T > self.max_tokens or S > self.max_seqs:
            raise ValueError(f"step of {T} tokens / {S} sequences does not fit (ids {len(ids)})")
        if any(e.q_start + e.q_len > cfg.max_model_len for e in entries):
            raise ValueError("sequence longer than max_model_len")
        ids_np = np.asarray(ids, np.int64)
        if ids_np.min() < 0 or ids_np.max() >= cfg.vocab:
            raise IndexError("token id out of range")
        # the executor's view of the step: each sequence's token ids (this step's known), block table, temperature
        seqs, ents, t = [], [], 0
        for i, e in enumerate(entries):
            tok = np.zeros(e.q_start + e.q_len, np.int32)
            tok[e.q_start:] = ids_np[t:t + e.q_len]
            t += e.q_len
            seqs.append(Hx.Sequence_(tok, list(e.block_table), 0.0 if temps is None else float(temps[i])))
            ents.append((i, e.q_start, e.q_len))
        decode = all(e.q_len == 1 for e in entries)  # every entry ends its sequence, so it emits
        n_tiles = 0 if decode else sum((e.q_len + self.pf_tile - 1) // self.pf_tile for e in entries)
        if seed is not None:
            self.step_seed = int(seed)
        buf, lay, self.step_seed, single = Hx.fill_meta(seqs, ents, S, n_tiles, self.pf_tile, cfg.block_size,
                                                        self.max_blocks, self.step_seed)
        self.meta_dev[:lay.total].copy_(torch.from_numpy(buf))  # one upload per step
        g = Hx.bind_step(self.meta_dev.data_ptr(), lay, T, S, n_tiles, decode, cfg.n_head, cfg.n_kv_head,
                         cfg.head_dim, cfg.block_size, self.max_blocks, cfg.max_model_len, self.part_o.data_ptr(),
                         self.part_ml.data_ptr(), self.sample_scratch.data_ptr(), hidden=cfg.hidden,
                         single_rows=single)
        d = self.device
        ids_ptr = self.meta_dev.data_ptr() + lay.ids
        H, nq, nkv, hd, F = cfg.hidden, cfg.n_head, cfg.n_kv_head, cfg.head_dim, cfg.ffn
        x = self._empty(T, H)
        xn, o = self._empty(T, H), self._empty(T, H)
        q, k, v = self._empty(T, nq, hd), self._empty(T, nkv, hd), self._empty(T, nkv, hd)
        attn = self._empty(T, nq, hd)
        gate, up = self._empty(T, F), self._empty(T, F)
        p = lambda t: t.data_ptr()  # noqa: E731
        W = self.w
        L.hip_embedding(p(x), ids_ptr, p(W["token_embd.weight"]), T, H)
        for i in range(cfg.n_layers):
            b = f"blk.{i}."
            L.hip_rmsnorm(p(xn), p(x), p(W[b + "attn_norm.weight"]), T, H, cfg.rms_eps)
            L.hip_linear(p(q), 0, p(xn), p(W[b + "attn_q.weight"]), T, nq * hd, H)
            L.hip_linear(p(k), 0, p(xn), p(W[b + "attn_k.weight"]), T, nkv * hd, H)
            L.hip_linear(p(v), 0, p(xn), p(W[b + "attn_v.weight"]), T, nkv * hd, H)
            kv = self.kv[i]
            if fused_qk:
                L.hip_qk_norm_rope_store_kv(p(q), p(kv.k), p(kv.v), p(q), p(k), p(v),
                                            p(W[b + "attn_q_norm.weight"]), p(W[b + "attn_k_norm.weight"]),
                                            cfg.rms_eps, p(self.cos), p(self.sin), g.pos, g.slots, T, nq, nkv, hd,
                                            cfg.block_size)
            else:
                L.hip_rmsnorm(p(q), p(q), p(W[b + "attn_q_norm.weight"]), T * nq, hd, cfg.rms_eps)
                L.hip_rmsnorm(p(k), p(k), p(W[b + "attn_k_norm.weight"]), T * nkv, hd, cfg.rms_eps)
                L.hip_rope(p(q), p(q), p(self.cos), p(self.sin), g.pos, T, nq, hd)
                L.hip_rope(p(k), p(k), p(self.cos), p(self.sin), g.pos, T, nkv, hd)
            Hx.paged_attention(g, attn, q, k, v, kv.k, kv.v, store_kv=not fused_qk)
            L.hip_linear(p(o), 0, p(attn), p(W[b + "attn_output.weight"]), T, H, nq * hd)
            L.hip_add(p(x), p(x), p(o), T * H)
            L.hip_rmsnorm(p(xn), p(x), p(W[b + "ffn_norm.weight"]), T, H, cfg.rms_eps)
            L.hip_linear(p(gate), 0, p(xn), p(W[b + "ffn_gate.weight"]), T, F, H)
            L.hip_linear(p(up), 0, p(xn), p(W[b + "ffn_up.weight"]), T, F, H)
            L.hip_silu(p(gate), p(gate), T * F)
            L.hip_mul(p(gate), p(gate), p(up), T * F)
            L.hip_linear(p(o), 0, p(gate), p(W[b + "ffn_down.weight"]), T, H, F)
            L.hip_add(p(x), p(x), p(o), T * H)
        L.hip_rmsnorm(p(xn), p(x), p(W["output_norm.weight"]), T, H, cfg.rms_eps)
        last = self._empty(S, H)
        L.hip_gather_rows(p(last), p(xn), g.last, S, H)
        logits = self._empty(S, cfg.vocab)
        L.hip_linear(p(logits), 0, p(last), p(W["token_embd.weight"]), S, cfg.vocab, H)
        out = torch.empty(S, dtype=torch.int32, device=d)
        L.hip_sample(p(out), p(logits), g.temps, g.seed, S, cfg.vocab, p(self.sample_scratch))
        self.last_logits = logits
        return out.cpu().tolist()
