"""CPU parity oracle for the llmgen attention hot path -- TEST INFRASTRUCTURE ONLY.

A ctypes front end over ``oracle/liboracle.so`` (built from ``attention_oracle.c`` by ``oracle/Makefile``), which
restates the reference CPU backend's attention (``src/backend/cpu/attention.zig:31-118``) and its bf16 helpers
(``src/backend/cpu/common.zig:55-65``).  Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import this package, and only as the checker; the product path in ``llmgen_amd`` never
does.

All arrays are numpy: bf16 tensors are ``uint16`` bit patterns, index tensors are ``int32``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> None:
    """Compile the C restatement (seconds)."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    P = ctypes.c_void_p
    I = ctypes.c_int64
    lib.ora_f32_to_bf16.restype = ctypes.c_uint16
    lib.ora_f32_to_bf16.argtypes = [ctypes.c_float]
    lib.ora_bf16_to_f32.restype = ctypes.c_float
    lib.ora_bf16_to_f32.argtypes = [ctypes.c_uint16]
    lib.ora_f32_to_bf16_array.argtypes = [P, P, I]
    lib.ora_store_kv.argtypes = [P, P, P, P, P, I, I, I, I]
    common = [P, P, P, P, P, P, P, P, I, I, I, I, I, I, ctypes.c_float]
    lib.ora_attend.argtypes = common
    lib.ora_attend.restype = ctypes.c_int
    lib.ora_attend_rows.argtypes = common + [P, I]
    lib.ora_attend_rows.restype = ctypes.c_int
    lib.ora_attend_rows_omp.argtypes = common + [P, I, ctypes.c_int]
    lib.ora_attend_rows_omp.restype = ctypes.c_int
    lib.ora_ref_two_pass.argtypes = [P, P, P, P, P, P, P, I, I, I, I, I, I, ctypes.c_float]
    lib.ora_ref_two_pass.restype = ctypes.c_int
    _lib = lib
    return lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _u16(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    assert a.dtype == np.uint16, f"bf16 tensors are uint16 bit patterns, got {a.dtype}"
    return a


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def f32_to_bf16(x) -> np.ndarray:
    """RNE f32 -> bf16 bits, NaN -> 0x7FC0 (common.zig:59-65)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    _load().ora_f32_to_bf16_array(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(b) -> np.ndarray:
    """bf16 bits -> f32 by a 16-bit left shift (common.zig:55-57)."""
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def store_kv(k, v, slots, kc: np.ndarray, vc: np.ndarray, nkv: int, hd: int, bs: int) -> None:
    """In-place paged write (cpu/attention.zig:31-44). k, v: [T, nkv, hd]; kc, vc: [blocks, nkv, bs, hd]."""
    k, v, slots = _u16(k), _u16(v), _i32(slots)
    assert kc.flags["C_CONTIGUOUS"] and vc.flags["C_CONTIGUOUS"]
    _load().ora_store_kv(_p(k), _p(v), _p(slots), _p(kc), _p(vc), slots.size, nkv, hd, bs)


def _common(q, kc, vc, block_tables, ctx_lens, cu_q):
    return _u16(q), _u16(kc), _u16(vc), _i32(block_tables), _i32(ctx_lens), _i32(cu_q)


def attend(q, kc, vc, block_tables, ctx_lens, cu_q, nq, nkv, hd, max_blocks, bs, scale):
    """cpu/attention.zig:64-118. Returns (out_bf16 [T,nq,hd] uint16, out_f32 [T,nq,hd] before rounding)."""
    q, kc, vc, bt, ctx, cuq = _common(q, kc, vc, block_tables, ctx_lens, cu_q)
    T = int(cuq[-1])
    out = np.zeros((T, nq, hd), np.uint16)
    out32 = np.zeros((T, nq, hd), np.float32)
    rc = _load().ora_attend(_p(out), _p(out32), _p(q), _p(kc), _p(vc), _p(bt), _p(ctx), _p(cuq),
                            ctx.size, nq, nkv, hd, max_blocks, bs, scale)
    if rc != 0:
        raise ValueError(f"oracle attend rejected shape nq={nq} nkv={nkv} hd={hd}")
    return out, out32


def attend_rows(q, kc, vc, block_tables, ctx_lens, cu_q, nq, nkv, hd, max_blocks, bs, scale, rows,
                threads: int = 1):
    """attend() restricted to token rows ``rows``. Returns (bf16 [R,nq,hd], f32 [R,nq,hd]) in ``rows`` order."""
    q, kc, vc, bt, ctx, cuq = _common(q, kc, vc, block_tables, ctx_lens, cu_q)
    rows = _i32(rows)
    T = int(cuq[-1])
    out = np.zeros((T, nq, hd), np.uint16)
    out32 = np.zeros((T, nq, hd), np.float32)
    lib = _load()
    args = (_p(out), _p(out32), _p(q), _p(kc), _p(vc), _p(bt), _p(ctx), _p(cuq),
            ctx.size, nq, nkv, hd, max_blocks, bs, scale, _p(rows), rows.size)
    rc = lib.ora_attend_rows_omp(*args, threads) if threads > 1 else lib.ora_attend_rows(*args)
    if rc != 0:
        raise ValueError("oracle attend_rows rejected shape")
    return out[rows], out32[rows]


def ref_two_pass(q, kc, vc, block_tables, ctx_lens, cu_q, nq, nkv, hd, max_blocks, bs, scale) -> np.ndarray:
    """kernel_test.zig:117-149 two-pass f32 reference over a varlen batch. Returns f32 [T,nq,hd]."""
    q, kc, vc, bt, ctx, cuq = _common(q, kc, vc, block_tables, ctx_lens, cu_q)
    T = int(cuq[-1])
    out = np.zeros((T, nq, hd), np.float32)
    rc = _load().ora_ref_two_pass(_p(out), _p(q), _p(kc), _p(vc), _p(bt), _p(ctx), _p(cuq),
                                  ctx.size, nq, nkv, hd, max_blocks, bs, scale)
    if rc != 0:
        raise ValueError("oracle ref_two_pass rejected shape")
    return out


# ---------------------------------------------------------------------------------------------------------------
# Non-attention ops of the CPU backend (model_oracle.c).  Arrays are uint16 (bf16 bits) or float32; the output
# dtype is chosen by ``out_bf16`` as the reference's output tensor dtype would be.
# ---------------------------------------------------------------------------------------------------------------
_DT = {np.dtype(np.uint16): 1, np.dtype(np.float32): 0}


def _t(a):
    a = np.ascontiguousarray(a)
    if a.dtype not in _DT:
        raise TypeError(f"oracle ops take uint16 (bf16) or float32 arrays, got {a.dtype}")
    return a, _DT[a.dtype]


def _out(shape, out_bf16):
    return np.empty(shape, np.uint16 if out_bf16 else np.float32)


def _model_sigs(lib):
    P, I, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float
    D = ctypes.c_int
    lib.ora_embedding.argtypes = [P, P, D, P, D, I, I, I]
    lib.ora_embedding.restype = ctypes.c_int
    lib.ora_rmsnorm.argtypes = [P, D, P, D, P, D, I, I, F, F]
    lib.ora_linear.argtypes = [P, D, P, D, P, D, I, I, I]
    lib.ora_rope_table.argtypes = [P, P, I, I, ctypes.c_double]
    lib.ora_rope.argtypes = [P, D, P, D, P, P, P, I, I, I, I]
    lib.ora_silu.argtypes = [P, D, P, D, I]
    lib.ora_add.argtypes = [P, D, P, D, P, D, I, I]
    lib.ora_mul.argtypes = [P, D, P, D, P, D, I, I]
    lib.ora_gather.argtypes = [P, P, P, I, I]
    lib.ora_sample.argtypes = [P, D, P, P, ctypes.c_uint64, I, I]
    lib.ora_splitmix64.argtypes = [ctypes.c_uint64]
    lib.ora_splitmix64.restype = ctypes.c_uint64


def _mlib():
    lib = _load()
    if not getattr(lib, "_model_sigs", False):
        _model_sigs(lib)
        lib._model_sigs = True
    return lib


def embedding(ids, table, out_bf16=True):
    """cpu/embedding.zig: out[s] = table[ids[s]]. Raises on an out-of-range id."""
    ids = _i32(ids)
    table, tdt = _t(table)
    vocab, hidden = table.shape
    out = _out((ids.size, hidden), out_bf16)
    if _mlib().ora_embedding(_p(ids), _p(table), tdt, _p(out), int(out_bf16), ids.size, vocab, hidden) != 0:
        raise IndexError("token id out of range")
    return out


def rmsnorm(x, gain, eps, out_bf16=None, w_offset=0.0):
    """cpu/norm.zig:57-89 over the last axis; output dtype defaults to the input's."""
    x, xdt = _t(x)
    gain, gdt = _t(gain)
    n = x.shape[-1]
    ob = xdt == 1 if out_bf16 is None else out_bf16
    out = _out(x.shape, ob)
    _mlib().ora_rmsnorm(_p(x), xdt, _p(gain), gdt, _p(out), int(ob), x.size // n, n, eps, w_offset)
    return out


def linear(x, w, out_bf16=None):
    """cpu/linear.zig:7-28: x [..., in] @ w[out, in]^T, f32 accumulation in index order."""
    x, xdt = _t(x)
    w, wdt = _t(w)
    out_dim, in_dim = w.shape
    assert x.shape[-1] == in_dim
    rows = x.size // in_dim
    ob = xdt == 1 if out_bf16 is None else out_bf16
    out = _out(x.shape[:-1] + (out_dim,), ob)
    _mlib().ora_linear(_p(x), xdt, _p(w), wdt, _p(out), int(ob), rows, in_dim, out_dim)
    return out


def rope_table(max_seq, head_dim, theta):
    """cpu/rope.zig:38-68: (cos, sin) f32 [max_seq, head_dim]."""
    c = np.empty((max_seq, head_dim), np.float32)
    s = np.empty((max_seq, head_dim), np.float32)
    _mlib().ora_rope_table(_p(c), _p(s), max_seq, head_dim, float(theta))
    return c, s


def rope(x, pos, cos_t, sin_t, out_bf16=None, rope_dim=None):
    """cpu/rope.zig:6-36: NEOX rotation of x [T, n_head, head_dim] at positions pos [T]."""
    x, xdt = _t(x)
    pos = _i32(pos)
    T, nh, hd = x.shape
    rd = hd if rope_dim is None else rope_dim
    cos_t = np.ascontiguousarray(cos_t, np.float32)
    sin_t = np.ascontiguousarray(sin_t, np.float32)
    assert cos_t.shape[1] == rd and int(pos.max(initial=0)) < cos_t.shape[0]
    ob = xdt == 1 if out_bf16 is None else out_bf16
    out = _out(x.shape, ob)
    _mlib().ora_rope(_p(x), xdt, _p(out), int(ob), _p(pos), _p(cos_t), _p(sin_t), T, nh, hd, rd)
    return out


def silu(x, out_bf16=None):
    x, xdt = _t(x)
    ob = xdt == 1 if out_bf16 is None else out_bf16
    out = _out(x.shape, ob)
    _mlib().ora_silu(_p(x), xdt, _p(out), int(ob), x.size)
    return out


def _binary(fn, a, b, out_bf16):
    a, adt = _t(a)
    b, bdt = _t(b)
    assert a.size % b.size == 0
    ob = adt == 1 if out_bf16 is None else out_bf16
    out = _out(a.shape, ob)
    fn(_p(a), adt, _p(b), bdt, _p(out), int(ob), a.size, b.size)
    return out


def add(a, b, out_bf16=None):
    """cpu/arithmetic.zig add (b broadcast by index modulo its size)."""
    return _binary(_mlib().ora_add, a, b, out_bf16)


def mul(a, b, out_bf16=None):
    """cpu/arithmetic.zig mul."""
    return _binary(_mlib().ora_mul, a, b, out_bf16)


def gather(x, last):
    """cpu/memcpy.zig GatherLast: rows last[s] of x [T, H]."""
    x = np.ascontiguousarray(x)
    last = _i32(last)
    assert int(last.max(initial=0)) < x.shape[0]
    out = np.empty((last.size,) + x.shape[1:], x.dtype)
    _mlib().ora_gather(_p(x), _p(out), _p(last), last.size, x[0].nbytes)
    return out


def sample(logits, temps=None, seed=0):
    """cpu/sample.zig:12-40: greedy (temp <= 0; ties keep the smaller index) or Gumbel-max per row."""
    logits, ldt = _t(logits)
    S, V = logits.shape
    temps = np.zeros(S, np.float32) if temps is None else np.ascontiguousarray(temps, np.float32)
    out = np.empty(S, np.int32)
    _mlib().ora_sample(_p(logits), ldt, _p(out), _p(temps), int(seed) & (2**64 - 1), S, V)
    return out


def splitmix64(x: int) -> int:
    """cpu/sample.zig:5-10 (one SplitMix64 output for state x)."""
    return int(_mlib().ora_splitmix64(int(x) & (2**64 - 1)))
