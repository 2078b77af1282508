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
