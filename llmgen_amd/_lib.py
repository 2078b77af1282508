"""ctypes binding of libllmgen_attn.so (the C-ABI declared in include/llmgen_attn.h and include/llmgen_model.h).

The library is loaded from the package directory (built in-tree by ``llmgen_amd.build``).  There is no fallback:
if the library is missing or fails to load, :func:`lib` raises, so nothing on the product path can silently run
elsewhere.
"""
from __future__ import annotations

import ctypes
import os

from .build import LIB_PATH

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_L = ctypes.c_long

# name -> (restype, argtypes); must match include/llmgen_attn.h and include/llmgen_model.h
SIGNATURES = {
    "hip_store_kv": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I]),
    "hip_attn_decode": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P, _P, _I, _I]),
    "hip_attn_decode_store_kv": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P, _P, _I,
                                        _I]),
    "hip_attn_decode_noalloc": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _I]),
    "hip_attn_prefill": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F]),
    "hip_attn_prefill_rows": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I]),
    "hip_attn_prefill_tile": (_I, []),
    "hip_attn_prefill_plan": (_I, [_I, _I, _I, _I, _I, _I]),
    "hip_attn_set_option": (_I, [_I, _I]),
    "hip_init": (_I, [_SZ]),
    "hip_sync": (None, []),
    "hip_last_error": (_I, []),
    "hip_graph_begin": (_I, []),
    "hip_graph_end": (_P, []),
    "hip_graph_launch": (None, [_P]),
    "hip_graph_destroy": (None, [_P]),
    "hip_device_count": (_I, []),
    "hip_mem_info": (None, [ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
    "hip_device_info": (None, [_I, ctypes.c_char_p, _I, ctypes.POINTER(_SZ), ctypes.POINTER(_I)]),
    "hip_set_stream": (None, [_P]),
    "hip_get_stream": (_P, []),
    "hip_malloc": (_P, [_SZ]),
    "hip_free": (None, [_P]),
    "hip_host_alloc": (_P, [_SZ]),
    "hip_host_free": (None, [_P]),
    "hip_h2d": (None, [_P, _P, _SZ]),
    "hip_d2h": (None, [_P, _P, _SZ]),
    "hip_d2d": (None, [_P, _P, _SZ]),
    "hip_h2d_async": (None, [_P, _P, _SZ]),
    "hip_d2h_async": (None, [_P, _P, _SZ]),
    "hip_timer_create": (_P, []),
    "hip_timer_record": (None, [_P]),
    "hip_timer_elapsed_ms": (_F, [_P, _P]),
    "hip_timer_destroy": (None, [_P]),
    # include/llmgen_model.h
    "hip_embedding": (None, [_P, _P, _P, _I, _I]),
    "hip_rmsnorm": (None, [_P, _P, _P, _L, _I, _F]),
    "hip_linear": (None, [_P, _I, _P, _P, _I, _I, _I]),
    "hip_rope": (None, [_P, _P, _P, _P, _P, _I, _I, _I]),
    "hip_silu": (None, [_P, _P, _SZ]),
    "hip_add": (None, [_P, _P, _P, _SZ]),
    "hip_mul": (None, [_P, _P, _P, _SZ]),
    "hip_gather_rows": (None, [_P, _P, _P, _I, _I]),
    "hip_sample": (None, [_P, _P, _P, _P, _I, _I, _P]),
    "hip_sample_scratch_bytes": (_SZ, [_I]),
    "hip_qk_norm_rope_store_kv": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
}

_lib = None
_lib_path = None


class LibraryMissing(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load libllmgen_attn.so (once) and attach the C signatures. Raises LibraryMissing if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    path = os.environ.get("LLMGEN_ATTN_LIB", LIB_PATH)  # an alternative build of the same library (A/B runs)
    if not os.path.exists(path):
        raise LibraryMissing(f"{path} is not built; run `python -m llmgen_amd.build` (hipcc, gfx950)")
    handle = ctypes.CDLL(path)
    alt = "LLMGEN_ATTN_LIB" in os.environ  # an A/B build may predate some entry points: bind what it has
    for name, (res, args) in SIGNATURES.items():
        if alt and not hasattr(handle, name):
            continue
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    global _lib_path
    _lib, _lib_path = handle, os.path.abspath(path)
    return handle


def loaded_library() -> dict:
    """Path and sha256 of the library this process loaded (recorded with every benchmark line)."""
    import hashlib

    lib()
    with open(_lib_path, "rb") as f:
        digest = hashlib.sha256(f.read()).hexdigest()
    return {"path": os.path.relpath(_lib_path, os.path.dirname(os.path.dirname(os.path.abspath(__file__)))),
            "sha256": digest}
