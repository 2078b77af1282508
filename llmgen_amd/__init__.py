"""llmgen_amd -- MI355X (gfx950) attention path for the llmgen engine.

Three hand-written HIP kernels behind the engine's C-ABI (include/llmgen_attn.h, built into
llmgen_amd/libllmgen_attn.so): paged-KV store, split-K flash decoding and FA2-style MFMA prefill.  The Python
modules mirror the host side the engine wraps around them: per-step metadata (``step``), the operator
(``attention.PagedAttentionImpl``), decode graph buckets (``graphs``) and seeded workloads (``workloads``).
"""
from .build import LIB_PATH, build  # noqa: F401
