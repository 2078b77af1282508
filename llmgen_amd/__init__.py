"""llmgen_amd -- MI355X (gfx950) attention path for the llmgen engine.

Three hand-written HIP kernels behind the engine's C-ABI (include/llmgen_attn.h, built into
llmgen_amd/libllmgen_attn.so): paged-KV store, split-K flash decoding and FA2-style MFMA prefill.  The host side
the engine wraps around them (step metadata, StepState, per-layer dispatch, decode graph buckets) is C++ in the
same library (include/llmgen_host.h), reached from Python through ``host``; ``attention`` keeps the operator's
Python names (``PagedAttentionImpl``, ``g_step``, ``kv_of``) over it.  ``step`` is an independent Python
restatement of the metadata that tests hold the C++ one against; ``workloads`` builds the seeded steps.
"""
from .build import LIB_PATH, build  # noqa: F401
