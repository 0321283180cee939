"""MI355X-native (gfx950) attention hot path of the Qwen3 inference engine.

Three hand-written HIP kernel families behind one C ABI
(include/qwen3_attn.h, built into libqwen3_attn.so next to this file):
paged decode attention with split-KV, varlen causal flash prefill, and the
paged KV-cache slot writes.  The Python modules mirror the reference engine's
kernel-wrapper and KV-cache interfaces so its call sites are a drop-in:

    qwen3_engine_from_scratch_amd.kernels.paged_attention      <- qwen3/kernels/paged_attention.py
    qwen3_engine_from_scratch_amd.kernels.flash_attention_varlen <- qwen3/kernels/flash_attention_varlen.py
    qwen3_engine_from_scratch_amd.PagedKVcache                 <- qwen3/PagedKVcache.py
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]
