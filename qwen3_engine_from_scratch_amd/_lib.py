"""ctypes binding of libqwen3_attn.so (the C ABI declared in include/qwen3_attn.h).

This module is the only place that touches the shared library.  There is no
fallback: if the library is missing or a tensor is not on a HIP device the
call raises, so a test or benchmark can never silently measure something else.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libqwen3_attn.so")

_c_i64p = ctypes.POINTER(ctypes.c_int64)
_c_i32p = ctypes.c_void_p  # device pointers travel as void*
_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64

# name -> (restype, argtypes)
_SIGNATURES = {
    "qwen3_attn_last_error": (ctypes.c_char_p, []),
    "qwen3_attn_abi_version": (_i, []),
    "qwen3_hbm_read_reference": (_i, [_vp, _i64, _i, _vp, _vp]),
    "qwen3_mfma_rate_reference": (_i, [_i, _vp, _c_i64p, _vp]),
    "qwen3_paged_decode_workspace_bytes": (ctypes.c_size_t, [_i, _i, _i, _i, _i64, _i]),
    "qwen3_paged_decode_bf16": (
        _i,
        [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _i64,
         _vp, _i64, _i64, _i64,
         _vp, _i, _vp,
         _vp, _c_i64p,
         _i, _i, _i, _i, _i, ctypes.c_float,
         _vp, ctypes.c_size_t, _vp],
    ),
    "qwen3_paged_decode_invariant_workspace_bytes": (ctypes.c_size_t,
                                                     [_i, _i, _i, _i, _i64, _i]),
    "qwen3_paged_decode_invariant_bf16": (
        _i,
        [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _i64,
         _vp, _i64, _i64, _i64,
         _vp, _i, _vp,
         _vp, _c_i64p,
         _i, _i, _i, _i, _i, ctypes.c_float,
         _vp, ctypes.c_size_t, _vp],
    ),
    "qwen3_paged_decode_noalloc_bf16": (
        _i,
        [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _i64,
         _vp, _i64, _i64, _i64,
         _vp, _i, _vp,
         _vp, _c_i64p,
         _i, _i, _i, _i, _i, ctypes.c_float, _vp],
    ),
    "qwen3_kv_write_decode_bf16": (
        _i,
        [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p,
         _i64, _i, _i, _vp, _vp, _i64, _i64, _i64, _vp,
         _i, _i, _i, _i, _vp],
    ),
    "qwen3_kv_write_range_bf16": (
        _i,
        [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p,
         _i64, _i, _i, _vp, _i64, _i64, _i64,
         _i, _i, _i, _vp],
    ),
    "qwen3_kv_write_slots_bf16": (
        _i,
        [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p,
         _i64, _i, _i, _vp, _i64,
         _i, _i, _i, _vp],
    ),
    "qwen3_varlen_prefill_workspace_bytes": (ctypes.c_size_t, []),
    "qwen3_varlen_prefill_bf16": (
        _i,
        [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p,
         _vp, _i, _i, _i64,
         _i, _i, _i, ctypes.c_float, _i, _vp, ctypes.c_size_t, _vp],
    ),
    "qwen3_qk_norm_rope_decode_bf16": (
        _i,
        [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _vp, ctypes.c_float,
         _vp, _vp, _i64, _i64,
         _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _i64, _i, _i,
         _vp, _vp, _i64, _i64, _i64, _vp, _vp,
         _i, _i, _i, _i, _i, _vp],
    ),
    "qwen3_qk_norm_rope_slots_bf16": (
        _i,
        [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _vp, ctypes.c_float,
         _vp, _vp, _i64, _i64, _vp, _vp,
         _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _i64, _i, _i,
         _i64, _i, _i, _i, _i, _vp],
    ),
    # include/qwen3_model_ops.h
    "qwen3_add_rms_norm_bf16": (
        _i,
        [_vp, _i64, _vp, _i64, _vp, _i64, _vp, ctypes.c_float, _vp, _i64,
         _vp, _i64, _i64, _i, _vp],
    ),
    "qwen3_silu_mul_bf16": (_i, [_vp, _i64, _vp, _i64, _i64, _i, _vp]),
    "qwen3_argmax_bf16": (_i, [_vp, _i64, _i64, _i64, _vp, _vp]),
    "qwen3_advance_seq_lens": (_i, [_vp, _i64, _vp, _i, _i, _i, _vp]),
    "qwen3_page_in_bf16": (_i, [_vp, _i64, _i64, _i64, _vp, _i, _vp, _vp, _i64, _i64, _vp]),
    "qwen3_sample_bf16": (_i, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, ctypes.c_uint64, _vp, _vp]),
    "qwen3_sample_workspace_bytes": (ctypes.c_size_t, [_i64, _i64]),
    "qwen3_sample_ws_bf16": (_i, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, ctypes.c_uint64, _vp, _vp,
                                  ctypes.c_size_t, _vp]),
    "qwen3_lm_head_argmax_workspace_bytes": (ctypes.c_size_t, []),
    "qwen3_lm_head_argmax_bf16": (_i, [_vp, _i64, _vp, _i, _vp, ctypes.c_float, _vp, _i64, _i,
                                       _i, _i, _vp, ctypes.c_size_t, _vp, _vp]),
    "qwen3_decode_linear_bf16": (
        _i,
        [_vp, _i64, _vp, _i, _vp, ctypes.c_float, _vp, _i64, _i, _i, _i, _i,
         _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i, _vp],
    ),
    "qwen3_embed_ss_bf16": (_i, [_vp, _vp, _i64, _i64, _i, _i, _vp, _i64, _vp, _vp]),
    "qwen3_decode_qkv_rope_bf16": (
        _i,
        [_vp, _i64, _vp, _i, _vp, ctypes.c_float, _vp, _i64, _i, _i, _i, _i, _i,
         _vp, _vp, ctypes.c_float, _vp, _vp, _i64, _i64, _vp,
         _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _i64, _i, _i,
         _vp, _vp, _i64, _i64, _i64, _vp, _i, _vp],
    ),
}

ABI_VERSION = 9

_lib = None


def load() -> ctypes.CDLL:
    """Loads the library once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python -m qwen3_engine_from_scratch_amd.build` "
                "(or __graft_entry__.build()) first")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.qwen3_attn_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH.name} ABI version {ver}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(rc: int, name: str) -> None:
    if rc != 0:
        msg = load().qwen3_attn_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed with code {rc}: {msg}")


def strides(t: torch.Tensor, dims) -> ctypes.Array:
    return (ctypes.c_int64 * len(dims))(*[t.stride(d) for d in dims])


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_hip(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one HIP device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"the HIP attention kernels need tensors on a GPU (got a tensor on {t.device}); "
                "there is no CPU fallback")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def stream_of(device: torch.device) -> int:
    """torch's current stream on `device` (so graph capture records our launches)."""
    return torch.cuda.current_stream(device).cuda_stream
