"""Fused pre-attention step on the gfx950 HIP kernel: QK-RMSNorm + RoPE + the
K/V pool write, one launch per layer.

The reference runs these as separate PyTorch / Triton steps between the QKV
projection and attention (qwen3/attention.py:91-96: q_norm, k_norm,
apply_rotary_pos_emb; then update_kv_batch_triton for decode,
qwen3/kernels/paged_attention.py:353-377, or PagedKVCache.update for
prefill, qwen3/PagedKVcache.py:177-214).  The arithmetic, including its
bf16 roundings, is the reference's (include/qwen3_attn.h states it); the
RoPE tables are the model's own fp32 cos/sin tables (qwen3/rope.py:42-58).
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["qk_norm_rope_decode", "qk_norm_rope_prefill", "rope_tables"]


def rope_tables(head_dim: int, base: float = 1e6, max_seq_len: int = 4096, device=None):
    """The model's fp32 cos/sin tables (max_seq_len, head_dim), as
    RotaryEmbedding builds them (qwen3/rope.py:42-58): inverse frequencies
    base^(-2i/head_dim), their outer product with the positions, repeated
    for both halves.  Computed on the CPU (like the reference's buffers) and
    moved to `device`."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32,
                                            device="cpu") / head_dim))
    positions = torch.arange(max_seq_len, dtype=torch.float32, device="cpu")
    freqs = torch.einsum("s,d->sd", positions, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    cos, sin = emb.cos(), emb.sin()
    if device is not None:
        cos, sin = cos.to(device), sin.to(device)
    return cos, sin


def _check_common(q, k, v, q_norm_weight, k_norm_weight, cos_table, sin_table):
    assert q.dtype == k.dtype == v.dtype == torch.bfloat16, "bf16 only"
    assert q_norm_weight.dtype == k_norm_weight.dtype == torch.bfloat16
    assert cos_table.dtype == sin_table.dtype == torch.float32
    assert cos_table.shape == sin_table.shape and cos_table.stride() == sin_table.stride()
    assert cos_table.stride(1) == 1 and q_norm_weight.is_contiguous() and k_norm_weight.is_contiguous()
    for t in (q, k, v):
        assert t.dim() == 3 and t.stride(2) == 1, "q/k/v must be (tokens, heads, head_dim) views"


def qk_norm_rope_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, eps: float,
                        cos_table: torch.Tensor, sin_table: torch.Tensor, pool, layer_idx: int,
                        row_ids: torch.Tensor | None = None,
                        out: torch.Tensor | None = None,
                        positions: torch.Tensor | None = None) -> torch.Tensor:
    """Decode step of one layer: returns the normalised, rotated q
    (B, Hq, D) and writes normalised, rotated k and raw v into `pool`
    (a KVCachePool) at position seq_lens[row], the position RoPE uses too
    (qwen3/model.py:76-78; qwen3/kernels/paged_attention.py:324-350).

    q: (B, Hq, D), k/v: (B, Hkv, D) bf16 views, e.g. slices of the fused
    QKV projection output; row_ids: int32 (B,) rows of pool.block_table_2d
    (None: row b for token b).  Pages must already be reserved.
    positions: int64 (B,) RoPE positions (the reference's position_ids);
    None rotates at seq_lens[row], the write position, which is what the
    reference's drivers pass.
    """
    _check_common(q, k, v, q_norm_weight, k_norm_weight, cos_table, sin_table)
    B, Hq, D = q.shape
    Hkv = k.shape[1]
    kb, vb = pool.k_buffer, pool.v_buffer
    dev = _lib.require_hip(q, k, v, q_norm_weight, kb, cos_table)
    if out is None:
        out = torch.empty(B, Hq, D, dtype=q.dtype, device=q.device)
    bt = pool.block_table_2d
    if row_ids is not None:
        assert row_ids.dtype == torch.int32 and row_ids.numel() == B
        row_ids = row_ids.contiguous()
    if positions is not None:
        assert positions.dtype == torch.int64 and positions.numel() == B
        positions = positions.reshape(-1)
        if positions.stride(0) != 1:
            positions = positions.contiguous()
    rc = _lib.load().qwen3_qk_norm_rope_decode_bf16(
        q.data_ptr(), _lib.strides(q, (0, 1)), k.data_ptr(), _lib.strides(k, (0, 1)),
        v.data_ptr(), _lib.strides(v, (0, 1)), q_norm_weight.data_ptr(),
        k_norm_weight.data_ptr(), float(eps), cos_table.data_ptr(), sin_table.data_ptr(),
        cos_table.stride(0), cos_table.shape[0],
        out.data_ptr(), _lib.strides(out, (0, 1)),
        kb.data_ptr(), _lib.strides(kb, (0, 1, 2, 3)), vb.data_ptr(), _lib.strides(vb, (0, 1, 2, 3)),
        kb.shape[0], int(layer_idx), kb.shape[1], pool.seq_lens.data_ptr(), bt.data_ptr(), bt.stride(0),
        bt.shape[0], bt.shape[1], _lib.ptr(row_ids), _lib.ptr(positions), B, Hq, Hkv, D,
        kb.shape[3],
        _lib.stream_of(dev))
    _lib.check(rc, "qwen3_qk_norm_rope_decode_bf16")
    return out


def qk_norm_rope_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, eps: float,
                         cos_table: torch.Tensor, sin_table: torch.Tensor,
                         positions: torch.Tensor, slot_mapping: torch.Tensor | None,
                         k_buffer: torch.Tensor, v_buffer: torch.Tensor, layer_idx: int,
                         q_out: torch.Tensor | None = None,
                         k_out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Prefill step of one layer over T packed tokens: returns the normalised,
    rotated (q, k) as (T, Hq, D) and (T, Hkv, D) for the varlen prefill kernel
    and writes k and raw v into the pool at slot_mapping[t] (int64 block *
    block_size + offset; negative entries, or no mapping, write nothing).
    positions: int64 (T,) RoPE positions (0..L-1 within each sequence for a
    fresh prefill, qwen3/model.py:132-136).
    """
    _check_common(q, k, v, q_norm_weight, k_norm_weight, cos_table, sin_table)
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    assert positions.dtype == torch.int64 and positions.numel() == T
    positions = positions.contiguous()
    if slot_mapping is not None:
        assert slot_mapping.dtype == torch.int64 and slot_mapping.numel() == T
        slot_mapping = slot_mapping.contiguous()
    dev = _lib.require_hip(q, k, v, q_norm_weight, k_buffer, cos_table, positions)
    if q_out is None:
        q_out = torch.empty(T, Hq, D, dtype=q.dtype, device=q.device)
    if k_out is None:
        k_out = torch.empty(T, Hkv, D, dtype=q.dtype, device=q.device)
    rc = _lib.load().qwen3_qk_norm_rope_slots_bf16(
        q.data_ptr(), _lib.strides(q, (0, 1)), k.data_ptr(), _lib.strides(k, (0, 1)),
        v.data_ptr(), _lib.strides(v, (0, 1)), q_norm_weight.data_ptr(),
        k_norm_weight.data_ptr(), float(eps), cos_table.data_ptr(), sin_table.data_ptr(),
        cos_table.stride(0), cos_table.shape[0], positions.data_ptr(), _lib.ptr(slot_mapping),
        q_out.data_ptr(), _lib.strides(q_out, (0, 1)), k_out.data_ptr(), _lib.strides(k_out, (0, 1)),
        k_buffer.data_ptr(), _lib.strides(k_buffer, (0, 1, 2, 3)),
        v_buffer.data_ptr(), _lib.strides(v_buffer, (0, 1, 2, 3)),
        k_buffer.shape[0], int(layer_idx), k_buffer.shape[1], T, Hq, Hkv, D, k_buffer.shape[3], _lib.stream_of(dev))
    _lib.check(rc, "qwen3_qk_norm_rope_slots_bf16")
    return q_out, k_out
