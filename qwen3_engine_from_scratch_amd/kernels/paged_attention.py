"""Paged decode attention and decode K/V write on gfx950 HIP kernels.

Drop-in for qwen3/kernels/paged_attention.py of the reference engine: the
function names, argument meanings, shapes, asserts and return contracts
are the reference's (file:line cited per function); the device work is the
HIP kernels behind include/qwen3_attn.h.  The reference's `triton_*` names
are kept as aliases so its call sites (qwen3/attention.py:27,
qwen3/PagedKVcache.py:16) resolve unchanged.
"""
from __future__ import annotations

import math

import torch

from .. import _lib

__all__ = [
    "paged_attention_decode_hip",
    "hip_paged_attention_decode",
    "hip_paged_attention_decode_batch",
    "update_kv_batch_hip",
    "paged_decode_workspace_bytes",
    # reference names
    "paged_attention_decode_triton",
    "triton_paged_attention_decode",
    "triton_paged_attention_decode_batch",
    "update_kv_batch_triton",
]


_INV_WORKSPACES: dict = {}
# Workspaces replaced by a larger one stay allocated: a graph captured
# earlier holds the old address and may still be replayed.
_SUPERSEDED: list = []


def _invariant_workspace(dev, stream: int, num_kv_heads: int, need: int) -> torch.Tensor:
    """The batch-invariant decode's workspace kept for this device, stream and
    KV-head count, grown as needed, zeroed when allocated (its hand-off
    tickets start at zero and every call leaves them there).  One per stream:
    calls on different streams may run at the same time and must not share
    tickets."""
    key = (str(dev), stream, num_kv_heads)
    ws = _INV_WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        if ws is not None:
            _SUPERSEDED.append(ws)
        ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=dev)
        _INV_WORKSPACES[key] = ws
    return ws


def paged_decode_workspace_bytes(batch: int, num_heads: int, num_kv_heads: int, head_dim: int,
                                 max_pages: int, block_size: int, *,
                                 batch_invariant: bool = False) -> int:
    """Workspace size of the decode on the current device; depends only on
    the launch shape, so a graph captured once stays valid for any live
    context lengths.  batch_invariant: the size for the batch-invariant
    kernel (one slot per 256-token partition of every (row, KV head) at the
    table's full row length, after the hand-off tickets)."""
    lib = _lib.load()
    fn = (lib.qwen3_paged_decode_invariant_workspace_bytes if batch_invariant
          else lib.qwen3_paged_decode_workspace_bytes)
    return int(fn(batch, num_heads, num_kv_heads, head_dim, max_pages, block_size))


def paged_attention_decode_hip(q, k_buffer, v_buffer, block_table_2d,
                               seq_lens_full, row_ids, block_size, *,
                               seq_len_bias: int = 1, scale: float | None = None,
                               out: torch.Tensor | None = None,
                               workspace: torch.Tensor | None = None,
                               batch_invariant: bool = False):
    """Bare kernel entry (reference: paged_attention_decode_triton,
    qwen3/kernels/paged_attention.py:132-178).

    q:              (B, num_heads, head_dim) bf16
    k_buffer/v_buffer: (num_blocks, num_kv_heads, block_size, head_dim) bf16,
                    the per-layer view pool.k_buffer[:, layer] (dim-0 stride
                    carries the layer interleave)
    block_table_2d: (max_requests, max_pages) int32 resident table
    seq_lens_full:  (max_requests,) int32, lengths BEFORE this step
    row_ids:        (B,) int32 rows of this batch (None = 0..B-1)
    Returns out (B, num_heads, head_dim) bf16.  Each sequence attends
    seq_lens_full[row] + seq_len_bias tokens (bias 1 = the reference's
    convention, :55).  The softmax scale is 1/sqrt(head_dim) as the reference
    recomputes it (:161) unless `scale` is given.

    batch_invariant: use the batch-invariant kernel (each sequence's output
    bits independent of the rest of the batch; qwen3_attn.h).  `workspace`:
    paged_decode_workspace_bytes(..., batch_invariant=...) bytes; for the
    batch-invariant kernel its leading ticket region must be zero before its
    first call (every call leaves it zero).  Default: a fresh one per call
    (default kernel) or one per device, stream and KV-head count kept by this
    module (batch-invariant kernel).
    """
    B, num_heads, head_dim = q.shape
    num_blocks, num_kv_heads, block_size_check, head_dim_check = k_buffer.shape
    assert block_size_check == block_size
    assert head_dim_check == head_dim
    assert v_buffer.shape == k_buffer.shape
    assert q.dtype == torch.bfloat16 and k_buffer.dtype == torch.bfloat16 \
        and v_buffer.dtype == torch.bfloat16, "HIP decode kernel is bf16 only"
    assert block_table_2d.dtype == torch.int32 and seq_lens_full.dtype == torch.int32
    assert block_table_2d.dim() == 2 and block_table_2d.stride(1) == 1, \
        "block_table_2d rows must be contiguous"
    dev = _lib.require_hip(q, k_buffer, v_buffer, block_table_2d, seq_lens_full, row_ids)
    if row_ids is not None:
        assert row_ids.dtype == torch.int32 and row_ids.numel() == B
        row_ids = row_ids.contiguous()
    seq_lens_full = seq_lens_full.contiguous()
    if q.stride(2) != 1:
        q = q.contiguous()
    assert k_buffer.stride(3) == 1 and v_buffer.stride(3) == 1
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    if out is None:
        out = torch.empty_like(q)
    else:
        assert out.shape == q.shape and out.dtype == torch.bfloat16 and out.stride(2) == 1, \
            "out must be a bf16 (B, num_heads, head_dim) tensor with unit last stride"
        _lib.require_hip(out)
    max_rows, max_pages = block_table_2d.shape
    need = paged_decode_workspace_bytes(B, num_heads, num_kv_heads, head_dim, max_pages,
                                        block_size, batch_invariant=batch_invariant)
    if workspace is None or workspace.numel() < need:
        if batch_invariant:
            workspace = _invariant_workspace(dev, _lib.stream_of(dev), num_kv_heads, need)
        else:
            workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    lib = _lib.load()
    fn = lib.qwen3_paged_decode_invariant_bf16 if batch_invariant else lib.qwen3_paged_decode_bf16
    rc = fn(
        q.data_ptr(), _lib.strides(q, (0, 1)),
        k_buffer.data_ptr(), _lib.strides(k_buffer, (0, 1, 2)),
        v_buffer.data_ptr(), _lib.strides(v_buffer, (0, 1, 2)),
        num_blocks,
        block_table_2d.data_ptr(), block_table_2d.stride(0), max_rows, max_pages,
        seq_lens_full.data_ptr(), seq_len_bias, _lib.ptr(row_ids),
        out.data_ptr(), _lib.strides(out, (0, 1)),
        B, num_heads, num_kv_heads, head_dim, block_size, float(scale),
        workspace.data_ptr(), workspace.numel(), _lib.stream_of(dev))
    _lib.check(rc, "qwen3_paged_decode_invariant_bf16" if batch_invariant
               else "qwen3_paged_decode_bf16")
    return out


def update_kv_batch_hip(k_new, v_new, k_buffer, v_buffer, seq_lens,
                        block_table_2d, row_ids, layer_idx):
    """Decode K/V write (reference: update_kv_batch_triton,
    qwen3/kernels/paged_attention.py:353-377).

    k_new, v_new: (B, num_kv_heads, head_dim) bf16, may be non-contiguous
                  slices of the fused QKV output (explicit strides, last dim 1)
    k_buffer/v_buffer: the full pool (num_blocks, num_layers, Hkv, bs, D)
    Writes in place at position seq_lens[row_ids[b]]; returns None.
    """
    B, num_kv_heads, head_dim = k_new.shape
    num_blocks, num_layers, _, block_size, _ = k_buffer.shape
    assert v_new.shape == k_new.shape and v_buffer.shape == k_buffer.shape
    assert k_buffer.dtype == torch.bfloat16 and k_new.dtype == torch.bfloat16
    assert 0 <= layer_idx < num_layers, f"layer_idx {layer_idx} out of range [0, {num_layers})"
    assert block_table_2d.dtype == torch.int32 and block_table_2d.stride(1) == 1
    dev = _lib.require_hip(k_new, v_new, k_buffer, v_buffer, seq_lens, block_table_2d, row_ids)
    if k_new.stride(2) != 1:
        k_new = k_new.contiguous()
    if v_new.stride(2) != 1:
        v_new = v_new.contiguous()
    if row_ids is not None:
        assert row_ids.dtype == torch.int32 and row_ids.numel() == B
        row_ids = row_ids.contiguous()
    max_rows, max_pages = block_table_2d.shape
    lib = _lib.load()
    rc = lib.qwen3_kv_write_decode_bf16(
        k_new.data_ptr(), _lib.strides(k_new, (0, 1)),
        v_new.data_ptr(), _lib.strides(v_new, (0, 1)),
        k_buffer.data_ptr(), _lib.strides(k_buffer, (0, 1, 2, 3)),
        v_buffer.data_ptr(), _lib.strides(v_buffer, (0, 1, 2, 3)),
        num_blocks, int(layer_idx), num_layers,
        seq_lens.contiguous().data_ptr(),
        block_table_2d.data_ptr(), block_table_2d.stride(0), max_rows, max_pages,
        _lib.ptr(row_ids), B, num_kv_heads, head_dim, block_size, _lib.stream_of(dev))
    _lib.check(rc, "qwen3_kv_write_decode_bf16")


def hip_paged_attention_decode(q, k_new, v_new, kv_cache, layer_idx, scaling):
    """Single-request decode (reference: triton_paged_attention_decode,
    qwen3/kernels/paged_attention.py:181-219).

    q: (B, Hq, 1, D) bf16; k_new/v_new: (B, Hkv, 1, D); kv_cache: PagedKVCache.
    Writes the new K/V first, then attends; returns (B, 1, Hq*D).
    """
    assert q.shape[2] == 1, "HIP decode kernel handles decode only (S == 1)"
    assert q.dtype == torch.bfloat16, "HIP decode kernel is bf16 only"
    pool = kv_cache._pool
    row_ids = torch.tensor([kv_cache.row_id], dtype=torch.int32, device=q.device)
    pool.update_kv_batch(layer_idx, k_new, v_new, row_ids)
    k_buffer = pool.k_buffer[:, layer_idx]
    v_buffer = pool.v_buffer[:, layer_idx]
    out = paged_attention_decode_hip(
        q.squeeze(2), k_buffer, v_buffer, pool.block_table_2d, pool.seq_lens,
        row_ids, pool.block_size)
    B, num_heads, head_dim = q.shape[0], q.shape[1], q.shape[3]
    return out.reshape(B, 1, num_heads * head_dim)


def hip_paged_attention_decode_batch(q, k_new, v_new, kv_caches, layer_idx, scaling,
                                     row_ids=None):
    """Batched decode, the hot call site (reference:
    triton_paged_attention_decode_batch, qwen3/kernels/paged_attention.py:222-289).

    q: (B, Hq, 1, D) bf16; k_new/v_new: (B, Hkv, 1, D) (non-contiguous fused-QKV
    slices are fine); kv_caches: list[PagedKVCache] of length B; row_ids: (B,)
    int32 resident-table rows, or None to reserve pages and build them here.
    Returns (B, 1, Hq*D).
    """
    assert q.shape[2] == 1, "HIP decode kernel handles decode only (S == 1)"
    assert q.dtype == torch.bfloat16, "HIP decode kernel is bf16 only"
    B = q.shape[0]
    assert len(kv_caches) == B, "kv_caches must have one entry per batch row"
    if row_ids is None:
        for c in kv_caches:
            c.reserve_next()
        row_ids = torch.tensor([c.row_id for c in kv_caches], dtype=torch.int32, device=q.device)
    pool = kv_caches[0]._pool
    pool.update_kv_batch(layer_idx, k_new, v_new, row_ids)
    k_buffer = pool.k_buffer[:, layer_idx]
    v_buffer = pool.v_buffer[:, layer_idx]
    out = paged_attention_decode_hip(
        q.squeeze(2), k_buffer, v_buffer, pool.block_table_2d, pool.seq_lens,
        row_ids, pool.block_size)
    num_heads, head_dim = q.shape[1], q.shape[3]
    return out.reshape(B, 1, num_heads * head_dim)


# Reference names (qwen3/kernels/paged_attention.py) for unchanged imports.
paged_attention_decode_triton = paged_attention_decode_hip
triton_paged_attention_decode = hip_paged_attention_decode
triton_paged_attention_decode_batch = hip_paged_attention_decode_batch
update_kv_batch_triton = update_kv_batch_hip
