"""KV slot-write oracle (numpy, bit-exact).  Test infrastructure only.

The pool is handled as raw uint16 (bf16 bit patterns), so every write is an
exact copy and results compare with ==.
  update_kv_batch_ref  update_kv_batch_kernel, qwen3/kernels/paged_attention.py:324-350
                       (row = row_ids[b], pos = seq_lens[row],
                        phys = block_table[row, pos // bs], off = pos % bs)
  paged_update_ref     PagedKVCache.update, qwen3/PagedKVcache.py:197-214
                       (pos = seq_len .. seq_len+S-1 through one table row)
  slots_write_ref      slot = phys * bs + off per token, negative = skipped
  gather_tokens        the independent read path (PagedKVCache.get_kv,
                       qwen3/PagedKVcache.py:164-175) used to pin the writes
"""
from __future__ import annotations

import numpy as np


def as_u16(t) -> np.ndarray:
    """bf16 torch tensor -> uint16 numpy view of its bits (copy on CPU)."""
    import torch

    return t.detach().cpu().contiguous().view(torch.uint16).numpy()


def update_kv_batch_ref(k_new: np.ndarray, v_new: np.ndarray, k_buf: np.ndarray,
                        v_buf: np.ndarray, seq_lens: np.ndarray, block_table: np.ndarray,
                        row_ids: np.ndarray, layer: int) -> None:
    """In place.  k_new/v_new (B, Hkv, D); k_buf/v_buf (num_blocks, layers, Hkv, bs, D)."""
    bs = k_buf.shape[3]
    for b in range(k_new.shape[0]):
        row = int(row_ids[b])
        pos = int(seq_lens[row])
        phys = int(block_table[row, pos // bs])
        off = pos % bs
        k_buf[phys, layer, :, off, :] = k_new[b]
        v_buf[phys, layer, :, off, :] = v_new[b]


def paged_update_ref(k_new: np.ndarray, v_new: np.ndarray, k_buf: np.ndarray,
                     v_buf: np.ndarray, table_row: np.ndarray, start_pos: int,
                     layer: int) -> None:
    """In place.  k_new/v_new (S, Hkv, D) token-major."""
    bs = k_buf.shape[3]
    pos = np.arange(start_pos, start_pos + k_new.shape[0])
    phys = table_row[pos // bs].astype(np.int64)
    off = pos % bs
    # numpy fancy assignment: (S,) x (S,) pairs select (S, Hkv, D) targets.
    k_buf[phys, layer, :, off, :] = k_new
    v_buf[phys, layer, :, off, :] = v_new


def slots_write_ref(k_new: np.ndarray, v_new: np.ndarray, k_buf: np.ndarray,
                    v_buf: np.ndarray, slot_mapping: np.ndarray, layer: int) -> None:
    """In place.  k_new/v_new (T, Hkv, D); slot < 0 skips the token."""
    bs = k_buf.shape[3]
    for t, slot in enumerate(slot_mapping.tolist()):
        if slot < 0:
            continue
        k_buf[slot // bs, layer, :, slot % bs, :] = k_new[t]
        v_buf[slot // bs, layer, :, slot % bs, :] = v_new[t]


def gather_tokens(buf: np.ndarray, layer: int, table_row: np.ndarray, L: int) -> np.ndarray:
    """Tokens 0..L-1 of one request: concatenate its pages in logical order
    and cut at L -> (Hkv, L, D)."""
    bs = buf.shape[3]
    n = (L + bs - 1) // bs
    if n == 0:
        return buf[:0, layer].reshape(buf.shape[2], 0, buf.shape[4])
    pages = [buf[int(table_row[j]), layer] for j in range(n)]
    return np.concatenate(pages, axis=1)[:, :L, :]
