"""Paged KV cache: one shared physical block pool plus per-request handles.

Drop-in for qwen3/PagedKVcache.py of the reference engine.  Host-side
bookkeeping (free lists, row slots, page reservation, sequence lengths) keeps
the reference's semantics line for line in behaviour; the two device writes
go to HIP kernels:
  KVCachePool.update_kv_batch -> qwen3_kv_write_decode_bf16
  PagedKVCache.update         -> qwen3_kv_write_range_bf16
and the batched prefill write, which the reference runs as a per-request
loop of PagedKVCache.update (qwen3/attention.py:160-161), is one
slot-mapped launch (write_prefill_batch / qwen3_kv_write_slots_bf16).

Pool layout (num_blocks, num_layers, num_kv_heads, block_size, head_dim):
one (block, layer, head) chunk is block_size * head_dim contiguous bf16
(4 KiB at 16 x 128), the unit the decode kernel streams.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .kernels.paged_attention import update_kv_batch_hip

__all__ = ["KVCachePool", "PagedKVCache", "prefill_slot_mapping", "write_prefill_batch",
           "reserve_pages_bulk", "set_seq_lens_bulk", "PageIn"]


class KVCachePool:
    """Process-wide physical block pool shared by all requests
    (reference: qwen3/PagedKVcache.py:19-114)."""

    def __init__(self, num_blocks: int, num_layers: int, block_size: int,
                 num_kv_heads: int, head_dim: int, device=None, dtype=None,
                 max_seq_len: int = 2048, max_requests: int = 256):
        self.num_layers = num_layers
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len

        max_pages = (max_seq_len + block_size - 1) // block_size
        self.block_table_2d = torch.full(
            (max_requests, max_pages), -1, dtype=torch.int32, device=device)
        self.seq_lens = torch.zeros(max_requests, dtype=torch.int32, device=device)
        self._free_rows = list(range(max_requests))
        self.max_requests = max_requests

        # Zero-initialised so never-written slots cannot hold NaN/inf.
        self.k_buffer = torch.zeros(num_blocks, num_layers, num_kv_heads,
                                    block_size, head_dim, device=device, dtype=dtype)
        self.v_buffer = torch.zeros(num_blocks, num_layers, num_kv_heads,
                                    block_size, head_dim, device=device, dtype=dtype)

        self.free_block_ids = list(range(num_blocks))
        self.total_blocks = num_blocks

    def alloc(self, n: int):
        """Pops n block ids (LIFO from the tail) and zeroes their K/V, so a
        request never reads another request's stale tokens (:58-73)."""
        if len(self.free_block_ids) < n:
            raise RuntimeError(
                f"OOM: requested {n} blocks, {len(self.free_block_ids)} / {self.total_blocks} free")
        allocated = self.free_block_ids[-n:]
        del self.free_block_ids[-n:]
        if allocated:
            idx = torch.tensor(allocated, dtype=torch.long, device=self.k_buffer.device)
            self.k_buffer.index_fill_(0, idx, 0)
            self.v_buffer.index_fill_(0, idx, 0)
        return allocated

    def take_blocks(self, n: int) -> list:
        """Pops n block ids like alloc, without touching the device: the
        caller zeroes them (PageIn does, batched)."""
        if len(self.free_block_ids) < n:
            raise RuntimeError(
                f"OOM: requested {n} blocks, {len(self.free_block_ids)} / {self.total_blocks} free")
        allocated = self.free_block_ids[-n:]
        del self.free_block_ids[-n:]
        return allocated

    def free(self, block_ids: list):
        self.free_block_ids.extend(block_ids)

    @property
    def free_count(self):
        return len(self.free_block_ids)

    def alloc_row(self) -> int:
        """Reserves a resident-table row for a new request; its seq_len is
        reset to 0 (:85-93)."""
        if not self._free_rows:
            raise RuntimeError(
                f"OOM: request rows exhausted (max_requests={self.max_requests}); "
                "raise KVCachePool(max_requests=...)")
        row = self._free_rows.pop()
        self.seq_lens[row] = 0
        return row

    def free_row(self, row: int):
        self._free_rows.append(row)

    def update_kv_batch(self, layer_idx: int, k_new: torch.Tensor, v_new: torch.Tensor,
                        row_ids: torch.Tensor):
        """Decode write of one token per request (:99-114).

        k_new, v_new: (B, num_kv_heads, 1, head_dim); row_ids: (B,) int32.
        Pages must already be reserved (reserve_next) for this step.
        """
        update_kv_batch_hip(k_new.squeeze(2), v_new.squeeze(2), self.k_buffer, self.v_buffer,
                            self.seq_lens, self.block_table_2d, row_ids, layer_idx)


class PagedKVCache:
    """Per-request handle over the shared pool (reference:
    qwen3/PagedKVcache.py:117-228)."""

    def __init__(self, pool: KVCachePool):
        self._pool = pool
        self.seq_len = 0
        self.block_table = []
        self.row_id = pool.alloc_row()
        self.block_table_tensor = pool.block_table_2d[self.row_id]
        self.num_pages = 0

    def _allocate_block(self):
        max_pages = self.block_table_tensor.shape[0]
        assert self.num_pages < max_pages, \
            f"request exceeds max_seq_len ({self._pool.max_seq_len} tokens / {max_pages} pages)"
        new = self._pool.alloc(1)
        self.block_table.append(new[0])
        self.block_table_tensor[self.num_pages] = new[0]
        self.num_pages += 1

    def reserve_next(self):
        """Reserves the page the next decode token lands in (:152-162)."""
        need = (self.seq_len + 1 + self._pool.block_size - 1) // self._pool.block_size
        if need > self.num_pages:
            self._allocate_block()

    def get_kv(self, layer_idx: int):
        """All cached K, V of a layer as (1, Hkv, seq_len, D) (:164-175)."""
        if self.seq_len == 0 or not self.block_table:
            return None, None
        k_pages = [self._pool.k_buffer[pid, layer_idx] for pid in self.block_table]
        v_pages = [self._pool.v_buffer[pid, layer_idx] for pid in self.block_table]
        k = torch.cat(k_pages, dim=1)[:, :self.seq_len, :]
        v = torch.cat(v_pages, dim=1)[:, :self.seq_len, :]
        return k.unsqueeze(0), v.unsqueeze(0)

    def update(self, layer_idx: int, k_new: torch.Tensor, v_new: torch.Tensor):
        """Writes S_new tokens at positions seq_len .. seq_len+S_new-1 (:177-214).

        k_new, v_new: (B, num_kv_heads, S_new, head_dim); as in the reference
        only batch row 0 is written.  Pages are reserved first.
        """
        _, _, S_new, _ = k_new.shape
        pool = self._pool
        end_pos = self.seq_len + S_new
        need_blocks = (end_pos + pool.block_size - 1) // pool.block_size
        while len(self.block_table) < need_blocks:
            self._allocate_block()
        if S_new == 0:
            return
        assert 0 <= layer_idx < pool.num_layers
        k0 = k_new[0].transpose(0, 1)  # (S_new, Hkv, D) view
        v0 = v_new[0].transpose(0, 1)
        if k0.stride(2) != 1:
            k0 = k0.contiguous()
        if v0.stride(2) != 1:
            v0 = v0.contiguous()
        dev = _lib.require_hip(k0, v0, pool.k_buffer)
        lib = _lib.load()
        rc = lib.qwen3_kv_write_range_bf16(
            k0.data_ptr(), _lib.strides(k0, (0, 1)),
            v0.data_ptr(), _lib.strides(v0, (0, 1)),
            pool.k_buffer.data_ptr(), _lib.strides(pool.k_buffer, (0, 1, 2, 3)),
            pool.v_buffer.data_ptr(), _lib.strides(pool.v_buffer, (0, 1, 2, 3)),
            pool.k_buffer.shape[0], int(layer_idx), pool.k_buffer.shape[1],
            self.block_table_tensor.data_ptr(), self.num_pages,
            self.seq_len, S_new, pool.num_kv_heads, pool.head_dim, pool.block_size,
            _lib.stream_of(dev))
        _lib.check(rc, "qwen3_kv_write_range_bf16")

    def reserve_slots(self, n: int):
        """Reserves the pages of positions seq_len .. seq_len + n - 1 (as
        update does, :186-190) and returns their pool slots, block *
        block_size + offset, as an int64 numpy array."""

        bs = self._pool.block_size
        end = self.seq_len + n
        while len(self.block_table) < (end + bs - 1) // bs:
            self._allocate_block()
        p = np.arange(self.seq_len, end, dtype=np.int64)
        table = np.asarray(self.block_table, dtype=np.int64)
        return table[p // bs] * bs + p % bs

    def advance_seq_len(self, n: int = 1):
        self.seq_len += n
        self._pool.seq_lens[self.row_id] = self.seq_len

    def free(self):
        if self.block_table:
            self._pool.free(self.block_table)
            self.block_table = []
            self.num_pages = 0
        self.seq_len = 0
        self._pool.free_row(self.row_id)


class PageIn:
    """Batched page reservation with no host synchronisation: new blocks are
    taken on the host, and their table entries plus the zeroing of their K/V
    go to the device as one asynchronous copy from pinned memory and one
    launch (qwen3_page_in_bf16).  Two pinned staging buffers alternate, so a
    buffer is rewritten only after the copy of the call before the previous
    one has run (the caller synchronises once per step, as the engine does)."""

    def __init__(self, pool: KVCachePool, capacity: int):
        assert pool.k_buffer.is_contiguous() and pool.v_buffer.is_contiguous()
        self.pool = pool
        self.cap = capacity
        self._host = [torch.empty(3 * capacity, dtype=torch.int32, pin_memory=True)
                      for _ in range(2)]
        self._dev = torch.empty(3 * capacity, dtype=torch.int32, device=pool.k_buffer.device)
        self._flip = 0

    def reserve(self, caches, tokens) -> int:
        """Gives every handle enough pages for tokens[i] tokens; returns the
        number of blocks mapped."""
        pool = self.pool
        bs = pool.block_size
        max_pages = pool.block_table_2d.shape[1]
        want = []
        for c, n in zip(caches, tokens):
            k = (int(n) + bs - 1) // bs - c.num_pages
            if k > 0:
                assert c.num_pages + k <= max_pages, \
                    f"request exceeds max_seq_len ({pool.max_seq_len} tokens / {max_pages} pages)"
                want.append((c, k))
        total = sum(k for _, k in want)
        if total == 0:
            return 0
        assert total <= self.cap, f"{total} new pages in one step (staging holds {self.cap})"
        ids = pool.take_blocks(total)
        h = self._host[self._flip]
        self._flip ^= 1
        # rows | page columns | block ids, filled through a numpy view of the
        # pinned buffer (element-wise tensor writes cost microseconds each)
        hn = h.numpy()
        counts = [k for _, k in want]
        hn[:total] = np.repeat([c.row_id for c, _ in want], counts)
        hn[total:2 * total] = np.concatenate(
            [np.arange(c.num_pages, c.num_pages + k) for c, k in want])
        hn[2 * total:3 * total] = ids
        i = 0
        for c, k in want:
            c.block_table.extend(ids[i:i + k])
            c.num_pages += k
            i += k
        d = self._dev[:3 * total]
        d.copy_(h[:3 * total], non_blocking=True)
        bt = pool.block_table_2d
        kb = pool.k_buffer
        rc = _lib.load().qwen3_page_in_bf16(
            bt.data_ptr(), bt.stride(0), bt.shape[0], bt.shape[1], d.data_ptr(), total,
            kb.data_ptr(), pool.v_buffer.data_ptr(), kb[0].numel(), kb.shape[0],
            _lib.stream_of(kb.device))
        _lib.check(rc, "qwen3_page_in_bf16")
        return total


def reserve_pages_bulk(caches, tokens: list) -> None:
    """Gives every handle enough pages for tokens[i] tokens with one pool
    allocation (one zeroing launch) and one block-table write for the whole
    batch, instead of a device write per page (_allocate_block).  Used by the
    batching engine once per step."""
    pool = caches[0]._pool
    bs = pool.block_size
    max_pages = pool.block_table_2d.shape[1]
    want = []
    for c, n in zip(caches, tokens):
        k = (int(n) + bs - 1) // bs - c.num_pages
        if k > 0:
            assert c.num_pages + k <= max_pages, \
                f"request exceeds max_seq_len ({pool.max_seq_len} tokens / {max_pages} pages)"
            want.append((c, k))
    total = sum(k for _, k in want)
    if total == 0:
        return
    ids = pool.alloc(total)
    rows, cols, vals = [], [], []
    for c, k in want:
        new, ids = ids[:k], ids[k:]
        rows += [c.row_id] * k
        cols += range(c.num_pages, c.num_pages + k)
        vals += new
        c.block_table.extend(new)
        c.num_pages += k
    idx = torch.tensor([rows, cols, vals], dtype=torch.int64).to(pool.block_table_2d.device)
    pool.block_table_2d.index_put_((idx[0], idx[1]), idx[2].to(torch.int32))


def set_seq_lens_bulk(caches) -> None:
    """Writes every handle's host seq_len into the resident seq_lens table
    with one copy (the batched form of advance_seq_len's device write)."""
    pool = caches[0]._pool
    idx = torch.tensor([[c.row_id for c in caches], [c.seq_len for c in caches]],
                       dtype=torch.int64).to(pool.seq_lens.device)
    pool.seq_lens.index_put_((idx[0],), idx[1].to(torch.int32))


def prefill_slot_mapping(caches, S: int, device) -> torch.Tensor:
    """Slot of every (request, padded position) of a right-padded prefill
    batch: the reference's per-request update writes all S positions from
    each request's seq_len (pads included, qwen3/attention.py:160-161), so the
    mapping covers them too.  Reserves the pages the same way."""
    bs = caches[0]._pool.block_size
    slots = np.empty((len(caches), S), dtype=np.int64)
    pos = np.arange(S, dtype=np.int64)
    for i, c in enumerate(caches):
        end_pos = c.seq_len + S
        need = (end_pos + bs - 1) // bs
        while len(c.block_table) < need:
            c._allocate_block()
        p = c.seq_len + pos
        table = np.asarray(c.block_table, dtype=np.int64)
        slots[i] = table[p // bs] * bs + p % bs
    return torch.from_numpy(slots.reshape(-1)).to(device, non_blocking=False)


def write_prefill_batch(caches, layer_idx: int, k: torch.Tensor, v: torch.Tensor,
                        slot_mapping: torch.Tensor | None = None):
    """One-launch equivalent of `for i, c in enumerate(caches): c.update(layer_idx,
    k[i:i+1], v[i:i+1])` (qwen3/attention.py:160-161).

    k, v: (B, Hkv, S, D).  `slot_mapping` (B*S,) int64 from prefill_slot_mapping
    can be built once per step and shared by every layer.
    """
    B, Hkv, S, D = k.shape
    pool = caches[0]._pool
    if slot_mapping is None:
        slot_mapping = prefill_slot_mapping(caches, S, k.device)
    assert slot_mapping.dtype == torch.int64 and slot_mapping.numel() == B * S
    assert 0 <= layer_idx < pool.num_layers
    # (B, Hkv, S, D) -> token-major (B*S, Hkv, D) view when strides allow.
    kt = k.transpose(1, 2).reshape(B * S, Hkv, D)
    vt = v.transpose(1, 2).reshape(B * S, Hkv, D)
    dev = _lib.require_hip(kt, vt, pool.k_buffer, slot_mapping)
    lib = _lib.load()
    rc = lib.qwen3_kv_write_slots_bf16(
        kt.data_ptr(), _lib.strides(kt, (0, 1)),
        vt.data_ptr(), _lib.strides(vt, (0, 1)),
        pool.k_buffer.data_ptr(), _lib.strides(pool.k_buffer, (0, 1, 2, 3)),
        pool.v_buffer.data_ptr(), _lib.strides(pool.v_buffer, (0, 1, 2, 3)),
        pool.k_buffer.shape[0], int(layer_idx), pool.k_buffer.shape[1],
        slot_mapping.contiguous().data_ptr(), B * S,
        Hkv, D, pool.block_size, _lib.stream_of(dev))
    _lib.check(rc, "qwen3_kv_write_slots_bf16")
