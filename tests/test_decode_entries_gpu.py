"""The reference's two decode entry points above the bare kernel, on the GPU:

  triton_paged_attention_decode        (qwen3/kernels/paged_attention.py:181-219)
      one request: write the step's K/V at seq_len, then attend seq_len + 1
      tokens; returns (B, 1, Hq*D); does not advance seq_len.
  triton_paged_attention_decode_batch  (:222-289) with row_ids=None
      the direct-call fallback (:257-264): reserve the next page of every
      handle and build row_ids itself.

Checked against the fp64 closed form over the pool contents the call leaves
(the write itself bit-exact against the numpy oracle), and the fallback
against the row_ids path of the same entry point.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from gpu_helpers import assert_close_attn
from oracle import decode as od
from oracle import kv_write as okw

pytestmark = pytest.mark.gpu

HQ, HKV, D, BS = 16, 8, 128, 16


def _pool(gpu, blocks=64, layers=3, max_requests=8):
    from qwen3_engine_from_scratch_amd.PagedKVcache import KVCachePool

    return KVCachePool(blocks, layers, BS, HKV, D, device=gpu, dtype=torch.bfloat16,
                       max_seq_len=1024, max_requests=max_requests)


def _prefilled(pool, lengths, layer, g):
    """Handles with `lengths` tokens of random K/V in `layer` (written with
    the range form, PagedKVCache.update) and seq_len advanced past them."""
    from qwen3_engine_from_scratch_amd.PagedKVcache import PagedKVCache

    caches = []
    for L in lengths:
        c = PagedKVCache(pool)
        k = torch.randn(1, HKV, L, D, generator=g).to(torch.bfloat16).to(pool.k_buffer.device)
        v = torch.randn(1, HKV, L, D, generator=g).to(torch.bfloat16).to(pool.k_buffer.device)
        c.update(layer, k, v)
        c.advance_seq_len(L)
        caches.append(c)
    return caches


def _dense_ref(pool, layer, caches, q):
    """fp64 softmax(q K^T / sqrt(D)) V over seq_len + 1 tokens of each handle,
    read from the pool through the host copy of its table."""
    kl = pool.k_buffer[:, layer].cpu()
    vl = pool.v_buffer[:, layer].cpu()
    mp = max(len(c.block_table) for c in caches)
    bt = torch.full((len(caches), mp), -1, dtype=torch.int32)
    for i, c in enumerate(caches):
        bt[i, :len(c.block_table)] = torch.tensor(c.block_table, dtype=torch.int32)
    sl = torch.tensor([c.seq_len for c in caches], dtype=torch.int32)
    return od.dense_decode_ref(q.cpu(), kl, vl, bt, sl, None, BS)


@pytest.mark.parametrize("name", ["hip_paged_attention_decode", "triton_paged_attention_decode"])
@pytest.mark.parametrize("L", [1, 16, 37, 300])
def test_single_request_decode_entry(gpu, name, L):
    from qwen3_engine_from_scratch_amd.kernels import paged_attention as pa

    fn = getattr(pa, name)
    g = torch.Generator().manual_seed(L)
    pool = _pool(gpu)
    _prefilled(pool, [23], 1, g)  # another request: the whole-pool compare covers its pages
    (c,) = _prefilled(pool, [L], 1, g)
    c.reserve_next()
    q = torch.randn(1, HQ, 1, D, generator=g).to(torch.bfloat16).to(gpu)
    qkv = torch.randn(1, HQ + 2 * HKV, 1, D, generator=g).to(torch.bfloat16).to(gpu)
    k_new, v_new = qkv[:, HQ:HQ + HKV], qkv[:, HQ + HKV:]  # fused-QKV slices
    ek, ev = okw.as_u16(pool.k_buffer), okw.as_u16(pool.v_buffer)
    table = np.asarray(c.block_table, np.int32)
    okw.paged_update_ref(okw.as_u16(k_new[0].transpose(0, 1)), okw.as_u16(v_new[0].transpose(0, 1)),
                         ek, ev, table, L, 1)
    announce(f"{name} L={L}")
    out = fn(q, k_new, v_new, c, 1, D ** -0.5)
    torch.cuda.synchronize()
    assert out.shape == (1, 1, HQ * D) and out.dtype == torch.bfloat16
    assert c.seq_len == L, "the entry point must not advance seq_len"
    assert np.array_equal(okw.as_u16(pool.k_buffer), ek), "K write not bit-exact"
    assert np.array_equal(okw.as_u16(pool.v_buffer), ev), "V write not bit-exact"
    ref = _dense_ref(pool, 1, [c], q[:, :, 0])
    assert_close_attn(out.view(1, HQ, D), ref, f"{name} L={L}")


def test_batch_entry_row_ids_none_fallback(gpu):
    """row_ids=None reserves each handle's next page itself (:257-264) and
    gives the bits of the row_ids path run on an identical pool."""
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import (
        triton_paged_attention_decode_batch)

    lens = [15, 16, 1, 47, 160]  # 16 and 160: the new token opens a page
    outs, pools, handles = [], [], []
    for use_rows in (False, True):
        g = torch.Generator().manual_seed(9)
        pool = _pool(gpu, blocks=96)
        caches = _prefilled(pool, lens, 2, g)
        q = torch.randn(len(lens), HQ, 1, D, generator=g).to(torch.bfloat16).to(gpu)
        k_new = torch.randn(len(lens), HKV, 1, D, generator=g).to(torch.bfloat16).to(gpu)
        v_new = torch.randn(len(lens), HKV, 1, D, generator=g).to(torch.bfloat16).to(gpu)
        pages_before = [c.num_pages for c in caches]
        rows = None
        if use_rows:
            for c in caches:
                c.reserve_next()
            rows = torch.tensor([c.row_id for c in caches], dtype=torch.int32, device=gpu)
        announce(f"decode batch entry row_ids={'given' if use_rows else 'None'} lens={lens}")
        out = triton_paged_attention_decode_batch(q, k_new, v_new, caches, 2, D ** -0.5,
                                                  row_ids=rows)
        torch.cuda.synchronize()
        assert [c.num_pages for c in caches] == [(L + 1 + BS - 1) // BS for L in lens]
        assert [c.num_pages - p for c, p in zip(caches, pages_before)] == \
            [int(L % BS == 0) for L in lens]
        assert out.shape == (len(lens), 1, HQ * D)
        assert_close_attn(out.view(len(lens), HQ, D), _dense_ref(pool, 2, caches, q[:, :, 0]),
                          f"batch entry rows={use_rows}")
        outs.append(out.cpu())
        pools.append((pool.k_buffer.cpu(), pool.v_buffer.cpu()))
        handles.append([c.block_table for c in caches])
    assert handles[0] == handles[1], "fallback reserved different pages"
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(pools[0][0], pools[1][0]) and torch.equal(pools[0][1], pools[1][1])
