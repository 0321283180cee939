"""Decode step (K/V write + paged attention) captured as a hipGraph through
torch.cuda.graph, the way the reference's GraphRunner captures it
(qwen3/graph_runner.py:137-151), replayed several times with new contents in
the static tensors and checked against an eager run after every replay."""
import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu


def _pool_with_requests(dev, lens, num_layers=2, seed=0):
    from qwen3_engine_from_scratch_amd.PagedKVcache import KVCachePool, PagedKVCache

    g = torch.Generator(device=dev).manual_seed(seed)
    pool = KVCachePool(256, num_layers, 16, 8, 128, device=dev, dtype=torch.bfloat16,
                       max_seq_len=1024, max_requests=16)
    caches = []
    for L in lens:
        c = PagedKVCache(pool)
        for layer in range(num_layers):
            k = torch.randn(1, 8, L, 128, generator=g, device=dev, dtype=torch.bfloat16)
            v = torch.randn(1, 8, L, 128, generator=g, device=dev, dtype=torch.bfloat16)
            c.update(layer, k, v)
        c.advance_seq_len(L)
        caches.append(c)
    return pool, caches


def test_decode_graph_replays_match_eager(gpu):
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import hip_paged_attention_decode_batch

    lens = [37, 200, 511, 64, 1]
    steps = 4
    B, Hq, Hkv, D, layer = len(lens), 16, 8, 128, 1
    announce("graph capture of the decode step, 4 replays")
    pool, caches = _pool_with_requests(gpu, lens)
    # Pages for every step are reserved before capture (no allocation inside).
    for c in caches:
        for s in range(steps):
            need = (c.seq_len + s + 1 + 15) // 16
            while c.num_pages < need:
                c._allocate_block()
    rows = torch.tensor([c.row_id for c in caches], dtype=torch.int32, device=gpu)
    q = torch.zeros(B, Hq, 1, D, dtype=torch.bfloat16, device=gpu)
    k_new = torch.zeros(B, Hkv, 1, D, dtype=torch.bfloat16, device=gpu)
    v_new = torch.zeros(B, Hkv, 1, D, dtype=torch.bfloat16, device=gpu)

    def step():
        return hip_paged_attention_decode_batch(q, k_new, v_new, caches, layer, D ** -0.5,
                                                row_ids=rows)

    # warm up eagerly (allocator and library load), then capture
    for _ in range(2):
        step()
    torch.cuda.synchronize()
    kb0, vb0 = pool.k_buffer.clone(), pool.v_buffer.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_static = step()
    torch.cuda.synchronize()
    pool.k_buffer.copy_(kb0)
    pool.v_buffer.copy_(vb0)

    gen = torch.Generator(device=gpu).manual_seed(7)
    for s in range(steps):
        q.copy_(torch.randn(q.shape, generator=gen, device=gpu, dtype=torch.bfloat16))
        k_new.copy_(torch.randn(k_new.shape, generator=gen, device=gpu, dtype=torch.bfloat16))
        v_new.copy_(torch.randn(v_new.shape, generator=gen, device=gpu, dtype=torch.bfloat16))
        kb_before, vb_before = pool.k_buffer.clone(), pool.v_buffer.clone()
        g.replay()
        torch.cuda.synchronize()
        got = out_static.clone()
        kb_graph, vb_graph = pool.k_buffer.clone(), pool.v_buffer.clone()
        # eager on the same starting pool
        pool.k_buffer.copy_(kb_before)
        pool.v_buffer.copy_(vb_before)
        ref = step()
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"replay {s}: output differs from eager"
        assert torch.equal(kb_graph, pool.k_buffer) and torch.equal(vb_graph, pool.v_buffer), \
            f"replay {s}: K/V write differs from eager"
        for c in caches:  # host-side advance between replays, as the engine does
            c.advance_seq_len(1)
