"""KV slot-write kernels vs the numpy oracle: bit-exact, whole pool compared."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import inputs as oi
from oracle import kv_write as ok

pytestmark = pytest.mark.gpu


def _u16(t):
    return ok.as_u16(t)


def _rand_bf16(shape, g, dev):
    return torch.randn(*shape, generator=g).to(torch.bfloat16).to(dev)


def test_decode_write_fused_qkv_slices(gpu):
    """k_new/v_new are slices of a fused (B, 1, Hq + 2 Hkv, D) QKV output (batch
    stride (Hq + 2 Hkv) * D), the layout that once broke batch rows >= 1."""
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import update_kv_batch_hip

    g = torch.Generator().manual_seed(0)
    B, Hq, Hkv, D, bs, nb, layers = 7, 16, 8, 128, 16, 40, 3
    qkv = _rand_bf16((B, Hq + 2 * Hkv, D), g, gpu)
    k_new, v_new = qkv[:, Hq:Hq + Hkv], qkv[:, Hq + Hkv:]
    kb = _rand_bf16((nb, layers, Hkv, bs, D), g, gpu)
    vb = _rand_bf16((nb, layers, Hkv, bs, D), g, gpu)
    rows_total, mp = 12, 6
    bt = torch.full((rows_total, mp), -1, dtype=torch.int32)
    perm = torch.randperm(nb, generator=g)
    bt[:, :3] = perm[:36].view(12, 3).to(torch.int32)
    seq_lens = torch.randint(0, 48, (rows_total,), generator=g, dtype=torch.int32)
    row_ids = torch.randperm(rows_total, generator=g)[:B].to(torch.int32)
    ek, ev = _u16(kb), _u16(vb)
    ok.update_kv_batch_ref(_u16(k_new), _u16(v_new), ek, ev, seq_lens.numpy(), bt.numpy(),
                           row_ids.numpy(), 2)
    announce("kv_write decode fused-qkv slices B=7")
    update_kv_batch_hip(k_new, v_new, kb, vb, seq_lens.to(gpu), bt.to(gpu), row_ids.to(gpu), 2)
    torch.cuda.synchronize()
    assert np.array_equal(_u16(kb), ek) and np.array_equal(_u16(vb), ev)


def test_range_write_matches_reference_update(gpu):
    """PagedKVCache.update path: S tokens from a nonzero seq_len across pages."""
    from qwen3_engine_from_scratch_amd.PagedKVcache import KVCachePool, PagedKVCache

    g = torch.Generator().manual_seed(1)
    pool = KVCachePool(32, 2, 16, 4, 128, device=gpu, dtype=torch.bfloat16, max_seq_len=512,
                       max_requests=4)
    c = PagedKVCache(pool)
    k1 = _rand_bf16((1, 4, 21, 128), g, gpu)
    v1 = _rand_bf16((1, 4, 21, 128), g, gpu)
    announce("kv_write range (PagedKVCache.update) 21 + 40 tokens")
    c.update(1, k1, v1)
    c.advance_seq_len(21)
    # second update from seq_len 21, as a transposed (non-contiguous) view
    k2 = _rand_bf16((1, 40, 4, 128), g, gpu).transpose(1, 2)
    v2 = _rand_bf16((1, 40, 4, 128), g, gpu).transpose(1, 2)
    c.update(1, k2, v2)
    torch.cuda.synchronize()
    ek = np.zeros(tuple(pool.k_buffer.shape), np.uint16)
    ev = np.zeros_like(ek)
    table = np.asarray(c.block_table, np.int32)
    ok.paged_update_ref(_u16(k1[0].transpose(0, 1)), _u16(v1[0].transpose(0, 1)), ek, ev, table, 0, 1)
    ok.paged_update_ref(_u16(k2[0].transpose(0, 1)), _u16(v2[0].transpose(0, 1)), ek, ev, table, 21, 1)
    assert np.array_equal(_u16(pool.k_buffer), ek) and np.array_equal(_u16(pool.v_buffer), ev)
    kk, vv = c.get_kv(1)
    assert kk.shape[2] == 21  # seq_len advanced by the first update only


def test_slots_write_with_padding(gpu):
    from qwen3_engine_from_scratch_amd import _lib

    g = torch.Generator().manual_seed(2)
    T, Hkv, D, bs, nb, layers = 300, 8, 128, 16, 64, 2
    k_new = _rand_bf16((T, Hkv, D), g, gpu)
    v_new = _rand_bf16((T, Hkv, D), g, gpu)
    kb = torch.zeros(nb, layers, Hkv, bs, D, dtype=torch.bfloat16, device=gpu)
    vb = torch.zeros_like(kb)
    slots = torch.randperm(nb * bs, generator=g)[:T].to(torch.int64)
    slots[::7] = -1
    ek = np.zeros(tuple(kb.shape), np.uint16)
    ev = np.zeros_like(ek)
    ok.slots_write_ref(_u16(k_new), _u16(v_new), ek, ev, slots.numpy(), 1)
    sm = slots.to(gpu)
    announce("kv_write slots T=300 with -1 padding")
    rc = _lib.load().qwen3_kv_write_slots_bf16(
        k_new.data_ptr(), _lib.strides(k_new, (0, 1)), v_new.data_ptr(), _lib.strides(v_new, (0, 1)),
        kb.data_ptr(), _lib.strides(kb, (0, 1, 2, 3)), vb.data_ptr(), _lib.strides(vb, (0, 1, 2, 3)),
        nb, 1, layers, sm.data_ptr(), T, Hkv, D, bs, _lib.stream_of(gpu))
    _lib.check(rc, "slots")
    torch.cuda.synchronize()
    assert np.array_equal(_u16(kb), ek) and np.array_equal(_u16(vb), ev)


def test_batched_prefill_write_equals_per_request_updates(gpu):
    """write_prefill_batch (one launch) == the reference's B-loop of update,
    padded positions included."""
    from qwen3_engine_from_scratch_amd.PagedKVcache import (KVCachePool, PagedKVCache,
                                                            write_prefill_batch)

    g = torch.Generator().manual_seed(3)
    B, S, Hkv = 3, 37, 8
    k = _rand_bf16((B, Hkv, S, 128), g, gpu)
    v = _rand_bf16((B, Hkv, S, 128), g, gpu)
    pa = KVCachePool(40, 2, 16, Hkv, 128, device=gpu, dtype=torch.bfloat16, max_seq_len=256, max_requests=8)
    pb = KVCachePool(40, 2, 16, Hkv, 128, device=gpu, dtype=torch.bfloat16, max_seq_len=256, max_requests=8)
    ca = [PagedKVCache(pa) for _ in range(B)]
    cb = [PagedKVCache(pb) for _ in range(B)]
    announce("kv_write batched prefill vs per-request updates")
    for i, c in enumerate(ca):
        c.update(0, k[i:i + 1], v[i:i + 1])
    write_prefill_batch(cb, 0, k, v)
    torch.cuda.synchronize()
    assert [c.block_table for c in ca] == [c.block_table for c in cb]
    assert torch.equal(pa.k_buffer, pb.k_buffer) and torch.equal(pa.v_buffer, pb.v_buffer)


def test_unaligned_rows_use_element_path(gpu):
    """A k_new view starting one element into its buffer cannot use 16-byte
    copies; the element path must still be bit-exact."""
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import update_kv_batch_hip

    g = torch.Generator().manual_seed(4)
    B, Hkv, D = 4, 2, 128
    base = _rand_bf16((B * Hkv * D + 1,), g, gpu)
    k_new = base[1:].view(B, Hkv, D)
    v_new = _rand_bf16((B, Hkv, D), g, gpu)
    kb = torch.zeros(8, 1, Hkv, 16, D, dtype=torch.bfloat16, device=gpu)
    vb = torch.zeros_like(kb)
    bt = torch.arange(8, dtype=torch.int32).view(4, 2)
    seq_lens = torch.tensor([0, 5, 17, 31], dtype=torch.int32)
    rows = torch.arange(4, dtype=torch.int32)
    ek = np.zeros(tuple(kb.shape), np.uint16)
    ev = np.zeros_like(ek)
    ok.update_kv_batch_ref(_u16(k_new), _u16(v_new), ek, ev, seq_lens.numpy(), bt.numpy(), rows.numpy(), 0)
    announce("kv_write unaligned element path")
    update_kv_batch_hip(k_new, v_new, kb, vb, seq_lens.to(gpu), bt.to(gpu), rows.to(gpu), 0)
    torch.cuda.synchronize()
    assert np.array_equal(_u16(kb), ek) and np.array_equal(_u16(vb), ev)


def test_slot_write_golden_fixture(gpu):
    from pathlib import Path

    from oracle import inputs as oi
    from qwen3_engine_from_scratch_amd import _lib

    f = np.load(Path(__file__).resolve().parent / "golden" / "slot_write.npz", allow_pickle=False)
    c = oi.make_prefill_case([40, 23], 16, 8, 128, seed=4)
    assert c.fingerprint() == str(f["sha256"])
    kb = torch.zeros(c.num_blocks + 2, 3, 8, 16, 128, dtype=torch.bfloat16, device=gpu)
    vb = torch.zeros_like(kb)
    k, v, sm = c.k.to(gpu), c.v.to(gpu), c.slot_mapping.to(gpu)
    announce("slot write vs golden fixture")
    rc = _lib.load().qwen3_kv_write_slots_bf16(
        k.data_ptr(), _lib.strides(k, (0, 1)), v.data_ptr(), _lib.strides(v, (0, 1)),
        kb.data_ptr(), _lib.strides(kb, (0, 1, 2, 3)), vb.data_ptr(), _lib.strides(vb, (0, 1, 2, 3)),
        kb.shape[0], 1, kb.shape[1], sm.data_ptr(), sm.numel(), 8, 128, 16, _lib.stream_of(gpu))
    _lib.check(rc, "slots")
    torch.cuda.synchronize()
    ku, vu = _u16(kb), _u16(vb)
    assert np.uint64(ku.astype(np.uint64).sum()) == f["k_checksum"]
    assert np.uint64(vu.astype(np.uint64).sum()) == f["v_checksum"]
    assert np.array_equal(np.argwhere(ku.any(axis=(2, 4))), f["touched"])


def test_config2_slot_write_full_size_bit_exact(gpu):
    """The Qwen3-0.6B prefill workload's slot write at its own size: 8
    sequences, 8,115 tokens, the seeded slot mapping through a permuted pool,
    into layer 1 of a 2-layer pool; the whole pool compared with the oracle
    (every written slot bit-exact, every other slot still zero)."""
    from qwen3_engine_from_scratch_amd import _lib

    c = oi.config2_prefill()
    T = int(c.cu_seqlens[-1])
    assert T == sum(c.lens) == 8115
    nb = c.num_blocks + 7  # a few blocks no sequence owns
    kb = torch.zeros(nb, 2, 8, 16, 128, dtype=torch.bfloat16, device=gpu)
    vb = torch.zeros_like(kb)
    ek = np.zeros(tuple(kb.shape), np.uint16)
    ev = np.zeros_like(ek)
    ok.slots_write_ref(_u16(c.k), _u16(c.v), ek, ev, c.slot_mapping.numpy(), 1)
    k, v, sm = c.k.to(gpu), c.v.to(gpu), c.slot_mapping.to(gpu)
    announce(f"config2 slot write T={T} lens={c.lens}")
    rc = _lib.load().qwen3_kv_write_slots_bf16(
        k.data_ptr(), _lib.strides(k, (0, 1)), v.data_ptr(), _lib.strides(v, (0, 1)),
        kb.data_ptr(), _lib.strides(kb, (0, 1, 2, 3)), vb.data_ptr(), _lib.strides(vb, (0, 1, 2, 3)),
        nb, 1, 2, sm.data_ptr(), T, 8, 128, 16, _lib.stream_of(gpu))
    _lib.check(rc, "slots")
    torch.cuda.synchronize()
    ku, vu = _u16(kb), _u16(vb)
    assert np.array_equal(ku, ek) and np.array_equal(vu, ev)
    # independent read path: each sequence gathered back through its pages
    cu = c.cu_seqlens.tolist()
    bs = 16
    for s, L in enumerate(c.lens):
        sl = c.slot_mapping[cu[s]:cu[s + 1]].numpy()
        table = sl[::bs] // bs
        got = ok.gather_tokens(ku, 1, table, L)  # (Hkv, L, D)
        assert np.array_equal(got, _u16(c.k[cu[s]:cu[s + 1]]).transpose(1, 0, 2))
