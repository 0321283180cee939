"""Fused QK-RMSNorm + RoPE + pool write on the GPU vs the oracle.

Bar: q/k within one bf16 ulp of the oracle with at least 99% of the values
bit-identical (only the fp32 sum of squares may associate differently), and
the pool bit-exact: k slots equal the kernel's own rotated k, v slots equal
v, every other slot untouched."""
import pytest
import torch

from conftest import announce
from oracle import pre_attention as opa

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _ordered(t):
    b = t.contiguous().view(torch.int16).to(torch.int32)
    return torch.where(b >= 0, b, -(b & 0x7FFF))


def assert_ulp_close(got, ref, what, max_ulps=1, min_exact=0.99):
    d = (_ordered(got.cpu()) - _ordered(ref.cpu())).abs()
    assert d.max().item() <= max_ulps, f"{what}: {d.max().item()} ulps"
    exact = (d == 0).float().mean().item()
    assert exact >= min_exact, f"{what}: only {exact:.4f} bit-identical"


def _qkv(T, hq, hkv, seed, scale=3.0):
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(T, (hq + 2 * hkv) * 128, generator=g) * scale).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    return qkv, qw, kw


def _split(qkv, hq, hkv):
    T = qkv.shape[0]
    q = qkv[:, :hq * 128].view(T, hq, 128)
    k = qkv[:, hq * 128:(hq + hkv) * 128].view(T, hkv, 128)
    v = qkv[:, (hq + hkv) * 128:].view(T, hkv, 128)
    return q, k, v


@pytest.mark.parametrize("hq,hkv,B", [(16, 8, 13), (32, 8, 64)])
def test_decode_form_vs_oracle(gpu, hq, hkv, B):
    from qwen3_engine_from_scratch_amd.PagedKVcache import KVCachePool, PagedKVCache
    from qwen3_engine_from_scratch_amd.kernels.pre_attention import qk_norm_rope_decode

    announce(f"pre-attention decode hq={hq} hkv={hkv} B={B}")
    g = torch.Generator().manual_seed(B)
    pool = KVCachePool(6 * B + 8, 2, 16, hkv, 128, device=gpu, dtype=torch.bfloat16,
                       max_seq_len=2048, max_requests=B + 3)
    caches = [PagedKVCache(pool) for _ in range(B)]
    for c in caches:
        c.seq_len = int(torch.randint(0, 60, (1,), generator=g))
        while c.num_pages < (c.seq_len + 16) // 16 + 1:
            c._allocate_block()
        pool.seq_lens[c.row_id] = c.seq_len
        c.reserve_next()
    row_ids = torch.tensor([c.row_id for c in caches], dtype=torch.int32, device=gpu)
    qkv, qw, kw = _qkv(B, hq, hkv, seed=B)
    cos, sin = opa.rope_tables(128, 1e6, 4096)
    q, k, v = _split(qkv.to(gpu), hq, hkv)
    out = qk_norm_rope_decode(q, k, v, qw.to(gpu), kw.to(gpu), EPS, cos.to(gpu), sin.to(gpu),
                              pool, 1, row_ids)
    torch.cuda.synchronize()
    pos = torch.tensor([c.seq_len for c in caches])
    qr, kr = opa.qk_norm_rope_ref(*_split(qkv, hq, hkv)[:2], qw, kw, EPS, cos, sin, pos)
    assert_ulp_close(out, qr, "q")
    kb, vb = pool.k_buffer.cpu(), pool.v_buffer.cpu()
    _, _, vh = _split(qkv, hq, hkv)
    written = torch.zeros(kb.shape[0], kb.shape[3], dtype=torch.bool)
    k_pool = torch.empty(B, hkv, 128, dtype=torch.bfloat16)
    for b, c in enumerate(caches):
        p = c.seq_len
        phys, off = c.block_table[p // 16], p % 16
        k_pool[b] = kb[phys, 1, :, off]
        assert torch.equal(vb[phys, 1, :, off], vh[b]), f"v slot of token {b}"
        written[phys, off] = True
    assert_ulp_close(k_pool, kr, "k in pool")
    assert not kb[:, 0].any() and not vb[:, 0].any(), "layer 0 touched"
    by_slot_k = kb[:, 1].permute(0, 2, 1, 3)  # (block, offset, head, D)
    by_slot_v = vb[:, 1].permute(0, 2, 1, 3)
    assert not by_slot_k[~written].any() and not by_slot_v[~written].any(), "other slots touched"


def test_slot_form_vs_oracle_and_pool_consistency(gpu):
    from qwen3_engine_from_scratch_amd.kernels.pre_attention import qk_norm_rope_prefill

    hq, hkv = 16, 8
    lens = [37, 1, 200, 64]
    T = sum(lens)
    announce(f"pre-attention prefill lens={lens}")
    qkv, qw, kw = _qkv(T, hq, hkv, seed=5)
    cos, sin = opa.rope_tables(128, 1e6, 4096)
    pos = torch.cat([torch.arange(L) for L in lens])
    g = torch.Generator().manual_seed(9)
    nblk = 40
    slots = torch.randperm(nblk * 16, generator=g)[:T].to(torch.int64)
    slots[::7] = -1  # no pool write for these tokens
    kb = torch.zeros(nblk, 3, hkv, 16, 128, dtype=torch.bfloat16, device=gpu)
    vb = torch.zeros_like(kb)
    q, k, v = _split(qkv.to(gpu), hq, hkv)
    qo, ko = qk_norm_rope_prefill(q, k, v, qw.to(gpu), kw.to(gpu), EPS, cos.to(gpu), sin.to(gpu),
                                  pos.to(gpu), slots.to(gpu), kb, vb, 2)
    torch.cuda.synchronize()
    qr, kr = opa.qk_norm_rope_ref(*_split(qkv, hq, hkv)[:2], qw, kw, EPS, cos, sin, pos)
    assert_ulp_close(qo, qr, "q")
    assert_ulp_close(ko, kr, "k")
    kbc, vbc = kb.cpu(), vb.cpu()
    _, _, vh = _split(qkv, hq, hkv)
    koc = ko.cpu()
    for t in range(T):
        s = int(slots[t])
        if s < 0:
            continue
        assert torch.equal(kbc[s // 16, 2, :, s % 16], koc[t])
        assert torch.equal(vbc[s // 16, 2, :, s % 16], vh[t])
    used = torch.zeros(nblk * 16, dtype=torch.bool)
    used[slots[slots >= 0]] = True
    flat_k = kbc[:, 2].permute(0, 2, 1, 3).reshape(nblk * 16, hkv, 128)
    assert not flat_k[~used].any() and not kbc[:, :2].any()


def test_decode_and_slot_forms_agree_bit_for_bit(gpu):
    from qwen3_engine_from_scratch_amd.PagedKVcache import KVCachePool, PagedKVCache
    from qwen3_engine_from_scratch_amd.kernels.pre_attention import (
        qk_norm_rope_decode, qk_norm_rope_prefill)

    hq, hkv, B = 16, 8, 6
    announce("pre-attention decode vs slot form")
    pool = KVCachePool(32, 1, 16, hkv, 128, device=gpu, dtype=torch.bfloat16, max_requests=8)
    caches = [PagedKVCache(pool) for _ in range(B)]
    for i, c in enumerate(caches):
        c.seq_len = 3 * i + 10
        pool.seq_lens[c.row_id] = c.seq_len
        while c.num_pages * 16 <= c.seq_len:
            c._allocate_block()
    qkv, qw, kw = _qkv(B, hq, hkv, seed=11)
    cos, sin = opa.rope_tables(128, 1e6, 1024)
    q, k, v = _split(qkv.to(gpu), hq, hkv)
    rows = torch.tensor([c.row_id for c in caches], dtype=torch.int32, device=gpu)
    qd = qk_norm_rope_decode(q, k, v, qw.to(gpu), kw.to(gpu), EPS, cos.to(gpu), sin.to(gpu),
                             pool, 0, rows)
    pos = torch.tensor([c.seq_len for c in caches], dtype=torch.int64, device=gpu)
    qs, ks = qk_norm_rope_prefill(q, k, v, qw.to(gpu), kw.to(gpu), EPS, cos.to(gpu),
                                  sin.to(gpu), pos, None, pool.k_buffer, pool.v_buffer, 0)
    torch.cuda.synchronize()
    assert torch.equal(qd.cpu(), qs.cpu())
    kb = pool.k_buffer.cpu()
    for b, c in enumerate(caches):
        p = c.seq_len
        assert torch.equal(kb[c.block_table[p // 16], 0, :, p % 16], ks[b].cpu())


def test_position_outside_tables_gives_zero_rows_and_no_write(gpu):
    from qwen3_engine_from_scratch_amd.kernels.pre_attention import qk_norm_rope_prefill

    hq, hkv = 8, 2
    announce("pre-attention out-of-table position")
    qkv, qw, kw = _qkv(3, hq, hkv, seed=2)
    cos, sin = opa.rope_tables(128, 1e6, 64)
    pos = torch.tensor([5, 64, -1], dtype=torch.int64, device=gpu)
    slots = torch.tensor([0, 1, 2], dtype=torch.int64, device=gpu)
    kb = torch.zeros(1, 1, hkv, 16, 128, dtype=torch.bfloat16, device=gpu)
    vb = torch.zeros_like(kb)
    q, k, v = _split(qkv.to(gpu), hq, hkv)
    qo, ko = qk_norm_rope_prefill(q, k, v, qw.to(gpu), kw.to(gpu), EPS, cos.to(gpu), sin.to(gpu),
                                  pos, slots, kb, vb, 0)
    torch.cuda.synchronize()
    assert qo[0].abs().sum() > 0 and not qo[1:].any() and not ko[1:].any()
    assert kb[0, 0, :, 0].any() and not kb[0, 0, :, 1:].any() and not vb[0, 0, :, 1:].any()
