"""Decode-attention oracle (CPU).  Test infrastructure only.

paged_attention_ref restates the reference's PyTorch decode path,
paged_attention() in qwen3/paged_attention.py:39-122, on the kernel's
interface (per-layer pool view + resident block table + seq_lens/row_ids
with the L = seq_lens[row] + 1 convention of
qwen3/kernels/paged_attention.py:54-56):
  - per request, walk its pages in logical order (:84);
  - zero K/V slots at or beyond L in the last page (:92-96);
  - repeat_kv for GQA (query head h -> KV head h // G) and cast to fp32
    (:98-99, qwen3/paged_attention.py:31-36);
  - s = q.float() @ K^T * scale, masked slots -> -inf (:68-73, :103-104);
  - online softmax m/l/acc in fp32 (:79-81, :108-118);
  - (acc / l).to(bf16) (:121).

dense_decode_ref is the independent closed form used to pin it: gather the L
tokens through the block table and take a plain softmax in fp64.
"""
from __future__ import annotations

import torch


def _repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """(1, Hkv, S, D) -> (1, Hkv * n_rep, S, D) (qwen3/paged_attention.py:31-36)."""
    if n_rep == 1:
        return x
    b, h, s, d = x.shape
    return x[:, :, None, :, :].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


def context_length(seq_lens, row_ids, b: int, bias: int = 1) -> tuple[int, int]:
    row = int(row_ids[b]) if row_ids is not None else b
    return row, int(seq_lens[row]) + bias


def paged_attention_ref(q, k_pool, v_pool, block_table, seq_lens, row_ids, block_size,
                        scale=None, bias: int = 1, out_fp32: bool = False):
    """q (B, Hq, D); k_pool/v_pool (num_blocks, Hkv, bs, D); block_table
    (rows, max_pages) int32; seq_lens (rows,) int32; row_ids (B,) or None.
    Returns (B, Hq, D) in q.dtype (or fp32 before the cast if out_fp32)."""
    B, H, D = q.shape
    Hk = k_pool.shape[1]
    groups = H // Hk
    if scale is None:
        scale = D ** -0.5
    outs = []
    for b in range(B):
        row, L = context_length(seq_lens, row_ids, b, bias)
        num_pages = (L + block_size - 1) // block_size
        qb = q[b:b + 1, :, None, :]  # (1, H, 1, D)
        m = torch.full((1, H, 1, 1), float("-inf"), dtype=torch.float32)
        l = torch.zeros((1, H, 1, 1), dtype=torch.float32)
        acc = torch.zeros((1, H, 1, D), dtype=torch.float32)
        slot_idx = torch.arange(block_size)
        for j in range(num_pages):
            phys = int(block_table[row, j])
            k_page = k_pool[phys].unsqueeze(0)  # (1, Hk, bs, D)
            v_page = v_pool[phys].unsqueeze(0)
            valid = min(block_size, L - j * block_size)
            slot_mask = (slot_idx < valid).view(1, 1, block_size, 1)
            k_page = k_page * slot_mask
            v_page = v_page * slot_mask
            k_page = _repeat_kv(k_page, groups).float()
            v_page = _repeat_kv(v_page, groups).float()
            s = torch.matmul(qb.float(), k_page.transpose(-2, -1)) * scale
            page_mask = torch.where(slot_idx < valid, 0.0, float("-inf")).view(1, 1, 1, block_size)
            s = s + page_mask
            m_new = torch.maximum(m, s.max(dim=-1, keepdim=True).values)
            alpha = torch.exp(m - m_new)
            p = torch.exp(s - m_new)
            l = l * alpha + p.sum(dim=-1, keepdim=True)
            acc = acc * alpha + torch.matmul(p, v_page)
            m = m_new
        o = (acc / l)[0, :, 0, :]
        outs.append(o if out_fp32 else o.to(q.dtype))
    if not outs:
        return torch.empty(0, H, D, dtype=torch.float32 if out_fp32 else q.dtype)
    return torch.stack(outs)


def gather_context(pool_layer: torch.Tensor, table_row, L: int, block_size: int) -> torch.Tensor:
    """Tokens 0..L-1 of one sequence gathered through its table row:
    (Hkv, L, D), the read path of PagedKVCache.get_kv (qwen3/PagedKVcache.py:164-175)."""
    num_pages = (L + block_size - 1) // block_size
    pages = [pool_layer[int(table_row[j])] for j in range(num_pages)]
    if not pages:
        return pool_layer.new_zeros(pool_layer.shape[1], 0, pool_layer.shape[3])
    return torch.cat(pages, dim=1)[:, :L, :]


def dense_decode_ref(q, k_pool, v_pool, block_table, seq_lens, row_ids, block_size,
                     scale=None, bias: int = 1, dtype=torch.float64):
    """Closed form: softmax(scale * q K_ctx^T) V_ctx per sequence in `dtype`,
    with query head h reading KV head h // G."""
    B, H, D = q.shape
    Hk = k_pool.shape[1]
    G = H // Hk
    if scale is None:
        scale = D ** -0.5
    out = torch.empty(B, H, D, dtype=dtype)
    for b in range(B):
        row, L = context_length(seq_lens, row_ids, b, bias)
        kc = gather_context(k_pool, block_table[row], L, block_size).to(dtype)  # (Hk, L, D)
        vc = gather_context(v_pool, block_table[row], L, block_size).to(dtype)
        for h in range(H):
            s = (kc[h // G] @ q[b, h].to(dtype)) * scale
            w = torch.softmax(s, dim=0)
            out[b, h] = w @ vc[h // G]
    return out
