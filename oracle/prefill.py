"""Prefill-attention oracle (CPU).  Test infrastructure only.

standard_attention_ref + prefill_mask restate the reference's PyTorch prefill
path selected by QWEN3_FLASH_ATTN=pytorch:
  prefill_mask            qwen3/model.py:150-161  ((B,1,S,S), -inf outside
                          the causal + length window, pad rows keep column 0)
  standard_attention_ref  qwen3/attention.py:193-207 (repeat_kv, q@k^T in the
                          input dtype, * scale, + mask, softmax in fp32 cast
                          back, @ v)
flash_varlen_ref restates the reference's Triton prefill algorithm
(qwen3/kernels/flash_attention_varlen.py:25-123: BLOCK_M x BLOCK_N tiles,
m_i = -1e10 start, masked scores -1e10, online softmax with exp, P rounded
to bf16 before P @ V) on the CPU.
varlen_attention_ref is the closed form used as the fp32 reference (and to
pin the others): per sequence, causal softmax(q k^T * scale) v.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    if n_rep == 1:
        return x
    b, h, s, d = x.shape
    return x[:, :, None, :, :].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


def prefill_mask(lens, S: int, dtype=torch.bfloat16) -> torch.Tensor:
    """(B, 1, S, S) additive mask of qwen3/model.py:150-161."""
    B = len(lens)
    row = torch.arange(S).view(1, S, 1)
    col = torch.arange(S).view(1, 1, S)
    lens_t = torch.tensor(lens).view(B, 1, 1)
    valid = (row < lens_t) & (col < lens_t) & (col <= row)
    pad_keep = (row >= lens_t) & (col == 0)
    mask = torch.full((B, S, S), float("-inf"), dtype=dtype)
    mask[valid | pad_keep] = 0
    return mask.unsqueeze(1)


def standard_attention_ref(q, k, v, attention_mask, scaling):
    """q (B, Hq, S, D), k/v (B, Hkv, S, D) -> (B, S, Hq * D)
    (qwen3/attention.py:193-207)."""
    groups = q.shape[1] // k.shape[1]
    k = _repeat_kv(k, groups)
    v = _repeat_kv(v, groups)
    w = torch.matmul(q, k.transpose(-2, -1)) * scaling
    w = w + attention_mask
    w = F.softmax(w, dim=-1, dtype=torch.float32).to(q.dtype)
    out = torch.matmul(w, v)
    B, S = q.shape[0], q.shape[2]
    return out.transpose(1, 2).reshape(B, S, -1)


def pad_batch(x: torch.Tensor, cu_seqlens, S: int) -> torch.Tensor:
    """Packed (T, H, D) -> right-padded (B, H, S, D) with zero pads."""
    B = len(cu_seqlens) - 1
    out = x.new_zeros(B, x.shape[1], S, x.shape[2])
    for b in range(B):
        s0, s1 = int(cu_seqlens[b]), int(cu_seqlens[b + 1])
        out[b, :, : s1 - s0] = x[s0:s1].transpose(0, 1)
    return out


def varlen_attention_ref(q, k, v, cu_seqlens, scale, causal: bool = True,
                         dtype=torch.float32) -> torch.Tensor:
    """Closed form on packed tensors: q (T, Hq, D), k/v (T, Hkv, D) ->
    (T, Hq, D) in `dtype`."""
    T, H, D = q.shape
    G = H // k.shape[1]
    out = torch.zeros(T, H, D, dtype=dtype)
    for s in range(len(cu_seqlens) - 1):
        s0, s1 = int(cu_seqlens[s]), int(cu_seqlens[s + 1])
        if s1 <= s0:
            continue
        qs = q[s0:s1].to(dtype).transpose(0, 1)                # (H, L, D)
        ks = k[s0:s1].to(dtype).transpose(0, 1).repeat_interleave(G, dim=0)
        vs = v[s0:s1].to(dtype).transpose(0, 1).repeat_interleave(G, dim=0)
        sc = (qs @ ks.transpose(-2, -1)) * scale
        if causal:
            L = s1 - s0
            tri = torch.ones(L, L, dtype=torch.bool).tril()
            sc = sc.masked_fill(~tri, float("-inf"))
        out[s0:s1] = (torch.softmax(sc, dim=-1) @ vs).transpose(0, 1)
    return out


def flash_varlen_ref(q, k, v, cu_seqlens, scale, block_m: int = 32, block_n: int = 32):
    """Tiled online-softmax restatement of flash_attention_varlen_kernel
    (qwen3/kernels/flash_attention_varlen.py:25-123); returns (T, Hq, D) bf16."""
    T, H, D = q.shape
    G = H // k.shape[1]
    out = torch.zeros(T, H, D, dtype=q.dtype)
    for s in range(len(cu_seqlens) - 1):
        s0, s1 = int(cu_seqlens[s]), int(cu_seqlens[s + 1])
        L = s1 - s0
        for h in range(H):
            kh = h // G
            for m0 in range(0, L, block_m):
                offs_m = torch.arange(m0, m0 + block_m)
                mask_m = offs_m < L
                qt = torch.zeros(block_m, D, dtype=torch.float32)
                qt[mask_m] = q[s0 + offs_m[mask_m], h].float()
                l_i = torch.zeros(block_m)
                m_i = torch.zeros(block_m) - 1e10
                acc = torch.zeros(block_m, D)
                for n0 in range(0, L, block_n):
                    offs_n = torch.arange(n0, n0 + block_n)
                    mask_n = offs_n < L
                    kt = torch.zeros(block_n, D)
                    vt = torch.zeros(block_n, D, dtype=q.dtype)
                    kt[mask_n] = k[s0 + offs_n[mask_n], kh].float()
                    vt[mask_n] = v[s0 + offs_n[mask_n], kh]
                    qk = (qt @ kt.T) * scale
                    causal = offs_m[:, None] >= offs_n[None, :]
                    qk = torch.where(causal & mask_n[None, :], qk, torch.tensor(-1e10))
                    m_new = torch.maximum(m_i, qk.max(dim=1).values)
                    alpha = torch.exp(m_i - m_new)
                    p = torch.exp(qk - m_new[:, None])
                    acc = acc * alpha[:, None]
                    acc = acc + p.to(q.dtype).float() @ vt.float()
                    l_i = l_i * alpha + p.sum(dim=1)
                    m_i = m_new
                o = (acc / l_i[:, None]).to(q.dtype)
                out[s0 + offs_m[mask_m], h] = o[mask_m]
    return out
