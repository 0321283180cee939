"""Seeded synthetic inputs for the hot-path workloads (CPU, torch.Generator).

Inputs are produced on the CPU with a seeded generator, so the same seed gives
the same bytes on any machine with this torch build; tests fingerprint them
(sha256) against the committed golden fixtures.

QK-RMSNorm and RoPE restate the reference math used upstream of the kernels:
  rms_norm        qwen3/norm.py:22-26
  rope_cos_sin    qwen3/rope.py:49-69   (cat(freqs, freqs) table, theta 1e6)
  apply_rope      qwen3/rope.py:72-110  (rotate-half pairing i <-> i + D/2)
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field

import numpy as np
import torch


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """fp32 RMSNorm over the last dim, cast back to x.dtype (qwen3/norm.py:22-26)."""
    xf = x.float()
    rms = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return ((xf * rms) * weight).to(x.dtype)


def rope_cos_sin(positions: torch.Tensor, head_dim: int, base: float = 1e6):
    """cos/sin tables gathered at `positions` (qwen3/rope.py:49-69)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    freqs = positions.to(torch.float32)[..., None] * inv_freq
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x * cos + rotate_half(x) * sin with cos/sin cast to x.dtype
    (qwen3/rope.py:106-110).  x: (..., T, H, D); cos/sin: (T, D)."""
    c = cos[:, None, :].to(x.dtype)
    s = sin[:, None, :].to(x.dtype)
    return x * c + _rotate_half(x) * s


def fingerprint(*tensors: torch.Tensor) -> str:
    h = hashlib.sha256()
    for t in tensors:
        t = t.detach().cpu().contiguous()
        h.update(str(tuple(t.shape)).encode())
        h.update(str(t.dtype).encode())
        h.update(t.view(torch.uint8).numpy().tobytes() if t.numel() else b"")
    return h.hexdigest()


@dataclass
class DecodeCase:
    """One paged-decode workload (one layer view of the pool).

    q (B, Hq, D) bf16; k_pool/v_pool (num_blocks, Hkv, bs, D) bf16;
    block_table (B, max_pages) int32, -1 where unallocated; seq_lens (B,)
    int32 holding L-1 (the reference's pre-step length, attended with +1);
    row_ids (B,) int32.
    """
    q: torch.Tensor
    k_pool: torch.Tensor
    v_pool: torch.Tensor
    block_table: torch.Tensor
    seq_lens: torch.Tensor
    row_ids: torch.Tensor
    lens: list
    block_size: int
    scale: float
    meta: dict = field(default_factory=dict)

    @property
    def num_heads(self):
        return self.q.shape[1]

    @property
    def num_kv_heads(self):
        return self.k_pool.shape[1]

    def fingerprint(self) -> str:
        return fingerprint(self.q, self.k_pool, self.v_pool, self.block_table,
                           self.seq_lens, self.row_ids)


def make_decode_case(lens, num_heads: int, num_kv_heads: int, head_dim: int = 128,
                     block_size: int = 16, num_blocks: int | None = None,
                     slack: float = 0.0, seed: int = 0, qk_norm: bool = False,
                     table: str = "sample", max_pages: int | None = None) -> DecodeCase:
    """Builds a decode workload.

    table="sample": each sequence's pages are a seeded sample without
    replacement from the pool; table="perm": the pool is a random permutation
    split across sequences.  qk_norm applies RMSNorm (eps 1e-6,
    gamma = 1 + 0.1 N(0,1)) to q and to the cached K before the bf16 cast.
    """
    g = torch.Generator().manual_seed(seed)
    lens = [int(x) for x in lens]
    B = len(lens)
    pages = [(L + block_size - 1) // block_size for L in lens]
    total_pages = sum(pages)
    if num_blocks is None:
        num_blocks = max(int(np.ceil(total_pages * (1.0 + slack))), total_pages, 1)
    assert num_blocks >= total_pages, "pool too small for the requested contexts"
    if max_pages is None:
        max_pages = max(pages) if pages else 1
    perm = torch.randperm(num_blocks, generator=g)
    table_t = torch.full((B, max_pages), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(pages):
        table_t[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = torch.randn(B, num_heads, head_dim, generator=g)
    k = torch.randn(num_blocks, num_kv_heads, block_size, head_dim, generator=g)
    v = torch.randn(num_blocks, num_kv_heads, block_size, head_dim, generator=g)
    if qk_norm:
        gq = 1.0 + 0.1 * torch.randn(head_dim, generator=g)
        gk = 1.0 + 0.1 * torch.randn(head_dim, generator=g)
        q = rms_norm(q, gq)
        k = rms_norm(k, gk)
    q = q.to(torch.bfloat16)
    k = k.to(torch.bfloat16)
    v = v.to(torch.bfloat16)
    seq_lens = torch.tensor([L - 1 for L in lens], dtype=torch.int32)
    row_ids = torch.arange(B, dtype=torch.int32)
    return DecodeCase(q=q, k_pool=k, v_pool=v, block_table=table_t, seq_lens=seq_lens,
                      row_ids=row_ids, lens=lens, block_size=block_size,
                      scale=1.0 / float(np.sqrt(head_dim)),
                      meta=dict(seed=seed, table=table, qk_norm=qk_norm, slack=slack))


def config1_decode() -> DecodeCase:
    """Qwen3-0.6B decode layer: 16/8 heads, D 128, B 4, L [37, 128, 511, 1024],
    pool of 512 blocks x 16, seeded per-sequence page samples, QK-RMSNorm."""
    return make_decode_case([37, 128, 511, 1024], 16, 8, 128, 16, num_blocks=512,
                            seed=0, qk_norm=True)


def seeded_lengths(n: int, lo: int, hi: int, seed: int) -> list:
    g = torch.Generator().manual_seed(seed)
    return [int(x) for x in torch.randint(lo, hi + 1, (n,), generator=g)]


def config3_lengths(seed: int = 0) -> list:
    """Qwen3-8B decode headline: 256 context lengths uniform in [1024, 8192]."""
    return seeded_lengths(256, 1024, 8192, seed)


def config4_lengths(seed: int = 0) -> list:
    """Long-context split-KV decode: 8 context lengths uniform in [32768, 131072]."""
    return seeded_lengths(8, 32768, 131072, seed)


@dataclass
class PrefillCase:
    """Packed varlen prefill: q (T, Hq, D), k/v (T, Hkv, D) bf16,
    cu_seqlens (S+1,) int32, plus the slot mapping of a block-16 pool."""
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    cu_seqlens: torch.Tensor
    lens: list
    slot_mapping: torch.Tensor
    num_blocks: int
    block_size: int
    scale: float
    meta: dict = field(default_factory=dict)

    def fingerprint(self) -> str:
        return fingerprint(self.q, self.k, self.v, self.cu_seqlens, self.slot_mapping)


def make_prefill_case(lens, num_heads: int = 16, num_kv_heads: int = 8, head_dim: int = 128,
                      seed: int = 0, qk_norm_rope: bool = True, block_size: int = 16,
                      rope_theta: float = 1e6) -> PrefillCase:
    """Packs sequences of the given lengths; Q/K/V ~ N(0,1), then (optionally)
    QK-RMSNorm and RoPE at positions 0..L-1 of each sequence.  The slot
    mapping sends each sequence through its own pages of a pool whose blocks
    are a seeded random permutation."""
    g = torch.Generator().manual_seed(seed)
    lens = [int(x) for x in lens]
    T = sum(lens)
    q = torch.randn(T, num_heads, head_dim, generator=g)
    k = torch.randn(T, num_kv_heads, head_dim, generator=g)
    v = torch.randn(T, num_kv_heads, head_dim, generator=g)
    if qk_norm_rope:
        gq = 1.0 + 0.1 * torch.randn(head_dim, generator=g)
        gk = 1.0 + 0.1 * torch.randn(head_dim, generator=g)
        q = rms_norm(q.to(torch.bfloat16), gq)
        k = rms_norm(k.to(torch.bfloat16), gk)
        pos = torch.cat([torch.arange(L) for L in lens]) if lens else torch.zeros(0)
        cos, sin = rope_cos_sin(pos, head_dim, rope_theta)
        q = apply_rope(q, cos, sin)
        k = apply_rope(k, cos, sin)
    q = q.to(torch.bfloat16)
    k = k.to(torch.bfloat16)
    v = v.to(torch.bfloat16)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    if lens:
        cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    pages = [(L + block_size - 1) // block_size for L in lens]
    num_blocks = max(sum(pages), 1)
    perm = torch.randperm(num_blocks, generator=g).to(torch.int64)
    slots = []
    off = 0
    for L, n in zip(lens, pages):
        table = perm[off:off + n]
        off += n
        p = torch.arange(L, dtype=torch.int64)
        slots.append(table[p // block_size] * block_size + p % block_size)
    slot_mapping = torch.cat(slots) if slots else torch.zeros(0, dtype=torch.int64)
    return PrefillCase(q=q, k=k, v=v, cu_seqlens=cu, lens=lens, slot_mapping=slot_mapping,
                       num_blocks=num_blocks, block_size=block_size,
                       scale=1.0 / float(np.sqrt(head_dim)),
                       meta=dict(seed=seed, qk_norm_rope=qk_norm_rope))


def config2_lengths(seed: int = 0) -> list:
    """Qwen3-0.6B varlen prefill: 8 lengths uniform in [64, 2048]."""
    return seeded_lengths(8, 64, 2048, seed)


def config2_prefill(seed: int = 0) -> PrefillCase:
    return make_prefill_case(config2_lengths(seed), 16, 8, 128, seed=seed)
