"""Oracle for the fused pre-attention step (QK-RMSNorm + RoPE + pool write).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Restates, on the CPU in
PyTorch, the reference's own modules in the order the attention layer calls
them: RMSNorm (qwen3/norm.py:22-26) on q and k, then apply_rotary_pos_emb
(qwen3/rope.py:88-110) with cos/sin gathered from the RotaryEmbedding
tables (qwen3/rope.py:42-58, 60-69) at each token's position; the pool write
that follows is kv_write.slots_write_ref.
"""
from __future__ import annotations

import torch

from .inputs import apply_rope, rms_norm


def rope_tables(head_dim: int, base: float = 1e6, max_seq_len: int = 4096):
    """The model's fp32 cos/sin tables (max_seq_len, head_dim), built the way
    RotaryEmbedding.__init__ builds them (qwen3/rope.py:42-58): inverse
    frequencies from even indices, an outer product over positions, and the
    frequencies repeated for both halves."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    positions = torch.arange(max_seq_len, dtype=torch.float32)
    freqs = torch.einsum("s,d->sd", positions, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def qk_norm_rope_ref(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor,
                     k_weight: torch.Tensor, eps: float, cos_table: torch.Tensor,
                     sin_table: torch.Tensor, positions: torch.Tensor):
    """q: (T, Hq, D), k: (T, Hkv, D) bf16; positions: (T,) int.  Returns the
    normalised, rotated (q, k) in bf16 (qwen3/attention.py:91-96)."""
    qn = rms_norm(q, q_weight, eps)
    kn = rms_norm(k, k_weight, eps)
    cos = cos_table[positions.long()]
    sin = sin_table[positions.long()]
    return apply_rope(qn, cos, sin), apply_rope(kn, cos, sin)


def rope_closed_form_fp64(n: torch.Tensor, positions: torch.Tensor, head_dim: int,
                          base: float = 1e6) -> torch.Tensor:
    """Independent check of RoPE: each pair (n_i, n_{i+D/2}) as the complex
    number n_i + j n_{i+D/2}, multiplied by exp(j * pos * base^(-2i/D)) in
    float64.  n: (T, H, D) (already normalised); returns (T, H, D) float64."""
    half = head_dim // 2
    i = torch.arange(half, dtype=torch.float64)
    theta = base ** (-2.0 * i / head_dim)
    ang = positions.to(torch.float64)[:, None, None] * theta[None, None, :]
    z = torch.complex(n[..., :half].double(), n[..., half:].double()) * torch.exp(1j * ang)
    return torch.cat((z.real, z.imag), dim=-1)


def rms_closed_form_fp64(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """x / sqrt(mean(x^2) + eps) * w in float64."""
    xd = x.double()
    return xd / torch.sqrt(xd.pow(2).mean(-1, keepdim=True) + eps) * w.double()
