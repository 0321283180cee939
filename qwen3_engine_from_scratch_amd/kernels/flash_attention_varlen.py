"""Varlen causal flash-attention prefill on the gfx950 HIP kernel.

Drop-in for qwen3/kernels/flash_attention_varlen.py of the reference engine:
same function names, arguments and return contracts (file:line per function),
device work in qwen3_varlen_prefill_bf16 (include/qwen3_attn.h).
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["flash_attention_prefill", "flash_attention_prefill_batched"]


_WORKSPACES: dict = {}


def _schedule_workspace(device, stream: int, lib) -> torch.Tensor:
    """The workspace of the item counters and of the items cut across
    workgroups (tickets and partial states) for this device and stream,
    zeroed once (every call leaves its counters and tickets at zero).  One
    per stream: calls on different streams may run at the same time and
    must not share tickets."""
    key = (str(device), stream)
    ws = _WORKSPACES.get(key)
    if ws is None:
        ws = torch.zeros(int(lib.qwen3_varlen_prefill_workspace_bytes()), dtype=torch.uint8,
                         device=device)
        _WORKSPACES[key] = ws
    return ws


def flash_attention_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                            cu_seqlens: torch.Tensor, scale: float, num_heads: int,
                            num_kv_heads: int, head_dim: int, *,
                            max_seqlen: int | None = None, causal: bool = True,
                            out: torch.Tensor | None = None,
                            workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Packed varlen prefill (reference: flash_attention_prefill,
    qwen3/kernels/flash_attention_varlen.py:126-194).

    q: (total_tokens, num_heads, head_dim); k, v: (total_tokens, num_kv_heads,
    head_dim); cu_seqlens: int32 (num_seqs + 1,) cumulative lengths.
    Returns (total_tokens, num_heads, head_dim).  `max_seqlen` (host int) avoids
    the reference's device->host read of cu_seqlens (:177-178); when omitted
    it is computed the same way the reference does.  A given max_seqlen must
    bound every sequence: rows of a longer one past max_seqlen (rounded up to
    a query tile) are left unwritten.  `workspace`: the item counters and
    the tickets and partial states of items cut across workgroups
    (qwen3_varlen_prefill_workspace_bytes() bytes, zeroed once; default: one
    per device and stream, kept by this module).  Without a workspace no
    item is cut: each runs whole in one workgroup.
    """
    assert q.dim() == 3 and q.shape[1] == num_heads and q.shape[2] == head_dim
    assert k.shape == (q.shape[0], num_kv_heads, head_dim) and v.shape == k.shape
    assert q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16, \
        "HIP prefill kernel is bf16 only"
    dev = _lib.require_hip(q, k, v, cu_seqlens)
    q = q if q.stride(2) == 1 else q.contiguous()
    k = k if k.stride(2) == 1 else k.contiguous()
    v = v if v.stride(2) == 1 else v.contiguous()
    if cu_seqlens.dtype != torch.int32:
        cu_seqlens = cu_seqlens.to(torch.int32)
    cu_seqlens = cu_seqlens.contiguous()
    num_seqs = cu_seqlens.shape[0] - 1
    if max_seqlen is None:
        cu_cpu = cu_seqlens.cpu()
        max_seqlen = int((cu_cpu[1:] - cu_cpu[:-1]).max().item()) if num_seqs > 0 else 0
    if out is None:
        out = torch.empty_like(q)
    else:
        assert out.shape == q.shape and out.dtype == torch.bfloat16 and out.stride(2) == 1, \
            "out must be a bf16 (total_tokens, num_heads, head_dim) tensor with unit last stride"
        _lib.require_hip(out)
    lib = _lib.load()
    stream = _lib.stream_of(dev)
    if workspace is None:
        workspace = _schedule_workspace(q.device, stream, lib)
    rc = lib.qwen3_varlen_prefill_bf16(
        q.data_ptr(), _lib.strides(q, (0, 1)),
        k.data_ptr(), _lib.strides(k, (0, 1)),
        v.data_ptr(), _lib.strides(v, (0, 1)),
        out.data_ptr(), _lib.strides(out, (0, 1)),
        cu_seqlens.data_ptr(), num_seqs, int(max_seqlen), q.shape[0],
        num_heads, num_kv_heads, head_dim, float(scale), 1 if causal else 0,
        workspace.data_ptr(), workspace.numel(), stream)
    _lib.check(rc, "qwen3_varlen_prefill_bf16")
    return out


def flash_attention_prefill_batched(q, k, v, lens, scaling, num_heads, num_kv_heads, head_dim):
    """Right-padded batch adaptor (reference: flash_attention_prefill_batched,
    qwen3/kernels/flash_attention_varlen.py:197-258).

    q: (B, num_heads, S, D); k, v: (B, num_kv_heads, S, D); lens: list[int]
    valid lengths (0 < lens[i] <= S).  Returns (B, S, num_heads * D) with pad
    rows zero.  The lengths are host data, so max_seqlen needs no device sync.
    """
    B, H, S, D = q.shape
    H_kv = k.shape[1]
    assert len(lens) == B, "lens must have one entry per batch row"
    assert all(0 < l <= S for l in lens), "lens out of range (need 0 < lens_i <= S)"
    q2 = q.permute(0, 2, 1, 3).reshape(B * S, H, D)
    k2 = k.permute(0, 2, 1, 3).reshape(B * S, H_kv, D)
    v2 = v.permute(0, 2, 1, 3).reshape(B * S, H_kv, D)
    if all(l == S for l in lens):
        cu = torch.arange(B + 1, device=q.device, dtype=torch.int32) * S
        out_f = flash_attention_prefill(q2, k2, v2, cu, scaling, num_heads, num_kv_heads,
                                        head_dim, max_seqlen=S)
        return out_f.reshape(B, S, H * D)
    s_idx = torch.arange(S, device=q.device)
    lens_t = torch.tensor(lens, device=q.device, dtype=torch.long)
    valid = (s_idx[None, :] < lens_t[:, None]).reshape(-1)
    q_f, k_f, v_f = q2[valid], k2[valid], v2[valid]
    cu = torch.zeros(B + 1, dtype=torch.int32, device=q.device)
    torch.cumsum(torch.tensor(lens, dtype=torch.int32, device=q.device), 0, out=cu[1:])
    out_f = flash_attention_prefill(q_f, k_f, v_f, cu, scaling, num_heads, num_kv_heads,
                                    head_dim, max_seqlen=max(lens))
    out = torch.zeros(B * S, H, D, dtype=q.dtype, device=q.device)
    out[valid] = out_f
    return out.reshape(B, S, H * D)
