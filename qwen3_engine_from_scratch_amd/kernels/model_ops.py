"""Kernels around the attention path of a Qwen3 decoder step, on the gfx950
HIP library (include/qwen3_model_ops.h): residual add + RMSNorm (also the
embedding lookup and the final-norm row selection), SwiGLU activation,
greedy token choice, the resident-length advance, and the decode-batch
linear layers with the norm / residual add / activation folded in.

Reference modules: qwen3/norm.py:22-26, qwen3/decoder.py:49,55,
qwen3/mlp.py:31-36, qwen3/attention.py:81,187, qwen3/model.py:212,241,
qwen3/sampling.py:256-258, qwen3/PagedKVcache.py:216-219.
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["add_rms_norm", "embed_rms_norm", "silu_mul", "argmax", "advance_seq_lens",
           "lm_head_argmax", "LM_HEAD_ARGMAX_MAX_K",
           "decode_linear", "decode_qkv_rope", "embed_ss", "DECODE_LINEAR_MAX_ROWS"]

DECODE_LINEAR_MAX_ROWS = 64
LM_HEAD_ARGMAX_MAX_K = 1024
_EPI = {"store": 0, "residual": 1, "silu": 2}


def _rows2d(t: torch.Tensor) -> torch.Tensor:
    assert t.dim() == 2 and t.stride(1) == 1, "expected a (rows, hidden) row-major view"
    return t


def add_rms_norm(x: torch.Tensor | None, residual: torch.Tensor, weight: torch.Tensor,
                 eps: float, *, residual_out: torch.Tensor | None = None,
                 out: torch.Tensor | None = None,
                 row_index: torch.Tensor | None = None) -> torch.Tensor:
    """h = residual + x (bf16; x None: h = residual), out = RMSNorm(h) * weight;
    h is stored in `residual_out` when given (pass `residual` itself for the
    in-place residual-stream update of a decoder layer).

    row_index (int64, optional): output row i reads source row row_index[i]
    (the final norm over the last token of each packed sequence).
    Returns `out` (rows, hidden) bf16.
    """
    residual = _rows2d(residual)
    if x is not None:
        x = _rows2d(x)
        assert x.shape == residual.shape
    hidden = residual.shape[1]
    if row_index is not None:
        assert row_index.dtype == torch.int64
        row_index = row_index.reshape(-1).contiguous()
        rows = row_index.numel()
    else:
        rows = residual.shape[0]
    assert weight.dtype == residual.dtype == torch.bfloat16 and weight.is_contiguous()
    dev = _lib.require_hip(x, residual, weight, residual_out, out, row_index)
    if out is None:
        out = torch.empty(rows, hidden, dtype=residual.dtype, device=residual.device)
    _rows2d(out)
    if residual_out is not None:
        _rows2d(residual_out)
        assert residual_out.shape == (rows, hidden)
    rc = _lib.load().qwen3_add_rms_norm_bf16(
        _lib.ptr(x), x.stride(0) if x is not None else 0,
        residual.data_ptr(), residual.stride(0),
        _lib.ptr(residual_out), residual_out.stride(0) if residual_out is not None else 0,
        weight.data_ptr(), float(eps), out.data_ptr(), out.stride(0),
        _lib.ptr(row_index), residual.shape[0], rows, hidden, _lib.stream_of(dev))
    _lib.check(rc, "qwen3_add_rms_norm_bf16")
    return out


def embed_rms_norm(ids: torch.Tensor, embed_weight: torch.Tensor, norm_weight: torch.Tensor,
                   eps: float, *, hidden_out: torch.Tensor | None = None,
                   out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Embedding lookup fused with layer 0's input RMSNorm: returns
    (hidden, normed), both (tokens, hidden) bf16.  ids: int64 token ids; an
    id outside the vocabulary gives zero rows."""
    ids = ids.reshape(-1)
    assert ids.dtype == torch.int64
    n = ids.numel()
    H = embed_weight.shape[1]
    if hidden_out is None:
        hidden_out = torch.empty(n, H, dtype=embed_weight.dtype, device=embed_weight.device)
    out = add_rms_norm(None, embed_weight, norm_weight, eps, residual_out=hidden_out, out=out,
                       row_index=ids)
    return hidden_out, out


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """SwiGLU activation of the fused gate/up projection (rows, 2*I) ->
    (rows, I): bf16(bf16(silu(gate)) * up)."""
    gate_up = _rows2d(gate_up)
    rows, two_i = gate_up.shape
    assert two_i % 2 == 0 and gate_up.dtype == torch.bfloat16
    inter = two_i // 2
    dev = _lib.require_hip(gate_up, out)
    if out is None:
        out = torch.empty(rows, inter, dtype=gate_up.dtype, device=gate_up.device)
    _rows2d(out)
    rc = _lib.load().qwen3_silu_mul_bf16(gate_up.data_ptr(), gate_up.stride(0), out.data_ptr(),
                                         out.stride(0), rows, inter, _lib.stream_of(dev))
    _lib.check(rc, "qwen3_silu_mul_bf16")
    return out


def argmax(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy choice over (rows, vocab) bf16 logits -> (rows,) int64: the
    first index of the maximum, NaN ranking highest (torch.argmax's rule)."""
    logits = _rows2d(logits)
    assert logits.dtype == torch.bfloat16
    rows, vocab = logits.shape
    dev = _lib.require_hip(logits, out)
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    assert out.dtype == torch.int64 and out.is_contiguous() and out.numel() == rows
    rc = _lib.load().qwen3_argmax_bf16(logits.data_ptr(), logits.stride(0), rows, vocab,
                                       out.data_ptr(), _lib.stream_of(dev))
    _lib.check(rc, "qwen3_argmax_bf16")
    return out


def lm_head_argmax_ok(hidden: int) -> bool:
    """Whether lm_head_argmax handles this hidden size."""
    return hidden % 512 == 0 and hidden <= LM_HEAD_ARGMAX_MAX_K


def lm_head_argmax(h: torch.Tensor, ss_in: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                   weight: torch.Tensor, *, out: torch.Tensor | None = None,
                   workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy tokens of a decode step, (M,) int64, for M <= 64 rows of the
    residual stream h (M, K) bf16: argmax over the vocabulary of
    bf16(RMSNorm(h) @ weight^T), the rms taken from ss_in (M, K/16) fp32
    per-16-column sums of h^2 (written by the last residual epilogue), in
    one pass over weight (V, K) without storing the logits.  Ties take the
    first index and NaN ranks highest (torch.argmax's rule)."""
    h = _rows2d(h)
    M, K = h.shape
    V = weight.shape[0]
    assert h.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
    assert norm_weight.dtype == torch.bfloat16 and norm_weight.is_contiguous()
    assert ss_in.dtype == torch.float32 and ss_in.is_contiguous() and ss_in.shape[0] == M
    assert weight.shape[1] == K and weight.stride(1) == 1
    assert M <= DECODE_LINEAR_MAX_ROWS and lm_head_argmax_ok(K)
    dev = _lib.require_hip(h, ss_in, norm_weight, weight, out, workspace)
    if out is None:
        out = torch.empty(M, dtype=torch.int64, device=h.device)
    assert out.dtype == torch.int64 and out.is_contiguous() and out.numel() == M
    lib = _lib.load()
    need = int(lib.qwen3_lm_head_argmax_workspace_bytes())
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=h.device)
    rc = lib.qwen3_lm_head_argmax_bf16(h.data_ptr(), h.stride(0), ss_in.data_ptr(),
                                       ss_in.shape[1], norm_weight.data_ptr(), float(eps),
                                       weight.data_ptr(), weight.stride(0), M, V, K,
                                       workspace.data_ptr(), workspace.numel(), out.data_ptr(),
                                       _lib.stream_of(dev))
    _lib.check(rc, "qwen3_lm_head_argmax_bf16")
    return out


def advance_seq_lens(seq_lens: torch.Tensor, row_ids: torch.Tensor, skip_row: int = -1,
                     delta: int = 1) -> None:
    """seq_lens[row_ids[i]] += delta on the device, except rows equal to
    skip_row; listed rows other than skip_row must be distinct."""
    assert seq_lens.dtype == torch.int32 and seq_lens.is_contiguous()
    assert row_ids.dtype == torch.int32 and row_ids.is_contiguous()
    dev = _lib.require_hip(seq_lens, row_ids)
    rc = _lib.load().qwen3_advance_seq_lens(seq_lens.data_ptr(), seq_lens.numel(),
                                            row_ids.data_ptr(), row_ids.numel(), int(skip_row),
                                            int(delta), _lib.stream_of(dev))
    _lib.check(rc, "qwen3_advance_seq_lens")


def decode_linear(x: torch.Tensor, weight: torch.Tensor, *, epilogue: str = "store",
                  ss_in: torch.Tensor | None = None, norm_weight: torch.Tensor | None = None,
                  eps: float = 1e-6, residual: torch.Tensor | None = None,
                  residual_out: torch.Tensor | None = None, ss_out: torch.Tensor | None = None,
                  out: torch.Tensor | None = None) -> torch.Tensor | None:
    """y = a @ weight^T for at most 64 rows (a decode batch), weight the
    (out, in) nn.Linear matrix.  With ss_in (rows, tiles) fp32 partial sums
    of x^2 and norm_weight, a = RMSNorm(x) computed on the fly.  Epilogues:
      "store"     returns y (rows, out) bf16;
      "residual"  residual_out = bf16(residual + bf16(y)) and ss_out
                  (rows, out/16) its per-16-column sums of squares; returns None;
      "silu"      weight holds gate then up rows (2I, in): returns
                  bf16(bf16(silu(gate)) * up), (rows, I).
    """
    x = _rows2d(x)
    M, K = x.shape
    assert weight.dim() == 2 and weight.stride(1) == 1 and weight.shape[1] == K
    assert x.dtype == weight.dtype == torch.bfloat16
    epi = _EPI[epilogue]
    N = weight.shape[0] // 2 if epilogue == "silu" else weight.shape[0]
    if ss_in is not None:
        assert ss_in.dtype == torch.float32 and ss_in.is_contiguous() and ss_in.shape[0] == M
        assert norm_weight is not None and norm_weight.is_contiguous() and norm_weight.numel() == K
    if epilogue == "residual":
        assert residual is not None and residual_out is not None and ss_out is not None
        assert residual.shape == residual_out.shape == (M, N)
        assert ss_out.dtype == torch.float32 and ss_out.is_contiguous() and ss_out.shape == (M, N // 16)
        assert residual_out.data_ptr() != residual.data_ptr(), "residual_out must not alias residual"
    elif out is None:
        out = torch.empty(M, N, dtype=x.dtype, device=x.device)
    dev = _lib.require_hip(x, weight, ss_in, norm_weight, residual, residual_out, ss_out, out)
    rc = _lib.load().qwen3_decode_linear_bf16(
        x.data_ptr(), x.stride(0), _lib.ptr(ss_in), ss_in.shape[1] if ss_in is not None else 0,
        _lib.ptr(norm_weight), float(eps), weight.data_ptr(), weight.stride(0), M, N, K, epi,
        _lib.ptr(out), out.stride(0) if out is not None else 0,
        _lib.ptr(residual), residual.stride(0) if residual is not None else 0,
        _lib.ptr(residual_out), residual_out.stride(0) if residual_out is not None else 0,
        _lib.ptr(ss_out), N if epilogue == "silu" else 0, _lib.stream_of(dev))
    _lib.check(rc, "qwen3_decode_linear_bf16")
    return out if epilogue != "residual" else None


def embed_ss(ids: torch.Tensor, embed_weight: torch.Tensor, *, h_out: torch.Tensor | None = None,
             ss_out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Embedding rows (tokens, hidden) bf16 plus their per-16-column sums of
    squares (tokens, hidden/16) fp32, the input of a normed decode_linear."""
    ids = ids.reshape(-1)
    assert ids.dtype == torch.int64 and ids.is_contiguous()
    V, H = embed_weight.shape
    M = ids.numel()
    if h_out is None:
        h_out = torch.empty(M, H, dtype=embed_weight.dtype, device=embed_weight.device)
    if ss_out is None:
        ss_out = torch.empty(M, H // 16, dtype=torch.float32, device=embed_weight.device)
    dev = _lib.require_hip(ids, embed_weight, h_out, ss_out)
    rc = _lib.load().qwen3_embed_ss_bf16(ids.data_ptr(), embed_weight.data_ptr(),
                                         embed_weight.stride(0), V, H, M, h_out.data_ptr(),
                                         h_out.stride(0), ss_out.data_ptr(), _lib.stream_of(dev))
    _lib.check(rc, "qwen3_embed_ss_bf16")
    return h_out, ss_out


def decode_qkv_rope(h: torch.Tensor, ss_in: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                    qkv_weight: torch.Tensor, num_heads: int, num_kv_heads: int,
                    q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, head_eps: float,
                    cos_table: torch.Tensor, sin_table: torch.Tensor, pool, layer_idx: int,
                    row_ids: torch.Tensor | None, positions: torch.Tensor | None = None,
                    q_out: torch.Tensor | None = None) -> torch.Tensor:
    """Input RMSNorm + qkv projection + QK-norm + RoPE + K/V pool write of a
    decode step for at most 64 tokens in one launch; returns q (M, Hq, 128)
    for the attention kernel (k and v go into `pool` at seq_lens[row])."""
    h = _rows2d(h)
    M, K = h.shape
    D = 128
    assert qkv_weight.shape == ((num_heads + 2 * num_kv_heads) * D, K)
    assert ss_in.dtype == torch.float32 and ss_in.is_contiguous() and ss_in.shape[0] == M
    assert cos_table.dtype == sin_table.dtype == torch.float32 and cos_table.stride(1) == 1
    kb, vb = pool.k_buffer, pool.v_buffer
    bt = pool.block_table_2d
    dev = _lib.require_hip(h, ss_in, qkv_weight, kb, cos_table, row_ids)
    if row_ids is not None:
        assert row_ids.dtype == torch.int32 and row_ids.is_contiguous() and row_ids.numel() == M
    if positions is not None:
        positions = positions.reshape(-1)
        assert positions.dtype == torch.int64 and positions.numel() == M
        positions = positions.contiguous()
    if q_out is None:
        q_out = torch.empty(M, num_heads, D, dtype=h.dtype, device=h.device)
    rc = _lib.load().qwen3_decode_qkv_rope_bf16(
        h.data_ptr(), h.stride(0), ss_in.data_ptr(), ss_in.shape[1], norm_weight.data_ptr(),
        float(eps), qkv_weight.data_ptr(), qkv_weight.stride(0), M, K, num_heads, num_kv_heads,
        D, q_norm_weight.data_ptr(), k_norm_weight.data_ptr(), float(head_eps),
        cos_table.data_ptr(), sin_table.data_ptr(), cos_table.stride(0), cos_table.shape[0],
        _lib.ptr(positions), q_out.data_ptr(), _lib.strides(q_out, (0, 1)),
        kb.data_ptr(), _lib.strides(kb, (0, 1, 2, 3)), vb.data_ptr(), _lib.strides(vb, (0, 1, 2, 3)),
        kb.shape[0], int(layer_idx), kb.shape[1], pool.seq_lens.data_ptr(), bt.data_ptr(), bt.stride(0),
        bt.shape[0], bt.shape[1], _lib.ptr(row_ids), kb.shape[3], _lib.stream_of(dev))
    _lib.check(rc, "qwen3_decode_qkv_rope_bf16")
    return q_out
