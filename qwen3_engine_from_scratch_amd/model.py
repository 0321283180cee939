"""Qwen3 causal LM whose decoder steps run on the gfx950 kernels of this
package.

Module tree and parameter names are the reference's (qwen3/model.py,
decoder.py, attention.py, mlp.py, norm.py, rope.py), so a state dict the
reference loads (fused qkv_proj / gate_up_proj) loads here unchanged.  The
forward passes are not module-by-module: one decoder layer is

    add_rms_norm -> qkv GEMM -> fused QK-norm/RoPE/pool write -> attention
    -> o_proj GEMM -> add_rms_norm -> gate_up GEMM -> silu_mul -> down GEMM

with the residual add folded into the next norm, the embedding lookup folded
into layer 0's norm, and the final norm applied only to the rows whose
logits are needed.  The GEMMs are plain library GEMMs (torch -> hipBLASLt);
everything else is a hand-written HIP kernel.  There is no CPU path.

Entry points:
  forward(input_ids, kv_cache, input_lens)          drop-in for
      Qwen3ForCausalLM.forward (qwen3/model.py:230-241 with :31-184)
  forward_decode(input_ids, position_ids, row_ids, caches)
      capture-friendly decode step (qwen3/model.py:243-251 with :186-217)
  decode_logits / prefill_logits                    the same steps on packed
      device inputs, used by the batching engine and the graph runner.
"""
from __future__ import annotations

import zlib

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from .config import Qwen3Config
from .kernels.flash_attention_varlen import flash_attention_prefill
from .kernels.model_ops import (DECODE_LINEAR_MAX_ROWS, add_rms_norm, argmax, decode_linear,
                                decode_qkv_rope, embed_rms_norm, embed_ss, lm_head_argmax,
                                lm_head_argmax_ok, silu_mul)
from . import _lib
from .kernels.paged_attention import paged_attention_decode_hip, paged_decode_workspace_bytes
from .kernels.pre_attention import qk_norm_rope_decode, qk_norm_rope_prefill, rope_tables

__all__ = ["Qwen3ForCausalLM", "Qwen3Model", "init_random_weights"]


class RMSNorm(nn.Module):
    """Parameter holder (qwen3/norm.py:15-20); the math is in add_rms_norm
    and the fused pre-attention kernel."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps


class RotaryEmbedding(nn.Module):
    """fp32 cos/sin tables (max_seq_len, head_dim) (qwen3/rope.py:42-58).
    Kept as plain fp32 tensors, not buffers, so casting the model to bf16
    leaves them alone: the kernels round cos/sin to bf16 themselves, as the
    reference's cast to q.dtype does."""

    def __init__(self, head_dim: int, base: float = 1e6, max_seq_len: int = 4096):
        super().__init__()
        self.head_dim, self.base, self.max_seq_len = head_dim, base, max_seq_len
        self._cpu = rope_tables(head_dim, base, max_seq_len)
        self._dev = {}

    def tables(self, device: torch.device):
        key = str(device)
        if key not in self._dev:
            self._dev[key] = tuple(t.to(device) for t in self._cpu)
        return self._dev[key]


class Qwen3Attention(nn.Module):
    def __init__(self, config: Qwen3Config, layer_idx: int):
        super().__init__()
        self.layer_idx = layer_idx
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        self.q_output_dim = self.num_heads * self.head_dim
        self.kv_output_dim = self.num_kv_heads * self.head_dim
        self.scaling = self.head_dim ** -0.5
        self.qkv_proj = nn.Linear(config.hidden_size, self.q_output_dim + 2 * self.kv_output_dim,
                                  bias=False)
        self.o_proj = nn.Linear(self.q_output_dim, config.hidden_size, bias=False)
        self.q_norm = RMSNorm(self.head_dim, config.rms_norm_eps)
        self.k_norm = RMSNorm(self.head_dim, config.rms_norm_eps)

    def split(self, qkv: torch.Tensor):
        """(T, q+k+v) fused projection -> (T, H, D) views of q, k, v."""
        T = qkv.shape[0]
        Q, KV, D = self.q_output_dim, self.kv_output_dim, self.head_dim
        return (qkv[:, :Q].view(T, self.num_heads, D),
                qkv[:, Q:Q + KV].view(T, self.num_kv_heads, D),
                qkv[:, Q + KV:].view(T, self.num_kv_heads, D))


class Qwen3MLP(nn.Module):
    def __init__(self, config: Qwen3Config):
        super().__init__()
        self.intermediate_size = config.intermediate_size
        self.gate_up_proj = nn.Linear(config.hidden_size, 2 * config.intermediate_size, bias=False)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=False)


class Qwen3DecoderLayer(nn.Module):
    def __init__(self, config: Qwen3Config, layer_idx: int):
        super().__init__()
        self.self_attn = Qwen3Attention(config, layer_idx)
        self.mlp = Qwen3MLP(config)
        self.input_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)


class Qwen3Model(nn.Module):
    def __init__(self, config: Qwen3Config):
        super().__init__()
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(
            [Qwen3DecoderLayer(config, i) for i in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.rotary_emb = RotaryEmbedding(config.head_dim, config.rope_theta,
                                          max_seq_len=config.max_position_embeddings)


class Qwen3ForCausalLM(nn.Module):
    def __init__(self, config: Qwen3Config):
        super().__init__()
        assert config.num_hidden_layers >= 1
        self.config = config
        self.model = Qwen3Model(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight
        self._workspace = None       # decode attention workspace of the current mode
        self._ws_mode = None
        self._superseded = []
        self._head_ws = None
        # Decode attention with the batch-invariant kernel: each sequence's
        # tokens independent of the rest of the batch (batched == serial),
        # at some HBM time where sequences are split across waves.
        self.decode_batch_invariant = False

    # ---- shared layer loop -------------------------------------------------

    def _run(self, ids: torch.Tensor, attend, final_index: torch.Tensor | None) -> torch.Tensor:
        """Embedding -> decoder layers -> final norm of the selected rows ->
        lm_head.  ids: (T,) int64 on the device; attend(i, attn_module, qkv)
        returns the attention output (T, Hq*D).  Returns logits (rows, V)."""
        eps = self.config.rms_norm_eps
        layers = self.model.layers
        residual, normed = embed_rms_norm(ids, self.model.embed_tokens.weight,
                                          layers[0].input_layernorm.weight, eps)
        d = None
        for i, layer in enumerate(layers):
            at = layer.self_attn
            qkv = F.linear(normed, at.qkv_proj.weight)
            o = F.linear(attend(i, at, qkv), at.o_proj.weight)
            normed = add_rms_norm(o, residual, layer.post_attention_layernorm.weight, eps,
                                  residual_out=residual)
            gu = F.linear(normed, layer.mlp.gate_up_proj.weight)
            d = F.linear(silu_mul(gu), layer.mlp.down_proj.weight)
            if i + 1 < len(layers):
                normed = add_rms_norm(d, residual, layers[i + 1].input_layernorm.weight, eps,
                                      residual_out=residual)
        final = add_rms_norm(d, residual, self.model.norm.weight, eps, row_index=final_index)
        return F.linear(final, self.lm_head.weight)

    # ---- decode ------------------------------------------------------------

    def reserve_decode_workspace(self, batch: int, pool) -> None:
        """Allocates the workspace of the decode attention (in the current
        mode, decode_batch_invariant) for up to `batch` rows once (a captured
        graph keeps using it)."""
        inv = bool(self.decode_batch_invariant)
        need = paged_decode_workspace_bytes(batch, self.config.num_attention_heads,
                                            self.config.num_key_value_heads,
                                            self.config.head_dim, pool.block_table_2d.shape[1],
                                            pool.block_size, batch_invariant=inv)
        if self._workspace is None or self._ws_mode != inv or self._workspace.numel() < need:
            if self._workspace is not None:
                # a graph captured earlier may still replay on the old buffer
                self._superseded.append(self._workspace)
            # zeroed once: the batch-invariant kernel's hand-off tickets start
            # at zero and every call leaves them there
            self._workspace = torch.zeros(max(need, 1), dtype=torch.uint8,
                                          device=pool.k_buffer.device)
            self._ws_mode = inv
        if self._head_ws is None:
            self._head_ws = torch.empty(int(_lib.load().qwen3_lm_head_argmax_workspace_bytes()),
                                        dtype=torch.uint8, device=pool.k_buffer.device)

    def fused_decode_ok(self, batch: int) -> bool:
        """Whether a decode step of `batch` rows runs on the fused decode
        linears (at most 64 rows; widths the kernels tile)."""
        c = self.config
        widths = (c.hidden_size, c.num_attention_heads * c.head_dim, c.intermediate_size)
        return (batch <= DECODE_LINEAR_MAX_ROWS and all(w % 128 == 0 for w in widths)
                and c.head_dim == 128 and c.hidden_size <= 4096)

    def _decode_fused(self, ids, row_ids, pool, positions) -> torch.Tensor:
        """Decode step on the fused kernels; returns the logits."""
        h, _ = self._decode_layers(ids, row_ids, pool, positions)
        # lm_head streams 311 MB of weights for few rows: the library GEMM
        # after a separate final norm
        final = add_rms_norm(None, h, self.model.norm.weight, self.config.rms_norm_eps)
        return F.linear(final, self.lm_head.weight)

    def _decode_layers(self, ids, row_ids, pool, positions):
        """The decoder layers of a decode step on the fused kernels: the
        residual stream ping-pongs between two buffers, each with its
        per-16-column sums of squares, so every RMSNorm is the prologue of
        the linear after it and every residual add the epilogue of the
        linear before it; the qkv projection also applies QK-norm and RoPE
        and writes K/V into the pool, leaving one attention launch (plus its
        merge) per layer.  Returns the last residual stream and its sums."""
        cfg = self.config
        eps = cfg.rms_norm_eps
        layers = self.model.layers
        B = ids.numel()
        Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        cos, sin = self.model.rotary_emb.tables(ids.device)
        ws = self._workspace
        h_a, ss_a = embed_ss(ids, self.model.embed_tokens.weight)
        h_b = torch.empty_like(h_a)
        ss_b = torch.empty_like(ss_a)
        for i, layer in enumerate(layers):
            at = layer.self_attn
            q = decode_qkv_rope(h_a, ss_a, layer.input_layernorm.weight, eps, at.qkv_proj.weight,
                                Hq, Hkv, at.q_norm.weight, at.k_norm.weight, eps, cos, sin, pool,
                                i, row_ids, positions)
            o = paged_attention_decode_hip(q, pool.k_buffer[:, i], pool.v_buffer[:, i],
                                           pool.block_table_2d, pool.seq_lens, row_ids,
                                           pool.block_size, workspace=ws,
                                           batch_invariant=self._ws_mode)
            decode_linear(o.view(B, Hq * D), at.o_proj.weight, epilogue="residual",
                          residual=h_a, residual_out=h_b, ss_out=ss_b)
            act = decode_linear(h_b, layer.mlp.gate_up_proj.weight, epilogue="silu", ss_in=ss_b,
                                norm_weight=layer.post_attention_layernorm.weight, eps=eps)
            decode_linear(act, layer.mlp.down_proj.weight, epilogue="residual",
                          residual=h_b, residual_out=h_a, ss_out=ss_a)
        return h_a, ss_a

    @torch.no_grad()
    def decode_greedy(self, ids: torch.Tensor, row_ids: torch.Tensor, pool,
                      positions: torch.Tensor | None = None,
                      out: torch.Tensor | None = None) -> torch.Tensor:
        """Greedy tokens (B,) int64 of one decode step, argmax of
        decode_logits(...).  On the fused path the final norm, lm_head and
        argmax run as one pass over the tied embedding that never stores the
        logits (qwen3_lm_head_argmax_bf16); out may alias ids (the ids are
        read before the tokens are written)."""
        B = ids.numel()
        cfg = self.config
        if out is None:
            out = torch.empty(B, dtype=torch.int64, device=ids.device)
        if self.fused_decode_ok(B) and lm_head_argmax_ok(cfg.hidden_size):
            self.reserve_decode_workspace(B, pool)
            rows = row_ids if row_ids is not None else torch.arange(
                B, dtype=torch.int32, device=ids.device)
            h, ss = self._decode_layers(ids.reshape(-1).contiguous(), rows.contiguous(), pool,
                                        positions)
            lm_head_argmax(h, ss, self.model.norm.weight, cfg.rms_norm_eps, self.lm_head.weight,
                           out=out.view(-1), workspace=self._head_ws)
            return out
        logits = self.decode_logits(ids, row_ids, pool, positions)
        return argmax(logits, out=out.view(-1))

    @torch.no_grad()
    def decode_logits(self, ids: torch.Tensor, row_ids: torch.Tensor, pool,
                      positions: torch.Tensor | None = None,
                      fused: bool | None = None) -> torch.Tensor:
        """One decode step for B requests: ids (B,) int64 (this step's input
        tokens), row_ids (B,) int32 resident-table rows.  Writes each token's
        K/V at position seq_lens[row] (pages must be reserved), attends over
        seq_lens[row] + 1 tokens and returns logits (B, V).  positions
        (B,) int64: RoPE positions (None: seq_lens[row]).  Does not advance
        seq_lens (the caller's job, as in the reference).  fused (None: when
        possible) selects the fused decode linears over the library GEMMs
        with separate norm / activation kernels."""
        B = ids.numel()
        cfg = self.config
        cos, sin = self.model.rotary_emb.tables(ids.device)
        self.reserve_decode_workspace(B, pool)
        ws = self._workspace
        Hq, D = cfg.num_attention_heads, cfg.head_dim

        def attend(i, at, qkv):
            q, k, v = at.split(qkv)
            qr = qk_norm_rope_decode(q, k, v, at.q_norm.weight, at.k_norm.weight,
                                     cfg.rms_norm_eps, cos, sin, pool, i, row_ids,
                                     positions=positions)
            o = paged_attention_decode_hip(qr, pool.k_buffer[:, i], pool.v_buffer[:, i],
                                           pool.block_table_2d, pool.seq_lens, row_ids,
                                           pool.block_size, workspace=ws,
                                           batch_invariant=self._ws_mode)
            return o.view(B, Hq * D)

        if fused is None:
            fused = self.fused_decode_ok(B)
        if fused:
            rows = row_ids if row_ids is not None else torch.arange(
                B, dtype=torch.int32, device=ids.device)
            return self._decode_fused(ids.reshape(-1).contiguous(), rows.contiguous(), pool,
                                      positions)
        return self._run(ids.reshape(-1), attend, None)

    @torch.no_grad()
    def forward_decode(self, input_ids: torch.Tensor, position_ids: torch.Tensor,
                       row_ids: torch.Tensor, caches: list) -> torch.Tensor:
        """Capture-friendly decode step (reference: Qwen3ForCausalLM.forward_decode,
        qwen3/model.py:243-251): no host state is touched; page reservation
        and seq_len advance are the caller's.  input_ids, position_ids: (B, 1)
        int64; row_ids: (B,) int32.  Returns logits (B, 1, V)."""
        B = input_ids.shape[0]
        pos = position_ids.reshape(B) if position_ids is not None else None
        logits = self.decode_logits(input_ids.reshape(B), row_ids, caches[0]._pool, pos)
        return logits.view(B, 1, -1)

    # ---- prefill -----------------------------------------------------------

    @torch.no_grad()
    def prefill_logits(self, ids: torch.Tensor, cu_seqlens: torch.Tensor, max_seqlen: int,
                       positions: torch.Tensor, slot_mapping: torch.Tensor | None, pool,
                       logit_rows: torch.Tensor | None) -> torch.Tensor:
        """Packed varlen prefill of n sequences (T tokens): ids (T,) int64,
        cu_seqlens (n+1,) int32, positions (T,) int64 RoPE positions,
        slot_mapping (T,) int64 pool slots (None or negative: not written).
        Returns logits of the rows in logit_rows (int64; None: every token)."""
        cfg = self.config
        cos, sin = self.model.rotary_emb.tables(ids.device)
        T = ids.numel()
        Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        kb = pool.k_buffer if pool is not None else None
        vb = pool.v_buffer if pool is not None else None
        if pool is None:  # no cache: the kernel still needs a pool to address
            kb = vb = torch.zeros(1, cfg.num_hidden_layers, Hkv, 16, D, dtype=torch.bfloat16,
                                  device=ids.device)
            slot_mapping = None

        def attend(i, at, qkv):
            q, k, v = at.split(qkv)
            qr, kr = qk_norm_rope_prefill(q, k, v, at.q_norm.weight, at.k_norm.weight,
                                          cfg.rms_norm_eps, cos, sin, positions, slot_mapping,
                                          kb, vb, i)
            o = flash_attention_prefill(qr, kr, v, cu_seqlens, at.scaling, Hq, Hkv, D,
                                        max_seqlen=max_seqlen)
            return o.view(T, Hq * D)

        return self._run(ids.reshape(-1), attend, logit_rows)

    # ---- drop-in forward ---------------------------------------------------

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, kv_cache=None,
                input_lens: list[int] | None = None) -> torch.Tensor:
        """Reference contract (qwen3/model.py:31-184, 230-241): input_ids
        (B, S), right-padded for a prefill batch with input_lens the valid
        lengths; kv_cache a PagedKVCache, a list of them (one per row) or None.
        Decode (S == 1 and seq_len > 0) reserves pages, writes K/V, attends and
        advances each handle by 1; prefill writes positions seq_len .. seq_len
        + len_i - 1 of each handle and advances it by len_i.  Returns logits
        (B, S, V); pad positions of a prefill batch are zero."""
        B, S = input_ids.shape
        dev = input_ids.device
        if kv_cache is None:
            caches = None
        elif isinstance(kv_cache, (list, tuple)):
            caches = list(kv_cache)
            assert len(caches) == B, "one kv cache handle per batch row"
        else:
            caches = [kv_cache]
        V = self.config.vocab_size

        if caches is not None and caches[0].seq_len > 0 and S == 1:
            for c in caches:
                c.reserve_next()
            pool = caches[0]._pool
            rows = torch.tensor([c.row_id for c in caches], dtype=torch.int32, device=dev)
            pos = torch.tensor([c.seq_len for c in caches], dtype=torch.int64, device=dev)
            logits = self.decode_logits(input_ids.reshape(B), rows, pool, pos)
            for c in caches:
                c.advance_seq_len(1)
            return logits.view(B, 1, V)

        lens = list(input_lens) if input_lens is not None else [S] * B
        assert len(lens) == B and all(0 < n <= S for n in lens)
        ids = torch.cat([input_ids[i, :n] for i, n in enumerate(lens)])
        cu = np.zeros(B + 1, dtype=np.int32)
        cu[1:] = np.cumsum(lens)
        # positions 0 .. len_i - 1 per request (qwen3/model.py:132-136)
        pos = np.concatenate([np.arange(n, dtype=np.int64) for n in lens])
        slots = None
        pool = None
        if caches is not None:
            pool = caches[0]._pool
            slots = np.concatenate([c.reserve_slots(n) for c, n in zip(caches, lens)])
            slots = torch.from_numpy(slots).to(dev)
        logits = self.prefill_logits(ids, torch.from_numpy(cu).to(dev), max(lens),
                                     torch.from_numpy(pos).to(dev), slots, pool, None)
        if caches is not None:
            for c, n in zip(caches, lens):
                c.advance_seq_len(n)
        out = torch.zeros(B, S, V, dtype=logits.dtype, device=dev)
        valid = torch.arange(S)[None, :] < torch.tensor(lens)[:, None]
        out[valid.to(dev)] = logits
        return out


def init_random_weights(model: Qwen3ForCausalLM, seed: int = 0, std: float = 0.02,
                        norm_jitter: float = 0.0) -> Qwen3ForCausalLM:
    """Seeded random initialisation in place (normal(0, std) projections and
    embeddings, RMSNorm weights 1 + norm_jitter * normal), generated on the
    parameters' device."""
    with torch.no_grad():
        for name, p in sorted(model.named_parameters(), key=lambda kv: kv[0]):
            g = torch.Generator(device=p.device).manual_seed(
                seed * 1000003 + zlib.crc32(name.encode()))
            if name.endswith("norm.weight"):
                p.copy_(1.0 + norm_jitter * torch.randn(p.shape, generator=g, device=p.device,
                                                        dtype=torch.float32))
            else:
                p.copy_(torch.randn(p.shape, generator=g, device=p.device,
                                    dtype=torch.float32) * std)
    return model
