"""Oracle for the whole Qwen3 forward — TEST INFRASTRUCTURE ONLY.

Restates, in PyTorch on the CPU, the reference Qwen3ForCausalLM forward for
one request over a fresh cache, in the order the reference calls its
modules:
  embedding                       qwen3/model.py:65
  per layer (qwen3/decoder.py:40-57):
    input_layernorm (RMSNorm)     qwen3/norm.py:22-26
    qkv_proj, split into heads    qwen3/attention.py:81-88
    q_norm, k_norm                qwen3/attention.py:91-92
    RoPE at positions 0..S-1      qwen3/rope.py:88-110, tables :42-58
    causal GQA attention          qwen3/attention.py:193-207 (+ the causal
                                  mask of qwen3/model.py:150-161)
    o_proj, residual add          qwen3/attention.py:187, decoder.py:49
    post_attention_layernorm, gate_up_proj, silu(gate) * up, down_proj,
    residual add                  qwen3/mlp.py:31-36, decoder.py:52-55
  final norm, lm_head             qwen3/model.py:184, 241
With teacher forcing, the logits of position s equal those of the decode
step that consumes token s, so one call checks a prefill and every decode
step after it.

dtype=float32 is the exact-arithmetic reference the GPU engine is measured
against; dtype=bfloat16 runs the same steps with the reference's bf16
roundings (bf16 GEMM outputs, norms in fp32 cast back, cos/sin cast to
bf16, softmax in fp32 cast to bf16), i.e. what the reference's own bf16
forward would produce up to GEMM summation order.  The fp32 form is pinned
against the independent Qwen3 implementation of the transformers library
(tests/test_oracle.py).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = ["qwen3_logits_ref", "generate_greedy_ref"]


def _rms(x, w, eps):
    xf = x.float()
    return ((xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)) * w.float()).to(x.dtype)


def _rope_tables(head_dim, base, n):
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    freqs = torch.outer(torch.arange(n, dtype=torch.float32), inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def _expand_kv(x, G):
    """(Hkv, S, D) -> (Hkv * G, S, D): query head h reads kv head h // G
    (repeat_kv, qwen3/attention.py:31-36)."""
    return x.repeat_interleave(G, dim=0).contiguous()


def qwen3_logits_ref(state: dict, cfg, ids, dtype=torch.float32) -> torch.Tensor:
    """state: parameter tensors under the reference's names (fused qkv_proj /
    gate_up_proj; lm_head.weight optional when embeddings are tied); cfg: a
    Qwen3Config; ids: (S,) token ids.  Returns fp32 logits (S, vocab)."""
    def W(name):
        return state[name].to(dtype)

    ids = torch.as_tensor(ids, dtype=torch.long).reshape(-1)
    S = ids.numel()
    Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    G = Hq // Hkv
    eps = cfg.rms_norm_eps
    cos, sin = _rope_tables(D, cfg.rope_theta, S)
    cos, sin = cos.to(dtype)[None], sin.to(dtype)[None]  # (1, S, D), .to(q.dtype)
    causal = torch.full((S, S), float("-inf")).triu(1)

    h = W("model.embed_tokens.weight")[ids]  # (S, hidden)
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        x = _rms(h, W(p + "input_layernorm.weight"), eps)
        qkv = x @ W(p + "self_attn.qkv_proj.weight").T
        q = qkv[:, :Hq * D].view(S, Hq, D).transpose(0, 1)          # (Hq, S, D)
        k = qkv[:, Hq * D:(Hq + Hkv) * D].view(S, Hkv, D).transpose(0, 1)
        v = qkv[:, (Hq + Hkv) * D:].view(S, Hkv, D).transpose(0, 1)
        q = _rms(q, W(p + "self_attn.q_norm.weight"), eps)
        k = _rms(k, W(p + "self_attn.k_norm.weight"), eps)
        q = q * cos + _rotate_half(q) * sin
        k = k * cos + _rotate_half(k) * sin
        k, v = _expand_kv(k, G), _expand_kv(v, G)
        s = torch.matmul(q, k.transpose(1, 2).contiguous()) * (D ** -0.5)
        a = F.softmax(s.float() + causal, dim=-1).to(dtype)
        o = torch.matmul(a, v).transpose(0, 1).reshape(S, Hq * D)
        h = h + o @ W(p + "self_attn.o_proj.weight").T
        x = _rms(h, W(p + "post_attention_layernorm.weight"), eps)
        gu = x @ W(p + "mlp.gate_up_proj.weight").T
        I = gu.shape[1] // 2
        h = h + (F.silu(gu[:, :I]) * gu[:, I:]) @ W(p + "mlp.down_proj.weight").T
    x = _rms(h, W("model.norm.weight"), eps)
    lm = state.get("lm_head.weight", state["model.embed_tokens.weight"]).to(dtype)
    return (x @ lm.T).float()


def generate_greedy_ref(state: dict, cfg, prompt, n_new: int, dtype=torch.float32):
    """Greedy generation of one request with a K/V cache, as the reference's
    serial generate() drives Qwen3ForCausalLM (generate.py: one prefill
    forward, then one token per decode forward over the cached K/V,
    qwen3/model.py:31-184; attention over the cache as in
    qwen3/paged_attention.py:39-122 without the paging).  Returns (tokens
    (n_new,), logits (n_new, vocab) fp32): logits[i] chose tokens[i].
    The timed CPU baseline of the serving line; its per-step logits equal
    qwen3_logits_ref's at the same positions (tests/test_oracle.py)."""
    Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    G = Hq // Hkv
    eps = cfg.rms_norm_eps
    L0 = len(prompt)
    cos_t, sin_t = _rope_tables(D, cfg.rope_theta, L0 + n_new)
    cos_t, sin_t = cos_t.to(dtype), sin_t.to(dtype)
    W = {k: v.to(dtype) for k, v in state.items()}
    lm = W.get("lm_head.weight", W["model.embed_tokens.weight"])
    cache = [[None, None] for _ in range(cfg.num_hidden_layers)]

    def forward(ids, start):
        S = ids.numel()
        cos, sin = cos_t[start:start + S][None], sin_t[start:start + S][None]
        h = W["model.embed_tokens.weight"][ids]
        for i in range(cfg.num_hidden_layers):
            p = f"model.layers.{i}."
            x = _rms(h, W[p + "input_layernorm.weight"], eps)
            qkv = x @ W[p + "self_attn.qkv_proj.weight"].T
            q = qkv[:, :Hq * D].view(S, Hq, D).transpose(0, 1)
            k = qkv[:, Hq * D:(Hq + Hkv) * D].view(S, Hkv, D).transpose(0, 1)
            v = qkv[:, (Hq + Hkv) * D:].view(S, Hkv, D).transpose(0, 1)
            q = _rms(q, W[p + "self_attn.q_norm.weight"], eps)
            k = _rms(k, W[p + "self_attn.k_norm.weight"], eps)
            q = q * cos + _rotate_half(q) * sin
            k = k * cos + _rotate_half(k) * sin
            if cache[i][0] is not None:
                k = torch.cat([cache[i][0], k], dim=1)
                v = torch.cat([cache[i][1], v], dim=1)
            cache[i] = [k, v]
            T = k.shape[1]
            ke, ve = _expand_kv(k, G), _expand_kv(v, G)
            s = torch.matmul(q, ke.transpose(1, 2).contiguous()) * (D ** -0.5)
            # query row r sits at position start + r and sees keys 0..start + r
            mask = torch.full((S, T), float("-inf")).triu(start + 1)
            a = F.softmax(s.float() + mask, dim=-1).to(dtype)
            o = torch.matmul(a, ve).transpose(0, 1).reshape(S, Hq * D)
            h = h + o @ W[p + "self_attn.o_proj.weight"].T
            x = _rms(h, W[p + "post_attention_layernorm.weight"], eps)
            gu = x @ W[p + "mlp.gate_up_proj.weight"].T
            I = gu.shape[1] // 2
            h = h + (F.silu(gu[:, :I]) * gu[:, I:]) @ W[p + "mlp.down_proj.weight"].T
        x = _rms(h[-1:], W["model.norm.weight"], eps)
        return (x @ lm.T).float()[0]

    ids = torch.as_tensor(prompt, dtype=torch.long).reshape(-1)
    tokens, logits = [], []
    lg = forward(ids, 0)
    for step in range(n_new):
        tok = int(torch.argmax(lg))
        tokens.append(tok)
        logits.append(lg)
        if step + 1 < n_new:
            lg = forward(torch.tensor([tok]), L0 + step)
    return torch.tensor(tokens), torch.stack(logits)
