"""Whole-model decode and prefill on the GPU: the row-wise kernels against
their oracle formulas, the model against the fp32 oracle (itself pinned to
the transformers Qwen3), the captured decode graphs against eager steps, and
greedy generation through the batching engine.

Bars:
  add_rms_norm, silu_mul   within one bf16 ulp of the oracle, >= 99% of the
                           values bit-identical (only fp32 summation order
                           and exp rounding may differ); the residual stream
                           and the embedding rows bit-exact.
  decode_linear            |got - ref| <= 2^-7 |ref| + 2^-9 max|ref| of the row
                           against the fp32 product rounded to bf16 (outputs
                           that nearly cancel move by more than an ulp when
                           the fp32 summation order changes).
  argmax                   the index torch.argmax returns, exactly.
  model logits             relative L2 error vs the fp32 oracle at most
                           max(2 x that of the reference's own bf16 forward
                           (the oracle's bf16 form), 0.03): the engine is no
                           further from exact arithmetic than the reference.
  graph replay             bit-identical to the eager step of the same
                           batch, on every replay.
  greedy tokens            each chosen token's fp32-oracle logit within
                           0.15 of that step's maximum (a near-tie may go
                           either way in bf16; a wrong token cannot); the
                           graph and eager engines token for token up to a
                           first difference at a near-tie.
"""
import pytest
import torch

from conftest import announce
from oracle import inputs as oi
from oracle import model as om

pytestmark = pytest.mark.gpu


def _ordered(t):
    b = t.contiguous().view(torch.int16).to(torch.int32)
    return torch.where(b >= 0, b, -(b & 0x7FFF))


def assert_ulp_close(got, ref, what, max_ulps=1, min_exact=0.99):
    d = (_ordered(got.cpu()) - _ordered(ref.cpu())).abs()
    assert d.max().item() <= max_ulps, f"{what}: {d.max().item()} ulps"
    exact = (d == 0).float().mean().item()
    assert exact >= min_exact, f"{what}: only {exact:.4f} bit-identical"


# ---- row-wise kernels --------------------------------------------------------

@pytest.mark.parametrize("rows,hidden", [(1, 1024), (37, 1024), (64, 4096), (5, 5120), (3, 264)])
def test_add_rms_norm_vs_oracle(gpu, rows, hidden):
    from qwen3_engine_from_scratch_amd.kernels.model_ops import add_rms_norm

    announce(f"add_rms_norm rows={rows} hidden={hidden}")
    g = torch.Generator().manual_seed(rows + hidden)
    x = (torch.randn(rows, hidden, generator=g) * 2).to(torch.bfloat16)
    r = (torch.randn(rows, hidden, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16)
    h_ref = (r.float() + x.float()).to(torch.bfloat16)
    n_ref = oi.rms_norm(h_ref, w, 1e-6)
    rd = r.to(gpu)
    out = add_rms_norm(x.to(gpu), rd, w.to(gpu), 1e-6, residual_out=rd)  # in place
    torch.cuda.synchronize()
    assert torch.equal(rd.cpu(), h_ref), "residual stream"
    assert_ulp_close(out, n_ref, "normed")
    # no add; strided rows
    big = torch.zeros(rows, hidden + 64, dtype=torch.bfloat16)
    big[:, :hidden] = r
    out2 = add_rms_norm(None, big.to(gpu)[:, :hidden], w.to(gpu), 1e-6)
    torch.cuda.synchronize()
    assert_ulp_close(out2, oi.rms_norm(r, w, 1e-6), "normed (no add)")


def test_embedding_and_row_selection(gpu):
    from qwen3_engine_from_scratch_amd.kernels.model_ops import add_rms_norm, embed_rms_norm

    announce("embed_rms_norm / row_index")
    g = torch.Generator().manual_seed(7)
    E = torch.randn(1000, 1024, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(1024, generator=g)).to(torch.bfloat16)
    ids = torch.tensor([5, 999, 0, 5, 1000, -3, 17], dtype=torch.int64)
    hid, normed = embed_rms_norm(ids.to(gpu), E.to(gpu), w.to(gpu), 1e-6)
    torch.cuda.synchronize()
    ok = (ids >= 0) & (ids < 1000)
    assert torch.equal(hid.cpu()[ok], E[ids[ok]])
    assert not hid.cpu()[~ok].any() and not normed.cpu()[~ok].any(), "out-of-range ids -> zero rows"
    assert_ulp_close(normed.cpu()[ok], oi.rms_norm(E[ids[ok]], w, 1e-6), "embedding norm")
    # final-norm row selection
    x = torch.randn(20, 1024, generator=g).to(torch.bfloat16)
    sel = torch.tensor([19, 0, 7], dtype=torch.int64)
    out = add_rms_norm(x.to(gpu), E[:20].to(gpu), w.to(gpu), 1e-6, row_index=sel.to(gpu))
    torch.cuda.synchronize()
    ref = oi.rms_norm((E[:20].float() + x.float()).to(torch.bfloat16)[sel], w, 1e-6)
    assert_ulp_close(out, ref, "selected rows")


@pytest.mark.parametrize("rows,inter", [(1, 3072), (64, 3072), (300, 8), (7, 12288)])
def test_silu_mul_vs_torch(gpu, rows, inter):
    from qwen3_engine_from_scratch_amd.kernels.model_ops import silu_mul

    announce(f"silu_mul rows={rows} inter={inter}")
    g = torch.Generator().manual_seed(rows * 7 + inter)
    gu = (torch.randn(rows, 2 * inter, generator=g) * 4).to(torch.bfloat16)
    ref = torch.nn.functional.silu(gu[:, :inter]) * gu[:, inter:]  # bf16 CPU, as qwen3/mlp.py:36
    out = silu_mul(gu.to(gpu))
    torch.cuda.synchronize()
    assert_ulp_close(out, ref, "silu_mul")


@pytest.mark.parametrize("rows,vocab", [(1, 151936), (64, 151936), (5, 1001), (3, 8)])
def test_argmax_matches_torch(gpu, rows, vocab):
    from qwen3_engine_from_scratch_amd.kernels.model_ops import argmax

    announce(f"argmax rows={rows} vocab={vocab}")
    g = torch.Generator().manual_seed(rows + vocab)
    x = torch.randn(rows, vocab, generator=g).to(torch.bfloat16)
    if rows >= 3:
        x[0] = 0.5                                  # all tied: first index
        x[1, vocab // 3] = x[1, -1] = 9.0           # tie between two maxima
        x[2] = float("-inf")
        x[2, vocab - 1] = -1e30
    if rows >= 5:
        x[3, vocab // 2] = float("nan")             # NaN ranks highest
        x[4] = -0.0
        x[4, 1] = 0.0                               # -0 == +0: first index
    got = argmax(x.to(gpu)).cpu()
    ref = torch.argmax(x, dim=-1)
    assert torch.equal(got, ref), (got, ref)


def test_advance_seq_lens(gpu):
    from qwen3_engine_from_scratch_amd.kernels.model_ops import advance_seq_lens

    announce("advance_seq_lens")
    sl = torch.arange(10, dtype=torch.int32, device=gpu)
    rows = torch.tensor([3, 9, 7, 7, 7, 0], dtype=torch.int32, device=gpu)
    advance_seq_lens(sl, rows, skip_row=7)
    torch.cuda.synchronize()
    assert sl.cpu().tolist() == [1, 1, 2, 4, 4, 5, 6, 7, 8, 10]


def _close(got, ref, what):
    """|got - ref| <= 2^-7 |ref| + 2^-9 max|ref| per row: one bf16 ulp of the
    output (a rounding that tips the other way) plus what a different fp32
    summation order, or a one-ulp change of a normalised input entry, moves an
    output that nearly cancels."""
    got, ref = got.float().cpu(), ref.float().cpu()
    bound = ref.abs() * 2 ** -7 + ref.abs().amax(-1, keepdim=True) * 2 ** -9
    bad = (got - ref).abs() > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} values off, max {(got - ref).abs().max():.3g}"


@pytest.mark.parametrize("M,K,N", [(1, 1024, 4096), (64, 1024, 4096), (37, 2048, 1024),
                                   (64, 3072, 1024), (5, 128, 16)])
def test_decode_linear_store_and_norm(gpu, M, K, N):
    from qwen3_engine_from_scratch_amd.kernels.model_ops import decode_linear

    announce(f"decode_linear M={M} K={K} N={N}")
    g = torch.Generator().manual_seed(M * 31 + K + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    wn = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
    y = decode_linear(x.to(gpu), W.to(gpu))
    ref = (x.float() @ W.float().T).to(torch.bfloat16)
    _close(y, ref, "plain")
    # norm prologue from per-16-column partial sums of squares
    ss = (x.float() ** 2).view(M, K // 16, 16).sum(-1).contiguous()
    yn = decode_linear(x.to(gpu), W.to(gpu), ss_in=ss.to(gpu), norm_weight=wn.to(gpu), eps=1e-6)
    refn = (oi.rms_norm(x, wn, 1e-6).float() @ W.float().T).to(torch.bfloat16)
    torch.cuda.synchronize()
    _close(yn, refn, "norm prologue")


@pytest.mark.parametrize("M", [17, 48, 64])
def test_decode_linear_norm_silu_all_rows(gpu, M):
    """SwiGLU linear with its RMSNorm prologue above 16 rows (every row in one
    workgroup per column tile, the rows normalised once into LDS), against
    y = bf16(bf16(silu(bf16 g)) * bf16 u) of the oracle norm; repeated calls
    give the same bits."""
    from qwen3_engine_from_scratch_amd.kernels.model_ops import decode_linear

    announce(f"decode_linear norm + SwiGLU M={M}")
    K, I = 1024, 3072
    g = torch.Generator().manual_seed(M + 5)
    x = (torch.randn(M, K, generator=g) * 2).to(torch.bfloat16)
    wn = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
    Wgu = (torch.randn(2 * I, K, generator=g) * 0.05).to(torch.bfloat16)
    ss = (x.float() ** 2).view(M, K // 16, 16).sum(-1).contiguous()
    args = dict(epilogue="silu", ss_in=ss.to(gpu), norm_weight=wn.to(gpu), eps=1e-6)
    act = decode_linear(x.to(gpu), Wgu.to(gpu), **args)
    a = oi.rms_norm(x, wn, 1e-6).float()
    gg = (a @ Wgu[:I].float().T).to(torch.bfloat16).float()
    uu = (a @ Wgu[I:].float().T).to(torch.bfloat16).float()
    ref = (torch.nn.functional.silu(gg).to(torch.bfloat16).float() * uu).to(torch.bfloat16)
    torch.cuda.synchronize()
    _close(act, ref, "norm + SwiGLU")
    again = decode_linear(x.to(gpu), Wgu.to(gpu), **args)
    torch.cuda.synchronize()
    assert torch.equal(again, act)


def test_decode_linear_residual_and_silu_epilogues(gpu):
    from qwen3_engine_from_scratch_amd.kernels.model_ops import decode_linear, embed_ss

    announce("decode_linear residual / silu epilogues, embed_ss")
    g = torch.Generator().manual_seed(99)
    M, K, N, I = 48, 2048, 1024, 3072
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    res = (torch.randn(M, N, generator=g) * 2).to(torch.bfloat16)
    h_out = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    ss_out = torch.empty(M, N // 16, dtype=torch.float32, device=gpu)
    decode_linear(x.to(gpu), W.to(gpu), epilogue="residual", residual=res.to(gpu),
                  residual_out=h_out, ss_out=ss_out)
    o = (x.float() @ W.float().T).to(torch.bfloat16)
    h_ref = (res.float() + o.float()).to(torch.bfloat16)
    _close(h_out, h_ref, "residual stream")
    ss_ref = (h_out.cpu().float() ** 2).view(M, N // 16, 16).sum(-1)
    torch.testing.assert_close(ss_out.cpu(), ss_ref, rtol=1e-5, atol=0)
    # repeated calls give the same bits (fixed summation order)
    for _ in range(3):
        h2 = torch.empty_like(h_out)
        ss2 = torch.empty_like(ss_out)
        decode_linear(x.to(gpu), W.to(gpu), epilogue="residual", residual=res.to(gpu),
                      residual_out=h2, ss_out=ss2)
        torch.cuda.synchronize()
        assert torch.equal(h2, h_out) and torch.equal(ss2, ss_out)
    # SwiGLU epilogue over a fused gate/up weight
    Wgu = (torch.randn(2 * I, N, generator=g) * 0.05).to(torch.bfloat16)
    act = decode_linear(h_out, Wgu.to(gpu), epilogue="silu")
    gu = (h_out.cpu().float() @ Wgu.float().T).to(torch.bfloat16)
    act_ref = torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]
    torch.cuda.synchronize()
    _close(act, act_ref, "silu epilogue")
    # embedding rows and their partial sums
    E = torch.randn(500, 1024, generator=g).to(torch.bfloat16)
    ids = torch.tensor([3, 499, 0, 500, 7], dtype=torch.int64)
    h, ss = embed_ss(ids.to(gpu), E.to(gpu))
    torch.cuda.synchronize()
    ok = ids < 500
    assert torch.equal(h.cpu()[ok], E[ids[ok]]) and not h.cpu()[~ok].any()
    torch.testing.assert_close(ss.cpu()[ok], (E[ids[ok]].float() ** 2).view(-1, 64, 16).sum(-1),
                               rtol=1e-5, atol=0)


@pytest.mark.parametrize("M,K", [(37, 1024), (64, 4096), (5, 2048)])
def test_decode_qkv_rope_vs_oracle(gpu, M, K):
    """Input RMSNorm + qkv projection + QK-norm + RoPE + pool write in one
    launch, against the oracle composition (fp32 projection rounded to bf16,
    then the pre-attention oracle)."""
    from oracle import pre_attention as opa
    from qwen3_engine_from_scratch_amd.PagedKVcache import KVCachePool, PagedKVCache
    from qwen3_engine_from_scratch_amd.kernels.model_ops import decode_qkv_rope

    announce(f"decode qkv + QK-norm + RoPE + pool write M={M} K={K}")
    g = torch.Generator().manual_seed(21 + K + M)
    Hq, Hkv = 16, 8
    h = (torch.randn(M, K, generator=g) * 2).to(torch.bfloat16)
    wn = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
    W = (torch.randn((Hq + 2 * Hkv) * 128, K, generator=g) * 0.03).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    ss = (h.float() ** 2).view(M, K // 16, 16).sum(-1).contiguous()
    cos, sin = opa.rope_tables(128, 1e6, 2048)
    pool = KVCachePool(4 * M + 8, 2, 16, Hkv, 128, device=gpu, dtype=torch.bfloat16,
                       max_seq_len=1024, max_requests=M + 2)
    caches = [PagedKVCache(pool) for _ in range(M)]
    for c in caches:
        c.seq_len = int(torch.randint(0, 40, (1,), generator=g))
        while c.num_pages < c.seq_len // 16 + 1:
            c._allocate_block()
        pool.seq_lens[c.row_id] = c.seq_len
    rows = torch.tensor([c.row_id for c in caches], dtype=torch.int32, device=gpu)
    q = decode_qkv_rope(h.to(gpu), ss.to(gpu), wn.to(gpu), 1e-6, W.to(gpu), Hq, Hkv, qw.to(gpu),
                        kw.to(gpu), 1e-6, cos.to(gpu), sin.to(gpu), pool, 1, rows)
    torch.cuda.synchronize()
    qkv = (oi.rms_norm(h, wn, 1e-6).float() @ W.float().T).to(torch.bfloat16)
    qr = qkv[:, :Hq * 128].view(M, Hq, 128)
    kr = qkv[:, Hq * 128:(Hq + Hkv) * 128].view(M, Hkv, 128)
    vr = qkv[:, (Hq + Hkv) * 128:].view(M, Hkv, 128)
    pos = torch.tensor([c.seq_len for c in caches])
    q_ref, k_ref = opa.qk_norm_rope_ref(qr, kr, qw, kw, 1e-6, cos, sin, pos)
    _close(q.reshape(M, -1), q_ref.reshape(M, -1), "q")
    kb, vb = pool.k_buffer.cpu(), pool.v_buffer.cpu()
    kp = torch.stack([kb[c.block_table[c.seq_len // 16], 1, :, c.seq_len % 16] for c in caches])
    vp = torch.stack([vb[c.block_table[c.seq_len // 16], 1, :, c.seq_len % 16] for c in caches])
    _close(kp.reshape(M, -1), k_ref.reshape(M, -1), "pool k")
    _close(vp.reshape(M, -1), vr.reshape(M, -1), "pool v")
    assert not kb[:, 0].any() and not vb[:, 0].any(), "other layers untouched"
    written = sum(1 for _ in caches)
    assert int((kb[:, 1].abs().sum(-1) > 0).sum()) == written * Hkv, "only the new slots written"


@pytest.mark.parametrize("M,V", [(1, 4096), (37, 1005), (64, 151936)])
def test_lm_head_argmax_vs_reference(gpu, M, V):
    """Final norm + lm_head + argmax in one pass: the chosen token's logit
    (fp32 reference rounded to bf16) is the row maximum up to one bf16 step,
    and the index equals the reference argmax except in near-ties."""
    from qwen3_engine_from_scratch_amd.kernels.model_ops import lm_head_argmax

    announce(f"lm_head argmax M={M} V={V}")
    K = 1024
    g = torch.Generator().manual_seed(M + V)
    h = (torch.randn(M, K, generator=g) * 2).to(torch.bfloat16)
    wn = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
    W = (torch.randn(V, K, generator=g) * 0.05).to(torch.bfloat16)
    ss = (h.float() ** 2).view(M, K // 16, 16).sum(-1).contiguous()
    out = lm_head_argmax(h.to(gpu), ss.to(gpu), wn.to(gpu), 1e-6, W.to(gpu)).cpu()
    ref = (oi.rms_norm(h, wn, 1e-6).float() @ W.float().T).to(torch.bfloat16).float()
    mx = ref.max(-1).values
    got = ref.gather(1, out.view(-1, 1)).view(-1)
    assert ((mx - got) <= mx.abs() * 2.0 ** -7 + 1e-6).all(), (mx - got).max()
    assert (out == ref.argmax(-1)).float().mean() >= 0.9


def test_lm_head_argmax_ties_and_nan(gpu):
    """Equal largest logits take the first index; a NaN logit wins."""
    from qwen3_engine_from_scratch_amd.kernels.model_ops import lm_head_argmax

    announce("lm_head argmax ties and NaN")
    M, K, V = 5, 512, 777
    g = torch.Generator().manual_seed(3)
    h = torch.ones(M, K, dtype=torch.bfloat16)
    wn = torch.ones(K, dtype=torch.bfloat16)
    W = (torch.randn(V, K, generator=g) * 0.01).to(torch.bfloat16)
    W[20] = W[700] = 0.1
    ss = (h.float() ** 2).view(M, K // 16, 16).sum(-1).contiguous()
    args = (h.to(gpu), ss.to(gpu), wn.to(gpu), 1e-6)
    assert lm_head_argmax(*args, W.to(gpu)).tolist() == [20] * M
    W[300, 7] = float("nan")
    assert lm_head_argmax(*args, W.to(gpu)).tolist() == [300] * M


def test_page_in_maps_and_zeroes_blocks(gpu):
    from qwen3_engine_from_scratch_amd.PagedKVcache import KVCachePool, PageIn, PagedKVCache

    announce("page-in: batched table entries + block zeroing")
    pool = KVCachePool(20, 3, 16, 2, 128, device=gpu, dtype=torch.bfloat16, max_seq_len=256,
                       max_requests=8)
    pool.k_buffer.fill_(1.0)
    pool.v_buffer.fill_(2.0)
    caches = [PagedKVCache(pool) for _ in range(3)]
    pages = PageIn(pool, capacity=32)
    assert pages.reserve(caches, [17, 0, 40]) == 2 + 0 + 3
    assert pages.reserve(caches, [17, 1, 48]) == 0 + 1 + 0
    torch.cuda.synchronize()
    bt = pool.block_table_2d.cpu()
    used = []
    for c in caches:
        assert bt[c.row_id, :c.num_pages].tolist() == c.block_table
        assert (bt[c.row_id, c.num_pages:] == -1).all()
        used += c.block_table
    kb, vb = pool.k_buffer.cpu(), pool.v_buffer.cpu()
    mask = torch.zeros(20, dtype=torch.bool)
    mask[used] = True
    assert not kb[mask].any() and not vb[mask].any(), "new blocks zeroed"
    assert (kb[~mask] == 1.0).all() and (vb[~mask] == 2.0).all(), "other blocks untouched"


# ---- whole model -------------------------------------------------------------

def _tiny(seed=0, layers=2, vocab=2048, hidden=512, inter=1024, hq=4, hkv=2):
    from qwen3_engine_from_scratch_amd.config import Qwen3Config
    from qwen3_engine_from_scratch_amd.model import Qwen3ForCausalLM, init_random_weights

    cfg = Qwen3Config(hidden_size=hidden, num_attention_heads=hq, num_key_value_heads=hkv,
                      head_dim=128, num_hidden_layers=layers, vocab_size=vocab,
                      intermediate_size=inter, rms_norm_eps=1e-6, rope_theta=1e6,
                      max_position_embeddings=1024, tie_word_embeddings=True)
    m = init_random_weights(Qwen3ForCausalLM(cfg), seed=seed, std=0.05, norm_jitter=0.2)
    m = m.to(torch.bfloat16)
    state = {k: v.detach().float().clone() for k, v in m.state_dict().items()}
    return m, state, cfg


def _rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


def _pool(cfg, gpu, blocks=64, max_seq_len=512, max_requests=16):
    from qwen3_engine_from_scratch_amd.PagedKVcache import KVCachePool

    return KVCachePool(blocks, cfg.num_hidden_layers, 16, cfg.num_key_value_heads, cfg.head_dim,
                       device=gpu, dtype=torch.bfloat16, max_seq_len=max_seq_len,
                       max_requests=max_requests)


def test_model_prefill_and_decode_vs_oracle(gpu):
    """Drop-in forward: a padded prefill batch, then teacher-forced decode
    steps; every position's logits against the fp32 oracle over the whole
    sequence."""
    from qwen3_engine_from_scratch_amd.PagedKVcache import PagedKVCache

    model, state, cfg = _tiny(seed=1)
    model = model.to(gpu)
    lens = [37, 1, 90]
    steps = 6
    g = torch.Generator().manual_seed(3)
    seqs = [torch.randint(0, cfg.vocab_size, (L + steps,), generator=g) for L in lens]
    announce(f"model prefill lens={lens} + {steps} decode steps")
    pool = _pool(cfg, gpu)
    caches = [PagedKVCache(pool) for _ in lens]
    S = max(lens)
    padded = torch.zeros(len(lens), S, dtype=torch.long)
    for i, L in enumerate(lens):
        padded[i, :L] = seqs[i][:L]
    out = [model(padded.to(gpu), kv_cache=caches, input_lens=lens).cpu()]
    for s in range(steps):
        ids = torch.stack([seqs[i][L + s] for i, L in enumerate(lens)])[:, None]
        out.append(model(ids.to(gpu), kv_cache=caches).cpu())
    torch.cuda.synchronize()
    assert [c.seq_len for c in caches] == [L + steps for L in lens]
    for i, L in enumerate(lens):
        got = torch.cat([out[0][i, :L]] + [o[i] for o in out[1:]]).float()
        ref = om.qwen3_logits_ref(state, cfg, seqs[i])
        ref16 = om.qwen3_logits_ref(state, cfg, seqs[i], dtype=torch.bfloat16)
        e, e16 = _rel(got, ref), _rel(ref16, ref)
        announce(f"  request {i}: rel err {e:.4f} (reference bf16 forward: {e16:.4f})")
        assert e <= max(2 * e16, 0.03), (i, e, e16)
        assert out[0][i, L:].abs().sum() == 0, "pad positions are zero"


def test_fused_and_library_decode_paths_agree(gpu):
    """The fused decode linears and the library-GEMM path compute the same
    step: both within the model bar of the fp32 oracle, and within bf16
    noise of each other."""
    from qwen3_engine_from_scratch_amd.PagedKVcache import PagedKVCache

    model, state, cfg = _tiny(seed=6)
    model = model.to(gpu)
    g = torch.Generator().manual_seed(8)
    lens = [30, 70, 5, 48]
    seqs = [torch.randint(0, cfg.vocab_size, (L + 1,), generator=g) for L in lens]
    announce("fused vs library decode step")
    pool = _pool(cfg, gpu)
    caches = [PagedKVCache(pool) for _ in lens]
    for c, sq, L in zip(caches, seqs, lens):
        model(sq[:L][None].to(gpu), kv_cache=c)
    for c in caches:
        c.reserve_next()
    rows = torch.tensor([c.row_id for c in caches], dtype=torch.int32, device=gpu)
    ids = torch.stack([sq[L] for sq, L in zip(seqs, lens)]).to(gpu)
    kb, vb = pool.k_buffer.clone(), pool.v_buffer.clone()
    fused = model.decode_logits(ids, rows, pool, fused=True).float().cpu()
    pool.k_buffer.copy_(kb)
    pool.v_buffer.copy_(vb)
    lib = model.decode_logits(ids, rows, pool, fused=False).float().cpu()
    for i, (sq, L) in enumerate(zip(seqs, lens)):
        ref = om.qwen3_logits_ref(state, cfg, sq)[L]
        ref16 = om.qwen3_logits_ref(state, cfg, sq, dtype=torch.bfloat16)[L]
        e16 = _rel(ref16, ref)
        ef, el = _rel(fused[i], ref), _rel(lib[i], ref)
        announce(f"  row {i}: fused {ef:.4f} library {el:.4f} reference bf16 {e16:.4f}")
        assert ef <= max(2 * e16, 0.03) and el <= max(2 * e16, 0.03)
    assert _rel(fused, lib) < 0.03


def test_graph_runner_matches_eager_decode(gpu):
    """The reference GraphRunner contract: replay(input_ids, positions, rows)
    for k rows in a bucket of b equals the eager forward_decode of the same b
    rows (dummy rows padding), bit for bit, on every replay."""
    from qwen3_engine_from_scratch_amd.PagedKVcache import PagedKVCache
    from qwen3_engine_from_scratch_amd.graph_runner import GraphRunner

    model, state, cfg = _tiny(seed=2)
    model = model.to(gpu)
    pool = _pool(cfg, gpu, blocks=96, max_requests=24)
    announce("graph runner: capture buckets 1,2,4,8")
    runner = GraphRunner(model, pool, [PagedKVCache(pool) for _ in range(8)], (1, 2, 4, 8),
                         reserve_pages=2)
    # live requests with some context
    g = torch.Generator().manual_seed(5)
    reqs = [PagedKVCache(pool) for _ in range(5)]
    for i, c in enumerate(reqs):
        L = 10 + 7 * i
        model(torch.randint(0, cfg.vocab_size, (1, L), generator=g).to(gpu), kv_cache=c)
    k_buf, v_buf = pool.k_buffer.clone(), pool.v_buffer.clone()
    for k in (5, 3, 1, 5):
        b = runner.bucket_for(k)
        act = reqs[:k]
        for c in act:
            c.reserve_next()
        ids = torch.randint(0, cfg.vocab_size, (k, 1), generator=g).to(gpu)
        pos = torch.tensor([[c.seq_len] for c in act], dtype=torch.long).to(gpu)
        rows = torch.tensor([c.row_id for c in act], dtype=torch.int32).to(gpu)
        announce(f"  replay k={k} bucket={b}")
        got = runner.replay(ids, pos, rows)[:k].clone()
        # eager on the same padded batch, from the same pool contents
        pool.k_buffer.copy_(k_buf)
        pool.v_buffer.copy_(v_buf)
        pad = torch.full((b,), runner.dummy_row, dtype=torch.int32, device=gpu)
        pad[:k] = rows
        pids = torch.zeros(b, 1, dtype=torch.long, device=gpu)
        pids[:k] = ids
        ppos = runner.graphs[b][1]["pos"].clone()
        ref = model.forward_decode(pids, ppos, pad, [reqs[0]] * b)[:k]
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"k={k}: replay differs from eager"
        for _ in range(2):  # replays after eager work give the same result
            again = runner.replay(ids, pos, rows)[:k]
            torch.cuda.synchronize()
            assert torch.equal(again, got)
        k_buf, v_buf = pool.k_buffer.clone(), pool.v_buffer.clone()
    runner.free()


def test_engine_greedy_generation_vs_oracle(gpu):
    """Continuous batching with captured decode graphs (greedy argmax and
    length advance inside the graph): every generated token is the fp32
    oracle's choice up to bf16 near-ties, and the eager engine agrees."""
    from qwen3_engine_from_scratch_amd.engine import Engine, GenRequest

    model, state, cfg = _tiny(seed=4)
    model = model.to(gpu)
    g = torch.Generator().manual_seed(11)
    lens = [5, 63, 17, 40, 1, 33]
    new = [12, 3, 20, 7, 9, 1]
    prompts = [torch.randint(0, cfg.vocab_size, (L,), generator=g).tolist() for L in lens]
    results = {}
    for use_graph in (True, False):
        pool = _pool(cfg, gpu, blocks=128, max_requests=32)
        announce(f"engine use_graph={use_graph}, max_batch=4, {len(lens)} requests")
        eng = Engine(model, pool, max_batch=4, use_graph=use_graph)
        reqs = [GenRequest(i, p, n) for i, (p, n) in enumerate(zip(prompts, new))]
        stats = eng.generate(reqs)
        eng.close()
        assert stats["output_tokens"] == sum(new)
        assert [len(r.output_ids) for r in reqs] == new
        assert pool.free_count == pool.total_blocks, "pages not returned"
        results[use_graph] = [r.output_ids for r in reqs]
    for i, (p, out) in enumerate(zip(prompts, results[True])):
        ref = om.qwen3_logits_ref(state, cfg, torch.tensor(p + out[:-1]))
        steps = ref[len(p) - 1:]
        chosen = steps[torch.arange(len(out)), torch.tensor(out)]
        gap = (steps.max(-1).values - chosen).max().item()
        assert gap <= 0.15, (i, gap)
    # graph and eager engines: token for token up to a first difference, which
    # may only come at a near-tie (the decode attention splits a padded bucket
    # differently from the unpadded eager batch; every other kernel of the
    # step is row-invariant)
    for i, (p, x, y) in enumerate(zip(prompts, results[True], results[False])):
        s = next((j for j, (a, b) in enumerate(zip(x, y)) if a != b), None)
        if s is None:
            continue
        ctx = torch.tensor(p + x[:s])
        ref = om.qwen3_logits_ref(state, cfg, ctx)[-1]
        ref16 = om.qwen3_logits_ref(state, cfg, ctx, dtype=torch.bfloat16)[-1]
        bar = 2 * (ref16 - ref).abs().max().item()
        d = abs(ref[x[s]].item() - ref[y[s]].item())
        announce(f"  request {i}: graph/eager first differ at step {s}, gap {d:.4f}, bar {bar:.4f}")
        assert d <= bar, (i, s, d, bar)

    # eos: a token the model does produce stops each request right after it,
    # also when it is seen one pipelined step late
    eos = results[True][2][4]
    pool = _pool(cfg, gpu, blocks=128, max_requests=32)
    eng = Engine(model, pool, max_batch=4, use_graph=True)
    reqs = [GenRequest(i, p, n, eos_token_id=eos) for i, (p, n) in enumerate(zip(prompts, new))]
    eng.generate(reqs)
    eng.close()
    assert pool.free_count == pool.total_blocks, "pages not returned"
    stopped = 0
    for r, n in zip(reqs, new):
        out = r.output_ids
        assert 1 <= len(out) <= n
        assert eos not in out[:-1], "tokens generated past eos"
        assert out[-1] == eos or len(out) == n
        stopped += out[-1] == eos and len(out) < n
    assert stopped >= 1, "no request stopped at eos"


def test_engine_graph_equals_eager_batch_invariant(gpu):
    """With the batch-invariant decode attention every kernel of a decode
    step is row-invariant, so the captured engine (padded power-of-two
    buckets with dummy rows) and the eager engine (unpadded batches) give
    the same tokens, token for token."""
    from qwen3_engine_from_scratch_amd.engine import Engine, GenRequest

    model, state, cfg = _tiny(seed=4)
    model = model.to(gpu)
    g = torch.Generator().manual_seed(11)
    lens = [5, 63, 17, 40, 1, 33]
    new = [12, 3, 20, 7, 9, 1]
    prompts = [torch.randint(0, cfg.vocab_size, (L,), generator=g).tolist() for L in lens]
    results = {}
    for use_graph in (True, False):
        pool = _pool(cfg, gpu, blocks=128, max_requests=32)
        announce(f"engine batch_invariant use_graph={use_graph}, max_batch=4")
        eng = Engine(model, pool, max_batch=4, use_graph=use_graph, batch_invariant=True)
        reqs = [GenRequest(i, p, n) for i, (p, n) in enumerate(zip(prompts, new))]
        eng.generate(reqs)
        eng.close()
        assert pool.free_count == pool.total_blocks, "pages not returned"
        results[use_graph] = [r.output_ids for r in reqs]
    model.decode_batch_invariant = False
    for i, (x, y) in enumerate(zip(results[True], results[False])):
        assert x == y, f"request {i}: graph and eager engines differ: {x} vs {y}"
