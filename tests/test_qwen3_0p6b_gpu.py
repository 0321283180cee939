"""The serving workload's own model on the GPU: Qwen3-0.6B at its real shape
(28 layers, hidden 1024, 16/8 heads of 128, SwiGLU 3072, vocab 151,936,
tied embeddings), random-init bf16 weights generated exactly as the serving
benchmark generates them (seed 0, std 0.02), prompts from the benchmark's
own length and token generators, cut to at most 160 tokens so the fp32 CPU
oracle stays cheap.  Reference driver: bench_batched.py:150-228 over
Qwen3ForCausalLM (qwen3/model.py:220-251).

Bars (calibrated against the reference's own bf16 arithmetic, restated in
oracle/model.py with dtype=bfloat16):
  teacher-forced logits   relative L2 error vs the fp32 oracle at most
                          max(2 x that of the reference's bf16 forward, 0.03)
                          (measured for the bf16 forward: 0.013-0.015).
  greedy tokens           each chosen token's fp32-oracle logit within
                          2 x (the reference bf16 forward's largest logit
                          error on that request) of the step's maximum: a
                          token the reference's own bf16 forward could have
                          chosen; at least 80% equal the fp32 argmax (the
                          bf16 forward itself: ~96%).
"""
import random

import pytest
import torch

from conftest import announce
from oracle import model as om

pytestmark = pytest.mark.gpu

N_PROMPTS, CAP, NEW = 40, 160, 10


@pytest.fixture(scope="module")
def qwen3_0p6b(gpu):
    from qwen3_engine_from_scratch_amd.config import qwen3_0p6b_config
    from qwen3_engine_from_scratch_amd.model import Qwen3ForCausalLM, init_random_weights

    cfg = qwen3_0p6b_config(max_position_embeddings=4096)
    announce("Qwen3-0.6B random init (seed 0, std 0.02) on the GPU")
    with torch.device(gpu):
        model = Qwen3ForCausalLM(cfg)
    init_random_weights(model, seed=0)
    model = model.to(torch.bfloat16).eval()
    state = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    # the serving benchmark's prompt generators: 64 lengths U[128, 1024] and
    # their tokens; the first N_PROMPTS, each cut to CAP tokens
    rng = random.Random(0)
    lens = [rng.randint(128, 1024) for _ in range(64)]
    g = torch.Generator().manual_seed(0)
    prompts = [torch.randint(0, cfg.vocab_size, (L,), generator=g).tolist() for L in lens]
    prompts = [p[:CAP] for p in prompts[:N_PROMPTS]]
    return model, state, cfg, prompts


def _pool(cfg, gpu, n_req, max_seq, graph_rows=0):
    """A pool for n_req requests of up to max_seq tokens, plus graph_rows
    placeholder handles (one page each) and the graph runner's dummy row."""
    from qwen3_engine_from_scratch_amd.PagedKVcache import KVCachePool

    bs = 16
    blocks = n_req * ((max_seq + bs - 1) // bs) + graph_rows + n_req + 16
    return KVCachePool(blocks, cfg.num_hidden_layers, bs, cfg.num_key_value_heads, cfg.head_dim,
                       device=gpu, dtype=torch.bfloat16, max_seq_len=max_seq,
                       max_requests=graph_rows + n_req + 8)


def _rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


def test_qwen3_0p6b_teacher_forced_logits_vs_oracle(gpu, qwen3_0p6b):
    """A padded prefill batch of 4 prompts through the drop-in forward, then
    4 teacher-forced decode steps; every position's logits vs the oracle."""
    from qwen3_engine_from_scratch_amd.PagedKVcache import PagedKVCache

    model, state, cfg, prompts = qwen3_0p6b
    steps = 4
    seqs = [torch.tensor(p) for p in prompts[:4]]
    lens = [len(s) - steps for s in seqs]
    announce(f"Qwen3-0.6B teacher-forced prefill lens={lens} + {steps} decode steps")
    pool = _pool(cfg, gpu, 4, CAP + 8)
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
    for i, L in enumerate(lens):
        got = torch.cat([out[0][i, :L]] + [o[i] for o in out[1:]]).float()
        ref = om.qwen3_logits_ref(state, cfg, seqs[i])
        ref16 = om.qwen3_logits_ref(state, cfg, seqs[i], dtype=torch.bfloat16)
        e, e16 = _rel(got, ref), _rel(ref16, ref)
        ed = _rel(got[L:], ref[L:])
        announce(f"  request {i}: rel err {e:.4f}, decode rows {ed:.4f} "
                 f"(reference bf16 forward: {e16:.4f})")
        assert e <= max(2 * e16, 0.03) and ed <= max(2 * e16, 0.03), (i, e, ed, e16)


def test_qwen3_0p6b_engine_greedy_vs_oracle(gpu, qwen3_0p6b):
    """Continuous batching through captured graphs (buckets up to 64; 40
    requests run in the 64-row bucket: a 64-row captured step, the 64-row
    gate/up kernel and a 64-sequence paged decode), greedy tokens checked
    against the fp32 oracle."""
    from qwen3_engine_from_scratch_amd.engine import Engine, GenRequest

    model, state, cfg, prompts = qwen3_0p6b
    pool = _pool(cfg, gpu, N_PROMPTS, CAP + NEW + 8, graph_rows=64)
    announce(f"Qwen3-0.6B engine: {N_PROMPTS} requests, prompts <= {CAP}, {NEW} greedy tokens")
    eng = Engine(model, pool, max_batch=64, use_graph=True)
    buckets = []
    bucket_for = eng.runner.bucket_for
    eng.runner.bucket_for = lambda k: buckets.append(bucket_for(k)) or buckets[-1]
    reqs = [GenRequest(i, p, NEW) for i, p in enumerate(prompts)]
    st = eng.generate(reqs)
    eng.close()
    assert st["output_tokens"] == N_PROMPTS * NEW
    assert buckets and set(buckets) == {64}, buckets
    assert pool.free_count == pool.total_blocks, "pages not returned"
    agree = total = 0
    worst = 0.0
    for r, p in zip(reqs, prompts):
        out = r.output_ids
        seq = torch.tensor(p + out[:-1])
        ref = om.qwen3_logits_ref(state, cfg, seq)[len(p) - 1:]
        ref16 = om.qwen3_logits_ref(state, cfg, seq, dtype=torch.bfloat16)[len(p) - 1:]
        bar = 2 * (ref16 - ref).abs().max().item()
        chosen = ref[torch.arange(len(out)), torch.tensor(out)]
        gap = (ref.max(-1).values - chosen).max().item()
        worst = max(worst, gap / bar)
        assert gap <= bar, (r.request_id, gap, bar)
        agree += int((ref.argmax(-1) == torch.tensor(out)).sum())
        total += len(out)
    announce(f"  greedy tokens: {agree}/{total} equal the fp32 argmax; worst gap "
             f"{worst:.2f} x the bar")
    assert agree >= 0.8 * total
