"""GPU token sampling (qwen3_sample_bf16) against the sampling oracle.

Bars: greedy rows equal torch.argmax exactly; every sampled token lies in
the oracle's kept set; over many independent draws the empirical frequency
of every token is within 5 standard deviations (plus 2/N) of the oracle's
probability; a fixed seed reproduces the draws."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import sampling as osm

pytestmark = pytest.mark.gpu


def _logits(B, V, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, V, generator=g) * scale).to(torch.bfloat16)


def test_greedy_rows_equal_argmax(gpu):
    from qwen3_engine_from_scratch_amd.sampling import sample_tokens

    announce("sampling: greedy rows")
    x = _logits(8, 151936, 1)
    x[3, 5] = x[3, 77] = 50.0  # tie: first index
    t = [0.0, 1.0, 0.0, 0.0, 0.8, 0.0, -1.0, 0.0]
    out = sample_tokens(x.to(gpu), temperature=t, top_k=50, top_p=0.9, seed=3).cpu().view(-1)
    ref = torch.argmax(x, -1)
    for r in range(8):
        if t[r] <= 0:
            assert out[r] == ref[r], r
    # all greedy: the argmax kernel
    assert torch.equal(sample_tokens(x.to(gpu)).cpu().view(-1), ref)


@pytest.mark.parametrize("V,top_k,top_p,temp", [(151936, 50, 0.9, 1.0), (151936, 0, 0.8, 0.7),
                                                 (4000, 1000, 1.0, 1.2), (4000, 0, 1.0, 0.9),
                                                 (1001, 7, 0.5, 1.0), (4000, 0, 0.0, 1.0),
                                                 (151936, 20, -0.5, 1.0), (151936, 5000, 1.0, 1.0),
                                                 (151936, 3000, 0.95, 1.0)])
def test_sampled_tokens_stay_in_the_kept_set(gpu, V, top_k, top_p, temp):
    from qwen3_engine_from_scratch_amd.sampling import sample_tokens

    announce(f"sampling support V={V} top_k={top_k} top_p={top_p} T={temp}")
    B = 16
    x = _logits(B, V, V + top_k)
    xd = x.to(gpu)
    kept = [osm.kept_set(x[r].float(), temp, top_k, top_p) for r in range(B)]
    for s in range(6):
        out = sample_tokens(xd, temperature=temp, top_k=top_k, top_p=top_p, seed=100 + s)
        out = out.cpu().view(-1).tolist()
        for r in range(B):
            assert out[r] in kept[r], (r, out[r])


@pytest.mark.parametrize("n_ties,top_k", [(2000, 1500), (1000, 900), (300, 0)])
def test_partial_cut_inside_many_ties(gpu, n_ties, top_k):
    """Many tokens share the top value: a top-k cut inside them keeps the
    lowest indices (more ties than one per thread takes the row pass); with
    top_k 0, a top-p cut inside them does the same."""
    from qwen3_engine_from_scratch_amd.sampling import sample_tokens

    announce(f"sampling: cut inside {n_ties} ties, top_k={top_k}")
    V, B = 8192, 32
    g = torch.Generator().manual_seed(n_ties)
    x = torch.full((V,), -8.0)
    x[torch.randperm(V, generator=g)[:n_ties]] = 3.0
    x = x.to(torch.bfloat16)
    top_p = 1.0 if top_k else 0.5
    kept = osm.kept_set(x.float(), 1.0, top_k, top_p)
    assert len(kept) == (top_k if top_k else n_ties // 2 + 1)
    out = sample_tokens(x.expand(B, V).contiguous().to(gpu), temperature=1.0, top_k=top_k,
                        top_p=top_p, seed=9)
    got = out.cpu().view(-1).tolist()
    assert all(t in kept for t in got), sorted(set(got) - kept)[:5]


def test_peaked_top_p_row(gpu):
    """A peaked row (few tokens carry the mass): the top-p pass keeps the
    candidates in LDS; draws stay in the kept set and follow it."""
    from qwen3_engine_from_scratch_amd.sampling import sample_tokens

    announce("sampling: peaked top-p")
    V, N = 151936, 4096
    g = torch.Generator().manual_seed(4)
    row = (torch.randn(V, generator=g) * 1.0)
    row[:12] += torch.linspace(14.0, 10.0, 12)
    row = row.to(torch.bfloat16)
    p = osm.sampling_distribution(row.float(), 1.0, 0, 0.9)
    out = sample_tokens(row.to(gpu).expand(N, V).contiguous(), temperature=1.0, top_p=0.9, seed=2)
    got = out.cpu().view(-1).numpy()
    assert (p[got] > 0).all()
    counts = np.bincount(got, minlength=V)[:12] / N
    tol = 5 * np.sqrt(p[:12] * (1 - p[:12]) / N) + 2.0 / N
    assert (np.abs(counts - p[:12]) <= tol).all()


@pytest.mark.parametrize("top_k,top_p,temp", [(0, 1.0, 1.0), (10, 1.0, 0.8), (0, 0.75, 1.0),
                                              (20, 0.9, 1.5)])
def test_draws_follow_the_oracle_distribution(gpu, top_k, top_p, temp):
    from qwen3_engine_from_scratch_amd.sampling import sample_tokens

    announce(f"sampling distribution top_k={top_k} top_p={top_p} T={temp}")
    V, N = 48, 16384
    row = (torch.linspace(-2.0, 2.5, V) + 0.3 * torch.sin(torch.arange(V) * 1.7)).to(torch.bfloat16)
    x = row.expand(N, V).contiguous().to(gpu)  # independent draws: the stream is keyed by row
    out = sample_tokens(x, temperature=temp, top_k=top_k, top_p=top_p, seed=7)
    counts = np.bincount(out.cpu().view(-1).numpy(), minlength=V) / N
    p = osm.sampling_distribution(row.float(), temp, top_k, top_p)
    tol = 5 * np.sqrt(p * (1 - p) / N) + 2.0 / N
    assert (np.abs(counts - p) <= tol).all(), np.abs(counts - p).max()
    assert counts[p == 0].sum() == 0


def test_boundary_ties_keep_the_lower_index_and_seed_reproduces(gpu):
    from qwen3_engine_from_scratch_amd.sampling import sample_tokens

    announce("sampling ties and seeds")
    x = torch.tensor([[5.0, 4.0, 4.0, 4.0, 1.0, 4.0] + [-20.0] * 10]).to(torch.bfloat16)
    xd = x.expand(4096, -1).contiguous().to(gpu)
    out = sample_tokens(xd, temperature=1.0, top_k=3, seed=11).cpu().view(-1)
    assert set(out.tolist()) <= {0, 1, 2} and {0, 1, 2} <= set(out.tolist())
    a = sample_tokens(xd, temperature=1.0, top_k=0, top_p=0.95, seed=5).cpu()
    b = sample_tokens(xd, temperature=1.0, top_k=0, top_p=0.95, seed=5).cpu()
    c = sample_tokens(xd, temperature=1.0, top_k=0, top_p=0.95, seed=6).cpu()
    assert torch.equal(a, b) and not torch.equal(a, c)
