"""GPU token sampling (qwen3_sample_bf16, qwen3_sample_ws_bf16) against the
sampling oracle, and the parallel form against the single-workgroup form.

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
    # all greedy: the parallel form's greedy path (8 rows: eight parts each)
    assert torch.equal(sample_tokens(x.to(gpu)).cpu().view(-1), ref)


@pytest.mark.parametrize("B", [1, 33, 64, 128, 129, 300])
def test_all_greedy_batches_equal_argmax(gpu, B):
    """All-greedy batches: up to 128 rows through the parallel form's
    greedy path (8, 4 or 2 parts per row), above that the argmax kernel;
    ties keep the first index, NaN ranks above every number, a row of -inf
    gives index 0."""
    from qwen3_engine_from_scratch_amd.sampling import sample_tokens

    announce(f"sampling: all greedy B={B}")
    x = _logits(B, 151936, 7 + B)
    x[0, 151935] = 60.0                          # maximum in the last token
    if B > 1:
        x[B - 1, 9000] = x[B - 1, 140000] = 55.0  # tie across parts: first index
    if B > 3:
        x[2, 100] = x[2, 30000] = float("nan")    # NaN ranks highest, first NaN
        x[3] = float("-inf")
    ref = torch.argmax(x, -1)
    assert ref[0] == 151935
    out = sample_tokens(x.to(gpu)).cpu().view(-1)
    assert torch.equal(out, ref), (out != ref).nonzero().view(-1)[:8].tolist()


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


def _both_forms(x, t, k, p, seed):
    """The draws of qwen3_sample_bf16 and of qwen3_sample_ws_bf16 for the
    same rows (x a (B, V) device view, t / k / p device arrays)."""
    from qwen3_engine_from_scratch_amd import _lib

    lib = _lib.load()
    B, V = x.shape
    dev = x.device
    stream = _lib.stream_of(dev)
    one = torch.empty(B, dtype=torch.int64, device=dev)
    par = torch.full((B,), -7, dtype=torch.int64, device=dev)
    _lib.check(lib.qwen3_sample_bf16(x.data_ptr(), x.stride(0), B, V, t.data_ptr(), k.data_ptr(),
                                     p.data_ptr(), seed, one.data_ptr(), stream),
               "qwen3_sample_bf16")
    need = int(lib.qwen3_sample_workspace_bytes(B, V))
    ws = torch.full((need,), 0xA5, dtype=torch.uint8, device=dev)  # stale contents are fine
    _lib.check(lib.qwen3_sample_ws_bf16(x.data_ptr(), x.stride(0), B, V, t.data_ptr(),
                                        k.data_ptr(), p.data_ptr(), seed, par.data_ptr(),
                                        ws.data_ptr(), need, stream), "qwen3_sample_ws_bf16")
    torch.cuda.synchronize()
    return one.cpu(), par.cpu()


@pytest.mark.parametrize("B,V,stride", [
    (64, 151936, 151936),   # four parts per row
    (1, 151936, 151936),    # eight parts
    (128, 151936, 151936),  # two parts
    (300, 151936, 151936),  # one part: the single-workgroup form
    (16, 151935, 151937),   # rows not 16-byte aligned: element loads
    (8, 20000, 20000),      # three rounds: three parts, the last one short
    (8, 5000, 5000),        # under one round: one part
])
def test_parallel_form_draws_the_same_tokens(gpu, B, V, stride):
    """Greedy rows, top-k + top-p, top-k alone (small and past the
    candidate list), top-p alone, top-k >= vocab and several temperatures
    in one batch: qwen3_sample_ws_bf16 draws exactly qwen3_sample_bf16's
    tokens."""
    g = torch.Generator().manual_seed(B + V)
    base = torch.randn(B, stride, generator=g) * 2
    if B >= 8:
        base[1, : V // 2] = 1.5    # many ties at the top-k boundary
        base[2] = base[2].round()  # a few hundred distinct values
    xb = base.to(torch.bfloat16)
    if B >= 16:  # NaNs of both signs (never drawn; greedy ranks them first)
        bits = xb.view(torch.int16)
        for r, sign_bit in ((0, 0), (3, 0), (6, 0), (9, 1), (10, 1), (14, 1), (16, 1)):
            if r >= B:
                continue
            cols = torch.tensor([7, 8191, V // 3, V - 2])
            bits[r, cols] = (0xFFC1 - 0x10000) if sign_bit else 0x7FC1
    x = xb.to(gpu)[:, :V]
    # top-k 1 to 200: unions of at most 1,024 entries (the sorted form); 600:
    # a longer union (the histogram passes over it); 5,000: lists past
    # their capacity (the row passes)
    kinds = [(0.0, 50, 0.9), (0.8, 50, 0.9), (1.0, 1, 1.0), (1.0, 5000, 1.0), (0.7, 0, 0.9),
             (1.2, V + 5, 0.95), (0.5, 3, 0.5), (2.0, 200, 0.99), (0.9, 600, 0.95)]
    t = torch.tensor([kinds[r % len(kinds)][0] for r in range(B)], device=gpu)
    k = torch.tensor([kinds[r % len(kinds)][1] for r in range(B)], dtype=torch.int32, device=gpu)
    p = torch.tensor([kinds[r % len(kinds)][2] for r in range(B)], device=gpu)
    announce(f"sampling parallel form B={B} V={V} stride={stride}")
    for seed in (1, 2):
        one, par = _both_forms(x, t, k, p, seed)
        assert torch.equal(one, par), f"B={B} V={V} seed={seed}: rows {(one != par).nonzero().view(-1)[:8].tolist()} differ"
