"""Batch invariance of the batch-invariant paged decode
(qwen3_paged_decode_invariant_bf16): a sequence's output bits depend only on
its own query, K/V pages and length, not on the batch around it.

The kernel cuts every sequence-head into 256-token partitions from its
first token, computes each partition's softmax state on its own and folds
the states in ascending order, whichever wave or launch path computed them;
the batch only decides which wave owns which partitions.  These tests hold
each sequence alone (batch 1) against the same sequence inside full batches
of the decode workloads, at other row positions, and across the two launch
paths (persistent waves up to 2,048 rows, one wave per partition above),
bit for bit.  The values themselves are checked against the fp32 reference
in test_decode_gpu.py.
"""
import pytest
import torch

from conftest import announce
from gpu_helpers import assert_close_attn, gpu_dense_decode_fp32
from oracle import inputs as oi
from test_decode_gpu import make_device_decode

pytestmark = pytest.mark.gpu


def _decode(t, rows):
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import paged_attention_decode_hip

    rows = torch.as_tensor(rows, dtype=torch.long, device=t["q"].device)
    return paged_attention_decode_hip(t["q"][rows], t["k"], t["v"], t["bt"], t["seq_lens"],
                                      t["row_ids"][rows], 16, batch_invariant=True)


def _alone_equals_batch(t, batch_out, rows, what):
    for i, b in enumerate(rows):
        alone = _decode(t, [b])
        torch.cuda.synchronize()
        assert torch.equal(alone[0], batch_out[i]), f"{what}: sequence {b} differs alone"


@pytest.mark.parametrize("cfg", ["config3", "config4"])
def test_decode_each_sequence_alone_equals_full_batch(gpu, cfg):
    """Every sequence of the Qwen3-8B decode workloads (256 contexts in
    [1024, 8192]; 8 in [32768, 131072]) alone vs inside the full batch."""
    lens = oi.config3_lengths() if cfg == "config3" else oi.config4_lengths()
    announce(f"decode batch invariance {cfg}: B={len(lens)} sumL={sum(lens)}")
    t = make_device_decode(lens, 32, 8, gpu, seed=0, slack=0.1)
    rows = list(range(len(lens)))
    full = _decode(t, rows)
    torch.cuda.synchronize()
    ref = gpu_dense_decode_fp32(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"], t["row_ids"], 16)
    assert_close_attn(full, ref, f"{cfg} batch-invariant vs fp32")
    _alone_equals_batch(t, full, rows, cfg)
    # other positions and company: the rows reversed, and every third row
    rev = rows[::-1]
    out = _decode(t, rev)
    torch.cuda.synchronize()
    assert torch.equal(out, full[rev]), f"{cfg}: reversed batch differs"
    sub = rows[1::3]
    out = _decode(t, sub)
    torch.cuda.synchronize()
    assert torch.equal(out, full[sub]), f"{cfg}: sub-batch differs"


def test_decode_partition_edges_invariant(gpu):
    """Lengths on and around partition edges (256 tokens) in batches of
    several sizes, so the waves' ranges end at different partitions."""
    lens = [1, 255, 256, 257, 511, 512, 513, 4096, 4097, 767, 768, 769, 3000, 17, 6000]
    announce(f"decode partition edges lens={lens}")
    t = make_device_decode(lens * 20, 16, 8, gpu, seed=5, slack=0.1)
    n = len(lens)
    ref = _decode(t, list(range(n)))
    torch.cuda.synchronize()
    _alone_equals_batch(t, ref, list(range(n)), "edges")
    for m in (3, 7, 20):  # the same sequences repeated: batches of 45, 105, 300
        rows = list(range(n * m))
        out = _decode(t, rows)
        torch.cuda.synchronize()
        assert torch.equal(out[:n], ref), f"edges x{m}: the first {n} rows differ"
        for b in range(n, n * m, 17):  # later rows (their own pages) alone
            alone = _decode(t, [b])
            torch.cuda.synchronize()
            assert torch.equal(alone[0], out[b]), f"edges x{m}: row {b} differs alone"


def test_decode_grid_path_equals_stream_path(gpu):
    """2,100 rows take the one-wave-per-partition path; the same sequences
    in batches of 1 and of 100 take the persistent path: the same bits."""
    g = torch.Generator().manual_seed(23)
    lens = [int(x) for x in torch.randint(1, 3000, (2100,), generator=g)]
    lens[7] = 9000
    announce(f"decode grid vs stream path B={len(lens)}")
    t = make_device_decode(lens, 32, 8, gpu, seed=6, slack=0.05)
    full = _decode(t, list(range(len(lens))))
    torch.cuda.synchronize()
    picks = [0, 7, 1, 255, 256, 1000, 2047, 2048, 2099] + list(range(3, 2100, 97))
    _alone_equals_batch(t, full[picks], picks, "grid path")
    rows = list(range(0, 2100, 21))
    out = _decode(t, rows)
    torch.cuda.synchronize()
    assert torch.equal(out, full[rows]), "stream batch of 100 differs from the grid path"


@pytest.mark.parametrize("B,lo,hi", [(64, 500, 900), (6, 20, 300), (3, 9000, 20000)])
def test_decode_invariant_workspace_contract(gpu, B, lo, hi):
    """Only the leading ticket region carries state between calls: zero before
    the first call and zero after every call, the rest may hold anything
    (0xFF bytes give the same bits); calls of other batch sizes in between
    keep the tickets where every batch size finds them."""
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import (
        paged_attention_decode_hip, paged_decode_workspace_bytes)

    g = torch.Generator().manual_seed(B)
    lens = [int(x) for x in torch.randint(lo, hi, (B,), generator=g)]
    announce(f"invariant decode workspace B={B} lens in [{lo},{hi})")
    t = make_device_decode(lens, 16, 8, gpu, seed=B, slack=0.1)
    need = paged_decode_workspace_bytes(B, 16, 8, 128, t["bt"].shape[1], 16, batch_invariant=True)
    tickets = -(-2048 * 8 * 4 // 256) * 256
    ws = torch.full((need,), 255, dtype=torch.uint8, device=gpu)
    ws[:tickets] = 0
    outs = []
    for rows in (list(range(B)), [0], list(range(B)), list(range(B))[::-1]):
        r = torch.tensor(rows, device=gpu)
        out = paged_attention_decode_hip(t["q"][r], t["k"], t["v"], t["bt"], t["seq_lens"],
                                         t["row_ids"][r], 16, workspace=ws, batch_invariant=True)
        torch.cuda.synchronize()
        assert not ws[:tickets].any(), "a call left a ticket set"
        outs.append((rows, out))
    full = outs[0][1]
    for rows, out in outs[1:]:
        assert torch.equal(out, full[torch.tensor(rows, device=gpu)])
    ref = gpu_dense_decode_fp32(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"], t["row_ids"], 16)
    assert_close_attn(full, ref, "invariant workspace contract")


@pytest.mark.parametrize("hq,hkv,bs", [(8, 8, 16), (32, 4, 16), (32, 2, 32), (16, 8, 32)])
def test_decode_invariant_group_sizes_and_blocks(gpu, hq, hkv, bs):
    """G = 1, 8, 16 and 2 with 16- and 32-token blocks: lengths around the
    256-token partitions, around 4,096 tokens (where partitions become 512
    tokens) and a long one; values against the fp32 reference, every row
    alone against the batch, and the batch reversed."""
    g = torch.Generator().manual_seed(hq * 100 + hkv + bs)
    lens = [1, 2, 255, 256, 257, 4095, 4096, 4097, 9000] + \
           [int(x) for x in torch.randint(1, 3000, (23,), generator=g)]
    announce(f"invariant decode hq={hq} hkv={hkv} bs={bs} B={len(lens)}")
    t = make_device_decode(lens, hq, hkv, gpu, seed=hq + bs, slack=0.1, block_size=bs)

    def run(rows):
        from qwen3_engine_from_scratch_amd.kernels.paged_attention import paged_attention_decode_hip
        r = torch.as_tensor(rows, dtype=torch.long, device=gpu)
        return paged_attention_decode_hip(t["q"][r], t["k"], t["v"], t["bt"], t["seq_lens"],
                                          t["row_ids"][r], bs, batch_invariant=True)

    rows = list(range(len(lens)))
    full = run(rows)
    torch.cuda.synchronize()
    ref = gpu_dense_decode_fp32(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"], t["row_ids"], bs)
    assert_close_attn(full, ref, f"invariant hq={hq} hkv={hkv} bs={bs}")
    for b in rows:
        alone = run([b])
        torch.cuda.synchronize()
        assert torch.equal(alone[0], full[b]), f"hq={hq} hkv={hkv} bs={bs}: row {b} differs alone"
    rev = rows[::-1]
    out = run(rev)
    torch.cuda.synchronize()
    assert torch.equal(out, full[rev]), f"hq={hq} hkv={hkv} bs={bs}: reversed batch differs"
