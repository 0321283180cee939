"""Seeded random shapes for the two attention kernels against fp32
references: prefill over batch sizes 1-30, lengths up to 2,500, G = 1, 2,
4, 5, 8, 16, causal and non-causal, on each schedule the batch selects and
on the wave-specialised tile; decode over batches of 1-300, contexts up to
9,000 tokens, 16- and 32-token blocks, on the default and the
batch-invariant kernel; and wider corners (over 256 prompts, prompts of
3-8k tokens, contexts of 10-40k tokens, batches above 2,048 rows).  Each
case is drawn from its own seed, so a failure names a reproducible shape."""
import random

import pytest
import torch

from conftest import announce
from gpu_helpers import assert_close_attn, gpu_dense_decode_fp32
from oracle import inputs as oi
from test_decode_gpu import make_device_decode
from test_prefill_gpu import _gpu_ref_fp32, _run

pytestmark = pytest.mark.gpu

_GROUPS = [(16, 8), (8, 8), (32, 8), (16, 2), (40, 8), (16, 1), (32, 4), (64, 8)]


def _prefill_case(i):
    rng = random.Random(7000 + i)
    hq, hkv = rng.choice(_GROUPS)
    ns = rng.choice([1, 1, 2, 3, 5, 8, 13, 30])
    mx = rng.choice([64, 300, 1200, 2500])
    lens = [rng.randint(1, mx) for _ in range(ns)]
    causal = rng.random() < 0.75
    tile = "ws" if i % 4 == 3 else ""
    return lens, hq, hkv, causal, tile


@pytest.mark.parametrize("i", range(16))
def test_prefill_random_shapes(gpu, monkeypatch, i):
    lens, hq, hkv, causal, tile = _prefill_case(i)
    if tile:
        monkeypatch.setenv("QWEN3_PREFILL_TILE", tile)
    announce(f"prefill random {i}: lens={lens} hq={hq} hkv={hkv} causal={causal} "
             f"tile={tile or 'default'}")
    c = oi.make_prefill_case(lens, hq, hkv, 128, seed=8000 + i)
    out = _run(c, gpu, hq, hkv, causal=causal)
    assert_close_attn(out, _gpu_ref_fp32(c, gpu, hq // hkv, causal), f"prefill random {i}")


@pytest.mark.parametrize("i", range(16))
def test_decode_random_shapes(gpu, i):
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import paged_attention_decode_hip

    rng = random.Random(9000 + i)
    hq, hkv = rng.choice(_GROUPS[:7])
    bs = rng.choice([16, 16, 32])
    B = rng.choice([1, 3, 17, 64, 150, 300])
    mx = rng.choice([100, 2000, 9000])
    lens = [rng.randint(1, mx) for _ in range(B)]
    inv = i % 2 == 1
    announce(f"decode random {i}: B={B} max_len={max(lens)} hq={hq} hkv={hkv} bs={bs} "
             f"invariant={inv}")
    t = make_device_decode(lens, hq, hkv, gpu, seed=9500 + i, slack=0.1, block_size=bs)
    out = paged_attention_decode_hip(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"], t["row_ids"],
                                     bs, batch_invariant=inv)
    torch.cuda.synchronize()
    ref = gpu_dense_decode_fp32(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"], t["row_ids"], bs)
    assert_close_attn(out, ref, f"decode random {i}")


# Wider corners: more than 256 prompts (the flat grid), prompts of 3-8k
# tokens, decode contexts of 10-40k tokens and batches above 2,048 rows
# (one wave per partition / the grid path).
_WIDE_GROUPS = [(16, 8), (8, 8), (32, 8), (16, 2), (40, 8), (16, 1), (32, 4), (64, 8), (32, 2)]


@pytest.mark.parametrize("i,kind", [(0, "many"), (1, "many"), (2, "long"), (3, "long"),
                                    (4, "mixed"), (5, "mixed")])
def test_prefill_wide_shapes(gpu, i, kind):
    rng = random.Random(11000 + i)
    hq, hkv = rng.choice(_WIDE_GROUPS)
    if kind == "many":
        lens = [rng.randint(1, 90) for _ in range(rng.randint(257, 400))]
    elif kind == "long":
        lens = [rng.randint(3000, 8000) for _ in range(rng.randint(1, 3))]
    else:
        lens = [rng.choice([1, 2, 63, 64, 65, 127, 128, 129, rng.randint(1, 5000)])
                for _ in range(rng.randint(2, 40))]
    causal = rng.random() < 0.8
    announce(f"prefill wide {i} ({kind}): n={len(lens)} sum={sum(lens)} max={max(lens)} "
             f"hq={hq} hkv={hkv} causal={causal}")
    c = oi.make_prefill_case(lens, hq, hkv, 128, seed=12000 + i)
    out = _run(c, gpu, hq, hkv, causal=causal)
    assert_close_attn(out, _gpu_ref_fp32(c, gpu, hq // hkv, causal), f"prefill wide {i}")


@pytest.mark.parametrize("i,kind", [(0, "long"), (1, "long"), (2, "grid"), (3, "grid"),
                                    (4, "mixed"), (5, "mixed")])
def test_decode_wide_shapes(gpu, i, kind):
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import paged_attention_decode_hip

    rng = random.Random(13000 + i)
    hq, hkv = rng.choice(_WIDE_GROUPS[:7] + [(32, 2)])
    bs = rng.choice([16, 32])
    if kind == "long":
        lens = [rng.randint(10000, 40000) for _ in range(rng.randint(1, 6))]
    elif kind == "grid":
        lens = [rng.randint(1, 400) for _ in range(rng.randint(2049, 2600))]
    else:
        lens = [rng.randint(1, 12000) for _ in range(rng.randint(1, 500))]
    inv = i % 2 == 1
    announce(f"decode wide {i} ({kind}): B={len(lens)} max={max(lens)} hq={hq} hkv={hkv} "
             f"bs={bs} invariant={inv}")
    t = make_device_decode(lens, hq, hkv, gpu, seed=14000 + i, slack=0.1, block_size=bs)
    out = paged_attention_decode_hip(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"], t["row_ids"],
                                     bs, batch_invariant=inv)
    torch.cuda.synchronize()
    ref = gpu_dense_decode_fp32(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"], t["row_ids"], bs)
    assert_close_attn(out, ref, f"decode wide {i}")
