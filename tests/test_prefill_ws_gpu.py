"""The wave-specialised prefill tile (QWEN3_PREFILL_TILE=ws: four matrix
waves and eight softmax waves per workgroup, scores and P^T through LDS)
against the fp32 closed form: query-head groups G = 1, 2, 4, 5, 8, 16,
causal and non-causal, ragged tails, single-token sequences and config 2."""
import pytest
import torch

from conftest import announce
from gpu_helpers import assert_close_attn
from oracle import inputs as oi
from test_prefill_gpu import _gpu_ref_fp32, _run

pytestmark = pytest.mark.gpu


@pytest.fixture
def ws_tile(monkeypatch):
    monkeypatch.setenv("QWEN3_PREFILL_TILE", "ws")


@pytest.mark.parametrize("lens,hq,hkv,causal", [
    ([1, 7, 64, 100], 16, 8, True),        # G = 2
    ([33, 129, 2], 8, 8, True),            # G = 1
    ([200, 65], 32, 8, True),              # G = 4
    ([150], 16, 2, True),                  # G = 8
    ([96, 31], 40, 8, True),               # G = 5
    ([129, 40], 16, 1, True),              # G = 16
    ([40, 90], 16, 8, False),
    ([300, 1000, 63], 16, 8, False),
    ([1500, 700, 2100], 16, 8, True),
])
def test_prefill_ws_vs_fp32(gpu, ws_tile, lens, hq, hkv, causal):
    c = oi.make_prefill_case(lens, hq, hkv, 128, seed=len(lens) + hq + 7)
    announce(f"prefill ws lens={lens} hq={hq} hkv={hkv} causal={causal}")
    out = _run(c, gpu, hq, hkv, causal=causal)
    assert_close_attn(out, _gpu_ref_fp32(c, gpu, hq // hkv, causal), f"ws lens={lens}")


def test_prefill_ws_single_token_sequences_return_v(gpu, ws_tile):
    c = oi.make_prefill_case([1, 1, 5, 1], 16, 8, 128, seed=4)
    announce("prefill ws single-token sequences")
    out = _run(c, gpu, 16, 8)
    for s in (0, 1, 3):
        t = int(c.cu_seqlens[s])
        for h in range(16):
            assert torch.equal(out[t, h], c.v[t, h // 2])


def test_prefill_ws_config2_vs_fp32(gpu, ws_tile):
    c = oi.config2_prefill()
    announce(f"prefill ws config2 lens={c.lens}")
    out = _run(c, gpu, 16, 8)
    assert_close_attn(out, _gpu_ref_fp32(c, gpu, 2), "ws config2")
