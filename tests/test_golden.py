"""Golden fixtures (tests/golden/*.npz): the seeded generators still produce
the same bytes, and the oracle still reproduces the stored outputs.  CPU only."""
from pathlib import Path

import numpy as np
import torch

from oracle import decode as od
from oracle import inputs as oi
from oracle import kv_write as okw
from oracle import prefill as op

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(GOLD / name, allow_pickle=False)


def test_decode_config1_fixture():
    f = load("decode_config1.npz")
    case = oi.config1_decode()
    assert case.fingerprint() == str(f["sha256"]), "input generator drifted"
    out = od.paged_attention_ref(case.q, case.k_pool, case.v_pool, case.block_table, case.seq_lens,
                                 case.row_ids, 16, out_fp32=True)
    assert np.allclose(out.numpy(), f["oracle_fp32"], atol=1e-6, rtol=0)
    assert np.abs(f["oracle_fp32"] - f["dense_fp64"]).max() < 2e-5


def test_prefill_fixture():
    from tests_golden_params import PREFILL_HEADS, PREFILL_LENS

    f = load("prefill_small.npz")
    c = oi.make_prefill_case(PREFILL_LENS, *PREFILL_HEADS, 128, seed=3)
    assert c.fingerprint() == str(f["sha256"]), "input generator drifted"
    ref = op.varlen_attention_ref(c.q, c.k, c.v, c.cu_seqlens, c.scale, dtype=torch.float64)
    stored = torch.from_numpy(f["closed_form_bf16"]).view(torch.bfloat16)
    assert torch.equal(ref.to(torch.bfloat16), stored)
    assert float(f["flash_restated_max_abs"]) < 2e-2 and float(f["flash_restated_mean_abs"]) < 2e-3


def test_slot_write_fixture():
    f = load("slot_write.npz")
    c = oi.make_prefill_case([40, 23], 16, 8, 128, seed=4)
    assert c.fingerprint() == str(f["sha256"])
    assert np.array_equal(c.slot_mapping.numpy(), f["slot_mapping"])
    kb = np.zeros((c.num_blocks + 2, 3, 8, 16, 128), np.uint16)
    vb = np.zeros_like(kb)
    okw.slots_write_ref(okw.as_u16(c.k), okw.as_u16(c.v), kb, vb, c.slot_mapping.numpy(), 1)
    assert np.uint64(kb.astype(np.uint64).sum()) == f["k_checksum"]
    assert np.uint64(vb.astype(np.uint64).sum()) == f["v_checksum"]
    assert np.array_equal(np.argwhere(kb.any(axis=(2, 4))), f["touched"])
