"""Writes the golden fixtures of tests/golden/ from the pinned CPU oracle.

    python tests/golden/make_golden.py

Each fixture stores the seed and shape of a seeded synthetic workload (the
inputs are regenerated from the seed by oracle.inputs, and their sha256 is
stored to detect any drift of the generator), the oracle's fp32 output and
the fp64 closed form.  The reference repository ships no fixtures of its own
for this path, so these are pinned by the oracle checks in tests/test_oracle.py.
"""
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import decode as od  # noqa: E402
from oracle import inputs as oi  # noqa: E402
from oracle import kv_write as okw  # noqa: E402
from oracle import prefill as op  # noqa: E402


def decode_fixture():
    case = oi.config1_decode()
    out = od.paged_attention_ref(case.q, case.k_pool, case.v_pool, case.block_table, case.seq_lens,
                                 case.row_ids, 16, out_fp32=True)
    dense = od.dense_decode_ref(case.q, case.k_pool, case.v_pool, case.block_table, case.seq_lens,
                                case.row_ids, 16)
    np.savez_compressed(HERE / "decode_config1.npz", sha256=case.fingerprint(),
                        oracle_fp32=out.numpy(), dense_fp64=dense.numpy())


sys.path.insert(0, str(HERE.parent))
from tests_golden_params import PREFILL_HEADS, PREFILL_LENS  # noqa: E402


def prefill_fixture():
    c = oi.make_prefill_case(PREFILL_LENS, *PREFILL_HEADS, 128, seed=3)
    ref = op.varlen_attention_ref(c.q, c.k, c.v, c.cu_seqlens, c.scale, dtype=torch.float64)
    fl = op.flash_varlen_ref(c.q, c.k, c.v, c.cu_seqlens, c.scale)
    d = (fl.double() - ref).abs()
    np.savez_compressed(HERE / "prefill_small.npz", sha256=c.fingerprint(),
                        closed_form_bf16=ref.to(torch.bfloat16).view(torch.int16).numpy(),
                        flash_restated_max_abs=d.max().item(), flash_restated_mean_abs=d.mean().item())


def slot_write_fixture():
    """Decode + range writes into a 3-layer pool; stores the bf16 bits of every
    written row and the slot it landed in."""
    c = oi.make_prefill_case([40, 23], 16, 8, 128, seed=4)
    kb = np.zeros((c.num_blocks + 2, 3, 8, 16, 128), np.uint16)
    vb = np.zeros_like(kb)
    okw.slots_write_ref(okw.as_u16(c.k), okw.as_u16(c.v), kb, vb, c.slot_mapping.numpy(), 1)
    touched = np.argwhere(kb.reshape(kb.shape[0], 3, 8, 16, 128).any(axis=(2, 4)))
    np.savez_compressed(HERE / "slot_write.npz", sha256=c.fingerprint(),
                        slot_mapping=c.slot_mapping.numpy(), touched=touched,
                        k_checksum=np.uint64(kb.astype(np.uint64).sum()),
                        v_checksum=np.uint64(vb.astype(np.uint64).sum()))


if __name__ == "__main__":
    decode_fixture()
    prefill_fixture()
    slot_write_fixture()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size, "bytes")
