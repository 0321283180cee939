"""bench.py defines its workloads without the oracle (which only its CPU
baseline leg may use); they must stay the ones the oracle and the GPU tests
use.  CPU only."""
import torch

import bench
from oracle import inputs as oi
from oracle import pre_attention as opa
from qwen3_engine_from_scratch_amd.kernels.pre_attention import rope_tables


def test_bench_lengths_equal_the_oracle_workloads():
    assert bench.workload_lengths("config2") == oi.config2_lengths()
    assert bench.workload_lengths("config3") == oi.config3_lengths()
    assert bench.workload_lengths("config4") == oi.config4_lengths()


def test_product_rope_tables_equal_the_oracle_tables():
    c1, s1 = rope_tables(128, 1e6, 512)
    c2, s2 = opa.rope_tables(128, 1e6, 512)
    assert torch.equal(c1, c2) and torch.equal(s1, s2)


def test_bench_config1_inputs_equal_the_oracle_case():
    c = bench.config1_inputs()
    o = oi.config1_decode()
    for name, a, b in (("q", c["q"], o.q), ("k", c["k"], o.k_pool), ("v", c["v"], o.v_pool),
                       ("bt", c["bt"], o.block_table), ("seq_lens", c["seq_lens"], o.seq_lens),
                       ("rows", c["row_ids"], o.row_ids)):
        assert torch.equal(a, b), name
