"""CPU oracle for the attention hot path — TEST INFRASTRUCTURE ONLY.

A restatement, in PyTorch on the CPU (fp32 math) and numpy (bit-exact slot
arithmetic), of the reference engine's own pure-PyTorch path for the three
hot-path operations.  Each function cites the reference file:line it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or, in bench.py, as the timed
CPU baseline).  The product package qwen3_engine_from_scratch_amd never
imports it: there is no CPU fallback.

Pinning (what fixes each function independently of its own formula; the tests
live in tests/test_oracle.py):
  decode.paged_attention_ref   fp64 dense softmax closed form; L=1 -> V[0];
                               constant K -> mean(V); GQA head map; page
                               permutation invariance; tail-slot garbage
                               ignored; planted-mistake variants are rejected.
  prefill.varlen_attention_ref torch scaled_dot_product_attention(is_causal)
                               per sequence in fp64; len=1 -> V[0]; packing
                               order independence.
  prefill.flash_varlen_ref     within bf16-P rounding of the fp64 closed form.
  prefill.standard_attention_ref  valid rows within bf16 rounding of the
                               closed form; pad rows equal V[:, 0].
  kv_write.*                   write -> gather round trip through the block
                               table (a separate read path, get_kv) is exact;
                               untouched slots stay zero; numpy and torch
                               index paths agree bit for bit.
  pre_attention.rope_tables    the frequency law cos/sin(pos * base^(-2i/D)) in
                               fp64; both halves equal.
  pre_attention.qk_norm_rope_ref  RMSNorm within one bf16 ulp of the fp64
                               closed form; RoPE within bf16 rounding of the
                               fp64 complex rotation of each (i, i + D/2)
                               pair; position 0 is the identity exactly;
                               adjacent pairing, a flipped sign, an off-by-one
                               position and norm-after-RoPE are rejected.
No function of this package is "parity unpinned".
"""
