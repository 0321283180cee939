"""Paged decode kernel vs the oracle (parity) on the GPU."""
import numpy as np
import pytest
import torch

from conftest import announce
from gpu_helpers import (assert_close_attn, decode_case_to_device, gpu_dense_decode_fp32)
from oracle import decode as od
from oracle import inputs as oi

pytestmark = pytest.mark.gpu


def _run(case, dev, **kw):
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import paged_attention_decode_hip

    t = decode_case_to_device(case, dev)
    out = paged_attention_decode_hip(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"],
                                     t["row_ids"], case.block_size, **kw)
    torch.cuda.synchronize()
    return out.cpu(), t


def test_decode_config1_vs_oracle_and_closed_form(gpu):
    case = oi.config1_decode()
    announce("decode config1 B=4 L=[37,128,511,1024] 16/8 heads")
    out, _ = _run(case, gpu)
    assert_close_attn(out, od.dense_decode_ref(case.q, case.k_pool, case.v_pool, case.block_table,
                                               case.seq_lens, case.row_ids, 16), "vs fp64")
    orc = od.paged_attention_ref(case.q, case.k_pool, case.v_pool, case.block_table,
                                 case.seq_lens, case.row_ids, 16, out_fp32=True)
    assert_close_attn(out, orc, "vs oracle")


@pytest.mark.parametrize("lens,hq,hkv,bs", [
    ([1, 2, 15, 16, 17, 63, 64, 65], 32, 8, 16),
    ([255, 256, 257, 300], 16, 8, 16),
    ([1000, 1, 700], 8, 8, 16),          # G = 1
    ([129, 40], 16, 1, 16),              # G = 16
    ([97, 500, 33], 40, 8, 16),          # G = 5 (Qwen3-14B shape)
    ([31, 32, 33, 200], 16, 8, 32),      # block_size 32 (two tiles per page)
])
def test_decode_shapes_vs_closed_form(gpu, lens, hq, hkv, bs):
    case = oi.make_decode_case(lens, hq, hkv, 128, bs, slack=0.3, seed=sum(lens) % 97)
    announce(f"decode shapes lens={lens} hq={hq} hkv={hkv} bs={bs}")
    out, _ = _run(case, gpu)
    ref = od.dense_decode_ref(case.q, case.k_pool, case.v_pool, case.block_table,
                              case.seq_lens, case.row_ids, bs)
    assert_close_attn(out, ref, f"lens={lens}")


def test_decode_split_kv_long_contexts(gpu):
    # several partitions per sequence plus the LSE merge
    case = oi.make_decode_case([4096, 20000, 777, 9000], 32, 8, 128, 16, slack=0.1, seed=11)
    announce("decode split-KV lens=[4096,20000,777,9000]")
    out, t = _run(case, gpu)
    ref = gpu_dense_decode_fp32(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"], t["row_ids"], 16)
    assert_close_attn(out, ref, "split-KV")


def test_decode_row_ids_and_dummy_row(gpu):
    """Rows addressed through row_ids in shuffled order inside a larger
    resident table; a dummy row with seq_len 0 reads exactly its page 0 slot 0."""
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import paged_attention_decode_hip

    case = oi.make_decode_case([50, 1, 300], 16, 8, 128, 16, slack=0.5, seed=12)
    t = decode_case_to_device(case, gpu, extra_rows=5)
    rows = torch.tensor([2, 0, 1, 1], dtype=torch.int32, device=gpu)
    q = torch.cat([t["q"], t["q"][:1]])
    announce("decode row_ids shuffled + dummy row")
    out = paged_attention_decode_hip(q, t["k"], t["v"], t["bt"], t["seq_lens"], rows, 16).cpu()
    ref = od.dense_decode_ref(q.cpu(), case.k_pool, case.v_pool, t["bt"].cpu(),
                              t["seq_lens"].cpu(), rows.cpu(), 16)
    assert_close_attn(out, ref, "row_ids")
    phys = int(case.block_table[1, 0])
    for h in range(16):  # L = 1: output is V[page 0, slot 0] exactly
        assert torch.equal(out[2, h], case.v_pool[phys, h // 2, 0])
        assert torch.equal(out[3, h], case.v_pool[phys, h // 2, 0])


def test_decode_tail_slots_cannot_leak(gpu):
    """NaN in slots at or beyond L of the last page never reaches the output."""
    case = oi.make_decode_case([19, 50, 16], 32, 8, 128, 16, seed=13)
    ref = od.dense_decode_ref(case.q, case.k_pool, case.v_pool, case.block_table,
                              case.seq_lens, case.row_ids, 16)
    for b, L in enumerate(case.lens):
        last = int(case.block_table[b, (L - 1) // 16])
        if L % 16:
            case.k_pool[last, :, L % 16:] = float("nan")
            case.v_pool[last, :, L % 16:] = float("nan")
    announce("decode NaN tail slots")
    out, _ = _run(case, gpu)
    assert_close_attn(out, ref, "tail")


def test_decode_zero_length_with_bias0_gives_zeros(gpu):
    case = oi.make_decode_case([5, 9], 16, 8, 128, 16, seed=14)
    case.seq_lens[0] = 0
    announce("decode bias=0, empty context")
    out, _ = _run(case, gpu, seq_len_bias=0)
    assert torch.equal(out[0], torch.zeros_like(out[0]))
    ref = od.dense_decode_ref(case.q[1:], case.k_pool, case.v_pool, case.block_table[1:],
                              case.seq_lens[1:], None, 16, bias=0)
    assert_close_attn(out[1:], ref, "bias0")


def test_decode_noncontiguous_q_and_out(gpu):
    """q sliced out of a fused (B, Hq + 2 Hkv, D) buffer, as the reference's
    QKV split produces it."""
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import paged_attention_decode_hip

    case = oi.make_decode_case([70, 200], 16, 8, 128, 16, seed=15)
    t = decode_case_to_device(case, gpu)
    fused = torch.zeros(2, 16 + 16, 128, dtype=torch.bfloat16, device=gpu)
    fused[:, :16] = t["q"]
    q = fused[:, :16]
    out_buf = torch.zeros(2, 40, 128, dtype=torch.bfloat16, device=gpu)
    out = out_buf[:, 4:20]
    announce("decode non-contiguous q/out")
    paged_attention_decode_hip(q, t["k"], t["v"], t["bt"], t["seq_lens"], t["row_ids"], 16,
                               out=out)
    ref = od.dense_decode_ref(case.q, case.k_pool, case.v_pool, case.block_table,
                              case.seq_lens, case.row_ids, 16)
    assert_close_attn(out.cpu(), ref, "strided")
    assert not out_buf[:, :4].any() and not out_buf[:, 20:].any()


def test_decode_page_permutation_bit_identical(gpu):
    case = oi.make_decode_case([300, 1200], 32, 8, 128, 16, slack=0.5, seed=16)
    base, _ = _run(case, gpu)
    g = torch.Generator().manual_seed(5)
    perm = torch.randperm(case.k_pool.shape[0], generator=g)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    case.k_pool = case.k_pool[perm].clone()
    case.v_pool = case.v_pool[perm].clone()
    m = case.block_table >= 0
    case.block_table[m] = inv[case.block_table[m].long()].to(torch.int32)
    announce("decode page permutation")
    out, _ = _run(case, gpu)
    assert torch.equal(out, base)


@pytest.mark.parametrize("cfg", ["config3", "config4"])
def test_decode_full_size_vs_fp32(gpu, cfg):
    """Headline shapes: Qwen3-8B 32/8 heads, block 16, scattered tables."""
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import paged_attention_decode_hip

    lens = oi.config3_lengths() if cfg == "config3" else oi.config4_lengths()
    announce(f"decode {cfg} B={len(lens)} sumL={sum(lens)}")
    t = make_device_decode(lens, 32, 8, gpu, seed=0, slack=0.1)
    out = paged_attention_decode_hip(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"],
                                     t["row_ids"], 16)
    torch.cuda.synchronize()
    # every sequence of the batch against the fp32 reference
    ref = gpu_dense_decode_fp32(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"], t["row_ids"], 16)
    assert_close_attn(out, ref, cfg)


def make_device_decode(lens, hq, hkv, dev, seed=0, slack=0.1, block_size=16):
    """Full-size decode inputs generated directly on the device (seeded)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    pages = [(L + block_size - 1) // block_size for L in lens]
    nb = int(np.ceil(sum(pages) * (1 + slack)))
    perm = torch.randperm(nb, generator=g, device=dev).to(torch.int32)
    mp = max(pages)
    bt = torch.full((len(lens), mp), -1, dtype=torch.int32, device=dev)
    off = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[off:off + n]
        off += n
    k = torch.randn(nb, hkv, block_size, 128, generator=g, device=dev, dtype=torch.bfloat16)
    v = torch.randn(nb, hkv, block_size, 128, generator=g, device=dev, dtype=torch.bfloat16)
    q = torch.randn(len(lens), hq, 128, generator=g, device=dev, dtype=torch.bfloat16)
    sl = torch.tensor([L - 1 for L in lens], dtype=torch.int32, device=dev)
    rows = torch.arange(len(lens), dtype=torch.int32, device=dev)
    return dict(q=q, k=k, v=v, bt=bt, seq_lens=sl, row_ids=rows)


def test_decode_stream_many_short_segments(gpu):
    """Many short sequences per wave, empty contexts mixed in (bias 0): every
    wave crosses several sequence-head boundaries and splits some."""
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import paged_attention_decode_hip

    g = torch.Generator().manual_seed(21)
    lens = [int(x) for x in torch.randint(0, 70, (700,), generator=g)]
    lens[5] = lens[300] = 0
    announce(f"decode stream many segments B={len(lens)}")
    t = make_device_decode([max(L, 1) for L in lens], 16, 8, gpu, seed=3, slack=0.2)
    t["seq_lens"] = torch.tensor(lens, dtype=torch.int32, device=gpu)  # bias 0: L = lens
    out = paged_attention_decode_hip(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"],
                                     t["row_ids"], 16, seq_len_bias=0)
    torch.cuda.synchronize()
    nz = [b for b, L in enumerate(lens) if L > 0]
    sel = torch.tensor(nz, device=gpu)
    ref = gpu_dense_decode_fp32(t["q"][sel], t["k"], t["v"], t["bt"], t["seq_lens"],
                                t["row_ids"][sel], 16, bias=0)
    assert_close_attn(out[sel], ref, "many segments")
    for b, L in enumerate(lens):
        if L == 0:
            assert not out[b].any()


def test_decode_grid_path_large_batch(gpu):
    """Batches above the stream path's table size use the grid kernel."""
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import paged_attention_decode_hip

    g = torch.Generator().manual_seed(22)
    lens = [int(x) for x in torch.randint(1, 3000, (2100,), generator=g)]
    announce(f"decode grid path B={len(lens)}")
    t = make_device_decode(lens, 32, 8, gpu, seed=4, slack=0.05)
    out = paged_attention_decode_hip(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"],
                                     t["row_ids"], 16)
    torch.cuda.synchronize()
    sel = torch.arange(0, 2100, 37, device=gpu)
    ref = gpu_dense_decode_fp32(t["q"][sel], t["k"], t["v"], t["bt"], t["seq_lens"],
                                t["row_ids"][sel], 16)
    assert_close_attn(out[sel], ref, "grid path")


def test_decode_config1_golden_fixture(gpu):
    from pathlib import Path

    f = np.load(Path(__file__).resolve().parent / "golden" / "decode_config1.npz", allow_pickle=False)
    case = oi.config1_decode()
    assert case.fingerprint() == str(f["sha256"])
    announce("decode config1 vs golden fixture")
    out, _ = _run(case, gpu)
    assert_close_attn(out, torch.from_numpy(f["dense_fp64"]), "golden fp64")
    assert_close_attn(out, torch.from_numpy(f["oracle_fp32"]), "golden oracle")


@pytest.mark.parametrize("B,lo,hi", [(64, 500, 900), (6, 20, 300)])
def test_decode_garbage_workspace_same_bits(gpu, B, lo, hi):
    """The split-KV workspace carries no state between calls: a workspace
    full of 0xFF bytes gives the same bits as a zeroed one, and so does a
    second call on the same workspace."""
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import (
        paged_attention_decode_hip, paged_decode_workspace_bytes)

    g = torch.Generator().manual_seed(B)
    lens = [int(x) for x in torch.randint(lo, hi, (B,), generator=g)]
    announce(f"decode garbage workspace B={B} lens in [{lo},{hi})")
    t = make_device_decode(lens, 16, 8, gpu, seed=B, slack=0.1)
    need = paged_decode_workspace_bytes(B, 16, 8, 128, t["bt"].shape[1], 16)
    outs = []
    ws = None
    for fill in (0, 255, None):
        if fill is not None:
            ws = torch.full((need,), fill, dtype=torch.uint8, device=gpu)
        out = paged_attention_decode_hip(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"],
                                         t["row_ids"], 16, workspace=ws)
        torch.cuda.synchronize()
        outs.append(out.cpu())
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    ref = gpu_dense_decode_fp32(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"], t["row_ids"], 16)
    assert_close_attn(outs[0], ref, "garbage workspace")
