"""Varlen prefill kernel vs the oracle / fp32 references on the GPU."""
from types import SimpleNamespace

import pytest
import torch

from conftest import announce
from gpu_helpers import assert_close_attn
from oracle import inputs as oi
from oracle import prefill as op

pytestmark = pytest.mark.gpu


def _run(c, dev, hq, hkv, causal=True):
    from qwen3_engine_from_scratch_amd.kernels.flash_attention_varlen import flash_attention_prefill

    out = flash_attention_prefill(c.q.to(dev), c.k.to(dev), c.v.to(dev), c.cu_seqlens.to(dev),
                                  c.scale, hq, hkv, 128, max_seqlen=max(c.lens), causal=causal)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("lens,hq,hkv", [
    ([1, 7, 64, 100], 16, 8),
    ([33, 129, 2], 8, 8),        # G = 1
    ([200, 65], 32, 8),          # G = 4
    ([150], 16, 2),              # G = 8
    ([96, 31], 40, 8),           # G = 5
])
def test_prefill_small_vs_closed_form(gpu, lens, hq, hkv):
    c = oi.make_prefill_case(lens, hq, hkv, 128, seed=len(lens) + hq)
    announce(f"prefill small lens={lens} hq={hq} hkv={hkv}")
    out = _run(c, gpu, hq, hkv)
    ref = op.varlen_attention_ref(c.q, c.k, c.v, c.cu_seqlens, c.scale, dtype=torch.float64)
    assert_close_attn(out, ref, f"lens={lens}")
    fl = op.flash_varlen_ref(c.q, c.k, c.v, c.cu_seqlens, c.scale)
    assert_close_attn(out, fl, "vs reference flash restatement")


def test_prefill_non_causal(gpu):
    c = oi.make_prefill_case([40, 90], 16, 8, 128, seed=3)
    announce("prefill non-causal")
    out = _run(c, gpu, 16, 8, causal=False)
    ref = op.varlen_attention_ref(c.q, c.k, c.v, c.cu_seqlens, c.scale, causal=False,
                                  dtype=torch.float64)
    assert_close_attn(out, ref, "non-causal")


def test_prefill_single_token_sequences_return_v(gpu):
    c = oi.make_prefill_case([1, 1, 5, 1], 16, 8, 128, seed=4)
    announce("prefill single-token sequences")
    out = _run(c, gpu, 16, 8)
    for s in (0, 1, 3):
        t = int(c.cu_seqlens[s])
        for h in range(16):
            assert torch.equal(out[t, h], c.v[t, h // 2])


def _gpu_ref_fp32(c, gpu, G, causal=True):
    """fp32 attention per sequence on the GPU (the closed form, GQA by
    repeating each KV head G times)."""
    q, k, v = c.q.to(gpu), c.k.to(gpu), c.v.to(gpu)
    ref = torch.empty(q.shape, dtype=torch.float32, device=gpu)
    for s in range(len(c.lens)):
        s0, s1 = int(c.cu_seqlens[s]), int(c.cu_seqlens[s + 1])
        L = s1 - s0
        qs = q[s0:s1].float().transpose(0, 1).contiguous()
        ks = k[s0:s1].float().transpose(0, 1).repeat_interleave(G, 0)
        vs = v[s0:s1].float().transpose(0, 1).repeat_interleave(G, 0).contiguous()
        sc = torch.matmul(qs, ks.transpose(1, 2).contiguous()) * c.scale
        if causal:
            sc.masked_fill_(~torch.ones(L, L, dtype=torch.bool, device=gpu).tril(), float("-inf"))
        ref[s0:s1] = torch.matmul(torch.softmax(sc, -1), vs).transpose(0, 1)
    return ref.cpu()


def test_prefill_config2_vs_fp32(gpu):
    """Qwen3-0.6B varlen prefill: 8 sequences, lengths uniform in [64, 2048]."""
    c = oi.config2_prefill()
    announce(f"prefill config2 lens={c.lens}")
    out = _run(c, gpu, 16, 8)
    assert_close_attn(out, _gpu_ref_fp32(c, gpu, 2), "config2")


@pytest.mark.parametrize("lens,hq,hkv,causal", [
    ([4096, 3000, 5000, 4500], 16, 8, True),
    ([2000, 7000], 32, 8, True),             # G = 4: 64-row items
    ([4000, 4000, 4000, 4000], 16, 8, False),
])
def test_prefill_large_batches_vs_fp32(gpu, lens, hq, hkv, causal):
    """Batches large enough for eight-wave workgroups (at least four of their
    work items per CU)."""
    c = oi.make_prefill_case(lens, hq, hkv, 128, seed=sum(lens) % 101)
    announce(f"prefill large lens={lens} hq={hq} hkv={hkv} causal={causal}")
    out = _run(c, gpu, hq, hkv, causal=causal)
    assert_close_attn(out, _gpu_ref_fp32(c, gpu, hq // hkv, causal), f"lens={lens}")


@pytest.mark.parametrize("lens", [
    [1215, 1488, 90, 1096, 641, 307, 1395, 1001, 1321, 540, 1453, 201],  # last round partial
    [2048, 2048, 2048, 2048],  # 1,024 items: two full rounds of 512 workgroups
])
def test_prefill_four_wave_rounds_vs_fp32(gpu, lens):
    """Four-wave workgroups in the static order over several rounds (a last
    round that does not fill the grid goes in the mirrored order)."""
    c = oi.make_prefill_case(lens, 16, 8, 128, seed=len(lens))
    announce(f"prefill four-wave rounds lens={lens}")
    out = _run(c, gpu, 16, 8)
    assert_close_attn(out, _gpu_ref_fp32(c, gpu, 2), f"lens={lens}")


def test_prefill_strided_views_of_fused_qkv(gpu):
    """q, k and v as head slices of one fused (T, 32, 128) projection (row
    stride 4096 elements) and the output into a slice of a wider buffer: the
    same bits as contiguous copies."""
    from qwen3_engine_from_scratch_amd.kernels.flash_attention_varlen import flash_attention_prefill

    lens = [300, 77, 1024, 5]
    c = oi.make_prefill_case(lens, 16, 8, 128, seed=21)
    T = sum(lens)
    fused = torch.empty(T, 32, 128, dtype=torch.bfloat16, device=gpu)
    fused[:, :16] = c.q.to(gpu)
    fused[:, 16:24] = c.k.to(gpu)
    fused[:, 24:] = c.v.to(gpu)
    q, k, v = fused[:, :16], fused[:, 16:24], fused[:, 24:]
    wide = torch.zeros(T, 20, 128, dtype=torch.bfloat16, device=gpu)
    out = wide[:, 2:18]
    cu = c.cu_seqlens.to(gpu)
    announce("prefill strided views")
    flash_attention_prefill(q, k, v, cu, c.scale, 16, 8, 128, max_seqlen=max(lens), out=out)
    ref = flash_attention_prefill(q.contiguous(), k.contiguous(), v.contiguous(), cu, c.scale,
                                  16, 8, 128, max_seqlen=max(lens))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert not wide[:, :2].any() and not wide[:, 18:].any()  # nothing outside the view
    assert_close_attn(out.cpu(), _gpu_ref_fp32(c, gpu, 2), "strided")


@pytest.mark.parametrize("n,lo,hi", [(260, 1, 40), (300, 1, 200)])
def test_prefill_many_sequences_flat_grid(gpu, n, lo, hi):
    """More sequences than the persistent kernel ranks in LDS (256): the flat
    grid, with four-wave (few tokens) and eight-wave (many) workgroups."""
    g = torch.Generator().manual_seed(n)
    lens = [int(x) for x in torch.randint(lo, hi + 1, (n,), generator=g)]
    c = oi.make_prefill_case(lens, 16, 8, 128, seed=n)
    announce(f"prefill flat grid n={n} tokens={sum(lens)}")
    out = _run(c, gpu, 16, 8)
    assert_close_attn(out, _gpu_ref_fp32(c, gpu, 2), f"n={n}")


def test_prefill_counter_schedule_matches_static(gpu):
    """Eight-wave workgroups (a batch of at least four of their items per
    CU): the item counters (a workspace) only reorder work, so the output is
    the same bits as the static order's, the counters end at zero, and a
    workspace holding garbage gives the same result."""
    from qwen3_engine_from_scratch_amd import _lib

    lens, hq, hkv = [4096] * 8, 16, 8
    c = oi.make_prefill_case(lens, hq, hkv, 128, seed=7)
    q, k, v = c.q.to(gpu), c.k.to(gpu), c.v.to(gpu)
    cu = c.cu_seqlens.to(gpu)
    lib = _lib.load()
    need = int(lib.qwen3_varlen_prefill_workspace_bytes())

    def call(ws):
        out = torch.empty_like(q)
        rc = lib.qwen3_varlen_prefill_bf16(
            q.data_ptr(), _lib.strides(q, (0, 1)), k.data_ptr(), _lib.strides(k, (0, 1)),
            v.data_ptr(), _lib.strides(v, (0, 1)), out.data_ptr(), _lib.strides(out, (0, 1)),
            cu.data_ptr(), len(lens), max(lens), q.shape[0], hq, hkv, 128, c.scale, 0,
            None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
            _lib.stream_of(gpu))
        _lib.check(rc, "qwen3_varlen_prefill_bf16")
        torch.cuda.synchronize()
        return out

    announce(f"prefill counter schedule lens={lens}")
    static = call(None)
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
    for _ in range(2):
        assert torch.equal(call(ws), static)
        assert not ws.any(), "the counters were not left at zero"
    ws.fill_(0xFF)
    assert torch.equal(call(ws), static)


TICKETS = 1152  # first byte of the range tickets inside the workspace


def _layout(lib):
    """(ticket bytes, first slot byte) of the workspace on this device."""
    need = int(lib.qwen3_varlen_prefill_workspace_bytes())
    slot = 4 * 64 * 66 * 4
    ranges = (need - TICKETS) // (4 + 2 * slot)
    tb = (ranges * 4 + 255) // 256 * 256
    assert need == TICKETS + tb + 2 * ranges * slot
    return slice(TICKETS, TICKETS + tb), TICKETS + tb


def _call(lib, gpu, c, hq, hkv, ws, causal=True):
    from qwen3_engine_from_scratch_amd import _lib

    q, k, v = c.q.to(gpu), c.k.to(gpu), c.v.to(gpu)
    cu = c.cu_seqlens.to(gpu)
    out = torch.empty_like(q)
    rc = lib.qwen3_varlen_prefill_bf16(
        q.data_ptr(), _lib.strides(q, (0, 1)), k.data_ptr(), _lib.strides(k, (0, 1)),
        v.data_ptr(), _lib.strides(v, (0, 1)), out.data_ptr(), _lib.strides(out, (0, 1)),
        cu.data_ptr(), len(c.lens), max(c.lens), q.shape[0], hq, hkv, 128, c.scale,
        1 if causal else 0, None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
        _lib.stream_of(gpu))
    _lib.check(rc, "qwen3_varlen_prefill_bf16")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("lens,hq,hkv,causal", [
    ([2048], 16, 8, True),               # one long prompt: items cut into up to five parts
    ([1500, 700], 16, 8, True),
    ([1200], 32, 8, True),               # G = 4: 32-row items
    ([2500], 8, 8, True),                # G = 1: 128-row items
    ([900], 40, 8, True),                # G = 5
    ([1500], 32, 2, True),               # G = 16
    ([1800, 40, 1], 16, 8, False),       # non-causal
])
def test_prefill_range_cut_items_vs_fp32(gpu, lens, hq, hkv, causal):
    """The range schedule (four-wave workgroups, given a workspace, fewer
    items than resident workgroups) cuts items across workgroups; their
    partial softmax states meet in the workspace.  The output matches the fp32 closed form, every call leaves
    the tickets at zero, and repeated calls give the same bits whichever
    part arrives last -- also with the partial-state slots filled with NaN
    before each call, so a part that folded a slot before its owner's saves
    landed would show."""
    from qwen3_engine_from_scratch_amd import _lib

    lib = _lib.load()
    c = oi.make_prefill_case(lens, hq, hkv, 128, seed=sum(lens) % 97)
    tickets, slots = _layout(lib)
    ws = torch.zeros(int(lib.qwen3_varlen_prefill_workspace_bytes()), dtype=torch.uint8,
                     device=gpu)
    announce(f"prefill range lens={lens} hq={hq} hkv={hkv} causal={causal}")
    first = _call(lib, gpu, c, hq, hkv, ws, causal)
    assert ws[slots:].any(), "no item was cut"
    assert not ws[tickets].any(), "range tickets not left at zero"
    assert_close_attn(first.cpu(), _gpu_ref_fp32(c, gpu, hq // hkv, causal), f"range lens={lens}")
    for _ in range(3):
        ws[slots:].fill_(0xFF)  # NaN in every float of every slot
        again = _call(lib, gpu, c, hq, hkv, ws, causal)
        assert torch.equal(again, first), "range output depends on the arrival order"
        assert not ws[tickets].any()


def test_prefill_range_matches_whole_items_when_uncut(gpu):
    """Items the range schedule does not cut (here: a batch of short
    prompts, at most four key tiles each) are computed exactly as the
    persistent grid computes whole items (no workspace): the same bits."""
    from qwen3_engine_from_scratch_amd import _lib

    lib = _lib.load()
    lens = [256, 17, 200, 131, 64, 1, 99, 250]
    c = oi.make_prefill_case(lens, 16, 8, 128, seed=11)
    ws = torch.zeros(int(lib.qwen3_varlen_prefill_workspace_bytes()), dtype=torch.uint8,
                     device=gpu)
    announce(f"prefill range vs whole items, {len(lens)} short prompts")
    assert torch.equal(_call(lib, gpu, c, 16, 8, ws), _call(lib, gpu, c, 16, 8, None))


def test_prefill_short_prompts_batch_invariant(gpu):
    """A prompt of at most 256 tokens gives the same bits alone and inside a
    larger batch (its items are never cut), as the reference's one program
    per query block does."""
    from qwen3_engine_from_scratch_amd import _lib

    lib = _lib.load()
    ws = torch.zeros(int(lib.qwen3_varlen_prefill_workspace_bytes()), dtype=torch.uint8,
                     device=gpu)
    big = oi.make_prefill_case([2048, 256, 1000, 130, 77], 16, 8, 128, seed=12)
    announce("prefill short prompts alone vs in a batch")
    both = _call(lib, gpu, big, 16, 8, ws)
    for s in (1, 3, 4):
        s0, s1 = int(big.cu_seqlens[s]), int(big.cu_seqlens[s + 1])
        alone = SimpleNamespace(q=big.q[s0:s1], k=big.k[s0:s1], v=big.v[s0:s1],
                                cu_seqlens=torch.tensor([0, s1 - s0], dtype=torch.int32),
                                lens=[s1 - s0], scale=big.scale)
        assert torch.equal(_call(lib, gpu, alone, 16, 8, ws), both[s0:s1]), f"sequence {s}"


def test_prefill_max_seqlen_is_an_upper_bound(gpu):
    """max_seqlen is a host-side bound (the contract in the header): the
    exact longest length, the wrapper's own derivation (None) and a larger
    bound give the same bits."""
    from qwen3_engine_from_scratch_amd.kernels.flash_attention_varlen import flash_attention_prefill

    lens = [300, 77, 1024, 5]
    c = oi.make_prefill_case(lens, 16, 8, 128, seed=5)
    q, k, v, cu = c.q.to(gpu), c.k.to(gpu), c.v.to(gpu), c.cu_seqlens.to(gpu)
    announce(f"prefill max_seqlen bound lens={lens}")
    outs = [flash_attention_prefill(q, k, v, cu, c.scale, 16, 8, 128, max_seqlen=m)
            for m in (max(lens), None, 4 * max(lens) + 3)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


def test_prefill_batched_adaptor_pads_zero(gpu):
    """flash_attention_prefill_batched on a right-padded batch: valid rows
    match the closed form, pad rows are zero (reference :252-258)."""
    from qwen3_engine_from_scratch_amd.kernels.flash_attention_varlen import \
        flash_attention_prefill_batched

    lens, S = [5, 48, 31], 48
    c = oi.make_prefill_case(lens, 16, 8, 128, seed=5)
    qp = op.pad_batch(c.q, c.cu_seqlens, S).to(gpu)
    kp = op.pad_batch(c.k, c.cu_seqlens, S).to(gpu)
    vp = op.pad_batch(c.v, c.cu_seqlens, S).to(gpu)
    announce("prefill batched adaptor")
    out = flash_attention_prefill_batched(qp, kp, vp, lens, c.scale, 16, 8, 128).cpu()
    out = out.view(3, S, 16, 128)
    ref = op.varlen_attention_ref(c.q, c.k, c.v, c.cu_seqlens, c.scale, dtype=torch.float64)
    for b, L in enumerate(lens):
        s0 = int(c.cu_seqlens[b])
        assert_close_attn(out[b, :L], ref[s0:s0 + L], f"row {b}")
        assert not out[b, L:].any()


def test_prefill_golden_fixture(gpu):
    from pathlib import Path

    import numpy as np
    from tests_golden_params import PREFILL_HEADS, PREFILL_LENS

    f = np.load(Path(__file__).resolve().parent / "golden" / "prefill_small.npz", allow_pickle=False)
    c = oi.make_prefill_case(PREFILL_LENS, *PREFILL_HEADS, 128, seed=3)
    assert c.fingerprint() == str(f["sha256"])
    announce("prefill vs golden fixture")
    out = _run(c, gpu, *PREFILL_HEADS)
    ref = torch.from_numpy(f["closed_form_bf16"]).view(torch.bfloat16)
    assert_close_attn(out, ref, "golden")
