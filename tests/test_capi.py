"""The C-ABI library loads, exports every function the headers under
include/ declare, and rejects bad arguments before launching anything.  CPU
only: no call here reaches a kernel launch."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from qwen3_engine_from_scratch_amd import _lib

HEADERS = sorted((Path(__file__).resolve().parent.parent / "include").glob("*.h"))


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(qwen3_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_the_abi():
    names = declared_functions()
    assert [h.name for h in HEADERS] == ["qwen3_attn.h", "qwen3_model_ops.h"]
    assert "qwen3_paged_decode_bf16" in names and "qwen3_varlen_prefill_bf16" in names
    assert "qwen3_argmax_bf16" in names
    assert sorted(names) == sorted(_lib.exported_symbols())


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.qwen3_attn_abi_version() == _lib.ABI_VERSION


def _cus() -> int:
    """CUs of the visible device (0 when there is none)."""
    import torch
    return torch.cuda.get_device_properties(0).multi_processor_count if torch.cuda.is_available() else 0


def test_workspace_bytes():
    lib = _lib.load()
    def a256(x):
        return -(-x // 256) * 256

    # batches up to 2048: two (128 + 1)-float partial slots per wave and
    # query head of the group, plus the (B + 1)-entry tile prefix: two
    # four-wave workgroups per CU of the current device, or the largest grid
    # (1024 workgroups) when no device can be queried
    waves = 4 * (min(2 * _cus(), 1024) if _cus() else 1024)
    for hq, hkv in ((32, 8), (16, 8), (16, 1)):
        G = hq // hkv
        expect = a256(waves * 2 * G * 128 * 4) + a256(waves * 2 * G * 4) + a256(257 * 4) + 256
        assert lib.qwen3_paged_decode_workspace_bytes(256, hq, hkv, 128, 512, 16) == expect
    # larger batches: one partial per (b, query head, 2048-token partition)
    slots = 4096 * 32 * -(-512 * 16 // 2048)
    assert lib.qwen3_paged_decode_workspace_bytes(4096, 32, 8, 128, 512, 16) == \
        a256(slots * 128 * 4) + a256(slots * 4)
    # the batch-invariant decode: tickets for 2048 rows x KV heads, then one
    # slot per (b, KV head, 256-token partition) of a full table row (G x 128
    # floats of output, G (max, denominator) pairs), the (B + 1)-entry tile
    # prefix and the tiles-per-wave word; the same on any device
    for B, hq, hkv, pages in ((256, 32, 8, 512), (256, 16, 8, 512), (256, 16, 1, 512),
                              (4096, 32, 8, 512), (3, 32, 8, 17)):
        G = hq // hkv
        slots = B * hkv * -(-pages * 16 // 256)
        expect = (a256(2048 * hkv * 4) + a256(slots * G * 128 * 4) + a256(slots * G * 8)
                  + a256((B + 1) * 4) + 256)
        assert lib.qwen3_paged_decode_invariant_workspace_bytes(B, hq, hkv, 128, pages, 16) == expect
    assert lib.qwen3_paged_decode_invariant_workspace_bytes(2, 32, 8, 128, 8, 64) == \
        65536 + a256(2 * 8 * 2 * 4 * 512) + a256(2 * 8 * 2 * 4 * 8) + 256 + 256  # 2 parts
    assert lib.qwen3_paged_decode_invariant_workspace_bytes(4, 16, 3, 128, 64, 16) == 0
    assert lib.qwen3_paged_decode_workspace_bytes(4, 16, 8, 64, 64, 16) == 0  # head_dim 64 not built
    assert lib.qwen3_paged_decode_workspace_bytes(4, 16, 8, 128, 64, 8) == 0  # block_size 8
    assert lib.qwen3_paged_decode_workspace_bytes(4, 16, 3, 128, 64, 16) == 0  # 16 % 3 != 0
    assert lib.qwen3_paged_decode_workspace_bytes(4, 34, 2, 128, 64, 16) == 0  # G = 17


def _s(*v):
    return (ctypes.c_int64 * len(v))(*v)


FAKE = 1 << 20  # a 16-byte aligned non-null address; never dereferenced on these paths


def test_decode_rejects_bad_arguments():
    lib = _lib.load()
    args = dict(q=FAKE, qs=_s(4096, 128), k=FAKE, ks=_s(65536, 2048, 128), v=FAKE,
                vs=_s(65536, 2048, 128), nb=64, bt=FAKE, bts=8, rows=4, mp=8, sl=FAKE, bias=1,
                rid=None, out=FAKE, os=_s(4096, 128), B=2, H=32, Hk=8, D=128, bs=16,
                scale=0.088, ws=FAKE, wsb=1 << 30, stream=None)

    def call(**over):
        a = dict(args, **over)
        return lib.qwen3_paged_decode_bf16(
            a["q"], a["qs"], a["k"], a["ks"], a["v"], a["vs"], a["nb"], a["bt"], a["bts"],
            a["rows"], a["mp"], a["sl"], a["bias"], a["rid"], a["out"], a["os"], a["B"], a["H"],
            a["Hk"], a["D"], a["bs"], a["scale"], a["ws"], a["wsb"], a["stream"])

    assert call(D=64) == -3
    assert call(bs=8) == -3
    assert call(H=30) == -3            # not a multiple of Hkv
    assert call(H=8 * 17) == -3        # group of 17 > 16
    assert call(q=None) == -1
    assert call(bts=4) == -1           # row stride shorter than the row
    assert call(q=FAKE + 2) == -2      # misaligned
    assert call(qs=_s(4097, 128)) == -2
    assert call(ws=None, mp=64, bts=64) == -4  # several partitions need the workspace
    assert "workspace" in lib.qwen3_attn_last_error().decode()


def test_prefill_rejects_bad_arguments():
    lib = _lib.load()
    s2 = _s(2048, 128)

    def call(D=128, H=16, Hk=8, q=FAKE, qs=s2, ws=None, wsb=0):
        return lib.qwen3_varlen_prefill_bf16(q, qs, FAKE, _s(1024, 128), FAKE, _s(1024, 128), FAKE, s2,
                                             FAKE, 2, 100, 150, H, Hk, D, 0.088, 1, ws, wsb, None)

    need = lib.qwen3_varlen_prefill_workspace_bytes()
    # 9 schedule counters 128 B apart, then for two ranges per CU (256 CUs
    # when no device is visible) one ticket each (256-aligned) and two
    # partial-state slots each of 4 waves x 64 lanes x 66 floats
    ranges = 2 * (_cus() or 256)
    assert need == 1152 + -(-ranges * 4 // 256) * 256 + 2 * ranges * 4 * 64 * 66 * 4
    assert call(ws=FAKE, wsb=need - 1) == -4  # a schedule workspace too small
    assert call(D=256) == -3
    assert call(H=12, Hk=8) == -3
    assert call(q=None) == -1
    assert call(qs=_s(2048, 129)) == -2


def test_pre_attention_rejects_bad_arguments():
    lib = _lib.load()
    qs, ks, c4 = _s(4096, 128), _s(4096, 128), _s(1 << 16, 1 << 14, 2048, 128)

    def dec(D=128, q=FAKE, q_strides=qs, tab_stride=128, bt_stride=8, layer=0, layers=4):
        return lib.qwen3_qk_norm_rope_decode_bf16(
            q, q_strides, FAKE, ks, FAKE, ks, FAKE, FAKE, 1e-6, FAKE, FAKE, tab_stride, 64,
            FAKE, _s(2048, 128), FAKE, c4, FAKE, c4, 16, layer, layers, FAKE, FAKE, bt_stride,
            4, 8, None, None, 2, 16, 8, D, 16, None)

    assert dec(D=64) == -3
    assert dec(q=None) == -1
    assert dec(q=FAKE + 2) == -2
    assert dec(q_strides=_s(4100, 128)) == -2
    assert dec(tab_stride=130) == -2
    assert dec(bt_stride=4) == -1  # table rows shorter than max_pages
    assert dec(layer=4) == -1 and dec(layer=-1) == -1  # layer outside the pool

    def slots(positions=FAKE, D=128, layer=0):
        return lib.qwen3_qk_norm_rope_slots_bf16(
            FAKE, qs, FAKE, ks, FAKE, ks, FAKE, FAKE, 1e-6, FAKE, FAKE, 128, 64, positions, None,
            FAKE, _s(2048, 128), None, None, FAKE, c4, FAKE, c4, 16, layer, 2, 5, 16, 8, D, 16,
            None)

    assert slots(positions=None) == -1
    assert slots(D=256) == -3
    assert slots(layer=2) == -1


def test_model_ops_reject_bad_arguments():
    lib = _lib.load()
    # hidden not a multiple of 8 / too large; misaligned rows; null weight
    assert lib.qwen3_add_rms_norm_bf16(None, 0, FAKE, 1024, None, 0, FAKE, 1e-6, FAKE, 1024,
                                       None, 0, 4, 1020, None) == -3
    assert lib.qwen3_add_rms_norm_bf16(None, 0, FAKE, 16384, None, 0, FAKE, 1e-6, FAKE, 16384,
                                       None, 0, 4, 16384, None) == -3
    assert lib.qwen3_add_rms_norm_bf16(FAKE, 1030, FAKE, 1024, None, 0, FAKE, 1e-6, FAKE, 1024,
                                       None, 0, 4, 1024, None) == -2
    assert lib.qwen3_add_rms_norm_bf16(None, 0, FAKE, 1024, None, 0, None, 1e-6, FAKE, 1024,
                                       None, 0, 4, 1024, None) == -1
    assert lib.qwen3_add_rms_norm_bf16(None, 0, FAKE, 1024, None, 0, FAKE, -1.0, FAKE, 1024,
                                       None, 0, 4, 1024, None) == -1
    assert lib.qwen3_silu_mul_bf16(FAKE, 6144, FAKE, 3072, 4, 3070, None) == -3
    assert lib.qwen3_silu_mul_bf16(FAKE + 2, 6144, FAKE, 3072, 4, 3072, None) == -2
    assert lib.qwen3_argmax_bf16(FAKE, 100, 4, 151936, FAKE, None) == -1  # row stride < vocab
    assert lib.qwen3_argmax_bf16(None, 151936, 4, 151936, FAKE, None) == -1
    assert lib.qwen3_advance_seq_lens(None, 8, FAKE, 4, -1, 1, None) == -1
    def lin(M=64, N=1024, K=2048, epi=0, y=FAKE, ss_in=None, nw=FAKE):
        return lib.qwen3_decode_linear_bf16(FAKE, K, ss_in, 64, nw, 1e-6, FAKE, K, M, N, K, epi,
                                            y, N, FAKE, N, FAKE + 4096, N, FAKE, 0, None)

    assert lin(M=65) == -1                 # more rows than a decode batch
    assert lin(N=1000) == -3 and lin(K=1000) == -3
    assert lin(epi=3) == -1
    assert lin(y=None) == -1
    assert lin(ss_in=FAKE, nw=None) == -1  # norm prologue without its weight
    assert lin(epi=2, N=1024) == -1        # silu: up half must start at or after row N
    assert lib.qwen3_sample_bf16(FAKE, 100, 4, 151936, None, None, None, 1, FAKE, None) == -1
    assert lib.qwen3_sample_bf16(None, 151936, 4, 151936, None, None, None, 1, FAKE, None) == -1
    assert lib.qwen3_sample_bf16(FAKE, 151936, 0, 151936, None, None, None, 1, FAKE, None) == 0
    need = int(lib.qwen3_sample_workspace_bytes(64, 151936))
    assert need == 64 * 4 * 32784          # 4 parts per row, one record per part
    assert int(lib.qwen3_sample_workspace_bytes(16, 151936)) == 16 * 8 * 32784
    assert int(lib.qwen3_sample_workspace_bytes(128, 151936)) == 128 * 2 * 32784
    assert int(lib.qwen3_sample_workspace_bytes(600, 151936)) == 0  # one workgroup per row
    assert int(lib.qwen3_sample_workspace_bytes(1, 1000)) == 0      # one round: one part
    assert int(lib.qwen3_sample_workspace_bytes(1, 20000)) == 1 * 3 * 32784  # three rounds
    assert lib.qwen3_sample_ws_bf16(FAKE, 151936, 64, 151936, None, None, None, 1, FAKE,
                                    FAKE, need - 16, None) == -4  # workspace too small
    assert lib.qwen3_sample_ws_bf16(FAKE, 151936, 64, 151936, None, None, None, 1, FAKE,
                                    FAKE + 8, need, None) == -2   # misaligned workspace
    assert lib.qwen3_sample_ws_bf16(FAKE, 100, 4, 151936, None, None, None, 1, FAKE,
                                    FAKE, need, None) == -1       # stride < vocab
    assert lib.qwen3_sample_ws_bf16(FAKE, 151936, 0, 151936, None, None, None, 1, FAKE,
                                    FAKE, need, None) == 0
    assert lib.qwen3_page_in_bf16(FAKE, 8, 4, 16, FAKE, 2, FAKE, FAKE, 100, 10, None) == -1  # stride < pages
    assert lib.qwen3_page_in_bf16(FAKE, 16, 4, 16, FAKE, 2, FAKE, FAKE, 100, 10, None) == -2  # odd block
    s2, s4 = _s(2048, 128), _s(1 << 16, 1 << 14, 2048, 128)

    def qkv(M=16, K=1024, D=128, ss=FAKE, bt_stride=8, layer=0):
        return lib.qwen3_decode_qkv_rope_bf16(
            FAKE, K, ss, 64, FAKE, 1e-6, FAKE, K, M, K, 16, 8, D, FAKE, FAKE, 1e-6, FAKE, FAKE,
            128, 64, None, FAKE, s2, FAKE, s4, FAKE, s4, 16, layer, 28, FAKE, FAKE, bt_stride,
            4, 8, None, 16, None)

    assert qkv(M=65) == -1 and qkv(D=64) == -3 and qkv(K=1000) == -3 and qkv(K=4160) == -3
    assert qkv(ss=None) == -1 and qkv(bt_stride=4) == -1
    assert qkv(layer=28) == -1
    ws = lib.qwen3_lm_head_argmax_workspace_bytes()
    assert ws > 0

    def head(M=16, K=1024, wsb=ws, out=FAKE):
        return lib.qwen3_lm_head_argmax_bf16(FAKE, K, FAKE, K // 16, FAKE, 1e-6, FAKE, K, M,
                                             151936, K, FAKE, wsb, out, None)

    assert head(M=65) == -1 and head(K=1000) == -3 and head(K=2048) == -3
    assert head(wsb=ws - 1) == -4 and head(out=None) == -1 and head(M=0) == 0
    # nothing to do: no launch, success
    assert lib.qwen3_add_rms_norm_bf16(None, 0, FAKE, 1024, None, 0, FAKE, 1e-6, FAKE, 1024,
                                       None, 0, 0, 1024, None) == 0
    assert lib.qwen3_argmax_bf16(FAKE, 16, 0, 16, FAKE, None) == 0


def test_kv_write_rejects_bad_arguments():
    lib = _lib.load()
    c4 = _s(1 << 16, 1 << 14, 2048, 128)
    n = _s(1024, 128)

    def rng(layer=0, layers=1, start=20):
        return lib.qwen3_kv_write_range_bf16(FAKE, n, FAKE, n, FAKE, c4, FAKE, c4, 64, layer,
                                             layers, FAKE, 2, start, 40, 8, 128, 16, None)

    assert rng() == -1  # positions 20..59 need 4 pages, the row has 2
    assert rng(start=0, layer=1, layers=1) == -1  # layer outside the pool
    assert rng(start=0, layer=-1, layers=4) == -1

    def dec(sl=FAKE, layer=0, layers=4):
        return lib.qwen3_kv_write_decode_bf16(FAKE, n, FAKE, n, FAKE, c4, FAKE, c4, 64, layer,
                                              layers, sl, FAKE, 8, 4, 8, None, 2, 8, 128, 16,
                                              None)

    assert dec(sl=None) == -1  # null seq_lens
    assert dec(layer=4) == -1 and dec(layer=7, layers=4) == -1
    slot = lambda layer, layers: lib.qwen3_kv_write_slots_bf16(  # noqa: E731
        FAKE, n, FAKE, n, FAKE, c4, FAKE, c4, 64, layer, layers, FAKE, 10, 8, 128, 16, None)
    assert slot(2, 2) == -1 and slot(0, 0) == -1


def test_wrappers_refuse_cpu_tensors():
    """No CPU fallback: the product path raises instead of computing on the host."""
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import paged_attention_decode_hip
    from qwen3_engine_from_scratch_amd.kernels.flash_attention_varlen import flash_attention_prefill

    q = torch.zeros(2, 16, 128, dtype=torch.bfloat16)
    kb = torch.zeros(8, 8, 16, 128, dtype=torch.bfloat16)
    bt = torch.zeros(2, 4, dtype=torch.int32)
    sl = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        paged_attention_decode_hip(q, kb, kb, bt, sl, None, 16)
    cu = torch.tensor([0, 2], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        flash_attention_prefill(q, q[:, :8], q[:, :8], cu, 0.088, 16, 8, 128, max_seqlen=2)


def test_hbm_read_reference_rejects_bad_arguments():
    lib = _lib.load()
    assert lib.qwen3_hbm_read_reference(None, 1 << 20, 1, FAKE, None) == -1
    assert lib.qwen3_hbm_read_reference(FAKE, 1 << 20, 1, None, None) == -1
    assert lib.qwen3_hbm_read_reference(FAKE, (1 << 20) + 8, 1, FAKE, None) == -1  # not 16 B units
    assert lib.qwen3_hbm_read_reference(FAKE, -16, 0, FAKE, None) == -1
    assert lib.qwen3_hbm_read_reference(FAKE + 8, 1 << 20, 0, FAKE, None) == -2   # misaligned
    assert lib.qwen3_hbm_read_reference(FAKE, 0, 1, FAKE, None) == 0              # nothing to read


def test_mfma_rate_reference_rejects_bad_arguments():
    lib = _lib.load()
    flops = ctypes.c_int64(0)
    assert lib.qwen3_mfma_rate_reference(0, FAKE, ctypes.byref(flops), None) == -1
    assert lib.qwen3_mfma_rate_reference((1 << 24) + 1, FAKE, ctypes.byref(flops), None) == -1
    assert lib.qwen3_mfma_rate_reference(10, None, ctypes.byref(flops), None) == -1
    assert lib.qwen3_mfma_rate_reference(10, FAKE, None, None) == -1
    assert lib.qwen3_mfma_rate_reference(10, FAKE + 4, ctypes.byref(flops), None) == -2
