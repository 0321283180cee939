"""qwen3_paged_decode_noalloc_bf16 (the allocation-free decode entry point)
against qwen3_paged_decode_bf16 with a caller workspace: the same kernels and
split, so the same bits, and both within the attention bar of the fp32
reference; two calls in a row, the second smaller, then the size limits."""
import ctypes

import pytest
import torch

from conftest import announce
from gpu_helpers import assert_close_attn, gpu_dense_decode_fp32
from test_decode_gpu import make_device_decode

pytestmark = pytest.mark.gpu


def _noalloc(lib, t, hq, hkv, out, bias=1):
    from qwen3_engine_from_scratch_amd import _lib

    B = t["q"].shape[0]
    return lib.qwen3_paged_decode_noalloc_bf16(
        t["q"].data_ptr(), _lib.strides(t["q"], (0, 1)),
        t["k"].data_ptr(), _lib.strides(t["k"], (0, 1, 2)),
        t["v"].data_ptr(), _lib.strides(t["v"], (0, 1, 2)), t["k"].shape[0],
        t["bt"].data_ptr(), t["bt"].stride(0), t["bt"].shape[0], t["bt"].shape[1],
        t["seq_lens"].data_ptr(), bias, t["row_ids"].data_ptr(),
        out.data_ptr(), _lib.strides(out, (0, 1)), B, hq, hkv, 128, 16,
        ctypes.c_float(128 ** -0.5), _lib.stream_of(t["q"].device))


@pytest.mark.parametrize("hq,hkv", [(32, 8), (16, 8)])
def test_noalloc_decode_equals_workspace_entry(gpu, hq, hkv):
    from qwen3_engine_from_scratch_amd import _lib
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import paged_attention_decode_hip

    lib = _lib.load()
    g = torch.Generator().manual_seed(hq)
    cases = [[int(x) for x in torch.randint(1000, 6000, (200,), generator=g)],
             [int(x) for x in torch.randint(1, 900, (37,), generator=g)]]  # second call smaller
    for i, lens in enumerate(cases):
        announce(f"noalloc decode call {i}: B={len(lens)} sumL={sum(lens)} heads {hq}/{hkv}")
        t = make_device_decode(lens, hq, hkv, gpu, seed=10 + i, slack=0.1)
        ref_ws = paged_attention_decode_hip(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"],
                                            t["row_ids"], 16)
        out = torch.full_like(t["q"], float("nan"))
        rc = _noalloc(lib, t, hq, hkv, out)
        _lib.check(rc, "qwen3_paged_decode_noalloc_bf16")
        torch.cuda.synchronize()
        assert torch.equal(out, ref_ws), f"call {i}: differs from the workspace entry point"
        ref = gpu_dense_decode_fp32(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"],
                                    t["row_ids"], 16)
        assert_close_attn(out, ref, f"noalloc call {i}")


def test_noalloc_decode_rejects_sizes_beyond_its_scratch(gpu):
    from qwen3_engine_from_scratch_amd import _lib

    lib = _lib.load()
    announce("noalloc decode size limits (rejected before any launch)")
    t = make_device_decode([20, 30], 16, 1, gpu, seed=3)  # G = 16: partials exceed 24 MiB
    out = torch.zeros_like(t["q"])
    rc = _noalloc(lib, t, 16, 1, out)
    assert rc == -4 and b"static scratch" in lib.qwen3_attn_last_error()
    big = make_device_decode([3] * 2049, 16, 8, gpu, seed=4)  # more rows than it serves
    out = torch.zeros_like(big["q"])
    assert _noalloc(lib, big, 16, 8, out) == -4
    torch.cuda.synchronize()
    assert not out.any(), "a rejected call launched work"
