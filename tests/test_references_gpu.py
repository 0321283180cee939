"""The two measurement references of the library on the GPU (no counterpart
in the reference engine): the streaming read (qwen3_hbm_read_reference) and
the matrix-core rate (qwen3_mfma_rate_reference).  They compute nothing the
caller uses, so the tests check that each call completes, that the read
path sums what it loads (a planted chunk whose sum is the kernel's store
condition makes it write its sink), and the reported flop count."""
import ctypes

import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu

MAGIC = 0x9E3779B9


def test_hbm_read_reference_reads_its_bytes(gpu):
    from qwen3_engine_from_scratch_amd import _lib

    lib = _lib.load()
    stream = _lib.stream_of(gpu)
    for nt in (1, 0):
        # 64 chunks: wave 0 reads them all, lane l chunk l; chunk 0 sums to the
        # store condition, every other chunk to zero
        buf = torch.zeros(64 * 4, dtype=torch.int64, device=gpu).view(torch.int32)
        buf[0] = torch.tensor(MAGIC, dtype=torch.int64).to(torch.int32)
        sink = torch.zeros(4, dtype=torch.int32, device=gpu)
        announce(f"hbm_read_reference: 1 KiB, nontemporal={nt}")
        rc = lib.qwen3_hbm_read_reference(buf.data_ptr(), 1024, nt, sink.data_ptr(), stream)
        assert rc == 0, _lib.load().qwen3_attn_last_error()
        torch.cuda.synchronize()
        assert int(sink[0].item()) & 0xFFFFFFFF == MAGIC
        # a larger, ragged buffer of ones: completes, sums never hit the condition
        big = torch.ones((3 << 20) + 16, dtype=torch.uint8, device=gpu)
        sink.zero_()
        announce(f"hbm_read_reference: {big.numel()} bytes, nontemporal={nt}")
        rc = lib.qwen3_hbm_read_reference(big.data_ptr(), big.numel(), nt, sink.data_ptr(),
                                          stream)
        assert rc == 0
        torch.cuda.synchronize()
        assert int(sink[0].item()) == 0


def test_mfma_rate_reference_flop_count(gpu):
    from qwen3_engine_from_scratch_amd import _lib

    lib = _lib.load()
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    sink = torch.zeros(4, dtype=torch.int32, device=gpu)
    flops = ctypes.c_int64(0)
    announce("mfma_rate_reference: 10 iterations")
    rc = lib.qwen3_mfma_rate_reference(10, sink.data_ptr(), ctypes.byref(flops),
                                       _lib.stream_of(gpu))
    assert rc == 0
    torch.cuda.synchronize()
    assert flops.value == cus * 2 * 4 * 10 * 16 * 2 * 32 * 32 * 16
    assert int(sink[0].item()) == 0
