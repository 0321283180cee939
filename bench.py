"""Benchmark of the MI355X attention hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                    [--only decode|prefill|pre_attention|sampling|e2e] [--workload config3|config4]

Headline (the JSON `value`): paged decode attention at the Qwen3-8B shape —
batch 256, 32 query / 8 KV heads, head_dim 128, bf16, block 16, context
lengths uniform in [1024, 8192] (seed 0), a pool of 1.1x the needed blocks and
random-permutation block tables.  One step = one decode-attention call over
the whole batch (the split-KV partition kernel plus the LSE merge), inputs
resident in HBM.  value = algorithmic bytes per step / time per step (GB/s).

Also reported on the same line:
  roofline      the decode call against the 8 TB/s HBM peak, timed with HIP
                events on the launch stream;
  decode_config1 one Qwen3-0.6B decode layer (B=4, contexts [37, 128, 511,
                1024]): time per call, parity against the oracle on the same
                tensors, and the oracle timed on the host (median of 10);
  cpu_baseline  the oracle's restatement of the reference's PyTorch decode path
                (qwen3/paged_attention.py:39-122) on the host cores, over a
                bounded sample (the first 64 sequences) of the same workload;
  decode_long_context  the same decode over 8 contexts in [32768, 131072];
  decode_batch_invariant  both decode workloads on the batch-invariant
                kernel (each sequence's output bits independent of the batch);
  prefill       varlen causal prefill at the Qwen3-0.6B shape (8 sequences,
                lengths uniform in [64, 2048], 16/8 heads) in TFLOP/s against
                the 2.5 PFLOP/s bf16 dense MFMA peak, plus its slot write and
                a single 2,048-token prompt;
  pre_attention the fused QK-RMSNorm + RoPE + pool write (prefill and decode
                forms) against the HBM peak;
  sampling      greedy and top-k / top-p token sampling over a 64 x 151936
                batch of logits, per call;
  e2e           the whole Qwen3-0.6B model (random-init bf16) serving 64
                requests by continuous batching, 256 greedy tokens each, in
                output tokens/s.
Lines whose working set is under 512 MB (config 1, pre-attention, the slot
write, sampling, and the prefill's flushed figure) read a 512 MiB buffer
before every timed rep, so their inputs come from HBM, and time each rep
with its own event pair; the per-rep pair adds about 5-6 us of dispatch
latency that back-to-back launches hide, so their back-to-back figures
ride along.  CPU baselines (the oracle, on the host cores) ride on the
decode, config-1, prefill and serving lines.
Prints exactly one JSON line on stdout (progress goes to stderr).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = "paged-decode attn GB/s & %HBM peak; varlen prefill TFLOPS & %MFMA peak"


def log(msg: str) -> None:
    sys.stderr.write(f"[bench] {msg}\n")
    sys.stderr.flush()


def decode_inputs(lens, hq, hkv, dev, seed=0, slack=0.1, block_size=16, head_dim=128):
    import numpy as np
    import torch

    g = torch.Generator(device=dev).manual_seed(seed)
    pages = [(L + block_size - 1) // block_size for L in lens]
    nb = int(np.ceil(sum(pages) * (1 + slack)))
    perm = torch.randperm(nb, generator=g, device=dev).to(torch.int32)
    bt = torch.full((len(lens), max(pages)), -1, dtype=torch.int32, device=dev)
    off = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[off:off + n]
        off += n
    k = torch.randn(nb, hkv, block_size, head_dim, generator=g, device=dev, dtype=torch.bfloat16)
    v = torch.randn(nb, hkv, block_size, head_dim, generator=g, device=dev, dtype=torch.bfloat16)
    q = torch.randn(len(lens), hq, head_dim, generator=g, device=dev, dtype=torch.bfloat16)
    sl = torch.tensor([L - 1 for L in lens], dtype=torch.int32, device=dev)
    rows = torch.arange(len(lens), dtype=torch.int32, device=dev)
    return dict(q=q, k=k, v=v, bt=bt, seq_lens=sl, row_ids=rows, pages=pages, nb=nb)


def decode_bytes(lens, hq, hkv, head_dim=128, block_size=16):
    """Algorithmic HBM bytes of one decode call: K and V of every attended
    token, q in, out, the block-table entries and per-row lengths/ids."""
    pages = sum((L + block_size - 1) // block_size for L in lens)
    B = len(lens)
    return (sum(lens) * hkv * head_dim * 2 * 2 + 2 * B * hq * head_dim * 2 + 4 * pages + 8 * B)


def time_steps(fn, steps, warmup):
    """W untimed warmups, then K timed steps bracketed by synchronize, and by
    one pair of HIP events on torch's current stream (where the kernels are
    launched) around the whole timed region.  Returns (wall ms/step, event
    ms/step = region / K).  One event pair per step would add each event's
    own cost to every step (about 6 us on a 70 us kernel)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    evt = start.elapsed_time(end) / steps
    return wall, evt


def warm_up(fn, seconds=0.3):
    """Runs fn (untimed) for about `seconds` of wall time, so the clocks
    have ramped up before a short kernel is timed (its first tens of calls
    after idle run up to ~10% slower)."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def time_graph(fn, steps, warmup):
    """Back-to-back rate of a short kernel without the host's launch cost:
    `steps` calls of fn captured into one HIP graph (after `warmup` eager
    calls), replayed once untimed and then timed by one event pair on
    torch's current stream around three replays.  Returns ms per call."""
    import torch

    for _ in range(max(warmup, 1)):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(steps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(3):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (3 * steps)


_FLUSH = {}


def flush_caches(dev) -> None:
    """Reads a 512 MiB scratch buffer (a max-reduction into one value),
    evicting the L2s and the 256 MB MALL, so the next kernel reads its
    inputs from HBM.  Reading rather than writing leaves no dirty lines
    behind, whose write-back would otherwise land in the timed interval
    (the event after the flush releases the caches)."""
    import torch

    buf = _FLUSH.get(str(dev))
    if buf is None:
        buf = _FLUSH[str(dev)] = torch.ones(64 << 20, dtype=torch.int64, device=dev)
        _FLUSH[str(dev) + "out"] = torch.empty((), dtype=torch.int64, device=dev)
    torch.amax(buf, dim=0, out=_FLUSH[str(dev) + "out"])


def time_steps_flushed(fn, steps, warmup, dev):
    """For working sets under 512 MB: W untimed warmups, then K reps, each
    after a cache flush and between its own pair of HIP events on torch's
    current stream (the launch stream).  Returns event ms per rep (the
    median of the K intervals); the flush itself is outside them."""
    import torch

    for _ in range(warmup):
        flush_caches(dev)
        fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    for a, b in evs:
        flush_caches(dev)
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    ts = sorted(a.elapsed_time(b) for a, b in evs)
    return ts[len(ts) // 2] if len(ts) % 2 else 0.5 * (ts[len(ts) // 2 - 1] + ts[len(ts) // 2])


def copy_reference(nbytes, dev, steps, warmup):
    """What a plain device copy (torch's copy kernel, nbytes / 2 read and
    nbytes / 2 written, contiguous) reaches at the same size: GB/s after a
    cache flush and back to back.  The ceiling a kernel of that many bytes
    is measured against."""
    import torch

    n = nbytes // 4
    src = torch.ones(n // 2, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    fn = lambda: dst.copy_(src)  # noqa: E731
    warm_up(fn)
    cold = time_steps_flushed(fn, steps, warmup, dev)
    hot = time_graph(fn, steps, warmup)
    b = 2 * src.numel() * 4
    return {"GB/s_flushed": round(b / (cold * 1e-3) / 1e9, 1),
            "GB/s_back_to_back": round(b / (hot * 1e-3) / 1e9, 1)}


def read_reference(nbytes, dev, reps=5):
    """What torch's own streaming reduction (a max over an int64 buffer of
    nbytes) reads per second: a plain full-device read of the decode call's
    byte count, the reference point of the decode line."""
    import torch

    buf = torch.ones(nbytes // 8, dtype=torch.int64, device=dev)
    warm_up(lambda: torch.amax(buf))
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        torch.amax(buf)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    del buf
    torch.cuda.empty_cache()
    return {"GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1), "ms": round(ms, 5),
            "kernel": f"torch.amax over {nbytes} bytes of int64"}


def stream_read_reference(nbytes, dev, nontemporal=True, reps=5):
    """What the library's streaming read reference (qwen3_hbm_read_reference:
    16-byte loads over a persistent grid, non-temporal like the decode's K/V
    loads or plain, no other work) reaches on nbytes: the device's read
    ceiling for the decode call's byte count."""
    import torch

    from qwen3_engine_from_scratch_amd import _lib

    lib = _lib.load()
    n = nbytes // 16 * 16
    buf = torch.ones(n // 8, dtype=torch.int64, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    stream = _lib.stream_of(dev)

    def call():
        _lib.check(lib.qwen3_hbm_read_reference(buf.data_ptr(), n, 1 if nontemporal else 0,
                                                sink.data_ptr(), stream),
                   "qwen3_hbm_read_reference")

    warm_up(call)  # as the decode line: untimed calls until the clocks have ramped
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        call()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    del buf
    torch.cuda.empty_cache()
    return {"GB/s": round(n / (ms * 1e-3) / 1e9, 1), "ms": round(ms, 5),
            "kernel": f"qwen3_hbm_read_reference over {n} bytes, "
                      f"{'non-temporal' if nontemporal else 'plain'} 16-byte loads"}


def mfma_rate_reference(dev, iters=2000, reps=5):
    """What the library's matrix-core rate reference (qwen3_mfma_rate_reference:
    back-to-back bf16 32x32x16 MFMAs from registers, two waves per SIMD as in
    the prefill kernel, no memory traffic) sustains: the practical bf16 ceiling
    at the clock the device holds under matrix-core load."""
    import ctypes

    import torch

    from qwen3_engine_from_scratch_amd import _lib

    lib = _lib.load()
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    flops = ctypes.c_int64(0)
    stream = _lib.stream_of(dev)

    def call():
        _lib.check(lib.qwen3_mfma_rate_reference(iters, sink.data_ptr(), ctypes.byref(flops),
                                                 stream), "qwen3_mfma_rate_reference")

    call()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        call()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    return {"TFLOP/s": round(flops.value / (ms * 1e-3) / 1e12, 1), "ms": round(ms, 5),
            "kernel": f"qwen3_mfma_rate_reference, {flops.value} flop per call "
                      "(bf16 32x32x16 MFMAs, two waves per SIMD, no memory traffic)"}


def seeded_lengths(n: int, lo: int, hi: int, seed: int = 0) -> list:
    """n lengths uniform in [lo, hi] from a seeded CPU generator."""
    import torch

    g = torch.Generator().manual_seed(seed)
    return [int(x) for x in torch.randint(lo, hi + 1, (n,), generator=g)]


# The workloads (seed 0): Qwen3-0.6B varlen prefill (8 lengths in [64, 2048]),
# the Qwen3-8B decode headline (256 contexts in [1024, 8192]) and the
# long-context decode (8 contexts in [32768, 131072]).
WORKLOAD_LENGTHS = {
    "config2": (8, 64, 2048),
    "config3": (256, 1024, 8192),
    "config4": (8, 32768, 131072),
}


def workload_lengths(name: str) -> list:
    return seeded_lengths(*WORKLOAD_LENGTHS[name])


def bench_decode(args, dev, batch_invariant=False):
    import torch

    from qwen3_engine_from_scratch_amd.kernels.paged_attention import (
        paged_attention_decode_hip, paged_decode_workspace_bytes)

    if args.workload == "config4":
        lens, wname = workload_lengths("config4"), ("long-context split-KV paged decode, Qwen3-8B "
                                                    "shape: B=8, L~U[32768,131072]")
    else:
        lens, wname = workload_lengths("config3"), ("paged decode attention, Qwen3-8B shape: "
                                                    "B=256, L~U[1024,8192]")
    if batch_invariant:
        wname += " on the batch-invariant kernel (qwen3_paged_decode_invariant_bf16)"
    hq, hkv = 32, 8
    log(f"decode inputs: B={len(lens)} sumL={sum(lens)}")
    t = decode_inputs(lens, hq, hkv, dev)
    out = torch.empty_like(t["q"])
    # zeroed: the batch-invariant kernel's tickets start at zero
    ws = torch.zeros(paged_decode_workspace_bytes(len(lens), hq, hkv, 128, t["bt"].shape[1], 16,
                                                  batch_invariant=batch_invariant),
                     dtype=torch.uint8, device=dev)

    def step():
        paged_attention_decode_hip(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"], t["row_ids"],
                                   16, out=out, workspace=ws, batch_invariant=batch_invariant)

    # untimed calls first, so the clocks have ramped up before the W warm-up
    # steps and the K timed ones (a cold first process measured 4% low)
    warm_up(step)
    wall_ms, evt_ms = time_steps(step, args.steps, args.warmup)
    nbytes = decode_bytes(lens, hq, hkv)
    log(f"decode: {evt_ms * 1e3:.1f} us/call (events), {wall_ms * 1e3:.1f} us/step (wall)")
    res = dict(lens=lens, wname=wname, bytes=nbytes, wall_ms=wall_ms, evt_ms=evt_ms, t=t)
    return res


def cpu_baseline_decode(res, n_seq=64):
    """The oracle (restated reference PyTorch decode path) on the host cores
    over the first n_seq sequences of the same workload (same bytes)."""
    import torch

    from oracle import decode as od

    t = res["t"]
    lens = res["lens"][:n_seq]
    pages = [(L + 15) // 16 for L in lens]
    bt = t["bt"][:n_seq].cpu()
    used = torch.cat([bt[b, :n].long() for b, n in enumerate(pages)])
    remap = torch.full((t["nb"],), -1, dtype=torch.long)
    remap[used] = torch.arange(used.numel())
    k_cpu = t["k"][used.to(t["k"].device)].cpu()
    v_cpu = t["v"][used.to(t["v"].device)].cpu()
    bt_small = torch.full_like(bt, -1)
    m = bt >= 0
    bt_small[m] = remap[bt[m].long()].to(torch.int32)
    q_cpu = t["q"][:n_seq].cpu()
    sl = t["seq_lens"][:n_seq].cpu()
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    log(f"cpu baseline: {n_seq} sequences, {sum(pages)} pages, {torch.get_num_threads()} threads")
    t0 = time.perf_counter()
    od.paged_attention_ref(q_cpu, k_cpu, v_cpu, bt_small, sl, None, 16)
    dt = time.perf_counter() - t0
    nbytes = decode_bytes(lens, 32, 8)
    return {"value": round(nbytes / dt / 1e9, 4), "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"first {n_seq} of {len(res['lens'])} sequences ({sum(lens)} tokens, "
                      f"{sum(pages)} pages), one pass of the oracle's per-page loop, "
                      f"{dt:.2f} s"}


def config1_inputs():
    """Qwen3-0.6B decode layer on the CPU (seed 0): 16 / 8 heads, head_dim 128,
    B=4 with contexts [37, 128, 511, 1024], a pool of 512 blocks x 16 whose
    pages each sequence takes in turn from a seeded permutation; q and K
    pass through RMSNorm (eps 1e-6, weight 1 + 0.1 N(0,1)) before the bf16
    cast.  The same bytes as the oracle's config-1 case (a CPU test checks)."""
    import torch

    lens, hq, hkv, D, bs, nb = [37, 128, 511, 1024], 16, 8, 128, 16, 512
    g = torch.Generator().manual_seed(0)
    pages = [(L + bs - 1) // bs for L in lens]
    perm = torch.randperm(nb, generator=g)
    bt = torch.full((len(lens), max(pages)), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = torch.randn(len(lens), hq, D, generator=g)
    k = torch.randn(nb, hkv, bs, D, generator=g)
    v = torch.randn(nb, hkv, bs, D, generator=g)
    gq = 1.0 + 0.1 * torch.randn(D, generator=g)
    gk = 1.0 + 0.1 * torch.randn(D, generator=g)

    def rms(x, w):
        return (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)) * w

    return dict(lens=lens, q=rms(q, gq).to(torch.bfloat16), k=rms(k, gk).to(torch.bfloat16),
                v=v.to(torch.bfloat16), bt=bt,
                seq_lens=torch.tensor([L - 1 for L in lens], dtype=torch.int32),
                row_ids=torch.arange(len(lens), dtype=torch.int32))


def bench_decode_config1(args, dev):
    """Config-1 decode (one Qwen3-0.6B layer, B=4): the kernel's time per
    call with caches flushed, its parity against the oracle's restatement of
    the reference decode on the same tensors, and that oracle timed on the
    host cores (median of 10)."""
    import torch

    from qwen3_engine_from_scratch_amd.kernels.paged_attention import paged_attention_decode_hip

    c = config1_inputs()
    t = {k: c[k].to(dev) for k in ("q", "k", "v", "bt", "seq_lens", "row_ids")}
    out = torch.empty_like(t["q"])

    def step():
        paged_attention_decode_hip(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"],
                                   t["row_ids"], 16, out=out)

    ms = time_steps_flushed(step, args.steps, args.warmup, dev)
    nbytes = decode_bytes(c["lens"], 16, 8)
    log(f"decode config1 (B=4, 16/8 heads): {ms * 1e3:.2f} us/call flushed")
    res = {"workload": "paged decode attention, one Qwen3-0.6B layer: B=4, L=[37,128,511,1024], "
                       "16 q / 8 kv heads, head_dim 128, bf16, block 16, pool 512 blocks, "
                       "QK-RMSNorm'd q/K",
           "us_per_call": round(ms * 1e3, 2), "bytes": nbytes,
           "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    if not args.no_cpu_baseline:
        res.update(cpu_baseline_config1(c, out.cpu()))
    return res


def cpu_baseline_config1(c, gpu_out):
    """The oracle (restated reference decode, qwen3/paged_attention.py:39-122)
    on the config-1 tensors, timed on the host cores (median of 10), and the
    GPU output's distance from it (the attention bar: max-abs 2e-2,
    mean-abs 2e-3)."""
    import statistics

    import torch

    from oracle import decode as od

    torch.set_num_threads(os.cpu_count() or 1)
    times = []
    ref = None
    for _ in range(10):
        t0 = time.perf_counter()
        ref = od.paged_attention_ref(c["q"], c["k"], c["v"], c["bt"], c["seq_lens"],
                                     c["row_ids"], 16, out_fp32=True)
        times.append(time.perf_counter() - t0)
    d = (gpu_out.double() - ref.double()).abs()
    med = statistics.median(times)
    log(f"decode config1 cpu: {med * 1e3:.2f} ms median of 10, parity max-abs "
        f"{d.max().item():.2e} mean-abs {d.mean().item():.2e}")
    return {"cpu_baseline": {"value": round(med * 1e3, 3), "unit": "ms/call",
                             "cores": torch.get_num_threads(), "kind": "port",
                             "sample": "the whole workload, median of 10 passes of the "
                                       "oracle's per-page loop"},
            "parity_vs_oracle": {"max_abs": float(f"{d.max().item():.3e}"),
                                 "mean_abs": float(f"{d.mean().item():.3e}"),
                                 "bar": {"max_abs": 2e-2, "mean_abs": 2e-3},
                                 "pass": bool(d.max().item() < 2e-2 and d.mean().item() < 2e-3)}}


PROFILE_DIR = Path(__file__).resolve().parent / "profiles"
TRAFFIC_PROFILE = "paged_decode_stream_b256_qwen3_8b.md"
PREFILL_PROFILE = "varlen_prefill_qwen3_0p6b.md"
PRE_ATTENTION_PROFILE = "pre_attention_qwen3.md"


def profiled_traffic(name: str):
    """HBM bytes per launch measured offline with rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE (scaled by a known-size copy) and recorded in profiles/<name>."""
    f = PROFILE_DIR / name
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def bench_pre_attention(args, dev):
    """Fused QK-RMSNorm + RoPE + pool write, HBM-bound: the slot form over the
    Qwen3-0.6B prefill batch (8,115 tokens, 16 / 8 heads) and the decode form
    for one Qwen3-8B layer at B=256 (32 / 8 heads; a few MB, launch-bound)."""
    import torch

    from qwen3_engine_from_scratch_amd.kernels.pre_attention import (
        qk_norm_rope_decode, qk_norm_rope_prefill, rope_tables)

    cos, sin = rope_tables(128, 1e6, 4096, device=dev)
    g = torch.Generator(device=dev).manual_seed(0)
    res = {}

    lens = workload_lengths("config2")
    T = sum(lens)
    hq, hkv = 16, 8
    qkv = torch.randn(T, (hq + 2 * hkv) * 128, device=dev, generator=g).to(torch.bfloat16)
    q = qkv[:, :hq * 128].view(T, hq, 128)
    k = qkv[:, hq * 128:(hq + hkv) * 128].view(T, hkv, 128)
    v = qkv[:, (hq + hkv) * 128:].view(T, hkv, 128)
    w = torch.ones(128, dtype=torch.bfloat16, device=dev)
    pos = torch.cat([torch.arange(L, device=dev) for L in lens])
    nblk = (T + 15) // 16 + 8
    slots = torch.randperm(nblk * 16, device=dev, generator=g)[:T]
    kb = torch.zeros(nblk, 1, hkv, 16, 128, dtype=torch.bfloat16, device=dev)
    vb = torch.zeros_like(kb)
    qo = torch.empty(T, hq, 128, dtype=torch.bfloat16, device=dev)
    ko = torch.empty(T, hkv, 128, dtype=torch.bfloat16, device=dev)

    def pstep():
        qk_norm_rope_prefill(q, k, v, w, w, 1e-6, cos, sin, pos, slots, kb, vb, 0, qo, ko)

    warm_up(pstep)
    p_evt = time_steps_flushed(pstep, args.steps, args.warmup, dev)
    p_hot = time_graph(pstep, args.steps, args.warmup)
    # per token: q, k, v read, one cos and one sin row, position + slot;
    # q_out, k_out, pool k and pool v written
    pbytes = T * ((hq + 2 * hkv) * 256 + 2 * 128 * 4 + 16 + (hq + 3 * hkv) * 256)
    gbs = pbytes / (p_evt * 1e-3) / 1e9
    log(f"pre-attention (prefill, {T} tokens): {p_evt * 1e3:.1f} us/call flushed "
        f"({p_hot * 1e3:.1f} back to back), {gbs:.0f} GB/s")
    res["prefill"] = {"workload": f"Qwen3-0.6B prefill batch, {T} tokens, 16/8 heads",
                      "ms_per_step": round(p_evt, 5), "ms_per_step_back_to_back": round(p_hot, 5),
                      "bytes": pbytes, "GB/s": round(gbs, 1),
                      "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                      "GB/s_back_to_back": round(pbytes / (p_hot * 1e-3) / 1e9, 1),
                      "copy_same_bytes": copy_reference(pbytes, dev, args.steps, args.warmup),
                      "traffic": profiled_traffic(PRE_ATTENTION_PROFILE),
                      "traffic_source": f"profiles/{PRE_ATTENTION_PROFILE}"}
    del qkv, q, k, v, kb, vb, qo, ko

    from qwen3_engine_from_scratch_amd.PagedKVcache import KVCachePool
    B, hq, hkv = 256, 32, 8
    pool = KVCachePool(B * 2 + 8, 1, 16, hkv, 128, device=dev, dtype=torch.bfloat16,
                       max_seq_len=4096, max_requests=B)
    lens_d = torch.randint(1, 4000, (B,), device=dev, generator=g, dtype=torch.int32)
    pool.seq_lens[:B] = lens_d
    pages = (lens_d.long() + 16) // 16
    tab = torch.randint(0, B * 2 + 8, (B, pool.block_table_2d.shape[1]), device=dev,
                        generator=g, dtype=torch.int32)
    pool.block_table_2d[:B] = torch.where(
        torch.arange(tab.shape[1], device=dev)[None, :] < pages[:, None], tab, -1)
    qkv = torch.randn(B, (hq + 2 * hkv) * 128, device=dev, generator=g).to(torch.bfloat16)
    q = qkv[:, :hq * 128].view(B, hq, 128)
    k = qkv[:, hq * 128:(hq + hkv) * 128].view(B, hkv, 128)
    v = qkv[:, (hq + hkv) * 128:].view(B, hkv, 128)
    rows = torch.arange(B, dtype=torch.int32, device=dev)
    qd = torch.empty(B, hq, 128, dtype=torch.bfloat16, device=dev)

    # A decode layer step is a few MB: time it as the engine runs it, inside
    # captured graphs, so host launch cost is not measured: one call per
    # replay after a cache flush, and ten calls per replay back to back
    # (inputs in cache, as inside a decode step).
    for _ in range(3):
        qk_norm_rope_decode(q, k, v, w, w, 1e-6, cos, sin, pool, 0, rows, qd)
    torch.cuda.synchronize()
    graphs = {}
    for n in (1, 10):
        graphs[n] = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graphs[n]):
            for _ in range(n):
                qk_norm_rope_decode(q, k, v, w, w, 1e-6, cos, sin, pool, 0, rows, qd)

    d_evt = time_steps_flushed(graphs[1].replay, args.steps, args.warmup, dev)
    _, d_hot = time_steps(graphs[10].replay, args.steps, args.warmup)
    d_hot /= 10
    dbytes = B * ((hq + 2 * hkv) * 256 + 2 * 128 * 4 + 16 + (hq + 2 * hkv) * 256)
    log(f"pre-attention (decode, B={B}, 32/8 heads, graph replay): {d_evt * 1e3:.2f} us/call "
        f"flushed, {d_hot * 1e3:.2f} back to back")
    res["decode"] = {"workload": f"one Qwen3-8B layer, B={B} decode tokens, 32/8 heads",
                     "ms_per_step": round(d_evt, 5), "bytes": dbytes,
                     "GB/s": round(dbytes / (d_evt * 1e-3) / 1e9, 1),
                     "ms_per_step_back_to_back": round(d_hot, 5)}
    return res


def bench_prefill(args, dev):
    import torch

    from qwen3_engine_from_scratch_amd import _lib
    from qwen3_engine_from_scratch_amd.kernels.flash_attention_varlen import flash_attention_prefill
    from qwen3_engine_from_scratch_amd.kernels.pre_attention import qk_norm_rope_prefill, rope_tables

    if args.prefill_workload == "steady":
        # 8 x 4096 tokens, non-causal: every query tile sweeps every key tile,
        # no masking and no ragged tail (the kernel's steady-state rate).
        lens = [4096] * 8
        g = torch.Generator(device=dev).manual_seed(0)
        q = torch.randn(sum(lens), 16, 128, device=dev, generator=g).to(torch.bfloat16)
        k = torch.randn(sum(lens), 8, 128, device=dev, generator=g).to(torch.bfloat16)
        v = torch.randn(sum(lens), 8, 128, device=dev, generator=g).to(torch.bfloat16)
        cu = torch.tensor([0] + [4096 * (i + 1) for i in range(8)], dtype=torch.int32, device=dev)
        out = torch.empty_like(q)

        def sstep():
            flash_attention_prefill(q, k, v, cu, 128 ** -0.5, 16, 8, 128, max_seqlen=4096,
                                    causal=False, out=out)

        warm_up(sstep)
        s_evt = time_graph(sstep, args.steps, args.warmup)
        flops = 4 * 128 * 16 * sum(L * L for L in lens)
        tflops = flops / (s_evt * 1e-3) / 1e12
        mref = mfma_rate_reference(dev)
        log(f"prefill (steady, 8x4096 non-causal): {s_evt * 1e3:.1f} us/call, {tflops:.1f} TFLOP/s")
        return {"workload": "varlen non-causal prefill, 8 x 4096 tokens, 16/8 heads, head_dim 128, bf16",
                "value": round(tflops, 2), "unit": "TFLOP/s", "ms_per_step": round(s_evt, 5),
                "timing": "graph replay of back-to-back calls, HIP events",
                "flops": flops,
                "roofline": {"bound": "mfma", "achieved": round(tflops, 2),
                             "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                             "mfma_rate_reference": mref,
                             "frac_of_mfma_rate": round(tflops / mref["TFLOP/s"], 4)}}

    # Qwen3-0.6B batch: N(0,1) projections, QK-RMSNorm (weights 1 + 0.1 N(0,1))
    # and RoPE at positions 0..L-1 applied by the fused pre-attention kernel.
    lens = workload_lengths("config2")
    T = sum(lens)
    g = torch.Generator(device=dev).manual_seed(0)
    qkv = torch.randn(T, 32 * 128, device=dev, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(128, device=dev, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(128, device=dev, generator=g)).to(torch.bfloat16)
    cos, sin = rope_tables(128, 1e6, 4096, device=dev)
    pos = torch.cat([torch.arange(L, device=dev) for L in lens])
    none_pool = torch.zeros(1, 1, 8, 16, 128, dtype=torch.bfloat16, device=dev)
    q, k = qk_norm_rope_prefill(qkv[:, :2048].view(T, 16, 128), qkv[:, 2048:3072].view(T, 8, 128),
                                qkv[:, 3072:].view(T, 8, 128), qw, kw, 1e-6, cos, sin, pos, None,
                                none_pool, none_pool, 0)
    v = qkv[:, 3072:].reshape(T, 8, 128).contiguous()
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32,
                      device=dev)
    out = torch.empty_like(q)
    mx = max(lens)
    scale = 128 ** -0.5

    def step():
        flash_attention_prefill(q, k, v, cu, scale, 16, 8, 128, max_seqlen=mx, out=out)

    # MFMA-bound: the line is the back-to-back rate (in a prefill its inputs
    # come straight from the pre-attention kernel), timed as a graph replay
    # so the host's per-call launch cost (Python wrapper + ctypes, as much as
    # the kernel itself) is not in it; the eager loop's rate and the rate
    # with q/k/v flushed out of the caches before every call ride along.
    warm_up(step)
    evt_ms = time_graph(step, args.steps, args.warmup)
    _, eager_ms = time_steps(step, args.steps, args.warmup)
    cold_ms = time_steps_flushed(step, args.steps, args.warmup, dev)
    flops = 2 * 128 * 16 * sum(L * (L + 1) for L in lens)
    tflops = flops / (evt_ms * 1e-3) / 1e12
    mref = mfma_rate_reference(dev)
    log(f"prefill: {evt_ms * 1e3:.1f} us/call back to back ({cold_ms * 1e3:.1f} flushed, "
        f"{eager_ms * 1e3:.1f} eager loop), {tflops:.1f} TFLOP/s")

    # slot write of the same prefill into a block-16 pool (one launch), through
    # a seeded random slot mapping over 1.25x the blocks needed
    nblk = (T + 15) // 16 * 5 // 4 + 1
    kb = torch.zeros(nblk, 1, 8, 16, 128, dtype=torch.bfloat16, device=dev)
    vb = torch.zeros_like(kb)
    sm = torch.randperm(nblk * 16, device=dev, generator=g)[:T]
    lib = _lib.load()

    def wstep():
        rc = lib.qwen3_kv_write_slots_bf16(
            k.data_ptr(), _lib.strides(k, (0, 1)), v.data_ptr(), _lib.strides(v, (0, 1)),
            kb.data_ptr(), _lib.strides(kb, (0, 1, 2, 3)), vb.data_ptr(),
            _lib.strides(vb, (0, 1, 2, 3)), nblk, 0, 1, sm.data_ptr(), sm.numel(), 8, 128,
            16, _lib.stream_of(dev))
        _lib.check(rc, "slots")

    warm_up(wstep)
    w_evt = time_steps_flushed(wstep, args.steps, args.warmup, dev)
    w_hot = time_graph(wstep, args.steps, args.warmup)
    wbytes = 8 * T * 8 * 128 + 8 * T
    wgbs = wbytes / (w_evt * 1e-3) / 1e9
    log(f"prefill slot write ({T} tokens): {w_evt * 1e3:.1f} us/call flushed "
        f"({w_hot * 1e3:.1f} back to back), {wgbs:.0f} GB/s")
    res = {"workload": f"varlen causal prefill, Qwen3-0.6B shape: 8 seqs lens={lens}, "
                       "16/8 heads, head_dim 128, bf16",
           "value": round(tflops, 2), "unit": "TFLOP/s", "ms_per_step": round(evt_ms, 5),
           "timing": "graph replay of back-to-back calls, HIP events",
           "ms_per_step_flushed": round(cold_ms, 5),
           "ms_per_step_eager_loop": round(eager_ms, 5), "flops": flops,
           "roofline": {"bound": "mfma", "achieved": round(tflops, 2),
                        "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                        "traffic": profiled_traffic(PREFILL_PROFILE),
                        "traffic_source": f"profiles/{PREFILL_PROFILE}",
                        "mfma_rate_reference": mref,
                        "frac_of_mfma_rate": round(tflops / mref["TFLOP/s"], 4)},
           "slot_write": {"GB/s": round(wgbs, 1), "frac_hbm_peak": round(wgbs / HBM_PEAK_GBS, 4),
                          "ms_per_step": round(w_evt, 5),
                          "ms_per_step_back_to_back": round(w_hot, 5), "bytes": wbytes,
                          "GB/s_back_to_back": round(wbytes / (w_hot * 1e-3) / 1e9, 1),
                          "copy_same_bytes": copy_reference(wbytes, dev, args.steps,
                                                            args.warmup)}}
    res["single_2048"] = bench_prefill_single(args, dev)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_prefill(lens, q, k, v, flops)
    return res


def bench_prefill_single(args, dev, L=2048):
    """One causal prompt of L tokens (Qwen3-0.6B heads): the small-batch case
    of the prefill, where the range schedule cuts the longest query tiles'
    items across workgroups; back-to-back graph replays, HIP events."""
    import torch

    from qwen3_engine_from_scratch_amd.kernels.flash_attention_varlen import flash_attention_prefill

    g = torch.Generator(device=dev).manual_seed(1)
    q = torch.randn(L, 16, 128, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(L, 8, 128, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(L, 8, 128, device=dev, generator=g).to(torch.bfloat16)
    cu = torch.tensor([0, L], dtype=torch.int32, device=dev)
    out = torch.empty_like(q)

    def step():
        flash_attention_prefill(q, k, v, cu, 128 ** -0.5, 16, 8, 128, max_seqlen=L, out=out)

    warm_up(step)
    evt_ms = time_graph(step, args.steps, args.warmup)
    flops = 2 * 128 * 16 * L * (L + 1)
    tflops = flops / (evt_ms * 1e-3) / 1e12
    log(f"prefill single {L}-token prompt: {evt_ms * 1e3:.1f} us/call, {tflops:.1f} TFLOP/s")
    return {"workload": f"varlen causal prefill, one {L}-token prompt, 16/8 heads, head_dim 128, "
                        "bf16", "value": round(tflops, 2), "unit": "TFLOP/s",
            "ms_per_step": round(evt_ms, 5), "flops": flops,
            "frac_mfma_peak": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "timing": "graph replay of back-to-back calls, HIP events"}


def cpu_baseline_prefill(lens, q, k, v, flops, reps=3):
    """The reference's batched prefill on the CPU, restated by the oracle:
    the padded batch through _standard_attention with the model's mask
    (qwen3/attention.py:193-207, qwen3/model.py:150-161) plus the per-request
    PagedKVCache.update of the padded K/V (qwen3/attention.py:160-161,
    qwen3/PagedKVcache.py:177-214), on the same q/k/v, all host cores,
    median of `reps` after one untimed pass."""
    import statistics

    import numpy as np
    import torch

    from oracle import kv_write as okw
    from oracle import prefill as op

    torch.set_num_threads(os.cpu_count() or 1)
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    cu = [0]
    for L in lens:
        cu.append(cu[-1] + L)
    S = max(lens)
    pages = (S + 15) // 16
    table = np.arange(len(lens) * pages, dtype=np.int32).reshape(len(lens), pages)
    kpool = np.zeros((len(lens) * pages, 1, kc.shape[1], 16, kc.shape[2]), np.uint16)
    vpool = np.zeros_like(kpool)

    def run():
        qp, kp, vp = (op.pad_batch(x, cu, S) for x in (qc, kc, vc))
        mask = op.prefill_mask(lens, S)
        for i in range(len(lens)):  # the reference writes S_max tokens per request
            okw.paged_update_ref(okw.as_u16(kp[i].transpose(0, 1)),
                                 okw.as_u16(vp[i].transpose(0, 1)), kpool, vpool, table[i], 0, 0)
        return op.standard_attention_ref(qp, kp, vp, mask, 128 ** -0.5)

    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    log(f"prefill cpu baseline: {med:.2f} s median of {reps}, {torch.get_num_threads()} threads")
    return {"value": round(flops / med / 1e12, 4), "unit": "TFLOP/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"the whole workload padded to {S} tokens (the reference's batched path), "
                      f"median of {reps} passes after one untimed pass, {med:.2f} s; the "
                      "causal algorithmic FLOPs divided by that time"}


def bench_sampling(args, dev):
    """Token sampling over one decode batch of Qwen3 logits (B=64 rows x
    151936 bf16): greedy (argmax kernel) and temperature 0.8 / top-k 50 /
    top-p 0.9 (the sampling kernel), per call; bytes = one read of the
    logits (the sampler re-reads them from L2 in its later passes)."""
    import torch

    from qwen3_engine_from_scratch_amd.sampling import sample_tokens

    B, V = 64, 151936
    g = torch.Generator(device=dev).manual_seed(0)
    x = (torch.randn(B, V, device=dev, generator=g) * 2).to(torch.bfloat16)
    t = torch.full((B,), 0.8, device=dev)
    k = torch.full((B,), 50, device=dev, dtype=torch.int32)
    p = torch.full((B,), 0.9, device=dev)
    res = {"workload": f"B={B} rows x {V} bf16 logits", "bytes": B * V * 2}
    for name, fn in (("greedy", lambda: sample_tokens(x)),
                     ("top_k50_top_p0.9_T0.8", lambda: sample_tokens(x, t, k, p, seed=1))):
        ms = time_steps_flushed(fn, args.steps, args.warmup, dev)
        res[name] = {"us_per_call": round(ms * 1e3, 2),
                     "GB/s": round(B * V * 2 / (ms * 1e-3) / 1e9, 1)}
        log(f"sampling {name}: {ms * 1e3:.1f} us/call flushed")
    return res


def bench_e2e(args, dev):
    """Whole Qwen3-0.6B (random-init bf16 weights) serving 64 requests with
    continuous batching: prompts of seeded lengths uniform in [128, 1024],
    256 greedy tokens each (the first from the prefill), prefill through the
    varlen kernel, decode through captured graphs per power-of-two bucket.
    Reports output tokens/s over the whole run (prefill included), after an
    untimed warm-up run of the same requests with 4 tokens each."""
    import random

    import torch

    from qwen3_engine_from_scratch_amd.PagedKVcache import KVCachePool
    from qwen3_engine_from_scratch_amd.config import qwen3_0p6b_config
    from qwen3_engine_from_scratch_amd.engine import Engine, GenRequest
    from qwen3_engine_from_scratch_amd.model import Qwen3ForCausalLM, init_random_weights

    n_req, lo, hi, new_tokens = 64, 128, 1024, args.e2e_tokens
    cfg = qwen3_0p6b_config(max_position_embeddings=4096)
    t0 = time.perf_counter()
    with torch.device(dev):
        model = Qwen3ForCausalLM(cfg)
    init_random_weights(model, seed=0)
    model = model.to(torch.bfloat16).eval()
    rng = random.Random(0)
    lens = [rng.randint(lo, hi) for _ in range(n_req)]
    g = torch.Generator().manual_seed(0)
    prompts = [torch.randint(0, cfg.vocab_size, (L,), generator=g).tolist() for L in lens]
    bs = 16
    max_seq = hi + new_tokens
    blocks = n_req * ((max_seq + bs - 1) // bs) + n_req + 1 + 16
    pool = KVCachePool(blocks, cfg.num_hidden_layers, bs, cfg.num_key_value_heads, cfg.head_dim,
                       device=dev, dtype=torch.bfloat16, max_seq_len=max_seq,
                       max_requests=2 * n_req + 8)
    t1 = time.perf_counter()
    engine = Engine(model, pool, max_batch=n_req, use_graph=True)
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    log(f"e2e: model init {t1 - t0:.1f} s, graph capture {t2 - t1:.1f} s")
    engine.generate([GenRequest(i, p, 4) for i, p in enumerate(prompts)])
    torch.cuda.synchronize()
    reqs = [GenRequest(i, p, new_tokens) for i, p in enumerate(prompts)]
    st = engine.generate(reqs)
    engine.close()
    dec_steps = max(st["decode_steps"], 1)
    log(f"e2e: {st['output_tokens']} tokens in {st['total_s']:.3f} s = "
        f"{st['tokens_per_s']:.0f} tok/s (prefill {st['prefill_s'] * 1e3:.1f} ms, "
        f"decode {st['decode_s'] * 1e3 / dec_steps:.3f} ms/step over {dec_steps} steps)")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_e2e(model, cfg, prompts[:2], 8)
    # bytes one decode step must read at the final context length: the weights
    # (the tied embedding once, as lm_head) and every live K/V token
    n_w = sum(p.numel() for p in model.parameters())
    ctx = sum(lens) + n_req * new_tokens
    kv_step = ctx * cfg.num_hidden_layers * cfg.num_key_value_heads * cfg.head_dim * 2 * 2
    return {"metric": "output tokens/s", "value": round(st["tokens_per_s"], 1),
            "unit": "tokens/s",
            "workload": "Qwen3-0.6B random-init bf16, 64 requests, prompts U[128,1024] "
                        f"(sum {sum(lens)}), {new_tokens} greedy tokens each, max batch 64, "
                        "decode in captured graphs (buckets 1..64)",
            "total_s": round(st["total_s"], 4), "output_tokens": st["output_tokens"],
            "prefill_ms": round(st["prefill_s"] * 1e3, 2),
            "decode_ms_per_step": round(st["decode_s"] * 1e3 / dec_steps, 4),
            "decode_steps": st["decode_steps"], "prefill_steps": st["prefill_steps"],
            "weight_bytes": 2 * n_w, "kv_bytes_last_step": kv_step, "cpu_baseline": cpu}


def cpu_baseline_e2e(model, cfg, prompts, n_new):
    """The same model served by the oracle's restatement of the reference's
    serial greedy generate() with a K/V cache (fp32 on the host cores), on a
    bounded sample: the first requests of the workload, n_new tokens each."""
    import torch

    from oracle import model as om

    torch.set_num_threads(os.cpu_count() or 1)
    state = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    t0 = time.perf_counter()
    for p in prompts:
        om.generate_greedy_ref(state, cfg, p, n_new)
    dt = time.perf_counter() - t0
    n = len(prompts) * n_new
    log(f"e2e cpu baseline: {n} tokens in {dt:.2f} s")
    return {"value": round(n / dt, 3), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{len(prompts)} requests (prompts of {[len(p) for p in prompts]} tokens), "
                      f"{n_new} greedy tokens each, one at a time with a K/V cache, fp32, "
                      f"{dt:.2f} s"}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["decode", "config1", "prefill", "pre_attention",
                                       "sampling", "e2e"],
                    default=None)
    ap.add_argument("--e2e-tokens", type=int, default=256,
                    help="greedy tokens per request in the whole-model serving line")
    ap.add_argument("--workload", choices=["config3", "config4"], default="config3")
    ap.add_argument("--prefill-workload", choices=["config2", "steady"], default="config2",
                    help="prefill line: the Qwen3-0.6B ragged causal batch, or 8 x 4096 tokens "
                         "non-causal (steady-state rate; profiling only, with --only prefill)")
    ap.add_argument("--cpu-sample", type=int, default=64, help="sequences in the CPU baseline sample")
    ap.add_argument("--no-invariant", action="store_true",
                    help="skip the batch-invariant decode lines")
    ap.add_argument("--decode-kernel", choices=["default", "invariant"], default="default",
                    help="kernel of the headline decode line (invariant: the batch-invariant "
                         "one, without the extra decode lines)")
    ap.add_argument("--no-long-context", action="store_true",
                    help="skip the secondary long-context (B=8, up to 128k tokens) decode line")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 1 GiB device copy (the known-size reference for "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args(argv)
    if args.prefill_workload != "config2" and args.only != "prefill":
        ap.error("--prefill-workload steady is a profiling line: use it with --only prefill")
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (MI355X)", file=sys.stderr)
        return 1
    from qwen3_engine_from_scratch_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()
    line = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) q/K/V, seeded lengths and block tables)"}
    if args.only in (None, "decode"):
        inv_main = args.decode_kernel == "invariant"
        res = bench_decode(args, dev, batch_invariant=inv_main)
        gbs = res["bytes"] / (res["wall_ms"] * 1e-3) / 1e9
        ach = res["bytes"] / (res["evt_ms"] * 1e-3) / 1e9
        line.update(value=round(gbs, 1), unit="GB/s", ms_per_step=round(res["wall_ms"], 5))
        line["config"] = {"workload": res["wname"] + ", 32 q / 8 kv heads, head_dim 128, bf16, "
                          "block 16, pool 1.1x pages, random-permutation block tables",
                          "batch": len(res["lens"]), "sum_context_tokens": sum(res["lens"]),
                          "bytes_per_step": res["bytes"]}
        traffic = (profiled_traffic(TRAFFIC_PROFILE) if args.workload == "config3" and not inv_main
                   else None)
        line["roofline"] = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                            "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                            "traffic": traffic, "kernel_ms": round(res["evt_ms"], 5),
                            "kernel": ("paged_decode_inv_stream_kernel (+ paged_decode_inv_merge_"
                                       "kernel when launched)" if inv_main else
                                       "paged_decode_stream_kernel + paged_decode_stream_merge_kernel")
                                      + " (one decode call), HIP events on the launch stream",
                            "traffic_source": f"profiles/{TRAFFIC_PROFILE}" if traffic else None}
        if not args.no_cpu_baseline:
            line["cpu_baseline"] = cpu_baseline_decode(res, args.cpu_sample)
        nbytes = res["bytes"]
        del res
        torch.cuda.empty_cache()
        line["roofline"]["read_reference"] = read_reference(nbytes, dev)
        line["roofline"]["stream_read_reference"] = stream_read_reference(nbytes, dev)
        line["roofline"]["frac_of_stream_read"] = round(
            line["roofline"]["achieved"] / line["roofline"]["stream_read_reference"]["GB/s"], 4)
        if args.workload == "config3" and not args.no_long_context and not inv_main:
            long_args = argparse.Namespace(**{**vars(args), "workload": "config4"})
            r4 = bench_decode(long_args, dev)
            line["decode_long_context"] = {
                "workload": r4["wname"] + ", 32 q / 8 kv heads, head_dim 128, bf16, block 16",
                "value": round(r4["bytes"] / (r4["evt_ms"] * 1e-3) / 1e9, 1), "unit": "GB/s",
                "ms_per_step": round(r4["evt_ms"], 5), "bytes_per_step": r4["bytes"],
                "frac_hbm_peak": round(r4["bytes"] / (r4["evt_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            del r4
            torch.cuda.empty_cache()
        if args.workload == "config3" and not args.no_invariant and not inv_main:
            for wl in ("config3", "config4"):
                ri = bench_decode(argparse.Namespace(**{**vars(args), "workload": wl}), dev,
                                  batch_invariant=True)
                gb = ri["bytes"] / (ri["evt_ms"] * 1e-3) / 1e9
                line.setdefault("decode_batch_invariant", {})[wl] = {
                    "workload": ri["wname"] + ": each sequence's bits independent of the batch",
                    "value": round(gb, 1), "unit": "GB/s", "ms_per_step": round(ri["evt_ms"], 5),
                    "frac_hbm_peak": round(gb / HBM_PEAK_GBS, 4)}
                del ri
                torch.cuda.empty_cache()
    if args.only in (None, "config1"):
        line["decode_config1"] = bench_decode_config1(args, dev)
        if args.only == "config1":
            c1 = line["decode_config1"]
            line.update(value=c1["GB/s"], unit="GB/s", ms_per_step=c1["us_per_call"] / 1e3,
                        config={"workload": c1["workload"]})
            print(json.dumps(line))
            return 0
        torch.cuda.empty_cache()
    if args.only in (None, "pre_attention"):
        line["pre_attention"] = bench_pre_attention(args, dev)
        if args.only == "pre_attention":
            pa = line["pre_attention"]["prefill"]
            line.update(value=pa["GB/s"], unit="GB/s", ms_per_step=pa["ms_per_step"],
                        config={"workload": pa["workload"]},
                        roofline={"bound": "hbm", "achieved": pa["GB/s"], "peak": HBM_PEAK_GBS,
                                  "unit": "GB/s", "frac": pa["frac_hbm_peak"],
                                  "traffic": pa["traffic"]})
            print(json.dumps(line))
            return 0
        torch.cuda.empty_cache()
    if args.only in (None, "prefill"):
        pf = bench_prefill(args, dev)
        if args.only == "prefill":
            line.update(value=pf["value"], unit=pf["unit"], ms_per_step=pf["ms_per_step"],
                        config={"workload": pf["workload"]}, roofline=pf["roofline"])
        line["prefill"] = pf
        torch.cuda.empty_cache()
    if args.only in (None, "sampling"):
        line["sampling"] = bench_sampling(args, dev)
        torch.cuda.empty_cache()
    if args.only in (None, "e2e"):
        e2e = bench_e2e(args, dev)
        if args.only == "e2e":
            line.update(value=e2e["value"], unit=e2e["unit"],
                        ms_per_step=e2e["decode_ms_per_step"], config={"workload": e2e["workload"]})
        line["e2e"] = e2e
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
